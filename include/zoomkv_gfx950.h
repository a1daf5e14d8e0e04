/*
 * zoomkv_gfx950.h -- C ABI of libzoomkv_gfx950.so, the MI355X (gfx950)
 * implementation of ZoomKV's quantized and sparse KV-cache decode path.
 *
 * All pointers are device pointers unless stated otherwise; all sizes are in
 * elements; strides are in elements of the pointed-to type.  Every entry point
 * launches asynchronously on the given HIP stream (0 = the legacy default
 * stream), never synchronises the host, never allocates device memory, and
 * returns 0 on success or a ZKV_E* code; zkv_last_error() then returns the
 * message of the last failure on the calling thread.
 *
 * dtypes: bf16 and fp16 values are passed as uint16_t bit patterns.
 *
 * Reference citations use Z/ = runtime/zoomkv_urania_runtime_20261011/ and
 * S = Z/cache_hub/polar_cache_quest_density_single_layer_kivi.py of
 * amy-77/zoomkv_revision.
 */
#ifndef ZOOMKV_GFX950_H_
#define ZOOMKV_GFX950_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* zkv_stream_t; /* == hipStream_t */

#define ZKV_OK 0
#define ZKV_EINVAL 1   /* bad shape / dtype / argument (TORCH_CHECK in the reference) */
#define ZKV_ELAUNCH 2  /* kernel launch failed (cudaGetLastError in the reference) */
#define ZKV_ESPACE 3   /* caller-provided workspace / output too small */

/* Message of the last failure on this thread ("" if none). */
const char* zkv_last_error(void);
/* Library / format version string. */
const char* zkv_version(void);

/* ------------------------------------------------------------------------
 * Format R: the reference's chunk-major KIVI K cache.
 *
 * zkv_chunk_encode replaces the full-chunk branch of
 * _compute_and_store_chunk_minmax + _kivi_pack_chunks (S:2119-2143,
 * S:1965-2020), which are pure torch in the reference.  For each of the
 * n_chunks chunks of g consecutive tokens of `keys` it writes, at chunk index
 * chunk_start + c: per-channel min / max / mean (bf16), valid = 1, and the
 * 4-bit codes in the chunk-major layout [.., n_chunks_max, 16, g] int32.
 *
 * keys      bf16 [bs, kv, n_tok >= n_chunks*g, 128] with strides
 *           (k_sb, k_sh, k_st), channel stride 1
 * chunk_min/chunk_max/chunk_centroid  bf16 [bs, kv, n_chunks_max, 128] contiguous
 * chunk_valid  uint8 (bool) [bs, kv, n_chunks_max]
 * packed_K  int32 [bs, kv, n_chunks_max, 16, g] contiguous
 * g in {8, 16, 32}.
 * ------------------------------------------------------------------------ */
int zkv_chunk_encode(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st,
                     int bs, int kv, int g, int n_chunks, int chunk_start, int n_chunks_max,
                     uint16_t* chunk_min, uint16_t* chunk_max, uint16_t* chunk_centroid,
                     uint8_t* chunk_valid, int32_t* packed_K, zkv_stream_t stream);

/* ------------------------------------------------------------------------
 * Format Q: 4-bit K (per channel, groups of 32 tokens) and V (per token,
 * groups of 32 channels) with fp16 scale / zero.  No reference counterpart
 * (the reference keeps V in bf16, S:561-571); the code ladder is the
 * reference's (S:2003-2009).  The cache is `groups` int32
 * [bs, kv, G_cap, 1280]: one contiguous 5120-byte record per 32-token group of
 * one KV head, holding
 *   words [0, 512)      K codes: word m*256 + l*4 + s, l = 16g + c: the
 *           nibbles of channels 8p..8p+7 (p = 4s + g) of token 32G + 16m + c
 *   words [512, 1024)   V codes: word (j/4)*256 + l*4 + j%4, l = 16r + c:
 *           channel 32(j/2) + 2c + j%2, nibble k = token 32G + TAU[r][2(k%4) + k/4]
 *   words [1024, 1152)  K scale / zero, fp16 [16, 2, 8] (p, scale|zero, slot):
 *           channel 8p + (0,4,1,5,2,6,3,7)[slot]
 *   words [1152, 1280)  V scale / zero, fp16 [4, 4, 2, 8] (channel group, r,
 *           scale|zero, e): token 32G + TAU[r][e], TAU[r] = (4r..4r+3, 16+4r..16+4r+3)
 * The code / metadata order is the MFMA operand order of the decode kernel,
 * and one record is one contiguous 5 KiB load.
 *
 * zkv_kivi4_pack quantizes tokens [32*g0, 32*(g0+n_groups)) of the cache
 * from src tokens [0, 32*n_groups) of k / v.
 * k, v     bf16 [bs, kv, n_tok, 128], strides (sb, sh, st), channel stride 1
 * range_status  (nullable) device uint32 the kernel ORs ZKV_RANGE_* bits into
 *          when a group's fp16 scale / zero cannot hold its values: ZKV_RANGE_K
 *          / ZKV_RANGE_V for a scale or zero beyond fp16 (|value| or range >
 *          65504), ZKV_RANGE_V_SCALE for a V scale above 2048 (a V range above
 *          30720 inside one 32-channel group, beyond the decode kernel's fp16
 *          V operand).  The caller clears it first; the packed records of a
 *          flagged call must not be attended.
 * ------------------------------------------------------------------------ */
#define ZKV_RANGE_K 1u
#define ZKV_RANGE_V 2u
#define ZKV_RANGE_V_SCALE 4u
int zkv_kivi4_pack(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                   const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                   int bs, int kv, int n_groups, int g0, int g_cap, int32_t* groups,
                   uint32_t* range_status, zkv_stream_t stream);

/* Prefill in one launch: zkv_kivi4_pack of tokens [0, 32*n_groups) of k / v
 * into groups [g0, g0 + n_groups), and tokens [32*n_groups, 32*n_groups +
 * res_len) copied as bf16 rows into rows [res_row0, res_row0 + res_len) of the
 * residual windows k_res / v_res (contiguous bf16 [bs, kv, r_cap, 128], the
 * decode attention's layout).  With res_len > 0 the k rows and the windows
 * must be 16-byte aligned.  No separate counterpart in the reference: its
 * prefill quantizes the full chunks and keeps the newest tokens as bf16 in
 * two steps (S:1379-1512). */
int zkv_kivi4_prefill(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                      const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                      int bs, int kv, int n_groups, int g0, int g_cap, int32_t* groups,
                      uint32_t* range_status, uint16_t* k_res, uint16_t* v_res, int r_cap,
                      int res_row0, int res_len, zkv_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused 4-bit decode attention over a Format Q cache plus a bf16 residual
 * window: out = softmax(q K^T * sm_scale) V, causal = False, with GQA
 * (hq / kv query heads per KV head, hq / kv <= 16, consecutive query heads
 * share a KV head).  Replaces flash_attn_with_kvcache_compat(q, k, v,
 * causal=False) (Z/attn_hub/flash_attn_compat.py:44-100, called at
 * S:1742-1747) for a quantized cache.
 *
 * q        bf16 [bs, hq, 128] with strides (q_sb, q_sh), channel stride 1
 * k_res, v_res  bf16 [bs, kv, R_cap, 128] contiguous; tokens [0, res_len) used
 * n_groups groups of the Format Q cache are attended (all bs share lengths)
 * out      [bs, hq, 128] contiguous, bf16 (out_f32 == 0) or fp32 (out_f32 != 0)
 * lse      optional (NULL to skip) fp32 [bs, hq]: natural-log LSE of the
 *          scaled scores, the layout of flash-attn's softmax_lse
 * n_splits context splits per (b, kv head); 0 = automatic
 * workspace device scratch of zkv_kivi4_attention_workspace_size() bytes
 *          (split partials, then one 8-byte arrival slot per (b, kv) when
 *          the plan has more than one split); no zeroing needed: each
 *          launch's slot value (epoch << 8 | count) has bit 63 set and a
 *          random per-process epoch base, so no non-negative int64 a reused
 *          buffer holds can read as a live slot, and other bytes match with
 *          probability 2^-55; calls that overlap on one workspace race.
 * With more than one split, the splits are merged inside the one launch by
 * the workgroup that completes each (b, kv) (same bits as the partial + merge
 * pair below); environment ZKV_SPLIT_MERGE=kernel selects a separate merge
 * launch instead, ZKV_SPLIT_MERGE=fence an in-launch merge ordered by
 * agent-scope fences (slower, same bits).
 * ------------------------------------------------------------------------ */
size_t zkv_kivi4_attention_workspace_size(int bs, int hq, int kv, int n_groups, int res_len,
                                          int n_splits);
int zkv_kivi4_decode_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                               const int32_t* groups, int g_cap,
                               const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                               int bs, int hq, int kv, int n_groups, int res_len,
                               float sm_scale, void* out, int out_f32, float* lse, int n_splits,
                               void* workspace, size_t workspace_bytes, zkv_stream_t stream);

/* zkv_kivi4_decode_attention without a workspace argument, allocating
 * nothing: no counterpart in the reference.  It is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The split partials live in a static
 * device array of ZKV_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends; a call whose split plan needs more (bs * hq * splits * 520 bytes,
 * plus bs * kv * 8 with more than one split) fails with ZKV_ESPACE.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (concurrent streams or threads) race.
 * Results equal zkv_kivi4_decode_attention's for the same arguments. */
#define ZKV_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int zkv_kivi4_decode_attention_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                       const int32_t* groups, int g_cap,
                                       const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                       int bs, int hq, int kv, int n_groups, int res_len,
                                       float sm_scale, void* out, int out_f32, float* lse,
                                       int n_splits, zkv_stream_t stream);

/* Stage 1 of zkv_kivi4_decode_attention: per context split, the unnormalised
 * partial output o, the running max m (log2 units, sm_scale*log2(e) folded in)
 * and the softmax denominator l of every (b, query head), written to
 * `workspace` as o fp32 [bs, kv, S, hq/kv, 128]
 * followed by (m, l) fp32 [bs, kv, S, hq/kv, 2].  *n_splits_used (host pointer, may be NULL) receives
 * the resolved split count S. */
int zkv_kivi4_attention_partial(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                const int32_t* groups, int g_cap,
                                const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                int bs, int hq, int kv, int n_groups, int res_len,
                                float sm_scale, int n_splits, void* workspace,
                                size_t workspace_bytes, int* n_splits_used, zkv_stream_t stream);

/* Stage 2: merge the n_splits partials of every (b, query head) with the LSE
 * rule of lse_merge_torch (Z/cache_hub/lse_merge/lse_merge.py:79-119):
 * out = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s.  out as in
 * zkv_kivi4_decode_attention. */
int zkv_attention_merge(const void* workspace, int bs, int hq, int kv, int n_splits,
                        void* out, int out_f32, zkv_stream_t stream);

/* ------------------------------------------------------------------------
 * Page scoring and selection
 * ------------------------------------------------------------------------ */

/* Quest upper bound score[b,h,c] = sum_d max(q_d*mn_d, q_d*mx_d) for chunks
 * c < n_chunks; invalid chunks (valid[b,h,c] == 0) score -inf.  Replaces
 * quest_kernel.quest_chunk_score(q, chunk_min, chunk_max, scores, n_chunks,
 * valid) (Z/cache_hub/quest/quest_chunk_score.cu:106-154, :536-540).
 * q bf16 [bs, kv, 128]; chunk_min/max [bs, kv, n_chunks_max, 128] bf16
 * (meta_fp16 == 0) or fp16 (meta_fp16 != 0); scores fp32 [bs, kv, n_chunks];
 * valid uint8 [bs, kv, n_chunks_max] or NULL; all contiguous. */
int zkv_quest_chunk_score(const uint16_t* q, const uint16_t* chunk_min, const uint16_t* chunk_max,
                          int meta_fp16, float* scores, int bs, int kv, int n_chunks,
                          int n_chunks_max, const uint8_t* valid, zkv_stream_t stream);

/* zkv_quest_chunk_score with its query formed in the same launch: the GQA-mean
 * query raw_q[b, h] = bf16(sum_i q[b, h*g + i] / g), g = hq / kv, of
 * zkv_gqa_mean_query is scored and also written to raw_q (bf16 [bs, kv, 128],
 * contiguous, for the later stages).  It fuses the two steps of S:1621-1626
 * and S:2223 (the torch mean, then quest_chunk_score,
 * Z/cache_hub/quest/quest_chunk_score.cu:106-154); no counterpart of its own in
 * the reference.  q bf16 [bs, hq, 128] at element strides (q_sb, q_sh),
 * multiples of 4; n_chunks >= 1; the other arguments as zkv_quest_chunk_score. */
int zkv_quest_chunk_score_gqa(const uint16_t* q, int64_t q_sb, int64_t q_sh, int hq, uint16_t* raw_q,
                              const uint16_t* chunk_min, const uint16_t* chunk_max, int meta_fp16,
                              float* scores, int bs, int kv, int n_chunks, int n_chunks_max,
                              const uint8_t* valid, zkv_stream_t stream);

/* zkv_quest_chunk_score_gqa and the row's exact top-k in one launch: the
 * float_topk_3d call of S:2168-2190 (Z/cache_hub/float_topk/float_topk.cu:51-271
 * semantics, as zkv_topk) on the scores just formed.  No counterpart of its
 * own in the reference.  out int64 [bs, kv, >= k] at row stride out_stride:
 * the k chunk indices of the largest scores in increasing index order (ties to
 * the lower index); rows with n_chunks <= k get 0 .. n_chunks - 1, then -1.
 * scores is still written (fp32 [bs, kv, n_chunks]).  1 <= n_chunks <= 4096.
 * slots: >= 4 * bs * kv bytes of arrival counters, zeroed once before the
 * first call and left zero by every call; calls that overlap on one slots
 * buffer race. */
int zkv_quest_chunk_topk_gqa(const uint16_t* q, int64_t q_sb, int64_t q_sh, int hq, uint16_t* raw_q,
                             const uint16_t* chunk_min, const uint16_t* chunk_max, int meta_fp16,
                             float* scores, int bs, int kv, int n_chunks, int n_chunks_max,
                             const uint8_t* valid, int k, int64_t* out, int64_t out_stride,
                             void* slots, size_t slots_bytes, zkv_stream_t stream);

/* Exact top-k of each of `rows` rows of L fp32 scores (row i at
 * scores + i*in_stride): out[i, 0..k) = the indices (or lut[i, index] when lut
 * != NULL) of the k largest scores, ties by lowest index, in increasing index
 * order; when L <= k, indices 0..L-1 then `sentinel`.  out[i, k..k+sk_count)
 * = skipped[i, 0..sk_count).  Replaces float_topk_3d (Z/cache_hub/topk/
 * float_topk.cu:280-346, sentinel -1) and float_topk_gather_concat_3d
 * (Z/cache_hub/topk/float_topk_gather_concat.cu:305-375, sentinel 0), whose
 * outputs are the same sets in unspecified order. */
int zkv_topk(const float* scores, int64_t in_stride, int rows, int L, int k, int64_t* out,
             int64_t out_stride, const int64_t* lut, int64_t lut_stride, const int64_t* skipped,
             int64_t sk_stride, int sk_count, int64_t sentinel, zkv_stream_t stream);

/* CDS density out[b,h,j] = centroid[b,h,chunk_ids[b,h,j]] . raw_q[b,h] (fp32,
 * 128-thread tree order), -1e30 for out-of-range ids.  Replaces
 * partial_chunk_density_scores (Z/cache_hub/rerank/rerank_topk.cu:627-689).
 * Strides are per batch / head (/ chunk) in elements; last dims contiguous. */
int zkv_chunk_density_scores(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                             const uint16_t* centroids, int64_t c_sb, int64_t c_sh, int64_t c_sc,
                             const uint16_t* raw_q, int64_t q_sb, int64_t q_sh, float* out,
                             int64_t o_sb, int64_t o_sh, int bs, int kv, int nk, int n_chunks,
                             zkv_stream_t stream);

/* mask[r, :] = 0 then mask[r, positions[r, j]] = 1 for in-range positions;
 * positions int64 [rows, n_dense], mask uint8 [rows, nk], contiguous.
 * Replaces mask_from_topk (Z/cache_hub/rerank/rerank_topk.cu:926-998). */
int zkv_dense_mask_from_topk(const int64_t* positions, uint8_t* mask, int rows, int n_dense, int nk,
                             zkv_stream_t stream);

/* The top k of each row (zkv_topk's selection, no lut / skipped tail) with
 * the dense mask written in the same launch: mask[r, :L] = 0, then 1 at every
 * selected index (mask uint8 [rows, >= L], row stride mask_stride).  It is
 * float_topk_3d followed by dense_mask_from_topk in one pass: no counterpart
 * of its own in the reference; it fuses the two calls of S:2360-2369
 * (float_topk.cu:51-346 + rerank_topk.cu:926-998). */
int zkv_topk_dense_mask(const float* scores, int64_t in_stride, int rows, int L, int k, int64_t* out,
                        int64_t out_stride, uint8_t* mask, int64_t mask_stride, zkv_stream_t stream);

/* GQA-mean query raw_q[b, h] = bf16(sum_i q[b, h*g + i] / g), g = hq / kv
 * (the torch mean of S:1621-1626).  q bf16 [bs, hq, 128] with strides
 * (q_sb, q_sh); out bf16 [bs, kv, 128] contiguous. */
int zkv_gqa_mean_query(const uint16_t* q, int64_t q_sb, int64_t q_sh, int bs, int hq, int kv,
                       uint16_t* out, zkv_stream_t stream);

/* KIVI stage-2 scorer (Format R): per selected chunk, bf16 dequant + bf16
 * products + fp32 sum, per-chunk descending bitonic sort, keep dense_topk /
 * sparse_topk, (-1e30, 0) elsewhere.  Replaces
 * partial_chunk_kivi_qk_dense_sparse (Z/cache_hub/kivi/kivi_qk_dot.cu:325-460):
 * chunk_ids int64 / dense_mask uint8 [bs, kv, nk]; packed_K int32 [bs, kv,
 * n_packed, 16, group_size] (chunk stride 16*group_size); chunk_min/max bf16
 * [bs, kv, n_chunks_max, 128] (chunk stride 128); raw_q bf16 [bs, kv, 128];
 * out_scores fp32 / out_indices int64 [bs, kv, >= nk*group_size].  Strides
 * are per batch / head in elements; group_size in {8, 16}. */
int zkv_kivi_qk_dense_sparse(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                             const uint8_t* dense_mask, int64_t dm_sb, int64_t dm_sh,
                             const int32_t* packed_K, int64_t pk_sb, int64_t pk_sh, int n_packed,
                             const uint16_t* chunk_min, const uint16_t* chunk_max, int64_t cm_sb,
                             int64_t cm_sh, int n_chunks_max, const uint16_t* raw_q, int64_t q_sb,
                             int64_t q_sh, int dense_topk, int sparse_topk, int group_size,
                             float* out_scores, int64_t* out_indices, int64_t o_sb, int64_t o_sh,
                             int bs, int kv, int nk, zkv_stream_t stream);

/* zkv_kivi_qk_dense_sparse with a compact output: slot i's lanes 0 ..
 * out_width-1 at i*out_width (max(dense_topk, sparse_topk) <= out_width <=
 * group_size; out_scores / out_indices [bs, kv, >= nk*out_width]).  No
 * counterpart in the reference: polar_cache.compute uses it so the global
 * top-k reads only the kept lanes (the entries it drops are the (-1e30, 0)
 * fillers, in the same relative order otherwise, so a top-k that takes no
 * filler selects the same tokens). */
int zkv_kivi_qk_dense_sparse_compact(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                                     const uint8_t* dense_mask, int64_t dm_sb, int64_t dm_sh,
                                     const int32_t* packed_K, int64_t pk_sb, int64_t pk_sh, int n_packed,
                                     const uint16_t* chunk_min, const uint16_t* chunk_max, int64_t cm_sb,
                                     int64_t cm_sh, int n_chunks_max, const uint16_t* raw_q, int64_t q_sb,
                                     int64_t q_sh, int dense_topk, int sparse_topk, int group_size,
                                     int out_width, float* out_scores, int64_t* out_indices, int64_t o_sb,
                                     int64_t o_sh, int bs, int kv, int nk, zkv_stream_t stream);

/* Quest page metadata of a paged cache in fp16: per (b, kv, page, channel)
 * min (rounded toward -inf) and max (toward +inf) of bf16 keys [bs, kv, n_tok,
 * 128] at element strides (k_sb, k_sh, k_st), pages of page_size tokens ->
 * page_min / page_max fp16 [bs, kv, n_pages_max, 128].  fp16 counterpart of
 * the chunk amin / amax of _compute_and_store_chunk_minmax (S:2025-2157) feeding
 * quest_chunk_score (Z/cache_hub/quest/quest_chunk_score.cu:31-154). */
int zkv_page_minmax_f16(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st, int bs,
                        int kv, int page_size, int n_pages, int n_pages_max, uint16_t* page_min,
                        uint16_t* page_max, zkv_stream_t stream);

/* Page-sparse decode attention: as zkv_kivi4_decode_attention, but the
 * quantized context of (b, kv) is the list pages int64 [bs, kv, n_sel]
 * (element strides pg_sb, pg_sh) of 16-token pages (page P = tokens 16P ..
 * 16P+15, i.e. half P & 1 of Format Q group P >> 1), followed by the bf16
 * residual window.  Equals attention over the gathered tokens of the listed
 * pages (a page listed twice counts twice; ids outside [0, 2 * n_groups) are
 * skipped); any two listed pages share one 32-token tile, in list order.
 * Counterpart of the Quest select -> gather -> flash_attn_with_kvcache
 * sequence (S:2195-2240, S:1723-1772). */
size_t zkv_kivi4_sparse_attention_workspace_size(int bs, int hq, int kv, int n_sel, int res_len,
                                                 int n_splits);
int zkv_kivi4_sparse_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh, const int32_t* groups,
                               int g_cap, const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                               int bs, int hq, int kv, int n_groups, int res_len, const int64_t* pages,
                               int64_t pg_sb, int64_t pg_sh, int n_sel, float sm_scale, void* out,
                               int out_f32, float* lse, int n_splits, void* workspace,
                               size_t workspace_bytes, zkv_stream_t stream);

/* Token-list decode attention over a Format Q cache plus bf16 rows, one
 * launch: the 4-bit counterpart of the reference's gather of sink + local +
 * selected tokens and flash_attn_with_kvcache(causal=False) (S:1723-1772;
 * the list is the output of float_topk_gather_concat_3d,
 * Z/cache_hub/topk/float_topk_gather_concat_ops.py:77-125).
 * toks     int64 [bs, kv, n_tok] at element strides (tk_sb, tk_sh), n_tok <=
 *          1024; per (b, kv), in any order: an id in [0, 32 n_groups) is that
 *          token of the Format Q records `groups` (int32 [bs, kv, g_cap,
 *          1280]); an id in [32 n_groups, 32 n_groups + n_tail) is the bf16
 *          row tail_row0 + (id - 32 n_groups) of k / v; other ids are
 *          skipped; a repeated id is attended again (as a repeated gathered
 *          row would be)
 * k, v     bf16 rows [bs, kv, n_rows, 128] at element strides (sb, sh, st),
 *          rows 16-byte aligned; rows [near_row0, near_row0 + near_len) are
 *          attended after the list
 * out, lse as zkv_kivi4_decode_attention; workspace of
 *          zkv_kivi4_token_attention_workspace_size() bytes (same layout and
 *          rules).
 * The workgroups sort each list in LDS, so the result does not depend on the
 * list's order beyond rounding of the online softmax (sorted order is the
 * computation order). */
size_t zkv_kivi4_token_attention_workspace_size(int bs, int hq, int kv, int n_tok, int near_len, int n_splits);
int zkv_kivi4_token_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh, const int32_t* groups, int g_cap,
                              int n_groups, const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                              const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int n_rows,
                              const int64_t* toks, int64_t tk_sb, int64_t tk_sh, int n_tok, int tail_row0,
                              int n_tail, int near_row0, int near_len, int bs, int hq, int kv, float sm_scale,
                              void* out, int out_f32, float* lse, int n_splits, void* workspace,
                              size_t workspace_bytes, zkv_stream_t stream);

/* Decode attention over bf16 K / V caches k, v [bs, n, kv, 128] at element
 * strides (sb = batch, st = token, sh = head; rows 16-byte aligned), causal
 * off, GQA hq = kv * gqa: the flash_attn_with_kvcache call of
 * flash_attn_with_kvcache_compat (Z/attn_hub/flash_attn_compat.py:44-100; call
 * sites S:1742-1747, S:1767-1772).  out bf16 or fp32 [bs, hq, 128]; lse
 * (optional, NULL to skip) fp32 [bs, hq] natural-log LSE of the scaled
 * scores, the layout of flash-attn's softmax_lse. */
size_t zkv_bf16_attention_workspace_size(int bs, int hq, int kv, int n, int n_splits);
int zkv_bf16_decode_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                              int64_t k_sb, int64_t k_st, int64_t k_sh, const uint16_t* v,
                              int64_t v_sb, int64_t v_st, int64_t v_sh, int bs, int hq, int kv, int n,
                              float sm_scale, void* out, int out_f32, float* lse, int n_splits,
                              void* workspace, size_t workspace_bytes, zkv_stream_t stream);

/* bf16 decode attention over a gathered token list without materialising the
 * gather: token t < n_idx of (b, kv) is row idx[b*idx_sb + kv*idx_sh + t] of
 * k / v (rows outside [0, n_rows) are masked out), and tokens n_idx ..
 * n_idx + tail_len - 1 are the contiguous rows tail_start ..  Replaces the
 * h2d_gather_kv / torch.gather -> torch.cat -> flash_attn_with_kvcache
 * sequence of compute() (S:1723-1747 offload, S:1752-1772 on-GPU).  Sizes
 * and workspace as zkv_bf16_decode_attention with n = n_idx + tail_len. */
int zkv_bf16_gather_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                              int64_t k_sb, int64_t k_st, int64_t k_sh, const uint16_t* v,
                              int64_t v_sb, int64_t v_st, int64_t v_sh, int n_rows, const int64_t* idx,
                              int64_t idx_sb, int64_t idx_sh, int n_idx, int tail_start, int tail_len,
                              int bs, int hq, int kv, float sm_scale, void* out, int out_f32, float* lse,
                              int n_splits, void* workspace, size_t workspace_bytes, zkv_stream_t stream);

/* LSE merge of two attention outputs [bs, 1, heads, dim] (contiguous, dtype 0
 * bf16 / 1 fp16 / 2 fp32) with fp32 natural-log LSEs [bs, heads]:
 * lse_merge_torch / lse_merge_cuda (Z/cache_hub/lse_merge/lse_merge.py:79-149). */
int zkv_lse_merge(const void* out_a, const float* lse_a, const void* out_b, const float* lse_b,
                  void* out, int dtype, int bs, int heads, int dim, zkv_stream_t stream);

/* ---- RaBitQ 1-bit sign codes -------------------------------------------------
 * The reference's RaBitQ keys are 4-bit sign + magnitude codes (ParisKV,
 * PC:1130-1195 batch_encode; rerank_rabitq_ref, Z/cache_hub/rerank/rerank.py:205-274).
 * This path keeps 1 bit per dimension of the SRHT-rotated vector, 16 bytes per
 * 128-dim key, plus fp16 (norm, correction) factors.
 *
 * Encode n fp16 vectors (rows of 128 at row_stride elements, 16-byte aligned)
 * with the +-1 SRHT sign vector signs (fp32 [128], device):
 *   codes uint8 [n, 16] (bit b of byte j = sign of rotated dim 8j + b),
 *   factors fp16 [n, 2] = (||x||, ||y|| sqrt(128) / sum|y|).
 * Replaces batch_encode (PC:1130-1195) / _encode_query_blocks (PC:1108-1124). */
int zkv_rabitq_encode(const uint16_t* x, int64_t row_stride, int64_t n, const float* signs,
                      uint8_t* codes, uint16_t* factors, zkv_stream_t stream);

/* Estimate matrix out fp32 [pools, queries, n]:
 *   ((nk*ck) * (nq*cq)) * (128 - 2 popc(xq ^ xk)) / 128
 * (the sign-sign identity of Z/cache_hub/rerank/coarse_2bit_score.cu:12-16 with
 * the RaBitQ corrections; counterpart of approx_scores in rerank.py:255-264).
 * codes_q [pools, queries, 16], codes_k [pools, n, 16], factors likewise. */
int zkv_rabitq_estimate(const uint8_t* codes_q, const uint16_t* factors_q, const uint8_t* codes_k,
                        const uint16_t* factors_k, int pools, int queries, int64_t n, float* out,
                        zkv_stream_t stream);

/* Workspace bytes zkv_rabitq_search needs (0 for invalid sizes). */
size_t zkv_rabitq_search_workspace_size(int pools, int queries, int64_t n, int topk);

/* Search: encode the fp16 queries q [pools, queries, 128], take the top-topk
 * keys by estimate (ties to the lower index) into cand_idx [pools, queries, topk]
 * (increasing index order), rerank them by the exact fp32 dot with the fp16
 * keys (keys + pool * k_pool_stride + index * k_row_stride) and write them in
 * (score desc, index asc) order to final_idx / final_scores.  Counterpart of
 * rerank_rabitq_ref's coarse filter -> score -> top-k
 * (Z/cache_hub/rerank/rerank.py:205-274).  Limits: topk <= min(n, 1024) and
 * ceil(n / 8192) * topk <= 8192. */
int zkv_rabitq_search(const uint16_t* q, const uint16_t* keys, int64_t k_pool_stride,
                      int64_t k_row_stride, const uint8_t* codes, const uint16_t* factors,
                      const float* signs, int pools, int queries, int64_t n, int topk,
                      int64_t* cand_idx, int64_t* final_idx, float* final_scores, void* workspace,
                      size_t workspace_bytes, zkv_stream_t stream);

/* ---- ParisKV 4-bit RaBitQ codes (1-bit sign + 3-bit magnitude) ---------------
 * The reference's production RaBitQ format.  Per key (bf16, 128 dims, rows
 * 16-byte aligned) and per block b of 8 rotated dimensions:
 *   code   uint8  (bit j = sign of dim 8b + j),       layout [..., 16, seq]
 *   packed uint32 (nibble j = sign << 3 | magnitude), layout [..., 16, seq]
 *          (4 bytes, byte k = v[2k] | v[2k+1] << 4)
 *   weight bf16   (r_b / alpha_b) * ||k||,            layout [..., 16, seq]
 * Strides are per (batch, head, block) in elements (uint32 units for packed);
 * the token stride is 1.  signs: the SRHT +-1 vector, bf16 [128]; the
 * magnitude levels: bf16 thresholds [7] and centers [8] (PC:266-270).
 * Every value is rounded to bf16 where the reference's torch ops round. */

/* Encode keys [bs, kv, n, 128] (element strides) into token positions
 * t0 .. t0 + n - 1 of the code / packed / weight arrays.
 * Replaces batch_encode (Z/cache_hub/polar_cache.py:1130-1195) with
 * _pack_4bit_codes (:1067-1084). */
int zkv_rabitq4_encode(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st, int bs, int kv,
                       int n, const uint16_t* signs, const uint16_t* mag_thresholds,
                       const uint16_t* mag_centers, uint8_t* code, int64_t c_sb, int64_t c_sh, int64_t c_sB,
                       uint8_t* packed, int64_t p_sb, int64_t p_sh, int64_t p_sB, uint16_t* weight,
                       int64_t w_sb, int64_t w_sh, int64_t w_sB, int t0, zkv_stream_t stream);

/* Query blocks: q bf16 rows (row stride q_sr elements) -> q_blocks bf16
 * [rows, 16, 8] (the SRHT-rotated unit query), q_norm bf16 [rows].
 * Replaces _encode_query_blocks (Z/cache_hub/polar_cache.py:1108-1124). */
int zkv_rabitq4_encode_query(const uint16_t* q, int64_t q_sr, int rows, const uint16_t* signs,
                             uint16_t* q_blocks, uint16_t* q_norm, zkv_stream_t stream);

/* 4-bit approximate inner products of the candidates cand int64 [bs, kv, C]
 * (strides cd_sb, cd_sh; unit stride along C) with the query blocks
 * [bs * kv, 16, 8] and q_norm [bs * kv]: per block the sequential bf16 sum of
 * bf16(+-center[t] * q), times the block weight, summed over the blocks in
 * bf16, times ||q||.  packed: strides p_sb, p_sh, p_sB, p_st in uint32 units;
 * weight: w_sb, w_sh, w_sB (unit token stride).  Outputs (any may be null,
 * not both scores): scores bf16 [bs, kv, C], scores_f32 (the same values),
 * v4b bf16 [bs, kv, 16, C, 8] (the decoded values).  A candidate outside
 * [0, kv_len) scores -inf.
 * workspace (optional, device, 16-byte aligned, at least
 * zkv_rabitq4_rerank_workspace_size(bs, kv, kv_len) bytes) enables the
 * streamed path for dense candidate lists (C >= kv_len / 16; scores only,
 * no v4b): its first F = ceil(bs * kv * ceil(kv_len / 1024) * 1024 / 256) * 256
 * bytes are token flags that must be all zero when the call starts and that
 * a successful call leaves all zero (a zero-filled buffer qualifies, and
 * stays qualified for calls of the same bs, kv and kv_len; zero its first F
 * bytes again before a call of another shape).  Calls that overlap on one
 * workspace race.  With a null workspace every call takes the direct path;
 * both give the same scores.
 * Replaces partial_rerank_cuda / partial_rerank_scores_cuda
 * (Z/cache_hub/rerank/rerank.py:352-440; kernel rerank.cu:52-143). */
int zkv_rabitq4_rerank(const int64_t* cand, int64_t cd_sb, int64_t cd_sh, int bs, int kv, int C,
                       const uint8_t* packed, int64_t p_sb, int64_t p_sh, int64_t p_sB, int64_t p_st,
                       int kv_len, const uint16_t* weight, int64_t w_sb, int64_t w_sh, int64_t w_sB,
                       const uint16_t* q_blocks, const uint16_t* q_norm, const uint16_t* mag_centers,
                       uint16_t* scores, float* scores_f32, uint16_t* v4b, void* workspace,
                       size_t workspace_bytes, zkv_stream_t stream);

/* Bytes of the rerank's streamed-path workspace: the token flags (above),
 * then one fp32 score per token.  0 for an invalid shape.
 * No reference counterpart (the reference's rerank has no workspace). */
size_t zkv_rabitq4_rerank_workspace_size(int bs, int kv, int kv_len);

/* ---------------------------------------------------------------------------
 * Host-to-device row gather (the UVA gather of
 * Z/cache_hub/gather_trans/trans_h2d.cu:43-188, trans_h2d.py:65-166).
 * src_k / src_v are pinned, mapped host buffers of bf16 rows
 * [bs, heads, src_len, 128] (the C ABI takes their host pointers and fails
 * with ZKV_EINVAL when they have no device alias); every other pointer is
 * device memory.  An index outside [0, src_len) leaves its destination row
 * untouched.
 * ------------------------------------------------------------------------- */

/* dst[b, h, slot] = src[b, h, indices[b, h, slot]] for slot < topk; dst is
 * [bs, heads, dst_len, 128], indices [bs, heads, topk] int64 (contiguous).
 * Replaces h2d_gather_kv (trans_h2d.py:65-103 -> trans_h2d.cu:84-188). */
int zkv_h2d_gather_kv(const void* src_k, const void* src_v, int bs, int heads, int src_len,
                      const int64_t* indices, int topk, void* dst_k, void* dst_v, int dst_len,
                      zkv_stream_t stream);

/* Variable-K gather into a packed varlen buffer [total_k, 128]: segment
 * vh = b * kv_heads + h takes indices_packed[cu_seqlens_topk[vh] ..
 * cu_seqlens_topk[vh + 1]) into rows cu_seqlens_k[vh] + sl_end + slot
 * (the first sl_end rows of each segment are the caller's).  global_k bounds
 * every segment's length.  Replaces h2d_gather_kv_packed
 * (trans_h2d.py:106-166 -> trans_h2d.cu:229-333). */
int zkv_h2d_gather_kv_packed(const void* src_k, const void* src_v, int bs, int kv_heads, int src_len,
                             void* dst_k_packed, void* dst_v_packed, int64_t total_k,
                             const int64_t* indices_packed, int64_t total_topk,
                             const int32_t* cu_seqlens_topk, const int32_t* cu_seqlens_k, int sl_end,
                             int global_k, zkv_stream_t stream);

/* Pitched copy on the stream's copy engine: rows x row_bytes from src (row
 * pitch src_pitch bytes) to dst (pitch dst_pitch), device memory or pinned
 * host memory on either side.  The offload flush's D2H move of the oldest
 * near-zone tokens into the pinned retrieval zone, one call per K / V
 * (replaces the strided dst_keys.copy_(src_keys, non_blocking=True) of
 * S:1465-1469). */
int zkv_copy_rows(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t row_bytes,
                  size_t rows, zkv_stream_t stream);

/* Pinned, device-mapped host memory of exactly `bytes` (*out; ZKV_ESPACE when
 * the host cannot pin that much) and its release: the offload retrieval zone
 * (S:561-571 allocates it with torch's pinned allocator, which rounds each
 * block up to a power of two). */
int zkv_host_alloc(size_t bytes, void** out);
int zkv_host_free(void* p);

/* ---- decode-step model layers (the C5 counterpart of layer_decode) ------ */

/* y = x . w^T for the M <= 16 rows of a decode batch: x [M, K] bf16 (row
 * stride x_ld, 16-byte aligned), w [N, K] bf16 contiguous, fp32 accumulate,
 * y [M, N] bf16 (or fp32 holding the bf16 value when out_f32), row stride
 * out_ld.  K must be a multiple of 128 and M * K * 2 bytes must fit the LDS (about 120 KiB).
 * norm_w (nullable): x is first replaced by bf16(x * rsqrt(mean(x^2) + eps) *
 * norm_w) per row.  epilogue 0: none; 1: y = bf16(residual + bf16(x . w^T))
 * (residual [M, N] bf16, row stride res_ld); 2: w rows [0, N/2) are gate and
 * [N/2, N) up, y [M, N/2] = bf16(bf16(silu(gate)) * up).
 * Replaces the torch rmsnorm + F.linear (+ residual add / silu * up) of
 * Z/model_hub/LLM.py:208-251 and the flashinfer rmsnorm / silu of
 * Z/model_hub/qwen.py:493-604. */
int zkv_decode_linear(const uint16_t* x, int64_t x_ld, int M, int K, const uint16_t* w, int N,
                      const uint16_t* norm_w, float eps, const uint16_t* residual, int64_t res_ld, void* out,
                      int64_t out_ld, int out_f32, int epilogue, zkv_stream_t stream);

/* qkv [bs, (hq + 2 hkv) * 128] bf16 (row stride qkv_ld): per-head RMSNorm of
 * the hq q heads (q_norm) and hkv k heads (k_norm), each rounded to bf16, then
 * rotate-half RoPE with the position's cos / sin rows (fp32 [64]) rounded to
 * bf16: q to q_out [bs, hq, 128]; k to k_dst + b * k_sb + h * k_sh and v
 * (copied) to v_dst + b * v_sb + h * v_sh (element strides; 128 contiguous
 * channels per row).  Replaces the q / k norms and RoPE of
 * Z/model_hub/qwen.py:493-545 and the cache append of decode_update_kv_cache
 * (S:1516-1583). */
int zkv_qk_norm_rope(const uint16_t* qkv, int64_t qkv_ld, int bs, int hq, int hkv, const uint16_t* q_norm,
                     const uint16_t* k_norm, float eps, const float* cos_row, const float* sin_row,
                     uint16_t* q_out, uint16_t* k_dst, int64_t k_sb, int64_t k_sh, uint16_t* v_dst,
                     int64_t v_sb, int64_t v_sh, zkv_stream_t stream);

/* Next-token sampling of one decode step over the top-window logits, one
 * launch: replaces the sampling chain of Z/model_hub/LLM.py:63-139
 * (temperature, top-k keeping ties at the k-th value, top-p keeping the token
 * that crosses top_p, softmax, torch.multinomial for one sample).
 * logits   fp32 [bs, vocab], row stride ld; scaled by inv_temperature (the
 *          fp32 reciprocal, as torch scales a CUDA tensor by a Python float)
 * window   k + W <= 64 (W = 16 in the decode step), with
 *          ceil(vocab / 8192) * window <= 2048: the row's `window` largest
 *          scaled logits under (value desc, index asc) are ranked; top-k and
 *          top-p act inside them
 * top_p    applied when 0 < top_p < 1
 * expo     fp32 [bs, vocab] (row stride expo_ld) of Exp(1) draws: the token is
 *          the lowest index of the largest p / expo over the window, the draw
 *          torch.multinomial(probs, 1) makes from the same Exp(1) row
 * tokens   int64 [bs]; overflow int32 [bs]: 1 when the window's last value
 *          equals the k-th (the tie group may reach past the window: the
 *          caller then draws over the whole vocabulary with the same expo)
 * workspace zkv_sample_window_workspace_size() bytes, 256-byte aligned: the
 *          per-row arrival counters (the first 4 bs bytes, rounded up to 256)
 *          must be zero before the first call with a given bs, and every call
 *          leaves them zero; the candidates follow.  Calls that overlap on
 *          one workspace race. */
size_t zkv_sample_window_workspace_size(int bs, int vocab, int window);
int zkv_sample_window(const float* logits, int64_t ld, int bs, int vocab, float inv_temperature, int top_k,
                      int window, float top_p, const float* expo, int64_t expo_ld, int64_t* tokens,
                      int32_t* overflow, void* workspace, size_t workspace_bytes, zkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZOOMKV_GFX950_H_ */
