// KIVI 4-bit quantize-and-pack kernels (gfx950).
//
// Format R (the reference's K cache): zkv_chunk_encode fuses the full-chunk
// part of _compute_and_store_chunk_minmax (S:2119-2143) -- per-channel
// amin / amax / mean over each chunk and the valid flag -- with
// _kivi_pack_chunks (S:1965-2020): the bf16 quantisation ladder of S:2003-2009
// and the chunk-major int32 packing of quant_pack.py:124-141 + S:2017.
//
// Format Q (north-star K + V cache): zkv_kivi4_pack quantizes K per channel
// over groups of 32 tokens and V per token over groups of 32 channels with the
// same ladder and stores fp16 scale / zero in the order the decode kernel's
// MFMA operands consume them (see decode_attention.hip).
//
// Both kernels are HBM-bound elementwise / small-reduction work: one
// workgroup of 128 lanes per (chunk | group, kv head, batch) reads the bf16
// keys once (coalesced 256 B rows), keeps the 4-bit codes in LDS and writes
// the packed words with coalesced dword stores.
#include "zkv_common.hpp"

namespace zkv {
namespace {

// ------------------------------- Format R ---------------------------------
template <int G>
__global__ __launch_bounds__(128) void chunk_encode_kernel(
    const uint16_t* __restrict__ keys, int64_t k_sb, int64_t k_sh, int64_t k_st, int kv,
    int chunk_start, int n_chunks_max, uint16_t* __restrict__ cmin, uint16_t* __restrict__ cmax,
    uint16_t* __restrict__ ccent, uint8_t* __restrict__ cvalid, int32_t* __restrict__ packed) {
  __shared__ uint8_t codes[G][128];
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
  const uint16_t* src = keys + b * k_sb + h * k_sh + static_cast<int64_t>(c) * G * k_st + d;
  float x[G];
#pragma unroll
  for (int t = 0; t < G; ++t) x[t] = bf16_to_f32(src[t * k_st]);
  float mn = x[0], mx = x[0], acc = 0.0f;
#pragma unroll
  for (int t = 0; t < G; ++t) {
    mn = fminf(mn, x[t]);
    mx = fmaxf(mx, x[t]);
    acc = acc + x[t];  // canonical sequential fp32 sum over the chunk's tokens
  }
  const float safe = kivi_safe(kivi_scale(mn, mx));
  if (safe < INFINITY) {
    const float r = 1.0f / safe;
#pragma unroll
    for (int t = 0; t < G; ++t) codes[t][d] = static_cast<uint8_t>(kivi_code_r(x[t], mn, safe, r));
  } else {
#pragma unroll
    for (int t = 0; t < G; ++t) codes[t][d] = static_cast<uint8_t>(kivi_code(x[t], mn, safe));
  }

  const int64_t bh = static_cast<int64_t>(b) * kv + h;
  const int64_t chunk = bh * n_chunks_max + chunk_start + c;
  cmin[chunk * 128 + d] = f32_to_bf16_bits(mn);
  cmax[chunk * 128 + d] = f32_to_bf16_bits(mx);
  ccent[chunk * 128 + d] = f32_to_bf16_bits(acc / static_cast<float>(G));
  if (d == 0) cvalid[chunk] = 1;
  __syncthreads();

  // word (p, t) = sum_j code[t][8p + j] << 4j, stored p-major: index p*G + t
  int32_t* dst = packed + chunk * (16 * G);
#pragma unroll
  for (int i = 0; i < (16 * G) / 128; ++i) {
    const int w = d + 128 * i;
    const int p = w / G, t = w % G;
    const uint64_t cb = *reinterpret_cast<const uint64_t*>(&codes[t][8 * p]);
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) word |= static_cast<uint32_t>((cb >> (8 * j)) & 0xF) << (4 * j);
    dst[w] = static_cast<int32_t>(word);
  }
}

// ------------------------------- Format Q ---------------------------------
// One 32-token group of one KV head is a 5120-byte record (int32 words):
//   [0, 512) K code words (half m = tokens 16m .. 16m + 15 at m*256),
//   [512, 1024) V code words (half m at 512 + m*256),
//   [1024, 1152) K scale/zero (fp16 pairs, shared by both halves),
//   [1152, 1280) V scale/zero (half m at 1152 + m*64).
// A 16-token page therefore reads 2816 of the 5120 bytes.
constexpr int kRecordWords = 1280;
// k_meta slot s of dim-block p holds channel 8p + KSLOT[s]; the inverse map of
// channel 8p + j is slot 2*(j % 4) + j / 4.

// fp16 bit pattern h is +-inf or NaN
__device__ __forceinline__ bool f16_nonfinite(uint16_t h) { return (h & 0x7C00u) == 0x7C00u; }
constexpr uint16_t kF16VScaleMax = 0x6800u;  // 2048.0: the decode kernel's V-scale limit

// The bf16 residual rows of a prefill (zkv_kivi4_prefill): tokens
// [32 n_groups, 32 n_groups + res_len) of k / v go to rows [res_row0, ..) of
// the contiguous [bs, kv, r_cap, 128] residual windows.  The pack launch runs
// them as extra workgroups (blockIdx.x >= n_groups), 32 tokens each, so a
// prefill is one launch.
struct ResidualCopy {
  uint16_t* k_res;
  uint16_t* v_res;
  int r_cap, res_row0, res_len, n_groups;
};

// 32 tokens x 256 bytes of K and of V: 16-byte chunks, 4 per thread per tensor.
__device__ __forceinline__ void copy_residual_rows(const uint16_t* __restrict__ k, int64_t k_sb, int64_t k_sh,
                                                   int64_t k_st, const uint16_t* __restrict__ v, int64_t v_sb,
                                                   int64_t v_sh, int64_t v_st, int kv, const ResidualCopy& rc,
                                                   int blk, int h, int b, int tid) {
  const int t0 = 32 * blk;  // first residual token of this workgroup
  const int64_t src_tok0 = static_cast<int64_t>(rc.n_groups) * 32 + t0;
  const int64_t dst_row0 = (static_cast<int64_t>(b) * kv + h) * rc.r_cap + rc.res_row0 + t0;
  u32x4_t kw[4], vw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 128 * i, t = c >> 4, part = c & 15;
    const bool ok = t0 + t < rc.res_len;
    const int64_t tok = src_tok0 + (ok ? t : 0);
    kw[i] = *reinterpret_cast<const u32x4_t*>(k + b * k_sb + h * k_sh + tok * k_st + 8 * part);
    vw[i] = *reinterpret_cast<const u32x4_t*>(v + b * v_sb + h * v_sh + tok * v_st + 8 * part);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 128 * i, t = c >> 4, part = c & 15;
    if (t0 + t < rc.res_len) {
      const int64_t o = (dst_row0 + t) * 128 + 8 * part;
      *reinterpret_cast<u32x4_t*>(rc.k_res + o) = kw[i];
      *reinterpret_cast<u32x4_t*>(rc.v_res + o) = vw[i];
    }
  }
}

__global__ __launch_bounds__(128) void kivi4_pack_kernel(
    const uint16_t* __restrict__ k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const uint16_t* __restrict__ v, int64_t v_sb, int64_t v_sh, int64_t v_st, int kv, int g0,
    int g_cap, int32_t* __restrict__ groups, uint32_t* __restrict__ range_status, const ResidualCopy rc) {
  __shared__ uint8_t kc[32][128];
  __shared__ uint8_t vc[32][128];
  const int g = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  if (g >= rc.n_groups) {  // (uniform) a residual-row workgroup of a prefill
    copy_residual_rows(k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, kv, rc, g - rc.n_groups, h, b, tid);
    return;
  }
  const int64_t bhg = (static_cast<int64_t>(b) * kv + h) * g_cap + g0 + g;
  int32_t* const rec = groups + bhg * kRecordWords;
  int32_t* const k_codes = rec;
  int32_t* const v_codes = rec + 512;
  uint16_t* const k_meta = reinterpret_cast<uint16_t*>(rec + 1024);
  uint16_t* const v_meta = reinterpret_cast<uint16_t*>(rec + 1152);

  // ---- K: lane = channel d, 32 tokens of the group ----
  {
    const int d = tid;
    const uint16_t* src = k + b * k_sb + h * k_sh + static_cast<int64_t>(g) * 32 * k_st + d;
    float x[32];
#pragma unroll
    for (int t = 0; t < 32; ++t) x[t] = bf16_to_f32(src[t * k_st]);
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int t = 1; t < 32; ++t) {
      mn = fminf(mn, x[t]);
      mx = fmaxf(mx, x[t]);
    }
    const float scale = kivi_scale(mn, mx);
    const float safe = kivi_safe(scale);
    if (safe < INFINITY) {
      const float r = 1.0f / safe;
#pragma unroll
      for (int t = 0; t < 32; ++t) kc[t][d] = static_cast<uint8_t>(kivi_code_r(x[t], mn, safe, r));
    } else {
#pragma unroll
      for (int t = 0; t < 32; ++t) kc[t][d] = static_cast<uint8_t>(kivi_code(x[t], mn, safe));
    }
    const int p = d >> 3, j = d & 7;
    const int slot = 2 * (j & 3) + (j >> 2);
    uint16_t* km = k_meta + p * 16;
    const uint16_t hs = f32_to_f16_bits(scale), hz = f32_to_f16_bits(mn);
    km[slot] = hs;
    km[8 + slot] = hz;
    if (range_status && (f16_nonfinite(hs) || f16_nonfinite(hz))) atomicOr(range_status, ZKV_RANGE_K);
  }
  // ---- V: lane = (token t, channel group gd), 32 channels ----
  {
    const int t = tid >> 2, gd = tid & 3;
    const uint16_t* src = v + b * v_sb + h * v_sh + (static_cast<int64_t>(g) * 32 + t) * v_st + 32 * gd;
    float x[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(src + 8 * i);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[8 * i + 2 * q] = __uint_as_float(w[q] << 16);
        x[8 * i + 2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
      }
    }
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
      mn = fminf(mn, x[i]);
      mx = fmaxf(mx, x[i]);
    }
    const float scale = kivi_scale(mn, mx);
    const float safe = kivi_safe(scale);
    if (safe < INFINITY) {
      const float r = 1.0f / safe;
#pragma unroll
      for (int i = 0; i < 32; ++i) vc[t][32 * gd + i] = static_cast<uint8_t>(kivi_code_r(x[i], mn, safe, r));
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) vc[t][32 * gd + i] = static_cast<uint8_t>(kivi_code(x[i], mn, safe));
    }
    // token t = 16m + 4r + i: half m's block, entry (gd, r) = 4 scales then 4 zeros
    const int m = t >> 4, r = (t >> 2) & 3, i = t & 3;
    uint16_t* vm = v_meta + m * 128 + (gd * 4 + r) * 8;
    const uint16_t hs = f32_to_f16_bits(scale), hz = f32_to_f16_bits(mn);
    vm[i] = hs;
    vm[4 + i] = hz;
    if (range_status) {
      const uint32_t bad = (f16_nonfinite(hs) || f16_nonfinite(hz) ? ZKV_RANGE_V : 0u) |
                           ((hs & 0x7FFFu) > kF16VScaleMax ? ZKV_RANGE_V_SCALE : 0u);
      if (bad) atomicOr(range_status, bad);
    }
  }
  __syncthreads();
  // ---- K words in MFMA lane order: w = m*256 + l*4 + s, l = 16g + c,
  //      word of dim block p = 4s + g for token t = 16m + c ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int w = tid + 128 * i;
    const int m = w >> 8, l = (w >> 2) & 63, s = w & 3;
    const int p = 4 * s + (l >> 4), t = 16 * m + (l & 15);
    const uint64_t cb = *reinterpret_cast<const uint64_t*>(&kc[t][8 * p]);
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) word |= static_cast<uint32_t>((cb >> (8 * j)) & 0xF) << (4 * j);
    k_codes[w] = static_cast<int32_t>(word);
  }
  // ---- V words in MFMA lane order: w = m*256 + l*4 + P, l = 16r + c: channels
  //      d = 32P + 2c and d + 1 (one 32-channel scale group) of tokens
  //      16m + 4r + i; nibbles (0, 4, 1, 5) = channel d, tokens i = 0..3,
  //      nibbles (2, 6, 3, 7) = channel d + 1 ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int w = tid + 128 * i;
    const int m = w >> 8, l = (w >> 2) & 63, P = w & 3;
    const int t0 = 16 * m + 4 * (l >> 4), d = 32 * P + 2 * (l & 15);
    uint32_t word = 0;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int tok = t0 + (n >> 2) + 2 * (n & 1), ch = d + ((n >> 1) & 1);
      word |= static_cast<uint32_t>(vc[tok][ch]) << (4 * n);
    }
    v_codes[w] = static_cast<int32_t>(word);
  }
}

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" int zkv_chunk_encode(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                int bs, int kv, int g, int n_chunks, int chunk_start,
                                int n_chunks_max, uint16_t* chunk_min, uint16_t* chunk_max,
                                uint16_t* chunk_centroid, uint8_t* chunk_valid, int32_t* packed_K,
                                zkv_stream_t stream) {
  ZKV_REQUIRE(keys && chunk_min && chunk_max && chunk_centroid && chunk_valid && packed_K,
              "zkv_chunk_encode: null pointer");
  ZKV_REQUIRE(g == 8 || g == 16 || g == 32, "zkv_chunk_encode: chunk size must be 8, 16 or 32; got %d", g);
  ZKV_REQUIRE(bs > 0 && kv > 0 && n_chunks >= 0 && chunk_start >= 0,
              "zkv_chunk_encode: bad sizes bs=%d kv=%d n_chunks=%d chunk_start=%d", bs, kv,
              n_chunks, chunk_start);
  ZKV_REQUIRE(chunk_start + n_chunks <= n_chunks_max,
              "zkv_chunk_encode: chunk_end=%d exceeds n_chunks_max=%d", chunk_start + n_chunks,
              n_chunks_max);
  if (n_chunks == 0) return ZKV_OK;
  dim3 grid(n_chunks, kv, bs);
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (g == 8)
    chunk_encode_kernel<8><<<grid, 128, 0, s>>>(keys, k_sb, k_sh, k_st, kv, chunk_start, n_chunks_max,
                                                chunk_min, chunk_max, chunk_centroid, chunk_valid, packed_K);
  else if (g == 16)
    chunk_encode_kernel<16><<<grid, 128, 0, s>>>(keys, k_sb, k_sh, k_st, kv, chunk_start, n_chunks_max,
                                                 chunk_min, chunk_max, chunk_centroid, chunk_valid, packed_K);
  else
    chunk_encode_kernel<32><<<grid, 128, 0, s>>>(keys, k_sb, k_sh, k_st, kv, chunk_start, n_chunks_max,
                                                 chunk_min, chunk_max, chunk_centroid, chunk_valid, packed_K);
  return check_launch("chunk_encode_kernel");
}

extern "C" int zkv_kivi4_pack(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                              const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int bs,
                              int kv, int n_groups, int g0, int g_cap, int32_t* groups,
                              uint32_t* range_status, zkv_stream_t stream) {
  ZKV_REQUIRE(k && v && groups, "zkv_kivi4_pack: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && n_groups >= 0 && g0 >= 0,
              "zkv_kivi4_pack: bad sizes bs=%d kv=%d n_groups=%d g0=%d", bs, kv, n_groups, g0);
  ZKV_REQUIRE(g0 + n_groups <= g_cap, "zkv_kivi4_pack: group end %d exceeds capacity %d",
              g0 + n_groups, g_cap);
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15) == 0 && (v_st % 8) == 0 && (v_sh % 8) == 0 &&
                  (v_sb % 8) == 0,
              "zkv_kivi4_pack: v rows must be 16-byte aligned");
  if (n_groups == 0) return ZKV_OK;
  dim3 grid(n_groups, kv, bs);
  const ResidualCopy rc{nullptr, nullptr, 0, 0, 0, n_groups};
  kivi4_pack_kernel<<<grid, 128, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, kv, g0, g_cap, groups, range_status, rc);
  return check_launch("kivi4_pack_kernel");
}

extern "C" int zkv_kivi4_prefill(const uint16_t* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                 const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int bs,
                                 int kv, int n_groups, int g0, int g_cap, int32_t* groups,
                                 uint32_t* range_status, uint16_t* k_res, uint16_t* v_res, int r_cap,
                                 int res_row0, int res_len, zkv_stream_t stream) {
  ZKV_REQUIRE(k && v && groups, "zkv_kivi4_prefill: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && n_groups >= 0 && g0 >= 0 && res_len >= 0 && res_row0 >= 0,
              "zkv_kivi4_prefill: bad sizes bs=%d kv=%d n_groups=%d g0=%d res_len=%d res_row0=%d", bs, kv,
              n_groups, g0, res_len, res_row0);
  ZKV_REQUIRE(g0 + n_groups <= g_cap, "zkv_kivi4_prefill: group end %d exceeds capacity %d", g0 + n_groups,
              g_cap);
  ZKV_REQUIRE(res_len == 0 || (k_res && v_res), "zkv_kivi4_prefill: null residual window");
  ZKV_REQUIRE(res_row0 + res_len <= r_cap, "zkv_kivi4_prefill: residual rows end %d exceed capacity %d",
              res_row0 + res_len, r_cap);
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15) == 0 && (v_st % 8) == 0 && (v_sh % 8) == 0 &&
                  (v_sb % 8) == 0,
              "zkv_kivi4_prefill: v rows must be 16-byte aligned");
  ZKV_REQUIRE(res_len == 0 || ((reinterpret_cast<uintptr_t>(k) & 15) == 0 && (k_st % 8) == 0 && (k_sh % 8) == 0 &&
                               (k_sb % 8) == 0 &&
                               ((reinterpret_cast<uintptr_t>(k_res) | reinterpret_cast<uintptr_t>(v_res)) & 15) == 0),
              "zkv_kivi4_prefill: k rows and the residual windows must be 16-byte aligned");
  const int res_blocks = (res_len + 31) / 32;
  if (n_groups + res_blocks == 0) return ZKV_OK;
  dim3 grid(n_groups + res_blocks, kv, bs);
  const ResidualCopy rc{k_res, v_res, r_cap, res_row0, res_len, n_groups};
  kivi4_pack_kernel<<<grid, 128, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, kv, g0, g_cap, groups, range_status, rc);
  return check_launch("kivi4_pack_kernel");
}
