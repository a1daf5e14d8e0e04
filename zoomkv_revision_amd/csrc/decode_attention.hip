// Fused 4-bit KV decode attention for gfx950 (MI355X).
//
// out[b, hq] = softmax(q[b, hq] . K[b, kv]^T * sm_scale) . V[b, kv], causal off,
// GQA: query heads hq = kv*gqa + c share KV head kv (the convention of
// flash_attn_with_kvcache at S:1742-1747 and of the GQA mean at S:1621-1626).
//
// K / V come from a Format Q cache (4-bit codes, fp16 scale / zero) plus a bf16
// residual window.  The work is HBM-bound (160 B per cached token per KV head
// against ~2 KFLOP), so the kernel streams every 32-token tile from HBM
// exactly once for all `gqa` query heads of its KV head:
//
//  * a workgroup of NW wave64s owns one (context split, kv head, batch); wave
//    w walks tiles T0 + w, T0 + w + NW, ...  In the dense kernels a lane
//    loads its 4 x 16 B of a tile's code words straight into a D-slot
//    register ring and only the tile's metadata KiB goes through a D-stage
//    LDS ring (global_load_lds_dwordx4); the page-sparse and bf16-only
//    kernels stream whole 5 KiB records through the LDS ring.  D-1 tiles per
//    wave are in flight;
//  * nibbles enter the matrix cores undequantized: one v_and_b32 per pair
//    turns them into exact fp16 subnormals (n * 2^-24 for the low nibble of a
//    byte, 16n * 2^-24 for the high one) and the scales move to the B operand:
//      S[t, c]  = sum_d n[t,d] (q[c,d] s_d)       + sum_d q[c,d] z_d
//      O[d, c] += sum_t n[d,t] (P[t,c] s_t,G(d))  + sum_t P[t,c] z_t,G(d)
//    The K-side product q*s (per channel) enters as an fp16 hi + lo pair
//    (lo = fp16(q*s - hi) from one fma, exact), so the scores carry no fp16
//    rounding of q*s: that rounding, scaled by the code, was the largest error
//    term of peaked softmaxes.  The V-side product 16*P*s (per token and
//    32-channel group) is one fp16 value.  Zero points go through their own
//    MFMAs on exact fp16 products;
//  * S^T[t, c] = sum_d Khat[t, d] q[c, d] and O^T[d, c] += sum_t Vhat[d, t] P[t, c]
//    run on the matrix cores as v_mfma_f32_16x16x32_f16 (query heads on the N
//    axis).  The Format Q word / metadata order is the MFMA operand order, so
//    the K-MFMA result lands in exactly the lanes the V-MFMA B operand needs;
//  * online softmax in fp32, base 2: q enters the MFMA as fp16(q / 8) (exact
//    for bf16 q in range) and the scale 8 * log2(e) * sm_scale is applied inside
//    the exponent's fma, so scores are not rounded to fp16; the O rescale is
//    skipped when no running max moved;
//  * the NW waves merge through LDS; with one split per KV head the kernel
//    writes the output, otherwise the splits merge inside the same launch:
//    each workgroup stores its partial with device-coherent (write-through)
//    stores and counts itself in on a per-(b, kv) arrival slot, and the
//    workgroup that completes the count merges every split's partial
//    (merge_splits_last), with the LSE rule of lse_merge_torch
//    (Z/cache_hub/lse_merge/lse_merge.py:79-119).  A separate merge kernel
//    (kivi4_combine_kernel) gives the same bits.
//
// MFMA 16x16x32 operand layout (lane l, c = l % 16, g = l / 16):
//   A: row c, k-slice g (8 halves);  B: k-slice g, column c;
//   D: rows 4g..4g+3, column c.
// K-MFMA: A = Khat (row = token c + 16m), B = q (column = query head c),
//   k-slice element e of dim block p = 4s + g is channel 8p + KSLOT[e],
//   KSLOT = (0,4,1,5,2,6,3,7).
// V-MFMA (one per j = 0..7): A = V codes^T (row c = channel 32(j/2) + 2c +
//   j%2, so each M-tile lies in one 32-channel scale group), B = P * scale,
//   k-slice element e of lane group g is token TAU[g][e] = 4g+e | 16+4g+e-4,
//   which is exactly where the K-MFMA left that token's score.  Elements 0-3
//   come from the V code word of the first 16-token half, 4-7 from the
//   second's: every half (one Quest page) has its own K codes, V codes and
//   V scale/zero block, so the page-sparse mode loads 2816 B for a page.
// Code operand element order (one int32 word, nibble k = bits 4k..4k+3):
//   (n0, n4, n1, n5, n2, n6, n3, n7); elements 2, 3, 6, 7 carry a factor 16,
//   which the B operands undo (1/16 on K's, 16 on V's other elements).
#include "zkv_common.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <cstdlib>
#include <mutex>
#include <random>

namespace zkv {
namespace {

constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegBig = -1.0e30f;

struct AttnParams {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const int32_t* groups;  // Format Q records [bs, kv, g_cap, 1280] int32
  const uint16_t* k_res;  // bf16 tiles: token t of (b, kv) at b*kr_sb + kv*kr_sh + t*kr_st
  const uint16_t* v_res;
  int g_cap;
  int64_t kr_sb, kr_sh, kr_st, vr_sb, vr_sh, vr_st;
  float* lse;      // optional natural-log LSE [bs, kv*gqa] of the scaled scores
  // optional index list of the bf16 tokens (see bf16_row)
  const int64_t* res_idx;
  int64_t ri_sb, ri_sh;
  int n_idx, tail_start, row_limit;
  int kv, gqa, n_groups, res_len, n_splits;
  int tiles_per_split;  // tiles of an even-numbered split
  int tiles_odd_split;  // tiles of an odd-numbered split
  float qscale;    // raw MFMA score * qscale = base-2 scaled score
  float* ws_o;     // [bs, kv, n_splits, gqa, 128]
  float* ws_ml;    // [bs, kv, n_splits, gqa, 2]
  void* out;       // [bs, kv*gqa, 128], written directly when n_splits == 1
  int out_f32;
  // in-launch split merge (out != nullptr, n_splits > 1): one arrival slot
  // per (b, kv) [bs*kv] = (epoch << 8) | splits arrived; the split that
  // completes the count merges all partials.  nullptr: partials only.
  unsigned long long* slots;
  unsigned long long epoch;  // distinct per launch, never 0
  int merge_fence;           // 1: plain partials ordered by agent-scope fences
  // page-sparse mode: the page list of (b, kv) at pages + b*pg_sb + h*pg_sh
  // (n_sel ids, any order; page 2g + m = tokens 16m .. 16m + 15 of group g).
  // Ids outside [0, 2 n_groups) are skipped; the others, in list order, pair
  // up into tiles of two pages (the last one alone when their count is odd);
  // a repeated id counts again.
  int page_sparse;  // the page-sparse kernel runs (also for an empty list)
  const int64_t* pages;
  int64_t pg_sb, pg_sh;
  int n_sel;
  // token-list mode (token_list != 0): `pages` holds n_sel int64 token ids
  // per (b, kv).  Ids in [0, 32 n_groups) are Format Q tokens; ids in
  // [32 n_groups, 32 n_groups + tok_n_tail) are the bf16 rows tok_tail_row0 +
  // (id - 32 n_groups); other ids are skipped; a repeated id counts again.
  // The bf16 tokens are the listed bf16 rows (ascending), then tok_near_len
  // contiguous rows from tail_start.
  int token_list;
  int tok_tail_row0, tok_n_tail, tok_near_len;
};

// Entries of a token list per (b, kv) (checked on the host).
constexpr int kMaxListTokens = 1024;

// One pipeline stage = one 32-token tile, a byte copy of its Format Q record:
//   [0, 2048)    K code words (lane order)   [2048, 4096) V code words
//   [4096, 4608) K scale/zero slots          [4608, 5120) V scale/zero
constexpr int kStageBytes = 5120;
constexpr int kRecordWords = kStageBytes / 4;
// A page-sparse stage holds two 16-token pages, each from any group, in the
// two halves' places of a record ([0, 5120) as above; a page B that is the
// first half of its group takes the second half's places, which the tile
// compute treats alike), plus page B's K scale/zero slots at [5120, 5632).
constexpr int kPairStageBytes = 5632;
// cache policy of the tile loads: nt (streamed once, not kept in the caches)
constexpr int kCachePolicyNT = 2;

typedef __attribute__((address_space(3))) void lds_void_t;

// 64 lanes x 16 B from per-lane global addresses straight into LDS at
// dst + 16*lane (global_load_lds_dwordx4): the prefetch ring costs no VGPRs.
__device__ __forceinline__ void dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(dst), 16, 0, kCachePolicyNT);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)(p)));
}

// The same DMA as inline asm, which the compiler's wait counting does not see.
// With the builtin, a loop that mixes these DMAs with VGPR loads gets a drain
// of every load in flight (vmcnt(0)) at one tile of each unrolled round.  The
// caller waits for the DMA with an explicit vmcnt; the compiler's own waits for
// VGPR loads issued around it count one op fewer per DMA, so they are
// stricter than needed, never short.  `dst` must be wave-uniform (it goes to
// M0; lane i lands at dst + 16 i).
__device__ __forceinline__ void dma16_untracked(const void* src, void* dst) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" : : "v"(src), "{m0}"(lds_addr(dst)) : "memory");
}

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits
// 15:14; expcnt / lgkmcnt left at "no wait").  The compiler does not track the
// LDS side of global_load_lds, so the ring's waits are explicit.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N & 0x30) << 10) | 0x0F70);
}

__device__ __forceinline__ void wait_tiles_in_flight(int later) {
  // 5 DMA ops per tile; `later` tiles were issued after the one needed now
  switch (later) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<5>(); break;
    case 2: wait_vmcnt<10>(); break;
    default: wait_vmcnt<15>(); break;
  }
  __builtin_amdgcn_sched_barrier(0);
}

// The same for tiles of 5 or 3 DMA ops: `ops` ops were issued after the last
// one of the tile needed now (at most 3 later tiles of 5).
__device__ __forceinline__ void wait_ops_in_flight(int ops) {
  switch (ops) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    default: wait_vmcnt<15>(); break;
  }
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ u32x4_t ld16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

using u32x2_t = uint32_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2_t ld8(const void* p) {
  return *reinterpret_cast<const u32x2_t*>(p);
}

// A tile's token mask: bit t = token t of the 32-token group is attended.
constexpr uint32_t kAllTokens = 0xFFFFFFFFu;

// Halves a token mask touches (bit m: tokens 16m .. 16m + 15): the blocks a
// tile loads.
__device__ __forceinline__ uint32_t halves_of(uint32_t tok_mask) {
  return ((tok_mask & 0xFFFFu) ? 1u : 0u) | ((tok_mask >> 16) ? 2u : 0u);
}

// DMA ops of a tile with token mask `tok_mask`
__device__ __forceinline__ int tile_dma_ops(uint32_t tok_mask) { return halves_of(tok_mask) == 3u ? 5 : 3; }

__device__ __forceinline__ void issue_tile(const AttnParams& p, int64_t bh, int gi, int lane,
                                           uint8_t* stage, uint32_t tok_mask = kAllTokens) {
  // the record is 5 contiguous KiB: 5 loads of 64 lanes x 16 B
  const uint8_t* rec = reinterpret_cast<const uint8_t*>(p.groups + (bh * p.g_cap + gi) * kRecordWords) + 16 * lane;
  const uint32_t mask = halves_of(tok_mask);
  if (mask == 3u) {
#pragma unroll
    for (int i = 0; i < 5; ++i) dma16(rec + 1024 * i, stage + 1024 * i);
  } else {
    // one 16-token half m: its K codes, its V codes, and of the metadata KiB
    // the K scale/zero (lanes 0-31) and its V scale/zero (lanes 32 + 16m ..)
    const int m = mask == 2u ? 1 : 0;
    dma16(rec + 1024 * m, stage + 1024 * m);
    dma16(rec + 2048 + 1024 * m, stage + 2048 + 1024 * m);
    if (lane < 32 || (lane >> 4) == 2 + m) dma16(rec + 4096, stage + 4096);
  }
}

// DMA ops of a paired-page tile: with page B, 6 (K codes A, K codes B, V codes
// A, V codes B, metadata A + V meta B, K meta B); without, 3.
__device__ __forceinline__ int pair_dma_ops(int page_b) { return page_b >= 0 ? 6 : 3; }

// Pages pa (always) and pb (or -1) of (b, kv) into a paired-page stage: page
// x = 2 gi + m is half m of group gi; its blocks go to the places of half 0
// (page A) or half 1 (page B) whatever m is.
__device__ __forceinline__ void issue_pair(const AttnParams& p, int64_t bh, int pa, int pb, int lane,
                                           uint8_t* stage) {
  const uint8_t* base = reinterpret_cast<const uint8_t*>(p.groups + bh * p.g_cap * kRecordWords) + 16 * lane;
  const uint8_t* ra = base + static_cast<int64_t>(pa >> 1) * kStageBytes;
  const int ma = pa & 1;
  dma16(ra + 1024 * ma, stage);
  dma16(ra + 2048 + 1024 * ma, stage + 2048);
  if (pb >= 0) {
    const uint8_t* rb = base + static_cast<int64_t>(pb >> 1) * kStageBytes;
    const int mb = pb & 1;
    dma16(rb + 1024 * mb, stage + 1024);
    dma16(rb + 2048 + 1024 * mb, stage + 3072);
    // lanes 0-31: A's K scale/zero; 32-47: A's V scale/zero; 48-63: B's
    const uint8_t* src = lane < 32 ? ra + 4096 : (lane < 48 ? ra + 4096 + 256 * ma : rb + 4096 + 256 * mb - 256);
    dma16(src, stage + 4096);
    if (lane < 32) dma16(rb + 4096, stage + 5120);
  } else {
    if (lane < 48) dma16(lane < 32 ? ra + 4096 : ra + 4096 + 256 * ma, stage + 4096);
  }
}

// One code word as an MFMA operand of exact fp16 subnormals:
// (n0, n4) * 2^-24, (n1, n5) * 16 * 2^-24, (n2, n6) * 2^-24, (n3, n7) * 16 * 2^-24.
// fp16 subnormal inputs are exact on the gfx950 matrix cores.
__device__ __forceinline__ half8_t codes8(uint32_t w) {
  const uint32_t w8 = w >> 8;
  const u32x4_t r = {w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u};
  return __builtin_bit_cast(half8_t, r);
}

// The V-MFMA code operand from the two halves' words of a channel pair:
// elements 0-3 from h0's nibbles (0, 4, 1, 5) >> shift, elements 4-7 from h1's
// (shift 0: the pair's first channel, 8: its second), same scaling as codes8.
__device__ __forceinline__ half8_t codes8_halves(uint32_t h0, uint32_t h1, int shift) {
  const uint32_t a = h0 >> shift, b = h1 >> shift;
  const u32x4_t r = {a & 0x000F000Fu, a & 0x00F000F0u, b & 0x000F000Fu, b & 0x00F000F0u};
  return __builtin_bit_cast(half8_t, r);
}

__device__ __forceinline__ half8_t as_half8(const u32x4_t& x) { return __builtin_bit_cast(half8_t, x); }

__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Max over the four 16-lane rows, for each lane position c: two gfx950
// permlane swaps (rows 0<->1 / 2<->3, then halves), no LDS round trip.
__device__ __forceinline__ float wave_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  return vmax(__uint_as_float(r2[0]), __uint_as_float(r2[1]));
}

// A running max is kept while a tile's max exceeds it by at most this many
// base-2 units (probabilities up to 2^0.5); O, L and OZ are rescaled only when
// some lane's max jumps further.  The bound keeps the quantized tiles' V-side
// products 16 * P * scale inside fp16 for every V scale up to 2048 (a V range
// of 30720 inside one 32-channel group; the pack reports larger ones).
constexpr float kLazyMaxBits = 0.5f;

// Online-softmax update for one tile.  The raw score of token TAU[g][e] for
// query head c is S * sc + bias (masked tokens have S = -inf); qs turns a raw
// score into a base-2 exponent and qsc = qs * sc.  m_run is kept in raw
// units.  Returns the fp32 probabilities P of the lane's 8 tokens relative to
// the (possibly updated) running max.  v_exp_f32 flushes results below 2^-126
// to zero, which only drops probabilities far below every operand's resolution.
// kTwoBias: the halves' scores carry their own bias (bias for S[0], bias1
// for S[1]: a paired-page tile's two pages have their own K zero points).
template <bool kTwoBias = false>
__device__ __forceinline__ void softmax_probs(const float4_t S[2], float sc, float bias, float qs,
                                              float qsc, float& m_run, float4_t& L, float4_t O[8],
                                              float4_t& OZ, float pr[8], float bias1 = 0.0f) {
  float sv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sv[i] = S[0][i];
    sv[4 + i] = S[1][i];
  }
  float mx;
  if constexpr (kTwoBias) {
    const float m0 = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    const float m1 = fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]));
    mx = wave_max16(fmaxf(__builtin_fmaf(m0, sc, bias), __builtin_fmaf(m1, sc, bias1)));
  } else {
    const float mx8 = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                            fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
    mx = wave_max16(__builtin_fmaf(mx8, sc, bias));
  }
  const bool up = (mx - m_run) * qs > kLazyMaxBits;
  if (__any(up)) {
    const float m_new = up ? mx : m_run;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * qs);
    m_run = m_new;
    L *= alpha;
    OZ *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) O[j] *= alpha;
  }
  const float b2 = (bias - m_run) * qs;
  const float b2h = kTwoBias ? (bias1 - m_run) * qs : b2;
#pragma unroll
  for (int e = 0; e < 8; ++e) pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[e], qsc, e < 4 ? b2 : b2h));
}

// The quantized tiles' P: one fp16 operand; L accumulates sum(P) with a
// ones-row MFMA on that same fp16 P (every row of L holds the column sum).
template <bool kTwoBias = false>
__device__ __forceinline__ half8_t softmax_step(const float4_t S[2], float sc, float bias, float qs,
                                                float qsc, float& m_run, float4_t& L, float4_t O[8],
                                                float4_t& OZ, float bias1 = 0.0f) {
  float pr[8];
  softmax_probs<kTwoBias>(S, sc, bias, qs, qsc, m_run, L, O, OZ, pr, bias1);
  half8_t pb;
#pragma unroll
  for (int e = 0; e < 8; ++e) pb[e] = static_cast<_Float16>(pr[e]);
  const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
  L = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb, L, 0, 0, 0);
  return pb;
}

// The bf16 tiles' P as a bf16 pair hi + lo (hi = bf16(P), lo = bf16(P - hi);
// the difference is exact in fp32), so P keeps 16 significant bits through
// the bf16 matrix cores; L sums both with ones-row MFMAs.
// S is q . K (q unscaled); the running max keeps the quantized tiles' raw
// units (q / 8), so the raw score is S / 8.
__device__ __forceinline__ void softmax_step_bf16(const float4_t S[2], float qs, float& m_run,
                                                  float4_t& L, float4_t O[8], float4_t& OZ,
                                                  bf16x8_t& phi, bf16x8_t& plo) {
  float pr[8];
  softmax_probs(S, 0.125f, 0.0f, qs, qs * 0.125f, m_run, L, O, OZ, pr);
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf16x2_t h2 = __builtin_convertvector(float2_t{pr[e], pr[e + 1]}, bf16x2_t);
    const float2_t hf = __builtin_convertvector(h2, float2_t);
    const bf16x2_t l2 = __builtin_convertvector(float2_t{pr[e] - hf[0], pr[e + 1] - hf[1]}, bf16x2_t);
    phi[e] = h2[0];
    phi[e + 1] = h2[1];
    plo[e] = l2[0];
    plo[e + 1] = l2[1];
  }
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  L = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, phi, L, 0, 0, 0);
  L = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, plo, L, 0, 0, 0);
}

constexpr float kTwo20 = 1048576.0f;
constexpr float kTwo24 = 16777216.0f;

// Per-lane constants of the quantized tiles.
struct TileConsts {
  half8_t qB[4];   // q / 8 (K-MFMA B operand for the zero points)
  half8_t qBm[4];  // q / 8 with 1/16 on elements 2, 3, 6, 7 (times the K scales)
  float qs, qs24;  // raw score -> base-2; the same for 2^-24-unit scores
};

// Code words of one tile held by a lane: K halves 0 / 1 (record bytes 16 lane
// and 1024 + 16 lane), V halves 0 / 1 (2048 + 16 lane, 3072 + 16 lane).
struct TileCodes {
  u32x4_t k0, k1, v0, v1;
};

__device__ __forceinline__ TileCodes codes_from_stage(const uint8_t* st, int lane) {
  return {ld16(st + 16 * lane), ld16(st + 1024 + 16 * lane), ld16(st + 2048 + 16 * lane),
          ld16(st + 3072 + 16 * lane)};
}

// Tile compute from the lane's code words and the record's metadata KiB in
// LDS (`meta`: K scale/zero slots at +0, V scale/zero at +512).  kPair: the
// halves are two pages of a paired-page stage, half 1's K scale/zero slots at
// meta + 1024 (its scores get their own hi / lo products and zero-point sum).
//   K: S = sum n * (hi + lo)(q s) in 2^-24 units (codes are subnormals);
//      Z (every row) = sum q z (raw units); score = S * 2^24 + Z.
//   V: O[j] += sum n * fp16(16 P s) in 2^-20 units; OZ row r = sum P z of
//      32-channel group r & 3.
template <bool kPair = false>
__device__ __forceinline__ void compute_tile(const TileCodes& cw, const uint8_t* meta, int c, int g,
                                             const TileConsts& tc, uint32_t tok_mask,
                                             float& m_run, float4_t& L, float4_t O[8],
                                             float4_t& OZ) {
  const u32x4_t kq0 = cw.k0, kq1 = cw.k1;
  float4_t S[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  float4_t Z = {0.0f, 0.0f, 0.0f, 0.0f};
  float4_t Z1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint8_t* km = meta + (4 * s + g) * 32;
    const u32x4_t ks = ld16(km);
    const u32x4_t kz = ld16(km + 16);  // zero points
    // q s as hi + lo fp16 pair: hi = fp16(q s), lo = fp16(q s - hi) by one fma (exact)
    const half8_t bp = as_half8(ks) * tc.qBm[s];
    const half8_t bl = __builtin_elementwise_fma(as_half8(ks), tc.qBm[s], -bp);
    Z = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(kz), tc.qB[s], Z, 0, 0, 0);
    const half8_t n0 = codes8(kq0[s]), n1 = codes8(kq1[s]);
    S[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n0, bp, S[0], 0, 0, 0);
    S[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n0, bl, S[0], 0, 0, 0);
    if constexpr (kPair) {
      const u32x4_t ks1 = ld16(km + 1024);
      const u32x4_t kz1 = ld16(km + 1024 + 16);
      const half8_t bp1 = as_half8(ks1) * tc.qBm[s];
      const half8_t bl1 = __builtin_elementwise_fma(as_half8(ks1), tc.qBm[s], -bp1);
      Z1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(kz1), tc.qB[s], Z1, 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n1, bp1, S[1], 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n1, bl1, S[1], 0, 0, 0);
    } else {
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n1, bp, S[1], 0, 0, 0);
      S[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(n1, bl, S[1], 0, 0, 0);
    }
  }
  // every row of Z holds sum q z (all A rows are the zero points)
  const float zc = Z[0];
  // S[m][i] holds token 16m + 4g + i: drop the tokens outside the tile's mask
  // (unselected pages, or unlisted tokens of a token-list tile)
  if (tok_mask != kAllTokens) {
    const uint32_t mb = tok_mask >> (4 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!((mb >> i) & 1u)) S[0][i] = -INFINITY;
      if (!((mb >> (16 + i)) & 1u)) S[1][i] = -INFINITY;
    }
  }
  const uint32_t half_mask = halves_of(tok_mask);
  // (a paired tile without page B keeps half 1's bias finite: its K slots
  // hold stale bytes, and its scores are -inf already)
  const half8_t pb = kPair ? softmax_step<true>(S, kTwo24, zc, tc.qs, tc.qs24, m_run, L, O, OZ,
                                                (half_mask & 2u) ? Z1[0] : zc)
                           : softmax_step(S, kTwo24, zc, tc.qs, tc.qs24, m_run, L, O, OZ);

  // V code words of channel pairs P = 0..3 of each half, and the halves' V
  // scale/zero blocks (entry (gd, r): 4 scales, then 4 zeros of tokens 16m + 4r
  // + i); the k-slice's elements 0-3 are half 0, 4-7 half 1.  An unselected
  // half was not loaded: its scale/zero enter as 0 (its P is 0 as well).
  const u32x4_t vh0 = cw.v0, vh1 = cw.v1;
  const uint8_t* vm = meta + 512;
  auto vmeta8 = [&](int entry, int off) {
    const u32x2_t a = ld8(vm + entry * 16 + off), b2 = ld8(vm + 256 + entry * 16 + off);
    const bool h0 = half_mask & 1u, h1 = half_mask & 2u;
    return u32x4_t{h0 ? a[0] : 0u, h0 ? a[1] : 0u, h1 ? b2[0] : 0u, h1 ? b2[1] : 0u};
  };
  const u32x4_t vz = vmeta8((c & 3) * 4 + g, 8);  // zero points of group c & 3
  OZ = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(vz), pb, OZ, 0, 0, 0);
  // P * 16 on the low-nibble elements 0, 1, 4, 5
  half8_t pm = pb;
  const half2_t sixteen = {(_Float16)16.0f, (_Float16)16.0f};
  {
    half2_t a = {pb[0], pb[1]}, b2 = {pb[4], pb[5]};
    a = a * sixteen;
    b2 = b2 * sixteen;
    pm[0] = a[0];
    pm[1] = a[1];
    pm[4] = b2[0];
    pm[5] = b2[1];
  }
#pragma unroll
  for (int G = 0; G < 4; ++G) {
    const half8_t bv = as_half8(vmeta8(4 * G + g, 0)) * pm;
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      const int j = 2 * G + jp;  // channel 32G + 2c + jp
      O[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes8_halves(vh0[G], vh1[G], 8 * jp), bv, O[j], 0, 0, 0);
    }
  }
}

// Row in the bf16 buffer of token t of (b, kv)'s bf16 list, or -1 (masked):
// tokens [0, n_idx) are the listed rows (rows outside [0, row_limit) masked),
// the rest are the contiguous rows tail_start, tail_start + 1, ...  Without a
// row index (n_idx = 0, tail_start = 0) token t is row t.
// In the token-list mode the bf16 list comes first: its n_l rows in LDS
// (l_rows), already resolved and in range.
__device__ __forceinline__ int bf16_row(const AttnParams& p, const int64_t* idx_bh, int t,
                                        const int32_t* l_rows = nullptr, int n_l = 0) {
  if (t < n_l) return l_rows[t];
  t -= n_l;
  if (t < p.n_idx) {  // n_idx > 0 only with a list (checked on the host)
    const int64_t r = idx_bh[t];
    return (r >= 0 && r < p.row_limit) ? static_cast<int>(r) : -1;
  }
  return p.tail_start + (t - p.n_idx);
}

// One bf16 tile: tokens [base, base + valid) of the list, on the bf16 matrix
// cores (K and V enter as stored: no conversion, any bf16 value).  Lane (c, g)
// loads the K rows of tokens c and c + 16 (the K-MFMA A rows, dims
// 8(4s+g) .. +7 in order, against the query qN in the same order) and the V
// rows of tokens TAU[g][e] (its V-MFMA k-slice), 16 B per row.
// M-tile j of the V-MFMA, row c: channel 32(j/2) + 2c + j%2 (the quantized
// tiles' order: dword 16(j/2) + c of the row, half j%2), or, when kBf16Only
// (no quantized tile in the kernel), channel 8c + j (dword 4c + j/2, half
// j%2) so that each V row is one 16-byte load per lane; O[j][i] of lane
// (c, g) is then channel 32g + 8i + j.
// A residual tile's rows in registers: K rows kx[s][m] (token c + 16m, dims
// 8(4s+g) .. +7), V rows vx[e] (token TAU[g][e]), and the tokens that exist
// (bit e: token TAU[g][e] is within the list and not masked).  Rows are loaded
// without branches: a missing token loads row 0 of the buffer (it exists
// whenever the wave has a residual tile), its score is masked and its V row
// zeroed before use (the row may hold any bits).
struct ResidualTile {
  u32x4_t kx[4][2];
  u32x4_t vx[8];
  uint32_t vvalid;
};

template <bool kBf16Only>
__device__ __forceinline__ void residual_rows(const AttnParams& p, int b, int h, int base, int valid, int c, int g,
                                              int (&krow)[2], int (&vrow)[8], const int32_t* l_rows = nullptr,
                                              int n_l = 0) {
  const int64_t* idx_bh = p.res_idx ? p.res_idx + b * p.ri_sb + h * p.ri_sh : nullptr;
#pragma unroll
  for (int m = 0; m < 2; ++m)
    krow[m] = c + 16 * m < valid ? bf16_row(p, idx_bh, base + c + 16 * m, l_rows, n_l) : -1;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int tok = (e < 4) ? (4 * g + e) : (16 + 4 * g + e - 4);
    vrow[e] = tok < valid ? bf16_row(p, idx_bh, base + tok, l_rows, n_l) : -1;
  }
}

// `dummy` (when not null) replaces every address: a wave without a residual
// tile issues the same loads, all lanes on one line, so that every wave has
// the same loads in flight (the compiler's wait counting then stays exact).
template <bool kBf16Only>
__device__ __forceinline__ void residual_load_v(const AttnParams& p, int b, int h, int c, const int (&vrow)[8],
                                                ResidualTile& rt, const void* dummy = nullptr) {
  const uint16_t* vr = p.v_res + b * p.vr_sb + h * p.vr_sh;
  rt.vvalid = 0;
  // every row address before the first load: the allocator otherwise reuses
  // a pending load's register as a don't-care operand of the 64-bit address
  // arithmetic, which makes the compiler wait for that load
  const uint32_t* row[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    rt.vvalid |= vrow[e] >= 0 ? 1u << e : 0u;
    row[e] = dummy ? reinterpret_cast<const uint32_t*>(dummy)
                   : reinterpret_cast<const uint32_t*>(vr + static_cast<int64_t>(max(vrow[e], 0)) * p.vr_st) +
                         (kBf16Only ? 4 * c : c);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (kBf16Only) {
      rt.vx[e] = ld16(row[e]);
    } else {
#pragma unroll
      for (int G = 0; G < 4; ++G) rt.vx[e][G] = row[e][dummy ? 0 : 16 * G];
    }
  }
}

template <bool kBf16Only>
__device__ __forceinline__ void residual_load_k(const AttnParams& p, int b, int h, int g, const int (&krow)[2],
                                                ResidualTile& rt, const void* dummy = nullptr) {
  const uint16_t* kr = p.k_res + b * p.kr_sb + h * p.kr_sh;
  const uint16_t* row[2];  // addresses first, as in residual_load_v
#pragma unroll
  for (int m = 0; m < 2; ++m)
    row[m] = dummy ? static_cast<const uint16_t*>(dummy)
                   : kr + static_cast<int64_t>(max(krow[m], 0)) * p.kr_st + 8 * g;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int m = 0; m < 2; ++m) rt.kx[s][m] = ld16(row[m] + (dummy ? 0 : 32 * s));
}

// Scores, online softmax and the V product of a residual tile whose K rows
// are loaded (and V rows too unless `vrow` is given: then they are requested
// after the softmax, when fewer registers are live).
template <bool kBf16Only>
__device__ __forceinline__ void residual_finish(const AttnParams& p, int b, int h, int c, ResidualTile& rt,
                                                const bf16x8_t qN[4], float qs, float& m_run, float4_t& L,
                                                float4_t O[8], float4_t& OZ, const int (*vrow)[8]) {
  float4_t S[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int m = 0; m < 2; ++m)
      S[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rt.kx[s][m]), qN[s], S[m], 0, 0,
                                                     0);
  // S[m][i] is token 4g + i + 16m = TAU[g][i + 4m]
  const uint32_t vvalid = vrow ? [&] {
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) v |= (*vrow)[e] >= 0 ? 1u << e : 0u;
    return v;
  }() : rt.vvalid;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (!(vvalid >> (i + 4 * m) & 1u)) S[m][i] = -INFINITY;
  bf16x8_t phi, plo;
  softmax_step_bf16(S, qs, m_run, L, O, OZ, phi, plo);
  if (vrow) residual_load_v<kBf16Only>(p, b, h, c, *vrow, rt);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (!(vvalid >> e & 1u)) rt.vx[e] = u32x4_t{0u, 0u, 0u, 0u};
  // V^T operand of M-tile j: element e = half j%2 of dword j/2 of token
  // TAU[g][e]'s loaded row (v_perm_b32 picks the halves of a token pair)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const u32x4_t a = {__builtin_amdgcn_perm(rt.vx[1][j >> 1], rt.vx[0][j >> 1], sel),
                       __builtin_amdgcn_perm(rt.vx[3][j >> 1], rt.vx[2][j >> 1], sel),
                       __builtin_amdgcn_perm(rt.vx[5][j >> 1], rt.vx[4][j >> 1], sel),
                       __builtin_amdgcn_perm(rt.vx[7][j >> 1], rt.vx[6][j >> 1], sel)};
    O[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), phi, O[j], 0, 0, 0);
    O[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), plo, O[j], 0, 0, 0);
  }
}

// One whole residual tile.  kEarlyV (kernels with registers to spare)
// requests the V rows together with the K rows: one memory round trip after
// the row indices, not two.
template <bool kBf16Only, bool kEarlyV>
__device__ __forceinline__ void residual_tile(const AttnParams& p, int b, int h, int base, int valid,
                                              int c, int g, const bf16x8_t qN[4], float qs,
                                              float& m_run, float4_t& L, float4_t O[8],
                                              float4_t& OZ, const int32_t* l_rows, int n_l) {
  int krow[2], vrow[8];
  residual_rows<kBf16Only>(p, b, h, base, valid, c, g, krow, vrow, l_rows, n_l);
  ResidualTile rt;
  residual_load_k<kBf16Only>(p, b, h, g, krow, rt);
  if constexpr (kEarlyV) {
    residual_load_v<kBf16Only>(p, b, h, c, vrow, rt);
    residual_finish<kBf16Only>(p, b, h, c, rt, qN, qs, m_run, L, O, OZ, nullptr);
  } else {
    residual_finish<kBf16Only>(p, b, h, c, rt, qN, qs, m_run, L, O, OZ, &vrow);
  }
}

__device__ __forceinline__ void store_out(const AttnParams& p, int64_t row, int d, float v) {
  if (p.out_f32)
    reinterpret_cast<float*>(p.out)[row * 128 + d] = v;
  else
    reinterpret_cast<uint16_t*>(p.out)[row * 128 + d] = f32_to_bf16_bits(v);
}

// Agent-scope (device-coherent) accesses of the split partials that are
// merged inside the launch: the splits of one (b, kv) run on different XCDs,
// whose L2s are not coherent with each other.  On gfx950 these are
// write-through stores and loads that do not hit stale L2 lines (sc1), so
// no whole-L2 writeback or invalidate is needed.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool kAgent>
__device__ __forceinline__ float load_partial(const float* p) {
  if constexpr (kAgent)
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

// LSE merge of the n_splits partials of one (b, query head) at channel d, in
// split order 0, 1, ...: the merge kernel and the in-launch merge run the
// same arithmetic, so they give the same bits.  Returns o; mmax and den are
// the merged base-2 max and denominator (for the LSE).  Up to kBatch splits,
// every partial is requested before any is used (unconditional loads, the
// split index clamped), so the merge costs one memory round trip; more
// splits take two per batch of kBatch.
template <bool kAgent>
__device__ __forceinline__ float combine_splits(const float* ws_o, const float* ws_ml, int64_t row0, int gqa,
                                                int n_splits, int d, float& mmax, float& den) {
  constexpr int kBatch = 8;
  float num = 0.0f;
  mmax = kNegBig;
  den = 0.0f;
  if (n_splits <= kBatch) {
    float mv[kBatch], lv[kBatch], ov[kBatch];
#pragma unroll
    for (int s = 0; s < kBatch; ++s) {
      const int64_t row = row0 + static_cast<int64_t>(min(s, n_splits - 1)) * gqa;
      mv[s] = load_partial<kAgent>(ws_ml + row * 2);
      lv[s] = load_partial<kAgent>(ws_ml + row * 2 + 1);
      ov[s] = load_partial<kAgent>(ws_o + row * 128 + d);
    }
#pragma unroll
    for (int s = 0; s < kBatch; ++s) mmax = s < n_splits ? fmaxf(mmax, mv[s]) : mmax;
#pragma unroll
    for (int s = 0; s < kBatch; ++s) {
      const float w = __builtin_amdgcn_exp2f(mv[s] - mmax);
      den = s < n_splits ? den + w * lv[s] : den;
      num = s < n_splits ? num + w * ov[s] : num;
    }
  } else {
    // batches of kBatch splits, each batch's loads issued together (the
    // split index clamped): two round trips per batch instead of one per
    // split; the same max and the same sums in split order
    for (int s0 = 0; s0 < n_splits; s0 += kBatch) {
      float mv[kBatch];
#pragma unroll
      for (int s = 0; s < kBatch; ++s)
        mv[s] = load_partial<kAgent>(ws_ml + (row0 + static_cast<int64_t>(min(s0 + s, n_splits - 1)) * gqa) * 2);
#pragma unroll
      for (int s = 0; s < kBatch; ++s) mmax = fmaxf(mmax, mv[s]);
    }
    for (int s0 = 0; s0 < n_splits; s0 += kBatch) {
      float mv[kBatch], lv[kBatch], ov[kBatch];
#pragma unroll
      for (int s = 0; s < kBatch; ++s) {
        const int64_t row = row0 + static_cast<int64_t>(min(s0 + s, n_splits - 1)) * gqa;
        mv[s] = load_partial<kAgent>(ws_ml + row * 2);
        lv[s] = load_partial<kAgent>(ws_ml + row * 2 + 1);
        ov[s] = load_partial<kAgent>(ws_o + row * 128 + d);
      }
#pragma unroll
      for (int s = 0; s < kBatch; ++s) {
        const float w = __builtin_amdgcn_exp2f(mv[s] - mmax);
        den = s0 + s < n_splits ? den + w * lv[s] : den;
        num = s0 + s < n_splits ? num + w * ov[s] : num;
      }
    }
  }
  return den > 0.0f ? num / den : 0.0f;
}

// In-launch split merge, run by every workgroup after its partial stores
// (store_agent).  Each workgroup waits until its own stores are complete,
// then one lane counts the workgroup in on the (b, kv) slot (arrive_last: a
// slot whose epoch is not this launch's is stale -- an earlier launch, or
// fresh memory -- and is claimed for this epoch at count 0, then every
// arrival adds 1; the last arrival resets the count to 0 under the launch's
// epoch).  The workgroup that brings the count to n_splits merges every
// split's partial with combine_splits, so which workgroup merges does not
// change the bits.
__device__ __forceinline__ void merge_splits_last(const AttnParams& p, int64_t bh, int tid, int nthreads,
                                                  int* s_last) {
  // this lane's partial stores are device-visible (the memory clobber keeps
  // the compiler from moving any store below the wait)
  if (!p.merge_fence) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    // fence variant: the workgroup's plain stores, ordered before this lane
    // by the barrier, are released at agent scope (an L2 writeback)
    if (p.merge_fence) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    // (the last arrival leaves the count at 0 under this epoch, so a replay
    // of the same launch, a captured graph keeps its epoch, counts from 0)
    const bool last = arrive_last(p.slots + bh, p.epoch, p.n_splits);
    if (last && p.merge_fence) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *s_last = last;
  }
  __syncthreads();
  if (!*s_last) return;
  for (int idx = tid; idx < p.gqa * 128; idx += nthreads) {
    const int cc = idx >> 7, d = idx & 127;
    const int64_t row0 = bh * p.n_splits * p.gqa + cc;
    float mmax, den;
    // (fence variant: plain loads after the acquire above)
    const float r = p.merge_fence ? combine_splits<false>(p.ws_o, p.ws_ml, row0, p.gqa, p.n_splits, d, mmax, den)
                                  : combine_splits<true>(p.ws_o, p.ws_ml, row0, p.gqa, p.n_splits, d, mmax, den);
    const int64_t qrow = bh * p.gqa + cc;  // b*hq + h*gqa + cc
    store_out(p, qrow, d, r);
    if (p.lse != nullptr && d == 0) p.lse[qrow] = (mmax + __log2f(den)) * kLn2;
  }
}

constexpr int kMetaBytes = 1024;  // the record's last KiB: K and V scale/zero
constexpr int kMaxGqa = 16;       // query heads per KV head (checked on the host)
// Row stride (floats) of the final merge's per-(wave, head) output rows: 4
// banks of skew between the heads' rows, so the 16-byte stores of the lanes
// of one channel block (one per head) hit different banks.
constexpr int kRedStride = 132;
// A bf16 residual tile (two dependent memory round trips, 16 KiB) takes a
// wave about as long as three quantized tiles; splits and waves are balanced
// with that weight.
constexpr int kResidualTileWeight = 3;
// Register budget of the dense kernels, as resident waves per SIMD: a 4-wave
// workgroup gets 168 VGPRs (3 waves per SIMD, 3 workgroups per CU); an 8-wave
// workgroup puts 2 waves on each SIMD, and 2 workgroups would need 128 VGPRs,
// which spills, so it keeps one workgroup per CU with up to 256 VGPRs.
constexpr int dense_waves_per_simd(int nw) { return nw == 8 ? 2 : 3; }

// LDS of a workgroup: the tile rings, reused by the final merge of the NW
// waves (o [NW][gqa][128] fp32, then m and l [NW][gqa] each).
//   dense quantized tiles (kVgpr): the 4 KiB of code words of a tile go
//     straight to VGPRs (a D-slot register ring); only the metadata KiB
//     streams through LDS (a D-stage DMA ring per wave).  An LDS-DMA-only
//     ring streams at ~76% of HBM on gfx950, code words in VGPRs at ~88%.
//   page-sparse tiles: a D-stage ring of paired-page stages (5.5 KiB).
//   token-list and bf16-only tiles: a D-stage ring of whole 5 KiB records.
template <int NW, int D, bool kSparse, bool kBf16Only, bool kToken = false>
struct KernelShape {
  static constexpr bool kVgpr = !kSparse && !kBf16Only;
  static constexpr bool kPaired = kSparse && !kToken;
  static constexpr int kStage = kVgpr ? kMetaBytes : (kPaired ? kPairStageBytes : kStageBytes);
  static constexpr int kRingBytes = NW * D * kStage;
  static constexpr int kMergeBytes = NW * kMaxGqa * (kRedStride + 2) * 4;
  static constexpr int kLdsBytes = std::max(kRingBytes, kMergeBytes);
  // resident waves per SIMD when LDS (160 KiB per CU) is the limit
  static constexpr int kWgPerCu = (160 * 1024) / kLdsBytes;
  static constexpr int kWavesPerSimd = std::max(1, std::min(4, (kWgPerCu * NW) / 4));
  // the occupancy the register allocation targets
  static constexpr int kWavesPerEu = kBf16Only ? 2 : (kVgpr ? dense_waves_per_simd(NW) : kWavesPerSimd);
};

using i32x4_t = int32_t __attribute__((ext_vector_type(4)));

// kToken (with kSparse): the token-list mode.  The workgroup sorts the list
// in LDS (rank sort: entry i goes to #{j : key_j < key_i} + #{j < i : key_j
// == key_i}), so the quantized tokens come first, ascending, then the listed
// bf16 rows.  A run of quantized tokens of one 32-token group is one tile
// with a token mask; a repeated token starts a new tile, so it counts once
// per listing.  The splits take contiguous tile ranges of equal weight,
// computed here from the actual tile counts.
template <int NW, int D, bool kSparse, bool kBf16Only = false, bool kToken = false>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(KernelShape<NW, D, kSparse, kBf16Only, kToken>::kWavesPerEu)))
void kivi4_attn_kernel(const AttnParams p) {
  static_assert(!kToken || kSparse, "the token-list mode streams whole records");
  using KS = KernelShape<NW, D, kSparse, kBf16Only, kToken>;
  constexpr bool kPaired = KS::kPaired;
  constexpr int kStage = KS::kStage;
  __shared__ __attribute__((aligned(16))) uint8_t smem[KS::kLdsBytes];
  __shared__ int s_prog[KS::kVgpr ? NW : 1];  // dense: tiles done per wave
  // token-list mode: list keys | sorted keys (the listed bf16 rows after the
  // quantized ones) | tile token masks | partial ranks | counters; tile
  // groups overwrite whichever key array is not the sorted one
  __shared__ __attribute__((aligned(16))) int32_t s_tok[kToken ? 4 * kMaxListTokens + 48 : 4];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  // wave index through readfirstlane: the compiler then keeps the ring and
  // tile bookkeeping in SGPRs (scalar branches, scalar DMA base addresses)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const bool col_ok = c < p.gqa;
  const int64_t bh = static_cast<int64_t>(b) * p.kv + h;

  int T0 = (split >> 1) * (p.tiles_per_split + p.tiles_odd_split) + (split & 1) * p.tiles_per_split;
  int T1_token = 0;  // token-list mode: the end of this split's tiles
  uint8_t (*ring)[kStage] = reinterpret_cast<uint8_t (*)[kStage]>(smem + wave * D * kStage);
  int n_qt = p.n_groups;  // quantized tiles of (b, kv)
  int res_len = p.res_len;
  const int32_t* l_rows = nullptr;  // token-list mode: rows of the listed bf16 tokens (LDS)
  int n_lrows = 0;
  const int32_t* s_groups = nullptr;  // token-list mode: group of each tile (LDS)
  if constexpr (kToken) {
    int32_t* s_key = s_tok;                        // list keys
    int32_t* s_sorted = s_tok + kMaxListTokens;    // sorted keys (when the list is not sorted)
    uint32_t* s_tmask = reinterpret_cast<uint32_t*>(s_tok + 2 * kMaxListTokens);
    int32_t* s_rank = s_tok + 3 * kMaxListTokens;  // partial ranks
    // per wave: [w] tiles started, [16 + w] entries kept, [24 + w] of them
    // quantized, [32 + w] whether the list descends in the wave's entries
    int* s_cnt = s_tok + 4 * kMaxListTokens;
    const int64_t* lst = p.pages + b * p.pg_sb + h * p.pg_sh;
    const int64_t q_end = 32ll * p.n_groups, t_end = q_end + p.tok_n_tail;
    const int n = p.n_sel;
    constexpr int kPer = kMaxListTokens / (64 * NW);
    // entry i and its predecessor (the same cache lines: one round trip)
    int64_t raw[kPer], prev[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int i = tid + e * 64 * NW;
      raw[e] = i < n ? lst[i] : -1;
      prev[e] = (i >= 1 && i < n) ? lst[i - 1] : -1;
    }
    auto key_of = [&](int64_t id) { return (id >= 0 && id < t_end) ? static_cast<int32_t>(id) : INT32_MAX; };
    // per-wave counts and "the list descends here" flags, one LDS slot per
    // wave each (summed after the barrier: no zeroing, no atomics)
    int kept = 0, kept_q = 0;
    bool descent = false;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int i = tid + e * 64 * NW;
      const int32_t k = key_of(raw[e]);
      s_key[i] = k;
      s_tmask[i] = 0u;
      s_rank[i] = 0;
      kept += __popcll(__ballot(k != INT32_MAX));
      kept_q += __popcll(__ballot(k < q_end));
      descent = descent || (i >= 1 && i < n && key_of(prev[e]) > k);
    }
    const bool wave_descent = __ballot(descent) != 0;
    if (lane == 0) {
      s_cnt[16 + wave] = kept;
      s_cnt[24 + wave] = kept_q;
      s_cnt[32 + wave] = wave_descent;
    }
    __syncthreads();
    int n_keep = 0, n_q = 0, unsorted = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      n_keep += s_cnt[16 + w];
      n_q += s_cnt[24 + w];
      unsorted |= s_cnt[32 + w];
    }
    // An ascending list (skipped ids last) is used as it is; otherwise a rank
    // sort: entry i goes to #{j : key_j < key_i} + #{j < i : key_j == key_i},
    // its comparisons split over (64 NW) / E threads (E = n rounded up to a
    // power of 2), partial ranks summed with LDS atomics.
    if (unsorted) {
      int E = 64;
      while (E < n) E <<= 1;
      const int S = E >= 64 * NW ? 1 : (64 * NW) / E;  // threads per entry
      const int n16 = (n + 15) & ~15;                  // keys past n are INT32_MAX
      const int jlen = ((n16 / 16 + S - 1) / S) * 16;
      const int part = E >= 64 * NW ? 0 : tid / E;
      const int j0 = part * jlen, j1 = min(n16, j0 + jlen);
      for (int i = E >= 64 * NW ? tid : tid % E; i < n; i += 64 * NW) {
        const int32_t k = s_key[i];
        if (k == INT32_MAX) continue;
        // (key, index) as one 64-bit key: j precedes i iff cj < ci (branch-free)
        const uint64_t ci = (static_cast<uint64_t>(static_cast<uint32_t>(k)) << 10) | static_cast<uint32_t>(i);
        int rank = 0;
        for (int j = j0; j < j1; j += 16) {
          i32x4_t kk[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) kk[u] = *reinterpret_cast<const i32x4_t*>(s_key + j + 4 * u);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const uint64_t cj = (static_cast<uint64_t>(static_cast<uint32_t>(kk[u][w])) << 10) |
                                  static_cast<uint32_t>(j + 4 * u + w);
              rank += cj < ci ? 1 : 0;
            }
        }
        if (rank) atomicAdd(&s_rank[i], rank);
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int i = tid + e * 64 * NW;
        const int32_t k = s_key[i];
        if (i < n && k != INT32_MAX) s_sorted[s_rank[i]] = k;
      }
    } else {
      s_sorted = s_key;
      s_key = s_tok + kMaxListTokens;
    }
    __syncthreads();
    // sorted positions r0 = 2 tid and r0 + 1 of the quantized part: a tile
    // starts at a new group or at a repeated token
    const int r0 = 2 * tid;
    const int32_t kp = (r0 >= 1 && r0 - 1 < n_q) ? s_sorted[r0 - 1] : -1;
    const int32_t k0 = r0 < n_q ? s_sorted[r0] : -1;
    const int32_t k1 = r0 + 1 < n_q ? s_sorted[r0 + 1] : -1;
    const bool st0 = r0 < n_q && (r0 == 0 || (k0 >> 5) != (kp >> 5) || k0 == kp);
    const bool st1 = r0 + 1 < n_q && ((k1 >> 5) != (k0 >> 5) || k1 == k0);
    const uint64_t b0 = __ballot(st0), b1 = __ballot(st1);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b0 >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b0), 0)) +
                      __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b1 >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b1), 0));
    if (lane == 0) s_cnt[wave] = __popcll(b0) + __popcll(b1);
    __syncthreads();
    int base = 0;
    n_qt = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int cw = s_cnt[w];
      base += w < wave ? cw : 0;
      n_qt += cw;
    }
    const int t0 = base + below + (st0 ? 1 : 0) - 1;  // tile of position r0
    const int t1 = t0 + (st1 ? 1 : 0);
    if (st0) s_key[t0] = k0 >> 5;  // from here on s_key[t] = group of tile t
    if (st1) s_key[t1] = k1 >> 5;
    s_groups = s_key;
    if (r0 < n_q) atomicOr(&s_tmask[t0], 1u << (k0 & 31));
    if (r0 + 1 < n_q) atomicOr(&s_tmask[t1], 1u << (k1 & 31));
    // the listed bf16 tokens' rows, in place after the quantized part
    for (int r = n_q + tid; r < n_keep; r += 64 * NW)
      s_sorted[r] = p.tok_tail_row0 + (s_sorted[r] - static_cast<int32_t>(q_end));
    __syncthreads();
    l_rows = s_sorted + n_q;
    n_lrows = n_keep - n_q;
    res_len = n_lrows + p.tok_near_len;
    // contiguous tile ranges of equal weight (a bf16 tile weighs
    // kResidualTileWeight quantized ones)
    const int n_rt = (res_len + kTile - 1) / kTile;
    const int W = n_qt + kResidualTileWeight * n_rt;
    auto tile_at = [&](int x) {
      return x <= n_qt ? x : n_qt + (x - n_qt + kResidualTileWeight - 1) / kResidualTileWeight;
    };
    T0 = tile_at((split * W + p.n_splits - 1) / p.n_splits);
    T1_token = tile_at(((split + 1) * W + p.n_splits - 1) / p.n_splits);
  } else if constexpr (kSparse) {
    // Every wave walks the page list (64 pages per step): the in-range pages,
    // in list order, pair up into tiles (ranks 2t and 2t + 1 form tile t, by
    // ballot ranks), and the wave keeps the page ids of its own tiles T0 +
    // wave + NW*k, k < 64, in its last ring stage, which no DMA has reached
    // yet (page B = -1: a tile of one page).
    int32_t* s_pa = reinterpret_cast<int32_t*>(ring[D - 1]);
    int32_t* s_pb = s_pa + 64;
    const int64_t* pg = p.pages + b * p.pg_sb + h * p.pg_sh;
    const int64_t n_pages = 2ll * p.n_groups;
    int base = 0;
    s_pb[lane] = -1;  // (a lane's own store first: it precedes the walk's)
    // one load per page: the next 64 pages are requested before this step's
    // ballot, so the first two steps share one memory round trip
    int64_t cur = lane < p.n_sel ? pg[lane] : -1;
    for (int i0 = 0; i0 < p.n_sel; i0 += 64) {
      const int i = i0 + lane;
      const int64_t ahead = i + 64 < p.n_sel ? pg[i + 64] : -1;
      const bool valid = i < p.n_sel && cur >= 0 && cur < n_pages;
      const uint64_t m = __ballot(valid);
      const int r = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      const int rel = (r >> 1) - T0 - wave;
      if (valid && rel >= 0 && rel % NW == 0 && rel / NW < 64)
        ((r & 1) ? s_pb : s_pa)[rel / NW] = static_cast<int32_t>(cur);
      base += __popcll(m);
      cur = ahead;
    }
    n_qt = (base + 1) >> 1;
  }
  const int n_tiles = n_qt + (res_len + kTile - 1) / kTile;
  const int T1 = kToken ? T1_token : min(T0 + ((split & 1) ? p.tiles_odd_split : p.tiles_per_split), n_tiles);
  const int TQ = min(T1, n_qt);  // quantized tiles of this workgroup: [T0, TQ)
  // this wave's quantized tiles: T0 + wave + NW*k, k < nq (nq <= 64 in sparse mode)
  const int nq = TQ > T0 + wave ? (TQ - (T0 + wave) + NW - 1) / NW : 0;
  // token-list mode: lane k holds the group and token mask of this wave's
  // tile k; page-sparse mode: its pages A and B (B = -1: none)
  int my_group = 0, my_mask = static_cast<int>(kAllTokens);
  if constexpr (kToken) {
    if (lane < nq) {
      my_group = s_groups[T0 + wave + NW * lane];
      my_mask = s_tok[2 * kMaxListTokens + T0 + wave + NW * lane];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
  } else if constexpr (kSparse) {
    const int32_t* s_group = reinterpret_cast<const int32_t*>(ring[D - 1]);
    if (lane < nq) {
      my_group = s_group[lane];
      my_mask = s_group[64 + lane];
    }
    // the stage is the DMA target of tile D - 1 from here on
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the descriptor reads are done
    __builtin_amdgcn_sched_barrier(0);
  }
  auto group_of = [&](int k) {
    if constexpr (kSparse)
      return __builtin_amdgcn_readlane(my_group, k);
    else
      return T0 + wave + NW * k;
  };
  auto mask_of = [&](int k) -> uint32_t {
    if constexpr (kPaired)
      return __builtin_amdgcn_readlane(my_mask, k) >= 0 ? kAllTokens : 0x0000FFFFu;
    else if constexpr (kSparse)
      return static_cast<uint32_t>(__builtin_amdgcn_readlane(my_mask, k));
    else
      return kAllTokens;
  };
  // the next tile of the LDS ring: token-list tiles are one group's record
  // (its halves per the token mask), page-sparse tiles two pages
  auto issue_next = [&](int k) {
    if constexpr (kPaired)
      issue_pair(p, bh, group_of(k), __builtin_amdgcn_readlane(my_mask, k), lane, ring[k % D]);
    else
      issue_tile(p, bh, group_of(k), lane, ring[k % D], mask_of(k));
  };
  auto dma_ops_of = [&](int k) {
    if constexpr (kPaired)
      return pair_dma_ops(__builtin_amdgcn_readlane(my_mask, k));
    else
      return tile_dma_ops(mask_of(k));
  };

  // dense tiles: tile k's code words into register slot k % D, its metadata
  // KiB into LDS stage k % D (4 loads + 1 DMA, in that order)
  TileCodes creg[KS::kVgpr ? D : 1];
  const uint8_t* rec0 = reinterpret_cast<const uint8_t*>(p.groups + bh * p.g_cap * kRecordWords) + 16 * lane;
  // tile k of this wave, k clamped to its last tile: the refills past the end
  // reload that one (record 0 of the sequence for a wave without tiles; the
  // dense kernels run only when there is at least one quantized group)
  auto issue_vgpr = [&](int k, TileCodes& cw, uint8_t* stage) {
    const int gi = nq > 0 ? T0 + wave + NW * min(max(k, 0), nq - 1) : 0;
    const uint8_t* rec = rec0 + static_cast<int64_t>(gi) * kStageBytes;
    cw.k0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec));
    cw.k1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec + 1024));
    cw.v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec + 2048));
    cw.v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec + 3072));
    dma16_untracked(rec + 4096, stage);
  };

  const uint16_t* qp = p.q + b * p.q_sb + static_cast<int64_t>(h * p.gqa + (col_ok ? c : 0)) * p.q_sh;
  // q (dims 8(4s+g) .. +7) ahead of the tile stream, whose first tiles would
  // otherwise have to land before q does
  u32x4_t q_raw[4];
  if constexpr (!kBf16Only) {
#pragma unroll
    for (int s = 0; s < 4; ++s) q_raw[s] = ld16(qp + 8 * (4 * s + g));
  }

  // 8-wave, 2-stage dense kernels (registers to spare) request the rows of their first
  // residual tile right after q and compute it when the first quantized
  // round begins: its memory round trip then overlaps the first tiles' loads
  // instead of running alone after the loop.  Waves without a residual tile
  // issue the same loads on q's line (no branch around loads: see
  // residual_load_v).
  constexpr bool kPrefetchRes = KS::kVgpr && NW == 8 && D == 2;  // (8x3 would spill)
  const bool has_res = kPrefetchRes && max(T0, n_qt) + wave < T1;
  bool res_pending = has_res;
  ResidualTile rt0;
  if constexpr (kPrefetchRes) {
    const int base = (max(T0, n_qt) + wave - n_qt) * kTile;
    int krow[2], vrow[8];
    if (has_res) {
      residual_rows<false>(p, b, h, base, min(kTile, p.res_len - base), c, g, krow, vrow);
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) krow[m] = -1;
#pragma unroll
      for (int e = 0; e < 8; ++e) vrow[e] = -1;
    }
    const void* dummy = has_res ? nullptr : static_cast<const void*>(p.q + b * p.q_sb + h * p.gqa * p.q_sh);
    residual_load_k<false>(p, b, h, g, krow, rt0, dummy);
    residual_load_v<false>(p, b, h, c, vrow, rt0, dummy);
  }

  float4_t O[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) O[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float4_t OZ = {0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegBig;
  float4_t L = {0.0f, 0.0f, 0.0f, 0.0f};

  // bf16 residual tiles of this wave (at most r_cap / 32 of them, in the last
  // splits; tile t goes to wave t - max(T0, n_qt) mod NW), in real units,
  // from the wave's `first`-th one on
  auto residual_tiles = [&](int first) {
    const int t0 = max(T0, n_qt) + wave + NW * first;
    if (t0 < T1) {
      // q as stored (bf16, dims 8(4s+g) .. +7 in order), the B operand of the bf16 K-MFMA
      bf16x8_t qN[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        qN[s] = __builtin_bit_cast(bf16x8_t, col_ok ? ld16(qp + 8 * (4 * s + g)) : u32x4_t{0u, 0u, 0u, 0u});
      for (int t = t0; t < T1; t += NW) {
        const int base = (t - n_qt) * kTile;
        residual_tile<kBf16Only, kBf16Only || kToken || (KS::kVgpr && NW == 8)>(p, b, h, base,
                                                                                 min(kTile, res_len - base),
                                                                       c, g, qN, p.qscale, m_run, L, O, OZ,
                                                                       l_rows, n_lrows);
      }
    }
  };

  // Start the HBM stream.
  int issued = 0;
  if constexpr (KS::kVgpr) {
    // (the dense stream starts inside its tile loop, in a first round that
    // only issues)
  } else {
#pragma unroll
    for (int k = 0; k < D - 1; ++k)
      if (issued < nq) {
        issue_next(issued);
        ++issued;
      }
  }

  if constexpr (!kBf16Only) {
    // ---- q as the K-MFMA B operand (element e of block 4s+g = channel 8(4s+g)+KSLOT[e]) ----
    TileConsts tc;
    {
      constexpr int kslot[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t raw = q_raw[s];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t wv = raw[kslot[e] >> 1];
          const float x = __uint_as_float((kslot[e] & 1) ? (wv & 0xFFFF0000u) : (wv << 16));
          tc.qB[s][e] = static_cast<_Float16>(col_ok ? x * 0.125f : 0.0f);
        }
      }
      const half8_t inv16 = {1, 1, 0.0625, 0.0625, 1, 1, 0.0625, 0.0625};
#pragma unroll
      for (int s = 0; s < 4; ++s) tc.qBm[s] = tc.qB[s] * inv16;
      tc.qs = p.qscale;
      tc.qs24 = p.qscale * kTwo24;
    }

    if constexpr (KS::kVgpr) {
      // ---- dense quantized tiles: D register slots + D metadata stages,
      // unrolled by D so that every slot index is static ----
      // Tile t sits in slot t % D.  Whole rounds of D tiles first, with no
      // exit inside a round: a conditional refill or an early exit makes the
      // compiler's wait counting drain every load (vmcnt(0)) at the next tile.
      //
      // Waves w and w + 4 of an 8-wave workgroup share a SIMD, whose issue
      // arbitration favours the older wave: left alone, waves 0-3 finish
      // their tiles ~6% of the loop ahead of waves 4-7, which then run with
      // half the SIMD idle.  Each wave publishes its progress (tiles done,
      // a residual tile counting kResidualTileWeight) and raises its priority
      // while it is behind its SIMD sibling.  Only the timing changes: every
      // wave computes the same tiles in the same order.
      constexpr bool kBalance = NW == 8;
      int prog = 0;
      if (kBalance && lane == 0) s_prog[wave] = prog;
      //
      // The loop starts one round early (k0 = -D): that round issues tiles
      // 0 .. D - 2 (and a reload of tile 0) and computes nothing.  With the
      // first issues inside the loop, each register slot has one definition
      // and the allocator adds no copies of in-flight loads before the loop
      // (a copy waits for its load: a separate prologue drained the stream).
      int k0 = -D;
      for (; k0 + D <= nq; k0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
          const int sib = kBalance ? s_prog[wave ^ 4] : 0;  // read early, used after the tile
          // refill the slot tile k0 + j - 1 used with tile k0 + j + D - 1
          issue_vgpr(k0 + j + D - 1, creg[(j + D - 1) % D], ring[(j + D - 1) % D]);
          if (k0 < 0) continue;
          if (j == 0 && res_pending) {
            // the prefetched residual tile, while tile 0 lands; the quantized
            // tiles accumulate O in 2^-20 units, so its part is scaled to
            // those units (exactly: a power of 2)
            bf16x8_t qN[4];  // q as stored, the B operand of the bf16 K-MFMA
#pragma unroll
            for (int s = 0; s < 4; ++s)
              qN[s] = __builtin_bit_cast(bf16x8_t, col_ok ? q_raw[s] : u32x4_t{0u, 0u, 0u, 0u});
            residual_finish<false>(p, b, h, c, rt0, qN, p.qscale, m_run, L, O, OZ, nullptr);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) O[jj] = O[jj] * (1.0f / kTwo20);
            res_pending = false;
            prog += kResidualTileWeight;
          }
          // 5 ops per tile, D - 1 tiles issued after tile k0 + j: its
          // metadata DMA (issued last) has landed once 5 (D - 1) ops remain
          wait_vmcnt<5 * (D - 1)>();
          __builtin_amdgcn_sched_barrier(0);
          compute_tile(creg[j], ring[j], c, g, tc, kAllTokens, m_run, L, O, OZ);
          if constexpr (kBalance) {
            ++prog;
            if (lane == 0) s_prog[wave] = prog;
            if (prog < __builtin_amdgcn_readfirstlane(sib))
              __builtin_amdgcn_s_setprio(1);
            else
              __builtin_amdgcn_s_setprio(0);
          }
        }
      }
      if constexpr (kBalance) __builtin_amdgcn_s_setprio(0);
      // the last nq - k0 < D tiles are in slots 0 .. nq - k0 - 1; this wait
      // also drains the reloads past the end, whose LDS the merge reuses
      wait_vmcnt<0>();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < D - 1; ++j)
        if (k0 + j < nq) compute_tile(creg[j], ring[j], c, g, tc, kAllTokens, m_run, L, O, OZ);
    } else {
      // ---- page-sparse tiles through this wave's D-stage LDS ring ----
      for (int k = 0; k < nq; ++k) {
        if (issued < nq) {
          issue_next(issued);
          ++issued;
        }
        const uint32_t tok_mask = mask_of(k);
        int later = 0;  // DMA ops issued after tile k's
        for (int t = k + 1; t < issued; ++t) later += dma_ops_of(t);
        wait_ops_in_flight(later);
        compute_tile<kPaired>(codes_from_stage(ring[k % D], lane), ring[k % D] + 4096, c, g, tc, tok_mask,
                              m_run, L, O, OZ);
      }
    }
    // O to real units: O * 2^20 + sum P z of the M-tile's group (OZ component
    // i = row 4g + i holds group i's sum; M-tile j lies in group j / 2)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) O[j][i] = __builtin_fmaf(O[j][i], kTwo20, OZ[j >> 1]);
  }

  // ---- bf16 residual tiles after the quantized ones: all of them in the
  // page-sparse and bf16-only kernels (q read here keeps registers free in
  // their loops); in the dense kernels the prefetched tile of a wave with no
  // full quantized round, and the wave's further residual tiles ----
  if constexpr (kPrefetchRes) {
    if (res_pending) {
      bf16x8_t qN[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        qN[s] = __builtin_bit_cast(bf16x8_t, col_ok ? ld16(qp + 8 * (4 * s + g)) : u32x4_t{0u, 0u, 0u, 0u});
      residual_finish<false>(p, b, h, c, rt0, qN, p.qscale, m_run, L, O, OZ, nullptr);
    }
    residual_tiles(1);
  } else {
    residual_tiles(0);
  }

  // ---- merge the NW waves through LDS (the rings are free now) ----
  const float l_tot = L[0];
  __syncthreads();
  float* red_o = reinterpret_cast<float*>(smem);  // [NW][gqa][kRedStride]
  float* red_m = red_o + NW * p.gqa * kRedStride;                    // [NW][gqa]
  float* red_l = red_m + NW * p.gqa;                          // [NW][gqa]
  if (col_ok) {
    if constexpr (kBf16Only) {
      // O[j][i] is channel 32g + 8i + j
      float* o = red_o + (wave * p.gqa + c) * kRedStride + 32 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *reinterpret_cast<float4_t*>(o + 8 * i) = float4_t{O[0][i], O[1][i], O[2][i], O[3][i]};
        *reinterpret_cast<float4_t*>(o + 8 * i + 4) = float4_t{O[4][i], O[5][i], O[6][i], O[7][i]};
      }
    } else {
      float* o = red_o + (wave * p.gqa + c) * kRedStride + 8 * g;
#pragma unroll
      for (int G = 0; G < 4; ++G) {
        // O[2G + jp][i] is channel 32G + 8g + 2i + jp
        *reinterpret_cast<float4_t*>(o + 32 * G) =
            float4_t{O[2 * G][0], O[2 * G + 1][0], O[2 * G][1], O[2 * G + 1][1]};
        *reinterpret_cast<float4_t*>(o + 32 * G + 4) =
            float4_t{O[2 * G][2], O[2 * G + 1][2], O[2 * G][3], O[2 * G + 1][3]};
      }
    }
    if (g == 0) {
      red_m[wave * p.gqa + c] = m_run * p.qscale;  // base-2 scaled units from here on
      red_l[wave * p.gqa + c] = l_tot;
    }
  }
  __syncthreads();

  const int n_out = p.gqa * 128;
  const bool final_out = p.out != nullptr && p.n_splits == 1;
  const bool fused_merge = p.out != nullptr && p.n_splits > 1 && p.slots != nullptr;
  for (int idx = tid; idx < n_out; idx += 64 * NW) {
    const int cc = idx >> 7, d = idx & 127;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) mm = fmaxf(mm, red_m[w * p.gqa + cc]);
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = __builtin_amdgcn_exp2f(red_m[w * p.gqa + cc] - mm);
      ll += wt * red_l[w * p.gqa + cc];
      oo += wt * red_o[(w * p.gqa + cc) * kRedStride + d];
    }
    if (final_out) {
      store_out(p, bh * p.gqa + cc, d, ll > 0.0f ? oo / ll : 0.0f);  // row b*hq + h*gqa + cc
      if (p.lse != nullptr && d == 0) p.lse[bh * p.gqa + cc] = (mm + __log2f(ll)) * kLn2;
    } else if (fused_merge && !p.merge_fence) {
      const int64_t row = (bh * p.n_splits + split) * p.gqa + cc;
      store_agent(p.ws_o + row * 128 + d, oo);
      if (d == 0) {
        store_agent(p.ws_ml + row * 2, mm);
        store_agent(p.ws_ml + row * 2 + 1, ll);
      }
    } else {
      const int64_t row = (bh * p.n_splits + split) * p.gqa + cc;
      p.ws_o[row * 128 + d] = oo;
      if (d == 0) {
        p.ws_ml[row * 2] = mm;
        p.ws_ml[row * 2 + 1] = ll;
      }
    }
  }
  // (the flag reuses the first word of smem: merge_splits_last writes it
  // only after a barrier that follows every read of the reduction above)
  if (fused_merge)
    merge_splits_last(p, bh, tid, 64 * NW, reinterpret_cast<int*>(smem));
}

// Merge the n_splits partials of every (b, query head) with the LSE rule
// (standalone second stage, used when the caller runs the stages separately).
__global__ __launch_bounds__(128) void kivi4_combine_kernel(const float* __restrict__ ws_o,
                                                            const float* __restrict__ ws_ml,
                                                            int kv, int gqa, int n_splits,
                                                            void* __restrict__ out, int out_f32,
                                                            float* __restrict__ lse) {
  const int bq = blockIdx.x;  // b * hq + hq_idx
  const int hq = kv * gqa;
  const int b = bq / hq, qh = bq % hq;
  const int h = qh / gqa, c = qh % gqa;
  const int d = threadIdx.x;
  const int64_t row0 = ((static_cast<int64_t>(b) * kv + h) * n_splits) * gqa + c;
  float mmax, den;
  const float r = combine_splits<false>(ws_o, ws_ml, row0, gqa, n_splits, d, mmax, den);
  if (lse != nullptr && d == 0) lse[bq] = (mmax + __log2f(den)) * kLn2;
  const int64_t oi = static_cast<int64_t>(bq) * 128 + d;
  if (out_f32)
    reinterpret_cast<float*>(out)[oi] = r;
  else
    reinterpret_cast<uint16_t*>(out)[oi] = f32_to_bf16_bits(r);
}


// Merge of two independently normalised attention outputs by their natural
// LSEs (lse_merge_torch, Z/cache_hub/lse_merge/lse_merge.py:79-119):
//   m = max(la, lb), wa = exp(la - m), wb = exp(lb - m),
//   out = (wa * a + wb * b) / (wa + wb), computed in fp32, stored as the inputs' type.
// Elementwise over [bs, 1, heads, dim]; lse [bs, heads].  dtype 0 bf16, 1 fp16, 2 fp32.
template <int kType>
__device__ __forceinline__ float load_val(const void* p, int64_t i) {
  if constexpr (kType == 0)
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (kType == 1)
    return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  else
    return static_cast<const float*>(p)[i];
}

template <int kType>
__device__ __forceinline__ void store_val(void* p, int64_t i, float v) {
  if constexpr (kType == 0)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else if constexpr (kType == 1)
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  else
    static_cast<float*>(p)[i] = v;
}

template <int kType>
__global__ __launch_bounds__(256) void lse_merge_kernel(const void* __restrict__ a, const float* __restrict__ la,
                                                        const void* __restrict__ b, const float* __restrict__ lb,
                                                        void* __restrict__ out, int64_t total, int dim) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t row = i / dim;  // b * heads + h
  const float x = la[row], y = lb[row];
  const float m = fmaxf(x, y);
  const float wa = expf(x - m), wb = expf(y - m);
  const float den = wa + wb;
  store_val<kType>(out, i, (wa * load_val<kType>(a, i) + wb * load_val<kType>(b, i)) / den);
}

struct SplitPlan {
  int n_splits, tiles_per_split;
  int tiles_odd_split;  // tiles of the odd-numbered splits (see xcd_skew)
};

// Page-sparse shape: a wave holds only a few paired-page tiles (C3: 2), so its
// loop is a chain of DMA round trips; a 3-stage ring issues them together
// (8 x 3 x 5.5 KiB = 132 KiB of LDS: one workgroup per CU, 2 waves per SIMD).
constexpr int kSparseNW = 8, kSparseD = 3;

constexpr float kXcdSkew = 0.03f;

// Kernel shape: NW waves per workgroup, D ring stages per wave.
// ZKV_ATTN_SHAPE=NWxD (e.g. 4x3) overrides the dense default for tuning sweeps.
struct Shape {
  int nw, d;
};

Shape attn_shape() {
  static Shape sh = [] {
    Shape s{8, 2};
    if (const char* e = getenv("ZKV_ATTN_SHAPE")) {
      int nw = 0, d = 0;
      if (sscanf(e, "%dx%d", &nw, &d) == 2 && (nw == 4 || nw == 8) && (d == 2 || d == 3)) s = {nw, d};
    }
    return s;
  }();
  return sh;
}

// Share of an odd split's tiles moved to its even partner (0 = equal
// splits).  ZKV_XCD_SKEW overrides it for tuning sweeps.
float xcd_skew() {
  static float v = [] {
    float x = kXcdSkew;
    if (const char* e = getenv("ZKV_XCD_SKEW")) x = std::max(0.0f, std::min(0.2f, static_cast<float>(atof(e))));
    return x;
  }();
  return v;
}

// Resident workgroups per CU: LDS (160 KiB per CU) and waves (4 SIMDs, at most
// `waves_per_simd` waves each at the kernel's register budget).
int wgs_per_cu(Shape sh, int stage_bytes, int waves_per_simd) {
  const int lds = std::max(sh.nw * sh.d * stage_bytes, sh.nw * kMaxGqa * (kRedStride + 2) * 4);
  return std::max(1, std::min((160 * 1024) / lds, 4 * waves_per_simd / sh.nw));
}

// Defaults: the dense kernels (metadata-only LDS stages).
SplitPlan plan_splits(int bs, int kv, int n_groups, int res_len, int n_splits, Shape sh = attn_shape(),
                      int stage_bytes = kMetaBytes, int waves_per_simd = 0, bool xcd_aware = true) {
  if (waves_per_simd <= 0) waves_per_simd = dense_waves_per_simd(sh.nw);
  const int n_tiles = std::max(n_groups + (res_len + kTile - 1) / kTile, 1);
  int ns = n_splits;
  if (ns <= 0) {
    // one resident workgroup per split on 256 CUs
    const int target = 256 * wgs_per_cu(sh, stage_bytes, waves_per_simd);
    const int units = bs * kv;
    ns = (target + units - 1) / units;
    if (n_groups > 0) {
      // at least one tile per wave of every split (short contexts at small
      // batch are latency-bound: more splits beat fuller waves)
      ns = std::min(ns, std::max(1, n_tiles / sh.nw));
    } else {
      // bf16 rows only: a tile is two dependent memory round trips, so one
      // workgroup per CU wins even with idle waves in each split
      ns = std::min((256 + units - 1) / units, n_tiles);
    }
  }
  ns = std::max(1, std::min(ns, n_tiles));
  // contiguous tile ranges [s * per, (s + 1) * per), the residual tiles last:
  // with quantized tiles present, per covers an equal share of the weighted
  // work, so the splits holding residual tiles get fewer quantized ones
  const int n_res_tiles = n_tiles - n_groups;
  const int64_t work = n_groups > 0 ? static_cast<int64_t>(n_groups) + int64_t{kResidualTileWeight} * n_res_tiles
                                    : n_tiles;
  int per = static_cast<int>(std::min<int64_t>((work + ns - 1) / ns, n_tiles));
  if ((n_tiles + per - 1) / per < ns) per = (n_tiles + ns - 1) / ns;  // keep the split count
  ns = (n_tiles + per - 1) / per;
  // With an even split count the grid (splits, kv, bs) puts every even split
  // on an even XCD (workgroups go to the 8 XCDs round-robin by linear id) and
  // every odd split on an odd one.  The odd XCDs stream more slowly (their
  // workgroups finish ~4% later at C2), so each (even, odd) pair of splits
  // moves a share of its tiles to the even split.
  int odd = per;
  const float skew = xcd_skew();
  if (xcd_aware && ns % 2 == 0 && n_groups > 0 && skew > 0.0f) {
    const int even = std::min(2 * per - 1, static_cast<int>(per * (1.0f + skew) + 0.5f));
    odd = 2 * per - even;
    per = even;
  }
  return {ns, per, odd};
}

// Workspace layout: split partials o fp32 [bs, kv, S, gqa, 128], then (m, l)
// fp32 [bs, kv, S, gqa, 2], then (S > 1) one 8-byte arrival slot per (b, kv)
// for the in-launch merge.  The slots need no initial value: each launch
// carries its own epoch, and a slot holding another epoch counts as empty.
//
// The splits merge inside the launch: the workgroup that completes a (b, kv)
// merges it.  Its partials go out with device-coherent (write-through)
// stores and are read back with device-coherent loads; a device-scope fence
// per workgroup (a whole-L2 writeback and invalidate on gfx950) cost more than
// the separate merge kernel it replaced (C2 148 us instead of 129).
// ZKV_SPLIT_MERGE=kernel keeps the separate merge kernel (for A/B timing);
// ZKV_SPLIT_MERGE=fence orders plain partial stores with agent-scope fences.
size_t partial_bytes_for(int bs, int hq, int n_splits) {
  return static_cast<size_t>(bs) * hq * n_splits * (128 + 2) * sizeof(float);
}

size_t workspace_bytes_for(int bs, int hq, int kv, int n_splits) {
  const size_t slots = n_splits > 1 ? static_cast<size_t>(bs) * kv * sizeof(unsigned long long) : 0;
  return partial_bytes_for(bs, hq, n_splits) + slots;
}

bool merge_in_launch() {  // read at every launch, so tests can compare both
  const char* e = getenv("ZKV_SPLIT_MERGE");
  return !(e && strcmp(e, "kernel") == 0);
}

bool merge_with_fence() {
  const char* e = getenv("ZKV_SPLIT_MERGE");
  return e && strcmp(e, "fence") == 0;
}


// Token-list shape: the rank sort's LDS (12 KiB) beside a 3-stage ring of
// whole records (8 x 3 x 5 KiB); a wave holds one or two tiles at C5.
constexpr int kTokenNW = 8, kTokenD = 3;

void launch_attn(const AttnParams& p, int bs, hipStream_t s) {
  const dim3 grid(p.n_splits, p.kv, bs);
  const Shape sh = attn_shape();
  if (p.token_list) {
    kivi4_attn_kernel<kTokenNW, kTokenD, true, false, true><<<grid, 64 * kTokenNW, 0, s>>>(p);
  } else if (p.page_sparse) {
    kivi4_attn_kernel<kSparseNW, kSparseD, true><<<grid, 64 * kSparseNW, 0, s>>>(p);
  } else if (p.n_groups == 0) {  // bf16 rows only: the 16-byte V layout
    kivi4_attn_kernel<8, 2, false, true><<<grid, 512, 0, s>>>(p);
  } else if (sh.nw == 8) {
    if (sh.d == 3)
      kivi4_attn_kernel<8, 3, false><<<grid, 512, 0, s>>>(p);
    else
      kivi4_attn_kernel<8, 2, false><<<grid, 512, 0, s>>>(p);
  } else if (sh.d == 3) {
    kivi4_attn_kernel<4, 3, false><<<grid, 256, 0, s>>>(p);
  } else {
    kivi4_attn_kernel<4, 2, false><<<grid, 256, 0, s>>>(p);
  }
}

// Element strides of the bf16 tiles: residual window or a whole bf16 cache.
struct ResidualLayout {
  int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
};

// Index list of the bf16 tokens: res_len = n_idx listed rows (+ tail).
struct RowIndex {
  const int64_t* idx;
  int64_t sb, sh;
  int n_idx, tail_start, row_limit;
};

// Page list of the page-sparse mode (pages int64 [bs, kv, n_sel] at strides).
struct SparsePages {
  const int64_t* pages;
  int64_t pg_sb, pg_sh;
  int n_sel;
};

// Token list of the token-list mode (toks int64 [bs, kv, n_tok] at strides)
// and where its bf16 tokens live (see AttnParams).
struct TokenList {
  const int64_t* toks;
  int64_t tk_sb, tk_sh;
  int n_tok;
  int tail_row0, n_tail, near_row0, near_len;
};


// Sparse mode: every split is planned for the longest page list (n_sel
// pages, (n_sel + 1) / 2 paired tiles); each wave keeps at most 64 tile
// descriptors in its lanes.
SplitPlan plan_sparse_splits(int bs, int kv, int n_sel, int res_len, int n_splits) {
  const int n_pair = (n_sel + 1) / 2;
  // (equal splits: a page-sparse split is a short latency chain)
  SplitPlan sp = plan_splits(bs, kv, n_pair, res_len, n_splits, Shape{kSparseNW, kSparseD}, kPairStageBytes, 4,
                             false);
  constexpr int kMaxPerSplit = 64 * kSparseNW;
  if (sp.tiles_per_split > kMaxPerSplit) {
    const int n_tiles = n_pair + (res_len + kTile - 1) / kTile;
    sp.n_splits = (n_tiles + kMaxPerSplit - 1) / kMaxPerSplit;
    sp.tiles_per_split = (n_tiles + sp.n_splits - 1) / sp.n_splits;
    sp.tiles_odd_split = sp.tiles_per_split;
  }
  return sp;
}

// Token-list mode: the split count of the sparse plan for the list's upper
// bounds (every entry its own quantized tile, every entry a bf16 row), raised
// so that no split's tile range (computed in the kernel from the actual
// counts) exceeds the 64 tiles per wave the kernel keeps descriptors for.
SplitPlan plan_token_splits(int bs, int kv, int n_tok, int near_len, int n_splits) {
  const int res_max = n_tok + near_len;
  SplitPlan sp = plan_splits(bs, kv, n_tok, res_max, n_splits, Shape{kTokenNW, kTokenD}, kStageBytes, 4, false);
  const int64_t w_max = int64_t{n_tok} + int64_t{kResidualTileWeight} * ((res_max + kTile - 1) / kTile);
  constexpr int64_t kMaxPerSplit = 64 * kTokenNW - 4;
  const int ns_min = static_cast<int>((w_max + kMaxPerSplit - 1) / kMaxPerSplit);
  sp.n_splits = std::max(std::max(sp.n_splits, ns_min), 1);
  return sp;
}

int attention_launch(const uint16_t* q, int64_t q_sb, int64_t q_sh, const int32_t* groups,
                     int g_cap, const uint16_t* k_res, const uint16_t* v_res, int r_cap, int bs,
                     int hq, int kv, int n_groups, int res_len, float sm_scale, int n_splits,
                     void* workspace, size_t workspace_bytes, int* n_splits_used, void* out,
                     int out_f32, hipStream_t s, const SparsePages* sparse = nullptr,
                     const ResidualLayout* rl = nullptr, float* lse = nullptr,
                     const RowIndex* ri = nullptr, const TokenList* tl = nullptr) {
  ZKV_REQUIRE(q && workspace, "zkv_kivi4_attention: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0,
              "zkv_kivi4_attention: bad heads bs=%d hq=%d kv=%d", bs, hq, kv);
  const int gqa = hq / kv;
  ZKV_REQUIRE(gqa <= 16, "zkv_kivi4_attention: at most 16 query heads per KV head; got %d", gqa);
  ZKV_REQUIRE(n_groups >= 0 && n_groups <= g_cap, "zkv_kivi4_attention: n_groups=%d g_cap=%d",
              n_groups, g_cap);
  ZKV_REQUIRE(res_len >= 0 && (rl != nullptr || res_len <= r_cap),
              "zkv_kivi4_attention: res_len=%d r_cap=%d", res_len, r_cap);
  const ResidualLayout res = rl ? *rl
                                : ResidualLayout{static_cast<int64_t>(kv) * r_cap * 128,
                                                 static_cast<int64_t>(r_cap) * 128, 128,
                                                 static_cast<int64_t>(kv) * r_cap * 128,
                                                 static_cast<int64_t>(r_cap) * 128, 128};
  ZKV_REQUIRE(res_len == 0 || ((res.k_sb | res.k_sh | res.k_st | res.v_sb | res.v_sh | res.v_st) % 8 == 0 &&
                               (reinterpret_cast<uintptr_t>(k_res) & 15) == 0 &&
                               (reinterpret_cast<uintptr_t>(v_res) & 15) == 0),
              "zkv_kivi4_attention: bf16 K / V rows must be 16-byte aligned (K strides %lld %lld %lld, "
              "V strides %lld %lld %lld)", (long long)res.k_sb, (long long)res.k_sh, (long long)res.k_st,
              (long long)res.v_sb, (long long)res.v_sh, (long long)res.v_st);
  ZKV_REQUIRE(sparse != nullptr || tl != nullptr || n_groups + res_len > 0, "zkv_kivi4_attention: empty context");
  ZKV_REQUIRE(n_groups == 0 || groups, "zkv_kivi4_attention: null cache pointer");
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(groups) & 15) == 0, "zkv_kivi4_attention: records must be 16-byte aligned");
  ZKV_REQUIRE(res_len == 0 || (k_res && v_res), "zkv_kivi4_attention: null residual pointer");
  ZKV_REQUIRE((q_sh % 8) == 0 && (q_sb % 8) == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0,
              "zkv_kivi4_attention: q rows must be 16-byte aligned");
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
              "zkv_kivi4_attention: workspace must be 16-byte aligned");
  if (sparse) {
    ZKV_REQUIRE(sparse->n_sel >= 0 && (sparse->n_sel == 0 || sparse->pages),
                "zkv_kivi4_sparse_attention: bad page list (n_sel=%d)", sparse->n_sel);
    ZKV_REQUIRE(g_cap <= (1 << 30), "zkv_kivi4_sparse_attention: g_cap=%d too large", g_cap);
  }
  if (tl) {
    ZKV_REQUIRE(tl->n_tok >= 0 && tl->n_tok <= kMaxListTokens && (tl->n_tok == 0 || tl->toks),
                "zkv_kivi4_token_attention: n_tok=%d (at most %d entries per (b, kv))", tl->n_tok,
                kMaxListTokens);
    ZKV_REQUIRE(tl->n_tail >= 0 && tl->near_len >= 0 && int64_t{32} * n_groups + tl->n_tail < (int64_t{1} << 31),
                "zkv_kivi4_token_attention: bad tail n_tail=%d near_len=%d", tl->n_tail, tl->near_len);
  }
  const SplitPlan sp = tl       ? plan_token_splits(bs, kv, tl->n_tok, tl->near_len, n_splits)
                       : sparse ? plan_sparse_splits(bs, kv, sparse->n_sel, res_len, n_splits)
                                : plan_splits(bs, kv, n_groups, res_len, n_splits);
  const size_t partial = workspace_bytes_for(bs, hq, kv, sp.n_splits);
  const size_t need = partial;
  if (workspace_bytes < need)
    return fail(ZKV_ESPACE, "zkv_kivi4_attention: workspace %zu < %zu bytes", workspace_bytes, need);
  AttnParams p;
  p.q = q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.groups = groups;
  p.k_res = k_res;
  p.v_res = v_res;
  p.g_cap = g_cap;
  p.kr_sb = res.k_sb;
  p.kr_sh = res.k_sh;
  p.kr_st = res.k_st;
  p.vr_sb = res.v_sb;
  p.vr_sh = res.v_sh;
  p.vr_st = res.v_st;
  p.lse = lse;
  p.res_idx = ri ? ri->idx : nullptr;
  p.ri_sb = ri ? ri->sb : 0;
  p.ri_sh = ri ? ri->sh : 0;
  p.n_idx = ri ? ri->n_idx : 0;
  p.tail_start = ri ? ri->tail_start : 0;
  p.row_limit = ri ? ri->row_limit : 0;
  p.kv = kv;
  p.gqa = gqa;
  p.n_groups = n_groups;
  p.res_len = res_len;
  p.n_splits = sp.n_splits;
  p.tiles_per_split = sp.tiles_per_split;
  p.tiles_odd_split = sp.tiles_odd_split;
  p.qscale = sm_scale * kLog2e * 8.0f;  // q enters the MFMA as q / 8
  p.ws_o = reinterpret_cast<float*>(workspace);
  p.ws_ml = p.ws_o + static_cast<size_t>(bs) * hq * sp.n_splits * 128;
  p.out = out;
  p.out_f32 = out_f32;
  p.slots = nullptr;
  p.epoch = 0;
  p.merge_fence = merge_with_fence();
  // (the slot counts arrivals in 8 bits)
  const bool merge_here = out != nullptr && sp.n_splits > 1 && sp.n_splits < 256 && merge_in_launch();
  if (merge_here) {
    p.slots = reinterpret_cast<unsigned long long*>(static_cast<uint8_t*>(workspace) +
                                                    partial_bytes_for(bs, hq, sp.n_splits));
    p.epoch = next_epoch();
  }
  p.page_sparse = sparse != nullptr;
  p.pages = sparse ? sparse->pages : nullptr;
  p.pg_sb = sparse ? sparse->pg_sb : 0;
  p.pg_sh = sparse ? sparse->pg_sh : 0;
  p.n_sel = sparse ? sparse->n_sel : 0;
  p.token_list = tl != nullptr;
  p.tok_tail_row0 = p.tok_n_tail = p.tok_near_len = 0;
  if (tl) {
    p.pages = tl->toks;
    p.pg_sb = tl->tk_sb;
    p.pg_sh = tl->tk_sh;
    p.n_sel = tl->n_tok;
    p.tok_tail_row0 = tl->tail_row0;
    p.tok_n_tail = tl->n_tail;
    p.tok_near_len = tl->near_len;
    p.tail_start = tl->near_row0;
    p.res_len = tl->n_tok + tl->near_len;  // (an upper bound; the kernel counts the listed bf16 rows)
  }
  if (n_splits_used) *n_splits_used = sp.n_splits;
  launch_attn(p, bs, s);
  int rc = check_launch("kivi4_attn_kernel");
  if (rc || out == nullptr || sp.n_splits == 1 || merge_here) return rc;
  kivi4_combine_kernel<<<bs * hq, 128, 0, s>>>(p.ws_o, p.ws_ml, kv, gqa, sp.n_splits, out, out_f32, lse);
  return check_launch("kivi4_combine_kernel");
}

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" size_t zkv_kivi4_attention_workspace_size(int bs, int hq, int kv, int n_groups,
                                                     int res_len, int n_splits) {
  if (bs <= 0 || kv <= 0 || hq <= 0) return 0;
  const SplitPlan sp = plan_splits(bs, kv, n_groups, res_len, n_splits);
  return workspace_bytes_for(bs, hq, kv, sp.n_splits);
}

extern "C" int zkv_kivi4_attention_partial(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                           const int32_t* groups, int g_cap,
                                           const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                           int bs, int hq, int kv, int n_groups, int res_len,
                                           float sm_scale, int n_splits, void* workspace,
                                           size_t workspace_bytes, int* n_splits_used,
                                           zkv_stream_t stream) {
  return attention_launch(q, q_sb, q_sh, groups, g_cap, k_res, v_res,
                          r_cap, bs, hq, kv, n_groups, res_len, sm_scale, n_splits, workspace,
                          workspace_bytes, n_splits_used, nullptr, 0,
                          reinterpret_cast<hipStream_t>(stream));
}

extern "C" int zkv_attention_merge(const void* workspace, int bs, int hq, int kv, int n_splits,
                                   void* out, int out_f32, zkv_stream_t stream) {
  ZKV_REQUIRE(workspace && out, "zkv_attention_merge: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0 && n_splits > 0,
              "zkv_attention_merge: bad sizes bs=%d hq=%d kv=%d n_splits=%d", bs, hq, kv, n_splits);
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
              "zkv_attention_merge: workspace must be 16-byte aligned");
  const float* ws_o = reinterpret_cast<const float*>(workspace);
  const float* ws_ml = ws_o + static_cast<size_t>(bs) * hq * n_splits * 128;
  kivi4_combine_kernel<<<bs * hq, 128, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      ws_o, ws_ml, kv, hq / kv, n_splits, out, out_f32, nullptr);
  return check_launch("kivi4_combine_kernel");
}

extern "C" int zkv_kivi4_decode_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                          const int32_t* groups, int g_cap,
                                          const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                          int bs, int hq, int kv, int n_groups, int res_len,
                                          float sm_scale, void* out, int out_f32, float* lse,
                                          int n_splits, void* workspace, size_t workspace_bytes,
                                          zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_kivi4_decode_attention: null output");
  return attention_launch(q, q_sb, q_sh, groups, g_cap, k_res, v_res,
                          r_cap, bs, hq, kv, n_groups, res_len, sm_scale, n_splits, workspace,
                          workspace_bytes, nullptr, out, out_f32,
                          reinterpret_cast<hipStream_t>(stream), nullptr, nullptr, lse);
}

// ---- allocation-free variant ----------------------------------------------
//
// The split partials of zkv_kivi4_decode_attention_noalloc live in this
// file-scope device array.  Each GPU the library runs on holds its own copy
// (until the process ends) at its own address; host code only ever uses that
// address, taken once per device with hipGetSymbolAddress -- the array's name
// in host code is a host-side stand-in, not a device pointer.
namespace zkv {
namespace {

constexpr size_t kNoAllocScratchBytes = ZKV_NOALLOC_SCRATCH_BYTES;  // 8 MiB per GPU
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of the current device's scratch array (taken once per
// device, with that device current), or nullptr with the error set.
void* scratch_for_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(ZKV_ELAUNCH, "zkv_kivi4_decode_attention_noalloc: no current HIP device (%s, device %d)",
         hipGetErrorString(e), dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      fail(ZKV_ELAUNCH, "zkv_kivi4_decode_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
           dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace zkv

extern "C" int zkv_kivi4_decode_attention_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                                  const int32_t* groups, int g_cap,
                                                  const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                                  int bs, int hq, int kv, int n_groups, int res_len,
                                                  float sm_scale, void* out, int out_f32, float* lse,
                                                  int n_splits, zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_kivi4_decode_attention_noalloc: null output");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0,
              "zkv_kivi4_decode_attention_noalloc: bad heads bs=%d hq=%d kv=%d", bs, hq, kv);
  const SplitPlan sp = plan_splits(bs, kv, n_groups, res_len, n_splits);
  const size_t need = workspace_bytes_for(bs, hq, kv, sp.n_splits);
  if (need > kNoAllocScratchBytes)
    return fail(ZKV_ESPACE,
                "zkv_kivi4_decode_attention_noalloc: %d splits x %d sequences x %d query heads need %zu bytes of "
                "split partials, beyond the %zu-byte static scratch (use zkv_kivi4_decode_attention with a "
                "workspace, or fewer splits)",
                sp.n_splits, bs, hq, need, kNoAllocScratchBytes);
  void* ws = scratch_for_current_device();
  if (ws == nullptr) return ZKV_ELAUNCH;
  return attention_launch(q, q_sb, q_sh, groups, g_cap, k_res, v_res, r_cap, bs, hq, kv, n_groups, res_len,
                          sm_scale, n_splits, ws, kNoAllocScratchBytes, nullptr, out, out_f32,
                          reinterpret_cast<hipStream_t>(stream), nullptr, nullptr, lse);
}

// ---- page-sparse mode -----------------------------------------------------

extern "C" size_t zkv_kivi4_sparse_attention_workspace_size(int bs, int hq, int kv, int n_sel,
                                                            int res_len, int n_splits) {
  if (bs <= 0 || kv <= 0 || hq <= 0 || n_sel < 0) return 0;
  const SplitPlan sp = plan_sparse_splits(bs, kv, n_sel, res_len, n_splits);
  return workspace_bytes_for(bs, hq, kv, sp.n_splits);
}

extern "C" int zkv_kivi4_sparse_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                          const int32_t* groups, int g_cap,
                                          const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                          int bs, int hq, int kv, int n_groups, int res_len,
                                          const int64_t* pages, int64_t pg_sb, int64_t pg_sh,
                                          int n_sel, float sm_scale, void* out, int out_f32,
                                          float* lse, int n_splits, void* workspace,
                                          size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_kivi4_sparse_attention: null output");
  const SparsePages sp{pages, pg_sb, pg_sh, n_sel};
  return attention_launch(q, q_sb, q_sh, groups, g_cap, k_res, v_res,
                          r_cap, bs, hq, kv, n_groups, res_len, sm_scale, n_splits, workspace,
                          workspace_bytes, nullptr, out, out_f32,
                          reinterpret_cast<hipStream_t>(stream), &sp, nullptr, lse);
}

// ---- bf16 K/V decode attention (flash_attn_with_kvcache counterpart) ------

extern "C" size_t zkv_bf16_attention_workspace_size(int bs, int hq, int kv, int n, int n_splits) {
  if (bs <= 0 || kv <= 0 || hq <= 0 || n < 0) return 0;
  const SplitPlan sp = plan_splits(bs, kv, 0, n, n_splits);
  return workspace_bytes_for(bs, hq, kv, sp.n_splits);
}

extern "C" int zkv_bf16_decode_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                         const uint16_t* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                                         const uint16_t* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                                         int bs, int hq, int kv, int n, float sm_scale, void* out,
                                         int out_f32, float* lse, int n_splits, void* workspace,
                                         size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_bf16_decode_attention: null output");
  ZKV_REQUIRE(n > 0, "zkv_bf16_decode_attention: empty key cache");
  const ResidualLayout rl{k_sb, k_sh, k_st, v_sb, v_sh, v_st};
  return attention_launch(q, q_sb, q_sh, nullptr, 0, k, v, n, bs, hq, kv, 0,
                          n, sm_scale, n_splits, workspace, workspace_bytes, nullptr, out, out_f32,
                          reinterpret_cast<hipStream_t>(stream), nullptr, &rl, lse);
}

// ---- token-list mode (4-bit cache + bf16 rows, one launch) -----------------

extern "C" size_t zkv_kivi4_token_attention_workspace_size(int bs, int hq, int kv, int n_tok, int near_len,
                                                           int n_splits) {
  if (bs <= 0 || kv <= 0 || hq <= 0 || n_tok < 0 || near_len < 0) return 0;
  const SplitPlan sp = plan_token_splits(bs, kv, n_tok, near_len, n_splits);
  return workspace_bytes_for(bs, hq, kv, sp.n_splits);
}

extern "C" int zkv_kivi4_token_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh, const int32_t* groups,
                                         int g_cap, int n_groups, const uint16_t* k, int64_t k_sb, int64_t k_sh,
                                         int64_t k_st, const uint16_t* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                                         int n_rows, const int64_t* toks, int64_t tk_sb, int64_t tk_sh, int n_tok,
                                         int tail_row0, int n_tail, int near_row0, int near_len, int bs, int hq,
                                         int kv, float sm_scale, void* out, int out_f32, float* lse, int n_splits,
                                         void* workspace, size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_kivi4_token_attention: null output");
  ZKV_REQUIRE(n_rows >= 0 && tail_row0 >= 0 && n_tail >= 0 && near_row0 >= 0 && near_len >= 0 &&
                  int64_t{tail_row0} + n_tail <= n_rows && int64_t{near_row0} + near_len <= n_rows,
              "zkv_kivi4_token_attention: tail rows [%d, +%d) or near rows [%d, +%d) outside the %d rows", tail_row0,
              n_tail, near_row0, near_len, n_rows);
  ZKV_REQUIRE(n_tail + near_len == 0 || (k && v), "zkv_kivi4_token_attention: null bf16 rows");
  const ResidualLayout rl{k_sb, k_sh, k_st, v_sb, v_sh, v_st};
  const TokenList tl{toks, tk_sb, tk_sh, n_tok, tail_row0, n_tail, near_row0, near_len};
  return attention_launch(q, q_sb, q_sh, groups, g_cap, k, v, n_rows, bs, hq, kv, n_groups, n_tok + near_len,
                          sm_scale, n_splits, workspace, workspace_bytes, nullptr, out, out_f32,
                          reinterpret_cast<hipStream_t>(stream), nullptr, &rl, lse, nullptr, &tl);
}

extern "C" int zkv_lse_merge(const void* out_a, const float* lse_a, const void* out_b, const float* lse_b,
                             void* out, int dtype, int bs, int heads, int dim, zkv_stream_t stream) {
  ZKV_REQUIRE(out_a && lse_a && out_b && lse_b && out, "zkv_lse_merge: null pointer");
  ZKV_REQUIRE(bs >= 0 && heads >= 0 && dim > 0, "zkv_lse_merge: bad sizes bs=%d heads=%d dim=%d", bs,
              heads, dim);
  ZKV_REQUIRE(dtype >= 0 && dtype <= 2, "zkv_lse_merge: dtype %d is not 0 (bf16), 1 (fp16) or 2 (fp32)",
              dtype);
  const int64_t total = static_cast<int64_t>(bs) * heads * dim;
  if (total == 0) return ZKV_OK;
  const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == 0)
    lse_merge_kernel<0><<<blocks, 256, 0, s>>>(out_a, lse_a, out_b, lse_b, out, total, dim);
  else if (dtype == 1)
    lse_merge_kernel<1><<<blocks, 256, 0, s>>>(out_a, lse_a, out_b, lse_b, out, total, dim);
  else
    lse_merge_kernel<2><<<blocks, 256, 0, s>>>(out_a, lse_a, out_b, lse_b, out, total, dim);
  return check_launch("lse_merge_kernel");
}

// ---- bf16 attention over an index list + a contiguous tail -----------------

extern "C" int zkv_bf16_gather_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                         const uint16_t* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                                         const uint16_t* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                                         int n_rows, const int64_t* idx, int64_t idx_sb, int64_t idx_sh,
                                         int n_idx, int tail_start, int tail_len, int bs, int hq, int kv,
                                         float sm_scale, void* out, int out_f32, float* lse, int n_splits,
                                         void* workspace, size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(out, "zkv_bf16_gather_attention: null output");
  ZKV_REQUIRE(n_idx >= 0 && tail_len >= 0 && n_idx + tail_len > 0 && n_rows > 0,
              "zkv_bf16_gather_attention: bad sizes n_idx=%d tail_len=%d n_rows=%d", n_idx, tail_len, n_rows);
  ZKV_REQUIRE(n_idx == 0 || idx, "zkv_bf16_gather_attention: null index list");
  ZKV_REQUIRE(tail_len == 0 || (tail_start >= 0 && static_cast<int64_t>(tail_start) + tail_len <= n_rows),
              "zkv_bf16_gather_attention: tail [%d, %d) outside the %d rows", tail_start, tail_start + tail_len,
              n_rows);
  const ResidualLayout rl{k_sb, k_sh, k_st, v_sb, v_sh, v_st};
  const RowIndex ri{idx, idx_sb, idx_sh, n_idx, tail_start, n_rows};
  return attention_launch(q, q_sb, q_sh, nullptr, 0, k, v, n_idx + tail_len, bs, hq,
                          kv, 0, n_idx + tail_len, sm_scale, n_splits, workspace, workspace_bytes, nullptr, out,
                          out_f32, reinterpret_cast<hipStream_t>(stream), nullptr, &rl, lse, &ri);
}

// ---- epochs of the in-launch arrival counts (declared in zkv_common.hpp) ----
namespace zkv {

// Epoch of a merging launch (56 bits): bit 55 set, the low 55 bits a random
// per-process base plus a launch counter, so distinct for every launch of the
// process.  A slot is (epoch << 8) | count, whose bit 63 is therefore set: no
// non-negative int64 a reused workspace may hold (a token index, a count, a
// small integer of the form (e << 8) | c) can read as a slot of a live
// launch, and another process's slots or arbitrary bytes match a given
// launch's epoch with probability 2^-55.
unsigned long long next_epoch() {
  static const unsigned long long base = [] {
    std::random_device rd;
    const unsigned long long hi = rd(), lo = rd();
    const unsigned long long t = static_cast<unsigned long long>(
        std::chrono::steady_clock::now().time_since_epoch().count());
    return (hi << 32) ^ lo ^ (t * 0x9E3779B97F4A7C15ull);
  }();
  static std::atomic<unsigned long long> counter{0};
  constexpr unsigned long long kLow55 = (1ull << 55) - 1;
  const unsigned long long n = counter.fetch_add(1, std::memory_order_relaxed) + 1;
  return ((base + n) & kLow55) | (1ull << 55);
}

}  // namespace zkv
