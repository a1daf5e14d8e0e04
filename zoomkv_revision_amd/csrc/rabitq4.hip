// ParisKV-compatible 4-bit RaBitQ codes on gfx950: key encode (1-bit sign +
// 3-bit magnitude per dimension, bf16 block weights), query blocks, and the
// 4-bit approximate inner-product rerank.
//
// Semantics (bf16 values rounded round-to-nearest-even at every point the
// reference's torch ops round):
//   key encode   Z/cache_hub/polar_cache.py:1130-1195 (batch_encode), with the
//                one-round SRHT of :1148-1151 and the fp32 butterfly of
//                Z/cache_hub/hadamard_fallback.py:16-26;
//   query blocks Z/cache_hub/polar_cache.py:1108-1124;
//   rerank       Z/cache_hub/rerank/rerank.cu:52-143: per candidate, for each
//                of the 16 blocks the sequential bf16 sum of the 8 bf16
//                products (+-center[t]) * q, times the block weight (bf16),
//                summed over the blocks in bf16, times ||q|| (bf16).
//
// Layouts (the reference's, PC:1137-1141): sign bytes [B=16, seq], 4-bit
// codes [16, seq] x 4 bytes (byte k = v[2k] | v[2k+1] << 4, v = sign << 3 |
// t), weights bf16 [16, seq]; each with its own (batch, head, block) strides
// and unit token stride.
#include "zkv_common.hpp"

namespace zkv {
namespace {

constexpr int kDim = 128;
constexpr int kBlk = 16;  // blocks of 8 dimensions
constexpr float kHadScale = 0.08838834764831845f;  // 1 / sqrt(128), as fp32 (PC:428)

// Lane xor-shuffle inside the 64-lane wave (ds_bpermute).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  const int lane = threadIdx.x & 63;
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

// One key (or query) per 16 lanes, lane b = block b (dimensions 8b .. 8b+7):
// returns the bf16 norm of the row and leaves in y[] the bf16 rotated unit
// row's block b.
//   norm   : per-lane sequential fp32 sum of the squares, then a butterfly
//            over the 16 lanes (xor 8, 4, 2, 1); sqrt; bf16
//   unit   : bf16(x / max(norm, bf16(1e-8)))
//   rotate : * sign (exact), fp32 butterfly h = 1, 2, 4 in the lane, then
//            h = 8, 16, 32, 64 across lanes (lower index a + b, upper a - b),
//            * 1/sqrt(128) in fp32, bf16
__device__ __forceinline__ float srht_unit_block(const float x[8], const float sg[8], int blk, float y[8]) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = s + x[j] * x[j];
#pragma unroll
  for (int d = 8; d >= 1; d >>= 1) s = s + shfl_xor(s, d);
  const float nrm = bf16r(__builtin_sqrtf(s));
  const float den = fmaxf(nrm, kBf16OneEm8);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = bf16r(x[j] / den) * sg[j];
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(i & h)) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
#pragma unroll
  for (int d = 1; d < kBlk; d <<= 1) {
    const bool upper = blk & d;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float o = shfl_xor(v[j], d);
      v[j] = upper ? o - v[j] : v[j] + o;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = bf16r(v[j] * kHadScale);
  return nrm;
}

struct EncodeParams {
  const uint16_t* keys;
  int64_t k_sb, k_sh, k_st;  // element strides
  int kv, n, t0;
  const uint16_t* signs;  // bf16 [128]
  uint8_t* code;
  int64_t c_sb, c_sh, c_sB;
  uint32_t* packed;
  int64_t p_sb, p_sh, p_sB;  // in 4-byte units
  uint16_t* weight;
  int64_t w_sb, w_sh, w_sB;
  int64_t rows;  // bs * kv * n
  // the 7 bucket thresholds and 8 reconstruction centers (bf16 [7], [8];
  // PC:266-270 holds them as bf16 tensors)
  const uint16_t* thr;
  const uint16_t* ctr;
};

__device__ __forceinline__ void load_row8(const uint16_t* p, float x[8]) {
  const u32x4_t r = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(r[i] << 16);
    x[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
  }
}

__global__ __launch_bounds__(256) void rabitq4_encode_kernel(const EncodeParams p) {
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 4;
  const int blk = threadIdx.x & 15;
  // rows past the end repeat the last row (every lane of a 16-lane group
  // takes part in the shuffles) and store nothing
  const int64_t r = row < p.rows ? row : p.rows - 1;
  const int64_t bh = r / p.n;
  const int t = static_cast<int>(r - bh * p.n);
  const int b = static_cast<int>(bh / p.kv), h = static_cast<int>(bh - static_cast<int64_t>(b) * p.kv);
  float x[8], sg[8], y[8];
  load_row8(p.keys + b * p.k_sb + h * p.k_sh + t * p.k_st + 8 * blk, x);
  load_row8(p.signs + 8 * blk, sg);
  const float knorm = srht_unit_block(x, sg, blk, y);
  float thr[7], ctr[8];
#pragma unroll
  for (int i = 0; i < 7; ++i) thr[i] = bf16_to_f32(p.thr[i]);
#pragma unroll
  for (int i = 0; i < 8; ++i) ctr[i] = bf16_to_f32(p.ctr[i]);

  // block radius, direction, magnitude bucket, alpha (PC:1166-1189)
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = s + y[j] * y[j];
  const float rad = bf16r(__builtin_sqrtf(s));
  const float den = fmaxf(rad, kBf16OneEm8);
  uint32_t code = 0, packed = 0;
  float alpha = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sb = y[j] >= 0.0f ? 1u : 0u;
    const float au = fabsf(bf16r(y[j] / den));
    uint32_t tq = 0;
#pragma unroll
    for (int i = 0; i < 7; ++i) tq += au > thr[i] ? 1u : 0u;
    float c = ctr[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) c = tq == static_cast<uint32_t>(i) ? ctr[i] : c;
    alpha = alpha + bf16r(c * au);
    code |= sb << j;
    packed |= ((sb << 3) | tq) << (4 * j);
  }
  alpha = fmaxf(alpha, 1e-6f);
  const float w = bf16r((rad / alpha) * knorm);
  if (row < p.rows) {
    const int tt = p.t0 + t;
    p.code[b * p.c_sb + h * p.c_sh + blk * p.c_sB + tt] = static_cast<uint8_t>(code);
    p.packed[b * p.p_sb + h * p.p_sh + blk * p.p_sB + tt] = packed;
    p.weight[b * p.w_sb + h * p.w_sh + blk * p.w_sB + tt] = f32_to_bf16_bits(w);
  }
}

__global__ __launch_bounds__(256) void rabitq4_query_kernel(const uint16_t* __restrict__ q, int64_t q_sr,
                                                             int rows, const uint16_t* __restrict__ signs,
                                                             uint16_t* __restrict__ q_blocks,
                                                             uint16_t* __restrict__ q_norm) {
  const int row = (blockIdx.x * 256 + threadIdx.x) >> 4;
  const int blk = threadIdx.x & 15;
  const int r = row < rows ? row : rows - 1;
  float x[8], sg[8], y[8];
  load_row8(q + r * q_sr + 8 * blk, x);
  load_row8(signs + 8 * blk, sg);
  const float nrm = srht_unit_block(x, sg, blk, y);
  if (row < rows) {
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = static_cast<uint32_t>(f32_to_bf16_bits(y[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(y[2 * i + 1])) << 16);
    *reinterpret_cast<u32x4_t*>(q_blocks + static_cast<int64_t>(r) * kDim + 8 * blk) = o;
    if (blk == 0) q_norm[r] = f32_to_bf16_bits(nrm);
  }
}

struct RerankParams {
  const int64_t* cand;
  int64_t cd_sb, cd_sh;
  int C, kv, kv_len;
  const uint32_t* packed;
  int64_t p_sb, p_sh, p_sB, p_st;  // 4-byte units
  const uint16_t* weight;
  int64_t w_sb, w_sh, w_sB;
  const uint16_t* q_blocks;  // [bs * kv, 16, 8] contiguous
  const uint16_t* q_norm;    // [bs * kv]
  const uint16_t* centers;   // bf16 [8]
  uint16_t* scores;          // bf16 [bs, kv, C] contiguous (optional)
  float* scores_f32;         // the same values as fp32 (optional)
  uint16_t* v4b;             // bf16 [bs, kv, 16, C, 8] (optional)
};

constexpr int kRerankThreads = 256;

// The bf16 products bf16(+-center[t] * q[b][j]) of every (block b, dimension
// j, 4-bit value v) into LDS at (8 b + j) * 16 + v: 16 consecutive fp32
// entries per (block, dimension), so any 4-bit values of a wave read 16
// distinct banks (conflict-free).
__device__ __forceinline__ void build_products(float* prod, const uint16_t* qb, const uint16_t* centers) {
  for (int e = threadIdx.x; e < kBlk * 8 * 16; e += blockDim.x) {
    const int v = e & 15, bj = e >> 4;  // bj = 8 * block + j
    const float c = bf16_to_f32(centers[v & 7]);
    prod[e] = bf16r((v & 8 ? c : -c) * bf16_to_f32(qb[bj]));
  }
}

// The score of one candidate from its 16 code words and 16 bf16 weights
// (all requested before the first is used): per block the sequential bf16
// sum of the 8 products, times the weight (bf16), added in block order
// (bf16), times ||q|| (bf16).
__device__ __forceinline__ float score_one(const float* prod, const uint32_t code[kBlk], const uint16_t wb[kBlk],
                                           float qn) {
  float res = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlk; ++i) {
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) dot = bf16r(dot + prod[(8 * i + j) * 16 + ((code[i] >> (4 * j)) & 15u)]);
    res = bf16r(res + bf16r(dot * bf16_to_f32(wb[i])));
  }
  return bf16r(res * qn);
}

// Direct path: one thread per candidate, its 16 code words and 16 weights
// gathered from wherever they lie.  A candidate index outside [0, kv_len)
// scores -inf and loads nothing.
__global__ __launch_bounds__(kRerankThreads) void rabitq4_rerank_kernel(const RerankParams p) {
  __shared__ float prod[kBlk * 8 * 16];
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * p.kv + h;
  build_products(prod, p.q_blocks + bh * kDim, p.centers);
  __syncthreads();
  const int ci = blockIdx.x * kRerankThreads + threadIdx.x;
  if (ci >= p.C) return;
  const int64_t idx = p.cand[b * p.cd_sb + h * p.cd_sh + ci];
  const int64_t out = bh * p.C + ci;
  const bool ok = idx >= 0 && idx < p.kv_len;
  float res = -INFINITY;
  if (ok) {
    const uint32_t* pk = p.packed + b * p.p_sb + h * p.p_sh + idx * p.p_st;
    const uint16_t* wt = p.weight + b * p.w_sb + h * p.w_sh + idx;
    uint32_t code[kBlk];
    uint16_t wb[kBlk];
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      code[i] = pk[i * p.p_sB];
      wb[i] = wt[i * p.w_sB];
    }
    res = score_one(prod, code, wb, bf16_to_f32(p.q_norm[bh]));
    if (p.v4b) {
      for (int i = 0; i < kBlk; ++i) {
        u32x4_t o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t two = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const uint32_t v = (code[i] >> (4 * (2 * k + e))) & 15u;
            const uint32_t cb = p.centers[v & 7];
            two |= (v & 8 ? cb : cb ^ 0x8000u) << (16 * e);
          }
          o[k] = two;
        }
        *reinterpret_cast<u32x4_t*>(p.v4b + ((bh * kBlk + i) * p.C + ci) * 8) = o;
      }
    }
  } else if (p.v4b) {
    for (int i = 0; i < kBlk; ++i)
      *reinterpret_cast<u32x4_t*>(p.v4b + ((bh * kBlk + i) * p.C + ci) * 8) = u32x4_t{0u, 0u, 0u, 0u};
  }
  if (p.scores) p.scores[out] = f32_to_bf16_bits(res);
  if (p.scores_f32) p.scores_f32[out] = res;
}

// ---- streamed path ----------------------------------------------------------
// In the reference's [16, seq] layout the 16 code words of a token lie 4*seq
// bytes apart, so a gather touches 32 lines per candidate; with the
// candidates a few percent of the tokens or more, nearly every line is read
// anyway.  The streamed path reads the layout in token order instead:
//   mark    : a flag byte per candidate token (plain stores; repeats store
//             the same 1);
//   stream  : each workgroup owns kStreamTokens tokens, reads their flags
//             (4 per thread), compacts the flagged tokens in LDS, clears the
//             flags it read (so the workspace is zero again for the next
//             call), scores the flagged tokens and writes one fp32 score per
//             flagged token;
//   collect : every candidate (repeats included) takes its token's score.
// The scores are the direct path's, bit for bit.
constexpr int kStreamThreads = 256;
constexpr int kStreamTokens = 4 * kStreamThreads;

// Flag bytes per (batch, head) row: kv_len rounded up to whole windows, so
// every window reads whole, in-bounds flag words (those past kv_len stay 0).
int64_t flag_row(int kv_len) {
  return (static_cast<int64_t>(kv_len) + kStreamTokens - 1) / kStreamTokens * kStreamTokens;
}

__global__ __launch_bounds__(256) void rabitq4_mark_kernel(const RerankParams p, uint8_t* __restrict__ flags,
                                                           int64_t frow) {
  const int ci = blockIdx.x * 256 + threadIdx.x;
  if (ci >= p.C) return;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t idx = p.cand[b * p.cd_sb + h * p.cd_sh + ci];
  if (idx < 0 || idx >= p.kv_len) return;
  flags[(static_cast<int64_t>(b) * p.kv + h) * frow + idx] = 1;
}

__global__ __launch_bounds__(kStreamThreads) void rabitq4_stream_kernel(const RerankParams p,
                                                                        uint8_t* __restrict__ flags, int64_t frow,
                                                                        float* __restrict__ tok_score) {
  __shared__ float prod[kBlk * 8 * 16];
  __shared__ int list[kStreamTokens];
  __shared__ int wave_total[kStreamThreads / 64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * p.kv + h;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kStreamTokens;
  // flags of tokens t0 + 4 tid .. t0 + 4 tid + 3 (bytes of 0 or 1), read first
  uint32_t* fw = reinterpret_cast<uint32_t*>(flags + bh * frow + t0) + tid;
  const uint32_t f = *fw;
  build_products(prod, p.q_blocks + bh * kDim, p.centers);
  // the tokens to score: flag bit 0 set and inside the row (a flag byte
  // other than 0 / 1, or one past kv_len, costs at most extra work and is
  // never counted without a list entry)
  uint32_t sel = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    sel |= (((f >> (8 * j)) & 1u) && t0 + 4 * tid + j < p.kv_len) ? 1u << j : 0u;
  const int cnt = __popc(sel);
  int inc = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {  // inclusive scan over the wave
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wave_total[wave] = inc;
  if (f) *fw = 0u;
  __syncthreads();
  int off = inc - cnt, n = 0;
#pragma unroll
  for (int w = 0; w < kStreamThreads / 64; ++w) {
    off += w < wave ? wave_total[w] : 0;
    n += wave_total[w];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if ((sel >> j) & 1u) list[off++] = 4 * tid + j;
  __syncthreads();
  const float qn = bf16_to_f32(p.q_norm[bh]);
  for (int i = tid; i < n; i += kStreamThreads) {
    const int64_t t = t0 + list[i];
    const uint32_t* pk = p.packed + b * p.p_sb + h * p.p_sh + t * p.p_st;
    const uint16_t* wt = p.weight + b * p.w_sb + h * p.w_sh + t;
    uint32_t code[kBlk];
    uint16_t wb[kBlk];
#pragma unroll
    for (int k = 0; k < kBlk; ++k) {
      code[k] = pk[k * p.p_sB];
      wb[k] = wt[k * p.w_sB];
    }
    tok_score[bh * p.kv_len + t] = score_one(prod, code, wb, qn);
  }
}

__global__ __launch_bounds__(256) void rabitq4_collect_kernel(const RerankParams p,
                                                              const float* __restrict__ tok_score) {
  const int ci = blockIdx.x * 256 + threadIdx.x;
  if (ci >= p.C) return;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * p.kv + h;
  const int64_t idx = p.cand[b * p.cd_sb + h * p.cd_sh + ci];
  const float s = (idx >= 0 && idx < p.kv_len) ? tok_score[bh * p.kv_len + idx] : -INFINITY;
  const int64_t out = bh * p.C + ci;
  if (p.scores) p.scores[out] = f32_to_bf16_bits(s);
  if (p.scores_f32) p.scores_f32[out] = s;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t stream_flag_bytes(int bs, int kv, int kv_len) {
  return (static_cast<int64_t>(bs) * kv * flag_row(kv_len) + 255) / 256 * 256;
}

size_t stream_workspace_bytes(int bs, int kv, int kv_len) {
  return static_cast<size_t>(stream_flag_bytes(bs, kv, kv_len) + static_cast<int64_t>(bs) * kv * kv_len * 4);
}

// The streamed path pays for reading every line of the codes; it wins once
// the candidates are dense enough that the direct gathers touch them all
// (C >= kv_len / 16).
bool use_stream(int C, int kv_len) { return static_cast<int64_t>(C) * 16 >= kv_len; }


}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" int zkv_rabitq4_encode(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st, int bs,
                                  int kv, int n, const uint16_t* signs, const uint16_t* mag_thresholds,
                                  const uint16_t* mag_centers, uint8_t* code, int64_t c_sb, int64_t c_sh,
                                  int64_t c_sB, uint8_t* packed, int64_t p_sb, int64_t p_sh, int64_t p_sB,
                                  uint16_t* weight, int64_t w_sb, int64_t w_sh, int64_t w_sB, int t0,
                                  zkv_stream_t stream) {
  ZKV_REQUIRE(keys && signs && mag_thresholds && mag_centers && code && packed && weight,
              "zkv_rabitq4_encode: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && n >= 0 && t0 >= 0, "zkv_rabitq4_encode: bad sizes bs=%d kv=%d n=%d t0=%d", bs,
              kv, n, t0);
  if (n == 0) return 0;
  ZKV_REQUIRE(aligned16(keys) && k_st % 8 == 0 && k_sh % 8 == 0 && k_sb % 8 == 0 && aligned16(signs),
              "zkv_rabitq4_encode: key rows and the sign vector must be 16-byte aligned (row stride %lld elements)",
              static_cast<long long>(k_st));
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(packed) & 3u) == 0,
              "zkv_rabitq4_encode: the 4-bit codes must be 4-byte aligned");
  EncodeParams p{};
  p.thr = mag_thresholds;
  p.ctr = mag_centers;
  p.keys = keys;
  p.k_sb = k_sb;
  p.k_sh = k_sh;
  p.k_st = k_st;
  p.kv = kv;
  p.n = n;
  p.t0 = t0;
  p.signs = signs;
  p.code = code;
  p.c_sb = c_sb;
  p.c_sh = c_sh;
  p.c_sB = c_sB;
  p.packed = reinterpret_cast<uint32_t*>(packed);
  p.p_sb = p_sb;
  p.p_sh = p_sh;
  p.p_sB = p_sB;
  p.weight = weight;
  p.w_sb = w_sb;
  p.w_sh = w_sh;
  p.w_sB = w_sB;
  p.rows = static_cast<int64_t>(bs) * kv * n;
  const int64_t blocks = (p.rows * 16 + 255) / 256;
  ZKV_REQUIRE(blocks < (1ll << 31), "zkv_rabitq4_encode: too many rows (%lld)", static_cast<long long>(p.rows));
  rabitq4_encode_kernel<<<static_cast<unsigned>(blocks), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(p);
  return check_launch("rabitq4_encode_kernel");
}

extern "C" int zkv_rabitq4_encode_query(const uint16_t* q, int64_t q_sr, int rows, const uint16_t* signs,
                                        uint16_t* q_blocks, uint16_t* q_norm, zkv_stream_t stream) {
  ZKV_REQUIRE(q && signs && q_blocks && q_norm, "zkv_rabitq4_encode_query: null pointer");
  ZKV_REQUIRE(rows >= 0, "zkv_rabitq4_encode_query: bad rows %d", rows);
  if (rows == 0) return 0;
  ZKV_REQUIRE(aligned16(q) && q_sr % 8 == 0 && aligned16(signs) && aligned16(q_blocks),
              "zkv_rabitq4_encode_query: query rows, the sign vector and q_blocks must be 16-byte aligned");
  const unsigned blocks = static_cast<unsigned>((static_cast<int64_t>(rows) * 16 + 255) / 256);
  rabitq4_query_kernel<<<blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(q, q_sr, rows, signs, q_blocks,
                                                                                   q_norm);
  return check_launch("rabitq4_query_kernel");
}

extern "C" size_t zkv_rabitq4_rerank_workspace_size(int bs, int kv, int kv_len) {
  if (bs <= 0 || kv <= 0 || kv_len < 0) return 0;
  return stream_workspace_bytes(bs, kv, kv_len);
}

extern "C" int zkv_rabitq4_rerank(const int64_t* cand, int64_t cd_sb, int64_t cd_sh, int bs, int kv, int C,
                                  const uint8_t* packed, int64_t p_sb, int64_t p_sh, int64_t p_sB, int64_t p_st,
                                  int kv_len, const uint16_t* weight, int64_t w_sb, int64_t w_sh, int64_t w_sB,
                                  const uint16_t* q_blocks, const uint16_t* q_norm, const uint16_t* mag_centers,
                                  uint16_t* scores, float* scores_f32, uint16_t* v4b, void* workspace,
                                  size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(bs > 0 && kv > 0 && C >= 0 && kv_len >= 0, "zkv_rabitq4_rerank: bad sizes bs=%d kv=%d C=%d kv_len=%d",
              bs, kv, C, kv_len);
  if (C == 0) return 0;  // (empty arrays may come as null pointers)
  // with kv_len == 0 every candidate scores -inf and no code is read
  ZKV_REQUIRE(cand && q_blocks && q_norm && mag_centers && (kv_len == 0 || (packed && weight)),
              "zkv_rabitq4_rerank: null pointer");
  ZKV_REQUIRE(scores || scores_f32, "zkv_rabitq4_rerank: no output");
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(packed) & 3u) == 0 && (!v4b || aligned16(v4b)),
              "zkv_rabitq4_rerank: the 4-bit codes must be 4-byte aligned and v4b 16-byte aligned");
  RerankParams p{};
  p.cand = cand;
  p.cd_sb = cd_sb;
  p.cd_sh = cd_sh;
  p.C = C;
  p.kv = kv;
  p.kv_len = kv_len;
  p.packed = reinterpret_cast<const uint32_t*>(packed);
  p.p_sb = p_sb;
  p.p_sh = p_sh;
  p.p_sB = p_sB;
  p.p_st = p_st;
  p.weight = weight;
  p.w_sb = w_sb;
  p.w_sh = w_sh;
  p.w_sB = w_sB;
  p.q_blocks = q_blocks;
  p.q_norm = q_norm;
  p.centers = mag_centers;
  p.scores = scores;
  p.scores_f32 = scores_f32;
  p.v4b = v4b;
  const dim3 grid((C + kRerankThreads - 1) / kRerankThreads, kv, bs);
  ZKV_REQUIRE(kv < 65536 && bs < 65536, "zkv_rabitq4_rerank: grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (workspace && !v4b && kv_len > 0 && use_stream(C, kv_len)) {
    const size_t need = stream_workspace_bytes(bs, kv, kv_len);
    ZKV_REQUIRE(workspace_bytes >= need && aligned16(workspace),
                "zkv_rabitq4_rerank: workspace of %zu bytes (16-byte aligned) needed, got %zu", need,
                workspace_bytes);
    const int64_t frow = flag_row(kv_len);
    uint8_t* flags = static_cast<uint8_t*>(workspace);
    float* tok = reinterpret_cast<float*>(flags + stream_flag_bytes(bs, kv, kv_len));
    rabitq4_mark_kernel<<<grid, 256, 0, s>>>(p, flags, frow);
    if (int rc = check_launch("rabitq4_mark_kernel")) return rc;
    const dim3 sgrid(static_cast<unsigned>(frow / kStreamTokens), kv, bs);
    rabitq4_stream_kernel<<<sgrid, kStreamThreads, 0, s>>>(p, flags, frow, tok);
    if (int rc = check_launch("rabitq4_stream_kernel")) return rc;
    rabitq4_collect_kernel<<<grid, 256, 0, s>>>(p, tok);
    return check_launch("rabitq4_collect_kernel");
  }
  rabitq4_rerank_kernel<<<grid, kRerankThreads, 0, s>>>(p);
  return check_launch("rabitq4_rerank_kernel");
}
