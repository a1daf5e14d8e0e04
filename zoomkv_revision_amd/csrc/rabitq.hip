// RaBitQ 1-bit sign codes and the estimate -> top-k -> exact-rerank search
// (gfx950).
//
// Code of a 128-dim fp16 vector x (one SRHT round, PC:1147-1160 pieces):
//   y = H (sigma * x), H the Sylvester Walsh-Hadamard butterfly
//   (Z/cache_hub/hadamard_fallback.py:16-23), sigma a +-1 vector;
//   bit b of byte j = (y[8j + b] >= 0);  factors (fp16) = (||x||, ||y|| sqrt(128) / sum|y|).
// Estimate of <q, k>:  ((nk*ck) * (nq*cq)) * (128 - 2 popc(xq ^ xk)) * 2^-7
//   (the sign-sign identity of Z/cache_hub/rerank/coarse_2bit_score.cu:12-16).
// Exact rerank: fp32 dot of the fp16 query and key, 16 lanes x 8 dims, then a
//   xor butterfly 8, 4, 2, 1.
//
// Search = three launches:
//   1. encode the queries (codes + factors into the workspace);
//   2. per (pool, query, slice of 4096 or 8192 keys): estimates computed on the fly
//      (nothing of size queries x keys is stored), exact top-k of the slice;
//   3. per (pool, query): exact top-k of the slices' candidates, exact rerank
//      of those k, bitonic sort by (score desc, index asc).
// The global top-k under the strict order (key desc, index asc) is the top-k
// of the union of per-slice top-k sets, so the two-level select is exact.
#include "zkv_common.hpp"

namespace zkv {
namespace {

constexpr int kD = 128;
constexpr float kSqrt128 = 11.313708498984761f;  // fp32(sqrt(128))

__device__ __forceinline__ uint32_t ordered_key_f(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ----------------------------------------------------------------------------
// Encode: one thread per vector (its sums are sequential in dimension order).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rabitq_encode_kernel(
    const uint16_t* __restrict__ x, int64_t row_stride, int64_t n, const float* __restrict__ signs,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ factors) {
  __shared__ float s_sign[kD];
  if (threadIdx.x < kD) s_sign[threadIdx.x] = signs[threadIdx.x];
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(x + i * row_stride);
  float y[kD];
  float nsq = 0.0f;
#pragma unroll
  for (int c = 0; c < kD / 8; ++c) {
    const u32x4_t w = row[c];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t h = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
      const float v = f16_to_f32(h);
      nsq = nsq + v * v;
      y[8 * c + e] = v * s_sign[8 * c + e];
    }
  }
#pragma unroll
  for (int h = 1; h < kD; h <<= 1) {
#pragma unroll
    for (int b0 = 0; b0 < kD; b0 += 2 * h) {
#pragma unroll
      for (int j = 0; j < h; ++j) {
        const float a = y[b0 + j], b = y[b0 + j + h];
        y[b0 + j] = a + b;
        y[b0 + j + h] = a - b;
      }
    }
  }
  float ysq = 0.0f, yabs = 0.0f;
  u32x4_t code = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int d = 0; d < kD; ++d) {
    ysq = ysq + y[d] * y[d];
    yabs = yabs + fabsf(y[d]);
    code[d >> 5] |= static_cast<uint32_t>(y[d] >= 0.0f) << (d & 31);
  }
  const float norm = sqrtf(nsq);
  const float corr = yabs > 0.0f ? (sqrtf(ysq) * kSqrt128) / yabs : 0.0f;
  *reinterpret_cast<u32x4_t*>(codes + i * 16) = code;
  reinterpret_cast<uint32_t*>(factors)[i] =
      static_cast<uint32_t>(f32_to_f16_bits(norm)) | (static_cast<uint32_t>(f32_to_f16_bits(corr)) << 16);
}

// Estimate of one (query, key) pair; q code / factor product held by the caller.
__device__ __forceinline__ float rabitq_estimate(u32x4_t qc, float fq, u32x4_t kc, uint32_t kf) {
  const int p = __popc(qc[0] ^ kc[0]) + __popc(qc[1] ^ kc[1]) + __popc(qc[2] ^ kc[2]) +
                __popc(qc[3] ^ kc[3]);
  const float fk = f16_to_f32(static_cast<uint16_t>(kf)) * f16_to_f32(static_cast<uint16_t>(kf >> 16));
  float t = fq * fk;
  t = t * static_cast<float>(kD - 2 * p);
  return t * 0.0078125f;
}

// popc(a ^ b) over 128 bits as one chain of count-and-add instructions
__device__ __forceinline__ int popc_xor128(u32x4_t a, u32x4_t b) {
  uint32_t pc;
  asm("v_bcnt_u32_b32 %0, %1, 0" : "=v"(pc) : "v"(a[0] ^ b[0]));
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(pc) : "v"(a[1] ^ b[1]), "v"(pc));
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(pc) : "v"(a[2] ^ b[2]), "v"(pc));
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(pc) : "v"(a[3] ^ b[3]), "v"(pc));
  return static_cast<int>(pc);
}

// lane L of v = the (uniform) value x
template <int L>
__device__ __forceinline__ void write_lane(uint32_t& v, uint32_t x) {
  asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(x), "n"(L));
}

// The filter's per-register step for the 32 x 32 result of query rows
// 32 RB .. 32 RB + 31: register R holds rows 8 (R / 4) + R % 4 (lanes 0-31)
// and + 4 (lanes 32-63) against column lane % 32; the compare's lane mask
// halves are those two queries' hit words, written into their lanes
template <int RB, int R>
struct FilterEpilogue {
  static __device__ __forceinline__ void run(const i32x16_t& acc, const float (&fqr)[16], const float (&tr)[16],
                                             float fk, uint32_t& h) {
    float e = fqr[R] * fk;  // rabitq_estimate's operations up to the 2^-7 scale
    e = e * static_cast<float>(acc[R]);
    const uint64_t m = __builtin_amdgcn_ballot_w64(!(e < tr[R]));  // NaN estimates are candidates too
    constexpr int q0 = 32 * RB + 8 * (R >> 2) + (R & 3);
    write_lane<q0>(h, static_cast<uint32_t>(m));
    write_lane<q0 + 4>(h, static_cast<uint32_t>(m >> 32));
    FilterEpilogue<RB, R + 1>::run(acc, fqr, tr, fk, h);
  }
};
template <int RB>
struct FilterEpilogue<RB, 16> {
  static __device__ __forceinline__ void run(const i32x16_t&, const float (&)[16], const float (&)[16], float,
                                             uint32_t&) {}
};

__device__ __forceinline__ float query_factor(const uint16_t* fac_q, int64_t pq) {
  const uint32_t f = reinterpret_cast<const uint32_t*>(fac_q)[pq];
  return f16_to_f32(static_cast<uint16_t>(f)) * f16_to_f32(static_cast<uint16_t>(f >> 16));
}

// Full estimate matrix out[pool, query, key] (a utility and the test hook for
// the estimate's bits).  Thread per key, grid (key tiles, query, pool).
__global__ __launch_bounds__(256) void rabitq_estimate_kernel(
    const uint8_t* __restrict__ codes_q, const uint16_t* __restrict__ fac_q,
    const uint8_t* __restrict__ codes_k, const uint16_t* __restrict__ fac_k, int64_t n, int queries,
    float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t pool = blockIdx.z;
  const int64_t pq = pool * queries + blockIdx.y;
  if (i >= n) return;
  const u32x4_t qc = *reinterpret_cast<const u32x4_t*>(codes_q + pq * 16);
  const float fq = query_factor(fac_q, pq);
  const int64_t row = pool * n + i;
  const u32x4_t kc = *reinterpret_cast<const u32x4_t*>(codes_k + row * 16);
  const uint32_t kf = reinterpret_cast<const uint32_t*>(fac_k)[row];
  out[pq * n + i] = rabitq_estimate(qc, fq, kc, kf);
}

// ----------------------------------------------------------------------------
// Wave primitives on DPP (row shifts / rotations / broadcasts inside the
// VALU) and ds_swizzle: no LDS bank traffic.
// ----------------------------------------------------------------------------
// lanes whose DPP source lies outside the row (or in a masked row) read 0
#define ZKV_DPP0(v, ctrl, row_mask) __builtin_amdgcn_update_dpp(0, (v), (ctrl), (row_mask), 0xF, false)
#define ZKV_ROR(v, n) __builtin_amdgcn_update_dpp((v), (v), 0x120 + (n), 0xF, 0xF, false)

// inclusive prefix sum over the wave's lanes
__device__ __forceinline__ int wave_incl_sum(int v) {
  v += ZKV_DPP0(v, 0x111, 0xF);  // row_shr:1
  v += ZKV_DPP0(v, 0x112, 0xF);  // row_shr:2
  v += ZKV_DPP0(v, 0x114, 0xF);  // row_shr:4
  v += ZKV_DPP0(v, 0x118, 0xF);  // row_shr:8: each 16-lane row scanned
  v += ZKV_DPP0(v, 0x142, 0xA);  // row_bcast:15 into rows 1, 3
  v += ZKV_DPP0(v, 0x143, 0xC);  // row_bcast:31 into rows 2, 3
  return v;
}

// every lane of each 16-lane row gets the row's max / min / sum
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 8)));
  v = max(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 4)));
  v = max(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 2)));
  return max(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 1)));
}
__device__ __forceinline__ uint32_t row_min_u32(uint32_t v) {
  v = min(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 8)));
  v = min(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 4)));
  v = min(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 2)));
  return min(v, static_cast<uint32_t>(ZKV_ROR(static_cast<int>(v), 1)));
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
// wave-uniform reductions
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row_max_u32(v);
  return max(max(lane_u32(v, 0), lane_u32(v, 16)), max(lane_u32(v, 32), lane_u32(v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = row_min_u32(v);
  return min(min(lane_u32(v, 0), lane_u32(v, 16)), min(lane_u32(v, 32), lane_u32(v, 48)));
}
// value of lane (l ^ X) inside the lane's 32-lane half (X < 32)
template <int X>
__device__ __forceinline__ int swizzle_xor(int v) {
  return __builtin_amdgcn_ds_swizzle(v, 0x1F | (X << 10));
}

// ----------------------------------------------------------------------------
// Block primitives for NT threads (multiple of 64)
// ----------------------------------------------------------------------------
template <int NT>
struct Block {
  static constexpr int kWaves = NT / 64;

  // exclusive prefix sum over threads (thread order) and the block total
  __device__ static int excl_scan(int v, int* s_tmp, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int incl = wave_incl_sum(v);
    if (lane == 63) s_tmp[wave] = incl;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int c = s_tmp[w];
      before += (w < wave) ? c : 0;
      total += c;
    }
    __syncthreads();
    return before + incl - v;
  }

  __device__ static void minmax(uint32_t& mn, uint32_t& mx, uint32_t* s_tmp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    mn = wave_min_u32(mn);
    mx = wave_max_u32(mx);
    if (lane == 0) {
      s_tmp[wave] = mn;
      s_tmp[kWaves + wave] = mx;
    }
    __syncthreads();
    mn = s_tmp[0];
    mx = s_tmp[kWaves];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      mn = min(mn, s_tmp[w]);
      mx = max(mx, s_tmp[kWaves + w]);
    }
    __syncthreads();
  }
};

struct SelectSmem {
  int* hist;        // [kWaves][256]
  uint32_t* tmp;    // >= 2 * kWaves words
  int* bin;         // 2 ints: bin, count above the bin
};

// k-th largest key among the valid items (thread t holds NI keys; valid_n
// counts its leading valid items).  Returns T and how many items == T are to
// be taken (lowest positions first).  Digits are taken from the current
// candidate range [lo, hi], 8 bits below its top bit, so a narrow
// distribution still spreads over the 256 bins; each round shrinks the range
// by at least 128x.  The block holds at least k valid items.
template <int NT, int NI>
__device__ void radix_select(const uint32_t (&key)[NI], int valid_n, int k, const SelectSmem& sm,
                             uint32_t& T, int& take_eq) {
  constexpr int W = Block<NT>::kWaves;
  const int tid = threadIdx.x, wave = tid >> 6;
  uint32_t lo = 0u, hi = 0xFFFFFFFFu;
  int rem = k;
  while (true) {
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if (j < valid_n && key[j] >= lo && key[j] <= hi) {
        mn = min(mn, key[j]);
        mx = max(mx, key[j]);
      }
    }
    Block<NT>::minmax(mn, mx, sm.tmp);
    lo = mn;
    hi = mx;
    if (lo == hi) break;
    const int bits = 32 - __clz(static_cast<int>(hi - lo));
    const int shift = bits > 8 ? bits - 8 : 0;
    for (int i = tid; i < W * 256; i += NT) sm.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if (j < valid_n && key[j] >= lo && key[j] <= hi)
        atomicAdd(&sm.hist[wave * 256 + ((key[j] - lo) >> shift)], 1);
    }
    __syncthreads();
    for (int b = tid; b < 256; b += NT) {
      int c = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) c += sm.hist[w * 256 + b];
      sm.hist[b] = c;
    }
    __syncthreads();
    if (tid < 64) {
      int c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = sm.hist[4 * tid + j];
      const int lane_sum = c[0] + c[1] + c[2] + c[3];
      int suf = lane_sum;  // inclusive suffix sum over lanes (lane 63 = top bins)
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_down(suf, off);
        if (tid + off < 64) suf += v;
      }
      int above = suf - lane_sum;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const int at_or_above = above + c[j];
        if (at_or_above >= rem && above < rem) {
          sm.bin[0] = 4 * tid + j;
          sm.bin[1] = above;
        }
        above = at_or_above;
      }
    }
    __syncthreads();
    const uint32_t b = static_cast<uint32_t>(sm.bin[0]);
    rem -= sm.bin[1];
    __syncthreads();
    const uint64_t new_lo = static_cast<uint64_t>(lo) + (static_cast<uint64_t>(b) << shift);
    const uint64_t new_hi = new_lo + (1ull << shift) - 1ull;
    lo = static_cast<uint32_t>(new_lo);
    hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
    if (shift == 0) break;
  }
  T = lo;
  take_eq = rem;
}

// Ordered compaction after radix_select: the selected items' slots in the
// block's output (positions in thread-major order = increasing item order).
// Calls emit(j, out_pos) for every selected item j of this thread.
template <int NT, int NI, typename Emit>
__device__ void compact_selected(const uint32_t (&key)[NI], int valid_n, uint32_t T, int take_eq_total,
                                 int* s_tmp, Emit&& emit) {
  int cnt_gt = 0, cnt_eq = 0;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    if (j < valid_n) {
      cnt_gt += key[j] > T;
      cnt_eq += key[j] == T;
    }
  }
  int eq_total = 0;
  const int eq_before = Block<NT>::excl_scan(cnt_eq, s_tmp, eq_total);
  int take = take_eq_total - eq_before;
  take = take < 0 ? 0 : (take > cnt_eq ? cnt_eq : take);
  int sel_total = 0;
  int pos = Block<NT>::excl_scan(cnt_gt + take, s_tmp, sel_total);
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    if (j < valid_n) {
      bool sel = key[j] > T;
      if (key[j] == T && take > 0) {
        sel = true;
        --take;
      }
      if (sel) emit(j, pos++);
    }
  }
}

// ----------------------------------------------------------------------------
// Stage 1: per (slice, query, pool) the exact top-k of the slice's NT * 16
// estimates.  Slices of 4096 keys (256 threads) when the per-query candidate
// list (slices x k) stays within kMaxCand2, else 8192 (512 threads): the
// smaller blocks' selection rounds are cheaper (C4: about 7% per search).
// Keys are loaded coalesced (position j*NT + t), their ordered estimates
// transposed through LDS so thread t owns positions t*NI .. t*NI+NI-1.
// Output: k (key, index) pairs in increasing index order; slices with fewer
// than k keys pad with index -1.
// ----------------------------------------------------------------------------
constexpr int kNI1 = 16;  // keys per thread (the LDS transpose pads one word per 16)
constexpr int kNT2 = 1024, kNI2 = 8, kMaxCand2 = kNT2 * kNI2;
constexpr int kMaxTopk = 1024;

template <int kNT1>
__global__ __launch_bounds__(kNT1) void rabitq_stage1_kernel(
    const uint8_t* __restrict__ codes_q, const uint16_t* __restrict__ fac_q,
    const uint8_t* __restrict__ codes_k, const uint16_t* __restrict__ fac_k, int64_t n, int queries,
    int k, uint32_t* __restrict__ cand_key, int32_t* __restrict__ cand_idx) {
  constexpr int W = Block<kNT1>::kWaves;
  constexpr int kSlice1 = kNT1 * kNI1;
  // LDS: the transposed keys (one pad word per 16), then reused as histograms
  __shared__ uint32_t s_keys[kSlice1 + kSlice1 / 16];
  __shared__ uint32_t s_tmp[2 * W + 2];
  const int tid = threadIdx.x;
  const int slice = blockIdx.x, n_slices = gridDim.x;
  const int64_t pool = blockIdx.z;
  const int64_t pq = pool * queries + blockIdx.y;
  const int64_t s0 = static_cast<int64_t>(slice) * kSlice1;
  const int n_here = static_cast<int>(n - s0 < kSlice1 ? n - s0 : kSlice1);

  const u32x4_t qc = *reinterpret_cast<const u32x4_t*>(codes_q + pq * 16);
  const float fq = query_factor(fac_q, pq);
  const u32x4_t* kc = reinterpret_cast<const u32x4_t*>(codes_k) + pool * n + s0;
  const uint32_t* kf = reinterpret_cast<const uint32_t*>(fac_k) + pool * n + s0;
#pragma unroll
  for (int j = 0; j < kNI1; ++j) {
    const int p = j * kNT1 + tid;
    if (p < n_here) s_keys[p + (p >> 4)] = ordered_key_f(rabitq_estimate(qc, fq, kc[p], kf[p]));
  }
  __syncthreads();
  uint32_t key[kNI1];
  const int base = tid * kNI1;
  const int valid_n = n_here - base < 0 ? 0 : (n_here - base > kNI1 ? kNI1 : n_here - base);
#pragma unroll
  for (int j = 0; j < kNI1; ++j) key[j] = s_keys[base + j + tid];  // (base+j) + (base+j)/16
  __syncthreads();

  uint32_t* out_key = cand_key + (pq * n_slices + slice) * static_cast<int64_t>(k);
  int32_t* out_idx = cand_idx + (pq * n_slices + slice) * static_cast<int64_t>(k);
  if (n_here <= k) {
    for (int j = 0; j < kNI1; ++j) {
      const int p = base + j;
      if (p < k) {
        out_key[p] = j < valid_n ? key[j] : 0u;
        out_idx[p] = j < valid_n ? static_cast<int32_t>(s0 + p) : -1;
      }
    }
    return;
  }
  SelectSmem sm{reinterpret_cast<int*>(s_keys), s_tmp, reinterpret_cast<int*>(s_tmp + 2 * W)};
  uint32_t T;
  int take_eq;
  radix_select<kNT1, kNI1>(key, valid_n, k, sm, T, take_eq);
  compact_selected<kNT1, kNI1>(key, valid_n, T, take_eq, reinterpret_cast<int*>(s_tmp),
                               [&](int j, int pos) {
                                 out_key[pos] = key[j];
                                 out_idx[pos] = static_cast<int32_t>(s0 + base + j);
                               });
}

// ----------------------------------------------------------------------------
// Exact rerank of the k selected indices (s_sel, increasing index order) and
// the bitonic sort by (score desc, index asc) -> out_idx / out_score.
// 16-lane groups: lane l holds dims 8l .. 8l+7 of the query and the key.
// ----------------------------------------------------------------------------
template <int NT>
__device__ void rerank_and_sort(const int32_t* s_sel, int k, const uint16_t* __restrict__ qrow,
                                const uint16_t* __restrict__ kp, int64_t k_row_stride, int64_t n_keys,
                                float* s_score, uint64_t* s_sort, int64_t* __restrict__ out_idx,
                                float* __restrict__ out_score) {
  const int tid = threadIdx.x;
  const int l = tid & 15;
  const u32x4_t qw = *reinterpret_cast<const u32x4_t*>(qrow + 8 * l);
  float qf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qf[e] = f16_to_f32(static_cast<uint16_t>(qw[e >> 1] >> (16 * (e & 1))));
  for (int c0 = 0; c0 < k; c0 += NT / 16) {
    const int c = c0 + (tid >> 4);
    float s = 0.0f;
    // the selection only yields indices inside the pool; a key row is read
    // only for such an index all the same
    const int64_t ki = c < k ? static_cast<int64_t>(s_sel[c]) : -1;
    if (ki >= 0 && ki < n_keys) {
      const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(kp + ki * k_row_stride + 8 * l);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = qf[e] * f16_to_f32(static_cast<uint16_t>(kw[e >> 1] >> (16 * (e & 1))));
        s = e == 0 ? pe : s + pe;
      }
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) s = s + __shfl_xor(s, off);
    if (c < k && l == 0) s_score[c] = s;
  }
  __syncthreads();

  // bitonic sort (descending) of (ordered score of +-0 -> +0, 0xFFFF - slot);
  // slots are in increasing index order, so ties go to the lower index
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = tid; i < P; i += NT)
    s_sort[i] = i < k ? (static_cast<uint64_t>(ordered_key_f(s_score[i] + 0.0f)) << 32) |
                            static_cast<uint64_t>(0xFFFFu - static_cast<uint32_t>(i))
                      : 0ull;
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int i = tid; i < P / 2; i += NT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = s_sort[lo], b = s_sort[hi];
        if ((a < b) == desc) {
          s_sort[lo] = b;
          s_sort[hi] = a;
        }
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < k; i += NT) {
    const int slot = static_cast<int>(0xFFFFu - static_cast<uint32_t>(s_sort[i] & 0xFFFFu));
    out_idx[i] = s_sel[slot];
    out_score[i] = s_score[slot];
  }
}

// ----------------------------------------------------------------------------
// Stage 2 of the slice path: per (query, pool): top-k of the n_cand
// candidates (positions are in increasing index order), exact rerank, sort by
// (score desc, index asc).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(kNT2) void rabitq_stage2_kernel(
    const uint32_t* __restrict__ cand_key, const int32_t* __restrict__ cand_idx, int n_cand, int n_real,
    int k, const uint16_t* __restrict__ q, const uint16_t* __restrict__ keys, int64_t k_pool_stride,
    int64_t k_row_stride, int64_t n_keys, int queries, int64_t* __restrict__ out_cand,
    int64_t* __restrict__ out_idx, float* __restrict__ out_score) {
  constexpr int W = Block<kNT2>::kWaves;
  __shared__ int s_hist[W * 256];
  __shared__ uint32_t s_tmp[2 * W + 2];
  __shared__ int32_t s_sel[kMaxTopk];
  __shared__ float s_score[kMaxTopk];
  __shared__ uint64_t s_sort[kMaxTopk];
  const int tid = threadIdx.x;
  const int64_t pool = blockIdx.y;
  const int64_t pq = pool * queries + blockIdx.x;
  const uint32_t* ck = cand_key + pq * n_cand;
  const int32_t* ci = cand_idx + pq * n_cand;

  // candidates [0, n_real) are real; only the last slice pads (index -1),
  // at its end, so every pad sits in the tail [n_real, n_cand)
  uint32_t key[kNI2];
  const int base = tid * kNI2;
  const int valid_n = n_real - base < 0 ? 0 : (n_real - base > kNI2 ? kNI2 : n_real - base);
#pragma unroll
  for (int j = 0; j < kNI2; ++j) key[j] = j < valid_n ? ck[base + j] : 0u;
  SelectSmem sm{s_hist, s_tmp, reinterpret_cast<int*>(s_tmp + 2 * W)};
  uint32_t T;
  int take_eq;
  radix_select<kNT2, kNI2>(key, valid_n, k, sm, T, take_eq);
  compact_selected<kNT2, kNI2>(key, valid_n, T, take_eq, reinterpret_cast<int*>(s_tmp),
                               [&](int j, int pos) { s_sel[pos] = ci[base + j]; });
  __syncthreads();
  for (int i = tid; i < k; i += kNT2) out_cand[pq * k + i] = s_sel[i];
  rerank_and_sort<kNT2>(s_sel, k, q + pq * kD, keys + pool * k_pool_stride, k_row_stride, n_keys, s_score,
                        s_sort, out_idx + pq * k, out_score + pq * k);
}

// ----------------------------------------------------------------------------
// Filter path (large pools, n >= 128 k): every code is read once per pass for
// all queries of its pool.
//   1. prep, per (query, pool), 4 waves: encode the query (wave 0: the FWHT
//      across lanes, the factor sums in dimension order by one lane, so the
//      bits equal rabitq_encode_kernel's), estimate a strided sample of
//      s = min(n, 2048) keys and take tau = the m-th largest sample key,
//      m = ceil(4 k s / n) (at least 8): about 4k keys of the pool are
//      expected at or above tau;
//   2. filter, one wave per 64 keys: each lane estimates its key against
//      every query (query code, factor and tau through scalar loads) and the
//      keys >= tau go to that (query, wave) list of up to kFiltCap entries in
//      increasing index order (ballot + mbcnt; no atomics, no barriers);
//   3. select, per (query, pool): the lists hold an exact superset of the
//      top-k whenever at least k keys reached tau and no list overflowed
//      (the k-th largest key is then >= tau): their exact top-k is the answer.
//      Otherwise (ties, adversarial layouts) the block selects over all n
//      keys, recomputing their estimates, so the result is exact either way.
//      Then the exact rerank and the sort by (score desc, index asc).
// ----------------------------------------------------------------------------
constexpr int kFiltWave = 64;         // keys per filter wave
constexpr int kFiltList = 256;        // keys per filter list (a 4-wave block)
constexpr int kBucketWords = 32;      // a list: 128 bytes = count, pad, 15 (key, index) pairs
constexpr int kFiltCap = 15;          // entries a list holds
constexpr int kSampleMax = 2048;      // prep: sample keys per query (64 runs of kSampleMax / 64)
constexpr int kBigNT = 1024;          // prep / select blocks
constexpr int kSelMaxPasses = 16;     // select: bucket chunks per thread (n <= 2048 lists of 256)

struct FilterPlan {
  int s_count, m;
};

// m = ceil(4 k s / n), at least 8: about 4k keys are expected at or above the
// m-th largest of s sample keys, and fewer than k only when m or more of the
// s samples land among the top k - 1 keys (expected m / 4).
FilterPlan filter_plan(int64_t n, int topk) {
  FilterPlan f{};
  f.s_count = static_cast<int>(n < kSampleMax ? n : kSampleMax);
  const int64_t m = (4ll * topk * f.s_count + n - 1) / n;
  f.m = static_cast<int>(m < 8 ? 8 : (m > f.s_count ? f.s_count : m));
  return f;
}

// select block: NT threads read NT / 8 buckets (NT 16-byte chunks) per pass,
// R passes.  1024 threads: the block's phases are latency-bound, and 16 waves
// hide more of it than 4 (256 threads took 21 us instead of 13.5 for C4)
struct SelectShape {
  int nt, passes;
};
SelectShape select_shape(int64_t n) {
  const int64_t lists = (n + kFiltList - 1) / kFiltList;
  const int nt = kBigNT;
  int r = 1;
  while (static_cast<int64_t>(nt / 8) * r < lists) r <<= 1;
  return {nt, r};
}

bool use_filter_path(int64_t n, int topk) { return n >= 128ll * topk && select_shape(n).passes <= kSelMaxPasses; }

// Threshold T and how many items equal to it to take (lowest positions
// first), such that the items > T and those taken == T are the top k among
// the valid items (bit j of `valid`: item j) of a block of NT threads holding
// NI keys each; the block holds at least k valid items, whose minimum and
// maximum are mn and mx.  T is the k-th largest item, or the lower edge of a
// bin that the top k take whole (the rounds stop there).  hist[0 .. 4095]
// must be zero, with a barrier since the clear; tmp holds W + 3 words.
// Radix rounds of 12-bit digits over LDS histograms of 4096 bins: the first
// digit is taken 12 bits below the top bit of the items' range [mn, mx],
// each later one 12 bits below the previous, so a 32-bit range takes at most
// three rounds.  Two histograms alternate (hist: 2 x 4096 ints), so a round
// clears the next one while it counts: three barriers per round.
// With first_counted the caller has done the first round's counting: every
// item into hist[(key - mn) >> radix12_first_shift(mn, mx)], hist[4096 ..
// 8191] cleared, a barrier since.
__device__ __forceinline__ int radix12_first_shift(uint32_t mn, uint32_t mx) {
  if (mn == mx) return 0;
  const int bits = 32 - __clz(static_cast<int>(mx - mn));
  return bits > 12 ? bits - 12 : 0;
}
template <int NT, int NI>
__device__ void block_radix_select12(const uint32_t (&key)[NI], uint32_t valid, int k, uint32_t mn, uint32_t mx,
                                     int* hist, uint32_t* tmp, uint32_t& T, int& take_eq,
                                     bool first_counted = false) {
  constexpr int W = NT / 64;
  constexpr int kBins = 4096, kPerT = kBins / NT;
  static_assert(kBins % NT == 0, "bins per thread");
  static_assert(NI <= 32, "validity mask");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t lo = mn, hi = mx;
  int rem = k;
  int shift = radix12_first_shift(mn, mx);
  int buf = 0;
  bool counted = first_counted;
  while (lo != hi) {
    int* h = hist + buf * kBins;
    int* h_next = hist + (buf ^ 1) * kBins;
    if (!counted) {
#pragma unroll
      for (int j = 0; j < kPerT; ++j) h_next[tid * kPerT + j] = 0;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        if (((valid >> j) & 1u) && key[j] >= lo && key[j] <= hi) atomicAdd(&h[(key[j] - lo) >> shift], 1);
      }
      __syncthreads();
    }
    counted = false;
    // thread t owns bins t*kPerT .. t*kPerT + kPerT - 1; higher threads hold higher bins
    int c[kPerT], own = 0;
#pragma unroll
    for (int j = 0; j < kPerT; ++j) {
      c[j] = h[tid * kPerT + j];
      own += c[j];
    }
    const int incl = wave_incl_sum(own);
    const int wave_total = __builtin_amdgcn_readlane(incl, 63);
    if (lane == 0) tmp[wave] = static_cast<uint32_t>(wave_total);
    __syncthreads();
    int waves_above = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) waves_above += w > wave ? static_cast<int>(tmp[w]) : 0;
    int above = waves_above + wave_total - incl;  // items in higher bins than this thread's
    if (above < rem && above + own >= rem) {       // the k-th largest lies in this thread's bins
#pragma unroll
      for (int j = kPerT - 1; j >= 0; --j) {
        const int at_or_above = above + c[j];
        if (at_or_above >= rem && above < rem) {
          tmp[W] = static_cast<uint32_t>(tid * kPerT + j);
          tmp[W + 1] = static_cast<uint32_t>(above);
          tmp[W + 2] = static_cast<uint32_t>(c[j]);
        }
        above = at_or_above;
      }
    }
    __syncthreads();
    const uint32_t b = tmp[W];
    rem -= static_cast<int>(tmp[W + 1]);
    const uint64_t new_lo = static_cast<uint64_t>(lo) + (static_cast<uint64_t>(b) << shift);
    const uint64_t new_hi = new_lo + (1ull << shift) - 1ull;
    lo = static_cast<uint32_t>(new_lo);
    hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
    if (shift == 0) break;
    // the top k take the whole bin: T = its lower edge, and rem (the bin's
    // count) covers every item == T
    if (rem == static_cast<int>(tmp[W + 2])) break;
    shift = shift > 12 ? shift - 12 : 0;
    buf ^= 1;
    // the next round's first barrier orders these reads of tmp before its rewrite
  }
  T = lo;
  take_eq = rem;
}

// ----------------------------------------------------------------------------
// 1. prep, per (query, pool), 1024 threads: every thread requests its sample
//    keys first -- s = min(n, 2048) keys in 64 runs of 32 consecutive keys
//    spread over the pool (or every key when n < 2048) -- while wave 0
//    encodes the query (the FWHT across lanes) and waves 0-2 form the three
//    factor sums in dimension order as lane chains (the bits of
//    rabitq_encode_kernel); then tau = the lower edge of the 4096-bin
//    histogram bin (over the samples' range) that holds the m-th largest
//    sample key.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(kBigNT) void rabitq_prep_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ signs, const uint8_t* __restrict__ codes_k,
    const uint16_t* __restrict__ fac_k, int64_t n, int queries, int s_count, int m,
    uint8_t* __restrict__ q_codes, uint16_t* __restrict__ q_fac, uint32_t* __restrict__ tau) {
  constexpr int NI = kSampleMax / kBigNT;
  __shared__ __attribute__((aligned(16))) float s_terms[3][kD + 4];  // x_d^2, y_d^2, |y_d| (rows 4 banks apart)
  __shared__ float s_sums[3];
  __shared__ u32x4_t s_qc;
  __shared__ int s_hist[2 * 4096];
  __shared__ uint32_t s_tmp[2 * (kBigNT / 64) + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t pool = blockIdx.y;
  const int64_t pq = pool * queries + blockIdx.x;
  // ---- sample rows first: item i of thread t is sample s = i * NT + t ----
  const u32x4_t* kc = reinterpret_cast<const u32x4_t*>(codes_k) + pool * n;
  const uint32_t* kf = reinterpret_cast<const uint32_t*>(fac_k) + pool * n;
  const int64_t blk = n / 64;  // sample run j starts at key j * blk (n >= kSampleMax)
  constexpr int kRun = kSampleMax / 64;
  u32x4_t sc[NI];
  uint32_t sf[NI];
  int valid_n = 0;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int s = i * kBigNT + tid;
    const int64_t p = s_count == kSampleMax ? (s / kRun) * blk + (s % kRun) : s;
    const bool ok = s < s_count;
    const int64_t pp = ok ? p : 0;
    sc[i] = kc[pp];
    sf[i] = kf[pp];
    valid_n += ok;  // valid items lead: s < s_count is monotone in i
  }
  if (tid < 64) {
    // ---- encode (wave 0): lane l holds dims 2l, 2l + 1 ----
    const uint32_t xw = reinterpret_cast<const uint32_t*>(q + pq * kD)[lane];
    const float x0 = f16_to_f32(static_cast<uint16_t>(xw)), x1 = f16_to_f32(static_cast<uint16_t>(xw >> 16));
    float y0 = x0 * signs[2 * lane], y1 = x1 * signs[2 * lane + 1];
    {  // h = 1: the pair sits in one lane
      const float a = y0, b = y1;
      y0 = a + b;
      y1 = a - b;
    }
    // h = 2 hl: partner lane l ^ hl (DPP for 1, 2; swizzles for 4, 8, 16)
    auto stage = [&](float p0, float p1, int hl) {
      const bool lower = (lane & hl) == 0;
      y0 = lower ? y0 + p0 : p0 - y0;
      y1 = lower ? y1 + p1 : p1 - y1;
    };
    auto fi = [](float v) { return __float_as_int(v); };
    stage(__int_as_float(__builtin_amdgcn_update_dpp(0, fi(y0), 0xB1, 0xF, 0xF, false)),
          __int_as_float(__builtin_amdgcn_update_dpp(0, fi(y1), 0xB1, 0xF, 0xF, false)), 1);
    stage(__int_as_float(__builtin_amdgcn_update_dpp(0, fi(y0), 0x4E, 0xF, 0xF, false)),
          __int_as_float(__builtin_amdgcn_update_dpp(0, fi(y1), 0x4E, 0xF, 0xF, false)), 2);
    stage(__int_as_float(swizzle_xor<4>(fi(y0))), __int_as_float(swizzle_xor<4>(fi(y1))), 4);
    stage(__int_as_float(swizzle_xor<8>(fi(y0))), __int_as_float(swizzle_xor<8>(fi(y1))), 8);
    stage(__int_as_float(swizzle_xor<16>(fi(y0))), __int_as_float(swizzle_xor<16>(fi(y1))), 16);
    stage(__shfl_xor(y0, 32), __shfl_xor(y1, 32), 32);
    // code bit d = (y_d >= 0): dims 2l / 2l + 1 are bit l of the two ballots
    const uint64_t be = __ballot(y0 >= 0.0f), bo = __ballot(y1 >= 0.0f);
    // the factor sums' terms, formed in parallel (the same products)
    s_terms[0][2 * lane] = x0 * x0;
    s_terms[0][2 * lane + 1] = x1 * x1;
    s_terms[1][2 * lane] = y0 * y0;
    s_terms[1][2 * lane + 1] = y1 * y1;
    s_terms[2][2 * lane] = fabsf(y0);
    s_terms[2][2 * lane + 1] = fabsf(y1);
    if (lane < 4) {  // word w = dims 32w .. 32w + 31 = ballot bits 16w .. 16w + 15, interleaved
      auto spread = [](uint32_t v) {  // bit i -> bit 2i (16 bits)
        v = (v | (v << 8)) & 0x00FF00FFu;
        v = (v | (v << 4)) & 0x0F0F0F0Fu;
        v = (v | (v << 2)) & 0x33333333u;
        return (v | (v << 1)) & 0x55555555u;
      };
      const uint32_t word = spread(static_cast<uint32_t>(be >> (16 * lane)) & 0xFFFFu) |
                            (spread(static_cast<uint32_t>(bo >> (16 * lane)) & 0xFFFFu) << 1);
      reinterpret_cast<uint32_t*>(q_codes + pq * 16)[lane] = word;
      reinterpret_cast<uint32_t*>(&s_qc)[lane] = word;
    }
  }
  __syncthreads();
  // ---- the factor sums (waves 0, 1, 2: sum w), each in dimension order as a
  //      chain along the lanes: step i hands the running sum from lane l - 1
  //      to lane l (DPP wave shift right), which adds dims 2l and 2l + 1; after
  //      64 steps lane 63 holds ((0 + t_0) + t_1) + ... + t_127, the encode
  //      kernel's order ----
  if (wave < 3) {
    const float2 t = reinterpret_cast<const float2*>(s_terms[wave])[lane];
    float acc = 0.0f;
#pragma unroll 16
    for (int i = 0; i < 64; ++i) {
      acc = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xF, 0xF, false)) + t.x;
      acc = acc + t.y;
    }
    if (lane == 63) s_sums[wave] = acc;
  }
  __syncthreads();
  const u32x4_t qc = s_qc;
  float fq;
  {  // the query factor (every thread; thread 0 stores it)
    const float nsq = s_sums[0], ysq = s_sums[1], yabs = s_sums[2];
    const float norm = sqrtf(nsq);
    const float corr = yabs > 0.0f ? (sqrtf(ysq) * kSqrt128) / yabs : 0.0f;
    const uint16_t hn = f32_to_f16_bits(norm), hc = f32_to_f16_bits(corr);
    if (tid == 0) reinterpret_cast<uint32_t*>(q_fac)[pq] = static_cast<uint32_t>(hn) | (static_cast<uint32_t>(hc) << 16);
    fq = f16_to_f32(hn) * f16_to_f32(hc);
  }
  uint32_t key[NI];
  uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    key[i] = ordered_key_f(rabitq_estimate(qc, fq, sc[i], sf[i]));
    if (i < valid_n) {
      mn = min(mn, key[i]);
      mx = max(mx, key[i]);
    }
  }
  constexpr int W = kBigNT / 64, kPerT = 4096 / kBigNT;
#pragma unroll
  for (int j = 0; j < kPerT; ++j) s_hist[tid * kPerT + j] = 0;
  // the samples' range: one barrier, which also orders the clear before the
  // counts (the reads of s_tmp here all precede the counts' barrier, after
  // which s_tmp is rewritten)
  mn = wave_min_u32(mn);
  mx = wave_max_u32(mx);
  if (lane == 0) {
    s_tmp[wave] = mn;
    s_tmp[W + wave] = mx;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < W; ++w) {
    mn = min(mn, s_tmp[w]);
    mx = max(mx, s_tmp[W + w]);
  }
  // one 12-bit histogram round over [mn, mx] (block_radix_select12's first
  // round): tau = the lower edge of the bin holding the m-th largest sample,
  // so at least m samples reach it; the thread owning that bin stores it
  if (mn == mx) {
    if (tid == 0) tau[pq] = mn;
    return;
  }
  const int shift = radix12_first_shift(mn, mx);
#pragma unroll
  for (int i = 0; i < NI; ++i)
    if (i < valid_n) atomicAdd(&s_hist[(key[i] - mn) >> shift], 1);
  __syncthreads();
  int c[kPerT], own = 0;
#pragma unroll
  for (int j = 0; j < kPerT; ++j) {
    c[j] = s_hist[tid * kPerT + j];
    own += c[j];
  }
  const int incl = wave_incl_sum(own);
  const int wave_total = __builtin_amdgcn_readlane(incl, 63);
  if (lane == 0) s_tmp[wave] = static_cast<uint32_t>(wave_total);
  __syncthreads();
  int above = wave_total - incl;  // samples in higher bins than this thread's
#pragma unroll
  for (int w = 0; w < W; ++w) above += w > wave ? static_cast<int>(s_tmp[w]) : 0;
  if (above < m && above + own >= m) {
#pragma unroll
    for (int j = kPerT - 1; j >= 0; --j) {
      const int at_or_above = above + c[j];
      if (at_or_above >= m && above < m)
        tau[pq] = static_cast<uint32_t>(static_cast<uint64_t>(mn) +
                                        (static_cast<uint64_t>(tid * kPerT + j) << shift));
      above = at_or_above;
    }
  }
}

// ----------------------------------------------------------------------------
// 2. filter: lane = query; a block of 4 waves covers 256 consecutive keys (a
//    list), each wave 64 of them; grid (lists, query groups of 64, pools).
//    Lane l of a wave loads key l of the wave's 64 (one coalesced request)
//    into LDS and holds query l's code, factor and tau.  The 64 x 64 +-1 dot
//    products come from int8 MFMAs, and each result register's compare gives
//    two queries' hit words over 32 keys (the mask lane = query, bit = key):
//    est >= tau compared as floats, before the final 2^-7 scale and the
//    order-preserving key, so the mask can only hold extra keys (+-0, the
//    2^-7 scale's underflow, NaN); the hits are re-checked with the exact
//    keys, unless tau is a positive normal float and every factor finite,
//    where the two compares agree.  One
//    barrier gives each wave its offset in the block's list per query.  A
//    list is a 128-byte bucket: word 0 the hit count, then the first 15 hits
//    in increasing index order as (key, index) word pairs from word 2, so
//    16-byte chunk c of a bucket holds entries 2c - 1 and 2c.  The block's 64
//    buckets are assembled in LDS and stored as whole lines.  No atomics.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rabitq_filter_kernel(
    const uint8_t* __restrict__ q_codes, const uint16_t* __restrict__ q_fac, const uint32_t* __restrict__ tau,
    const uint8_t* __restrict__ codes_k, const uint16_t* __restrict__ fac_k, int64_t n, int queries,
    int n_lists, uint32_t* __restrict__ buckets) {
  __shared__ u32x4_t s_kc[4][kFiltWave];
  __shared__ float s_fk[4][kFiltWave];
  __shared__ __attribute__((aligned(16))) float s_qf[4][2][64];  // per wave: the queries' factors, tau * 2^7
  __shared__ uint64_t s_lut[4][256];                             // per wave: byte -> 8 +-1 bytes
  __shared__ int s_cnt[4][64];
  __shared__ uint32_t s_bkt[64][kBucketWords + 1];  // the block's 64 buckets; odd stride: per-lane rows conflict-free
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int list = blockIdx.x;
  const int64_t pool = blockIdx.z;
  const int64_t p0 = static_cast<int64_t>(list) * kFiltList + wave * kFiltWave;
  const int nk = n - p0 < kFiltWave ? static_cast<int>(n - p0 > 0 ? n - p0 : 0) : kFiltWave;
  float fk;
  {
    const int64_t row = pool * n + (lane < nk ? p0 + lane : 0);
    const u32x4_t c = reinterpret_cast<const u32x4_t*>(codes_k)[row];
    const uint32_t f = reinterpret_cast<const uint32_t*>(fac_k)[row];
    s_kc[wave][lane] = c;
    fk = f16_to_f32(static_cast<uint16_t>(f)) * f16_to_f32(static_cast<uint16_t>(f >> 16));
    s_fk[wave][lane] = fk;
  }
  const int qi = blockIdx.y * 64 + lane;
  const bool q_ok = qi < queries;
  const int64_t pq = pool * queries + (q_ok ? qi : 0);
  const u32x4_t qc = *reinterpret_cast<const u32x4_t*>(q_codes + pq * 16);
  const float fq = query_factor(q_fac, pq);
  const uint32_t t = tau[pq];
  // tau as an unscaled float: est * 2^-7 >= tau  <=>  est >= tau * 2^7 (exact
  // scaling), with the float compare putting -0 with +0
  const float t128 = __uint_as_float((t & 0x80000000u) ? (t & 0x7FFFFFFFu) : ~t) * 128.0f;
  const int half = lane >> 5, col = lane & 31;
  s_qf[wave][0][lane] = fq;
  s_qf[wave][1][lane] = t128;
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // lut[x]: byte i = +1 if bit i of x, else -1
    const uint32_t x = static_cast<uint32_t>(lane + 64 * e);
    const uint32_t lo = ((x & 15u) * 0x204081u) & 0x01010101u, hi = ((x >> 4) * 0x204081u) & 0x01010101u;
    s_lut[wave][x] = static_cast<uint64_t>(~(lo * 0xFEu)) | (static_cast<uint64_t>(~(hi * 0xFEu)) << 32);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  // ---- the +-1 dot products 128 - 2 popc(q ^ k) of 64 queries (rows) x the
  //      wave's 64 keys (columns), exact in int8 MFMAs (32 x 32 x 16): two
  //      row blocks of 32 queries, two column blocks of 32 keys.  Lane l
  //      supplies row / column l % 32, dims 16 s + 8 (l / 32) .. + 7 of K
  //      step s; register r of a 32 x 32 result holds row 8 (r / 4) + 4 (l /
  //      32) + r % 4, column l % 32.  Then per register: the estimate's two
  //      multiplies (fq fk) dot, the compare with tau * 2^7 as one lane mask,
  //      whose halves are the hit words of two queries over 32 keys, written
  //      into those queries' lanes ----
  // A operands: query 32 rb + col's code (this lane's own for rb = half, the
  // lane 32 apart's for the other) as +-1 bytes
  int64_t qa[2][8];
  {
    u32x4_t other;
#pragma unroll
    for (int w = 0; w < 4; ++w) other[w] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(qc[w]), 32));
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const u32x4_t c = rb == half ? qc : other;
#pragma unroll
      for (int st = 0; st < 8; ++st)
        qa[rb][st] = static_cast<int64_t>(s_lut[wave][(c[st >> 1] >> (8 * ((2 * st + half) & 3))) & 255u]);
    }
  }
  int64_t kb[2][8];
  float fkc[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const u32x4_t c = s_kc[wave][32 * cb + col];
    fkc[cb] = s_fk[wave][32 * cb + col];
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const uint32_t x = (c[st >> 1] >> (8 * ((2 * st + half) & 3))) & 255u;
      kb[cb][st] = static_cast<int64_t>(s_lut[wave][x]);
    }
  }
  uint32_t h[2] = {0u, 0u};  // bit j of h[j / 32] (this lane's query): key j of the wave's 64 may reach tau
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    i32x16_t acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[cb] = i32x16_t{};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        acc[cb] = __builtin_amdgcn_mfma_i32_32x32x16_i8(qa[rb][st], kb[cb][st], acc[cb], 0, 0, 0);
    }
    float fqr[16], tr[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 f4 = *reinterpret_cast<const float4*>(&s_qf[wave][0][32 * rb + 8 * g + 4 * half]);
      const float4 t4 = *reinterpret_cast<const float4*>(&s_qf[wave][1][32 * rb + 8 * g + 4 * half]);
      fqr[4 * g] = f4.x; fqr[4 * g + 1] = f4.y; fqr[4 * g + 2] = f4.z; fqr[4 * g + 3] = f4.w;
      tr[4 * g] = t4.x; tr[4 * g + 1] = t4.y; tr[4 * g + 2] = t4.z; tr[4 * g + 3] = t4.w;
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      if (rb == 0)
        FilterEpilogue<0, 0>::run(acc[cb], fqr, tr, fkc[cb], h[cb]);
      else
        FilterEpilogue<1, 0>::run(acc[cb], fqr, tr, fkc[cb], h[cb]);
    }
  }
  uint64_t hits = h[0] | (static_cast<uint64_t>(h[1]) << 32);
  hits &= nk >= 64 ? ~0ull : ((1ull << nk) - 1ull);
  // exact re-check of the (few) candidates, in index order.  None is needed
  // when tau * 2^7 is a normal float in [2^-100, FLT_MAX] and no estimate can
  // be NaN (the query's and the 64 keys' factors finite, so every product is
  // finite): then a hit's estimate is >= 2^-100, its 2^-7 scale is exact and
  // ordered the same as the float compare, and a miss scales to below tau
  const bool keys_finite = __builtin_amdgcn_ballot_w64(!__builtin_isfinite(fk)) == 0;
  const bool direct = keys_finite && __builtin_isfinite(fq) && t128 >= 0x1p-100f && t128 <= 0x1.fffffep127f;
  uint64_t exact = direct ? hits : 0;
  for (uint64_t m = direct ? 0 : hits; m != 0; m &= m - 1) {
    const int j = __builtin_ctzll(m);
    const u32x4_t c = s_kc[wave][j];
    const int pc = __popc(qc[0] ^ c[0]) + __popc(qc[1] ^ c[1]) + __popc(qc[2] ^ c[2]) + __popc(qc[3] ^ c[3]);
    float est = fq * s_fk[wave][j];
    est = est * static_cast<float>(kD - 2 * pc);
    if (ordered_key_f(est * 0.0078125f) >= t) exact |= 1ull << j;
  }
  const int mine = __popcll(exact);
  s_cnt[wave][lane] = mine;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int c = s_cnt[w][lane];
    before += w < wave ? c : 0;
    total += c;
  }
  uint32_t* row = s_bkt[lane];
  if (wave == 0) row[0] = static_cast<uint32_t>(total);
  // two entries per step, both keys' LDS reads first
  auto put = [&](int e, int j, const u32x4_t c, float f) {
    float est = fq * f;
    est = est * static_cast<float>(kD - 2 * popc_xor128(qc, c));
    row[2 + 2 * e] = ordered_key_f(est * 0.0078125f);
    row[3 + 2 * e] = static_cast<uint32_t>(p0 + j);
  };
  int e = before;
  for (uint64_t m = exact; m != 0 && e < kFiltCap;) {
    const int j0 = __builtin_ctzll(m);
    m &= m - 1;
    const bool two = m != 0 && e + 1 < kFiltCap;
    const int j1 = two ? __builtin_ctzll(m) : j0;
    if (two) m &= m - 1;
    const u32x4_t c0 = s_kc[wave][j0], c1 = s_kc[wave][j1];
    const float f0 = s_fk[wave][j0], f1 = s_fk[wave][j1];
    put(e, j0, c0, f0);
    if (two) put(e + 1, j1, c1, f1);
    e += two ? 2 : 1;
  }
  __syncthreads();
  // ---- the buckets out: 4 threads per bucket, 8 words each, as two 16-byte
  //      stores (entries past the count are left unspecified) ----
  {
    const int b = threadIdx.x >> 2, part = threadIdx.x & 3;
    const int qb = blockIdx.y * 64 + b;
    if (qb < queries) {
      const uint32_t* src = s_bkt[b] + 8 * part;
      u32x4_t lo, hi;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        lo[w] = src[w];
        hi[w] = src[4 + w];
      }
      u32x4_t* dst = reinterpret_cast<u32x4_t*>(buckets + ((pool * queries + qb) * n_lists + list) * kBucketWords +
                                                8 * part);
      dst[0] = lo;
      dst[1] = hi;
    }
  }
}

// Exact k-th largest key over all n positions of a pool, keys recomputed by
// key_at(p) each round (the select kernel's fallback): the radix_select rounds
// with the items streamed from the codes instead of held in registers.
template <int NT, typename KeyAt>
__device__ void radix_select_stream(KeyAt&& key_at, int64_t n, int k, const SelectSmem& sm, uint32_t& T,
                                    int& take_eq) {
  constexpr int W = Block<NT>::kWaves;
  const int tid = threadIdx.x, wave = tid >> 6;
  uint32_t lo = 0u, hi = 0xFFFFFFFFu;
  int rem = k;
  while (true) {
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
    for (int64_t p = tid; p < n; p += NT) {
      const uint32_t key = key_at(p);
      if (key >= lo && key <= hi) {
        mn = min(mn, key);
        mx = max(mx, key);
      }
    }
    Block<NT>::minmax(mn, mx, sm.tmp);
    lo = mn;
    hi = mx;
    if (lo == hi) break;
    const int bits = 32 - __clz(static_cast<int>(hi - lo));
    const int shift = bits > 8 ? bits - 8 : 0;
    for (int i = tid; i < W * 256; i += NT) sm.hist[i] = 0;
    __syncthreads();
    for (int64_t p = tid; p < n; p += NT) {
      const uint32_t key = key_at(p);
      if (key >= lo && key <= hi) atomicAdd(&sm.hist[wave * 256 + ((key - lo) >> shift)], 1);
    }
    __syncthreads();
    for (int b = tid; b < 256; b += NT) {
      int c = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) c += sm.hist[w * 256 + b];
      sm.hist[b] = c;
    }
    __syncthreads();
    if (tid < 64) {
      int c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = sm.hist[4 * tid + j];
      const int lane_sum = c[0] + c[1] + c[2] + c[3];
      int suf = lane_sum;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_down(suf, off);
        if (tid + off < 64) suf += v;
      }
      int above = suf - lane_sum;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const int at_or_above = above + c[j];
        if (at_or_above >= rem && above < rem) {
          sm.bin[0] = 4 * tid + j;
          sm.bin[1] = above;
        }
        above = at_or_above;
      }
    }
    __syncthreads();
    const uint32_t b = static_cast<uint32_t>(sm.bin[0]);
    rem -= sm.bin[1];
    __syncthreads();
    const uint64_t new_lo = static_cast<uint64_t>(lo) + (static_cast<uint64_t>(b) << shift);
    const uint64_t new_hi = new_lo + (1ull << shift) - 1ull;
    lo = static_cast<uint32_t>(new_lo);
    hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
    if (shift == 0) break;
  }
  T = lo;
  take_eq = rem;
}

// ----------------------------------------------------------------------------
// 3. select, per (query, pool), 1024 threads.
//    Gather: pass r reads chunks r*1024 + t of the query's buckets (coalesced);
//    chunk c of a bucket holds its entries 2c - 1 and 2c, so every thread owns
//    2 items per pass, straight from the load, in increasing index order
//    (pass, thread, item); the bucket's count comes from its chunk 0 through
//    a lane swizzle.  One block reduction gives the overflow flag, the key
//    range and, from per-pass entry counts scanned over the threads, every
//    entry's position in index order.  Up to 4 NT entries move to LDS there
//    (thread t then holds entries t*C .. t*C + C - 1, C = ceil(entries / NT)),
//    and the exact k-th key comes from the radix rounds over those, one scan
//    of packed (above, equal) counts placing the selected indices in index
//    order; more entries stay in the registers, with one scan per pass.
//    Otherwise (a list beyond kFiltCap, or fewer than k keys at or above
//    tau) the block selects over all n keys, estimates recomputed per pass.
//    Then the exact rerank and the sort by (score desc, index asc).
// ----------------------------------------------------------------------------
template <int NT, int R>
__global__ __launch_bounds__(NT) void rabitq_select_kernel(
    const uint32_t* __restrict__ buckets, int n_lists,
    const uint8_t* __restrict__ q_codes, const uint16_t* __restrict__ q_fac, const uint8_t* __restrict__ codes_k,
    const uint16_t* __restrict__ fac_k, int k, const uint16_t* __restrict__ q, const uint16_t* __restrict__ keys,
    int64_t k_pool_stride, int64_t k_row_stride, int64_t n, int queries, int64_t* __restrict__ out_cand,
    int64_t* __restrict__ out_idx, float* __restrict__ out_score) {
  constexpr int W = NT / 64, NI = 2 * R;
  __shared__ int s_hist[2 * 4096];
  constexpr int kCap = 4 * NT;  // compacted entries: up to 4 per thread
  __shared__ __attribute__((aligned(16))) uint32_t s_tmp[(R > 4 ? R : 4) * W + 2];
  __shared__ __attribute__((aligned(16))) uint32_t s_red[4 * W];
  __shared__ uint32_t s_ckey[kCap];
  __shared__ int32_t s_cidx[kCap];
  __shared__ int32_t s_sel[kMaxTopk];
  __shared__ float s_score[kMaxTopk];
  __shared__ __attribute__((aligned(16))) uint64_t s_rkey[kMaxTopk + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t pool = blockIdx.y;
  const int64_t pq = pool * queries + blockIdx.x;

  // ---- gather ----
  const u32x4_t* bq = reinterpret_cast<const u32x4_t*>(buckets + pq * n_lists * kBucketWords);
  const int n_chunks = n_lists * (kBucketWords / 4);
#pragma unroll
  for (int j = 0; j < 4096 / NT; ++j) s_hist[tid * (4096 / NT) + j] = 0;  // the radix's first histogram
  const int part = tid & 7;  // chunk of the bucket
  // item j: key[j]; its index = bucket * 256 + byte j of idx8 (a bucket is one
  // 256-key list)
  uint32_t key[NI], idx8[(NI + 3) / 4], valid = 0u;
#pragma unroll
  for (int j = 0; j < (NI + 3) / 4; ++j) idx8[j] = 0u;
  int overflow = 0;
  uint32_t mn = 0xFFFFFFFFu, mx = 0u;
  constexpr int RB = R < 8 ? R : 8;  // chunks in flight per thread
#pragma unroll
  for (int r0 = 0; r0 < R; r0 += RB) {
    u32x4_t ch[RB];
    // (a clamped address, then zero past the last bucket: no branch per load)
#pragma unroll
    for (int b = 0; b < RB; ++b) ch[b] = bq[min((r0 + b) * NT + tid, n_chunks - 1)];
#pragma unroll
    for (int b = 0; b < RB; ++b)
      if ((r0 + b) * NT + tid >= n_chunks) ch[b] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = r0 + b;
      // the bucket's count from its chunk 0 (lane & ~7 of this 32-lane half);
      // chunks past the last bucket are zero
      const int c = __builtin_amdgcn_ds_swizzle(static_cast<int>(ch[b][0]), 0x18);
      const int kept = c < kFiltCap ? c : kFiltCap;
      overflow |= c > kFiltCap;
      key[2 * r] = ch[b][0];      // entry 2 * part - 1 (chunk 0: count and pad)
      key[2 * r + 1] = ch[b][2];  // entry 2 * part
      idx8[r >> 1] |= ((ch[b][1] & 255u) | ((ch[b][3] & 255u) << 8)) << (16 * (r & 1));
      // packed here, so the chunk's index words die now (with 16 passes the
      // compiler would otherwise keep them all until the placement)
      if constexpr (R > 8) asm volatile("" : "+v"(idx8[r >> 1]));
      if (part >= 1 && 2 * part - 1 < kept) valid |= 1u << (2 * r);
      if (2 * part < kept) valid |= 1u << (2 * r + 1);
    }
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    if ((valid >> j) & 1u) {
      mn = min(mn, key[j]);
      mx = max(mx, key[j]);
    }
  }
  // per-pass entry counts scanned over the threads: entry positions in index
  // order (pass, thread, item); with 16 passes the in-wave prefixes are
  // recomputed where they are used instead of kept live
  constexpr bool kKeepExcl = R <= 8;
  auto pass_entries = [&](int r) { return __popc((valid >> (2 * r)) & 3u); };
  int pos_ex[kKeepExcl ? R : 1];  // within the wave
  int total = 0;
  {  // block reduction: overflow, key range, entry offsets (also orders the clear)
    const uint32_t w_ovf = wave_max_u32(static_cast<uint32_t>(overflow));
    const uint32_t w_mn = wave_min_u32(mn), w_mx = wave_max_u32(mx);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int cnt = pass_entries(r);
      const int incl = wave_incl_sum(cnt);
      if constexpr (kKeepExcl) pos_ex[r] = incl - cnt;
      if (lane == 63) s_tmp[r * W + wave] = static_cast<uint32_t>(incl);
    }
    if (lane == 0) {
      s_red[4 * wave] = w_ovf;
      s_red[4 * wave + 1] = w_mn;
      s_red[4 * wave + 2] = w_mx;
    }
    __syncthreads();
    if (wave == 0) {  // (pass, wave) totals -> exclusive offsets; the sum after them
      int carry = 0;
      for (int i0 = 0; i0 < R * W; i0 += 64) {
        const bool in = i0 + lane < R * W;
        const int v = in ? static_cast<int>(s_tmp[i0 + lane]) : 0;
        const int inc = wave_incl_sum(v);
        if (in) s_tmp[i0 + lane] = static_cast<uint32_t>(carry + inc - v);
        carry += __builtin_amdgcn_readlane(inc, 63);
      }
      if (lane == 0) s_tmp[R * W] = static_cast<uint32_t>(carry);
    }
    overflow = 0;
    mn = 0xFFFFFFFFu;
    mx = 0u;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const u32x4_t v = reinterpret_cast<const u32x4_t*>(s_red)[w];
      overflow |= static_cast<int>(v[0]);
      mn = min(mn, v[1]);
      mx = max(mx, v[2]);
    }
    __syncthreads();
    total = static_cast<int>(s_tmp[R * W]);
    valid = (overflow == 0 && total >= k) ? valid : 0u;
    overflow = overflow != 0 || total < k;  // from here: the fallback is needed
  }

  if (!overflow && total <= kCap) {
    // compaction: the entries move to LDS in index order, then thread t
    // holds entries t*C .. t*C + C - 1 (C = ceil(total / NT) <= 4), so the
    // later radix rounds and the placement touch ~total / NT slots per
    // thread instead of all 2 R; the radix's first round counts here, from
    // the registers, and clears its second histogram
    const int shift0 = radix12_first_shift(mn, mx);
#pragma unroll
    for (int j = 0; j < 4096 / NT; ++j) s_hist[4096 + tid * (4096 / NT) + j] = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int ex;
      if constexpr (kKeepExcl) {
        ex = pos_ex[r];
      } else {
        const int cnt = pass_entries(r);
        ex = wave_incl_sum(cnt) - cnt;
      }
      int p = static_cast<int>(s_tmp[r * W + wave]) + ex;
      const int32_t list0 = ((r * NT + tid) >> 3) * kFiltList;
#pragma unroll
      for (int j = 2 * r; j < 2 * r + 2; ++j) {
        if ((valid >> j) & 1u) {
          s_ckey[p] = key[j];
          s_cidx[p] = list0 + static_cast<int32_t>((idx8[j >> 2] >> (8 * (j & 3))) & 255u);
          ++p;
          atomicAdd(&s_hist[(key[j] - mn) >> shift0], 1);
        }
      }
    }
    __syncthreads();
    const int C = (total + NT - 1) / NT;
    uint32_t ck[4], cv = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int sl = tid * C + j;
      const bool ok = j < C && sl < total;
      ck[j] = ok ? s_ckey[sl] : 0u;
      cv |= static_cast<uint32_t>(ok) << j;
    }
    uint32_t T;
    int take_eq;
    block_radix_select12<NT, 4>(ck, cv, k, mn, mx, s_hist, s_tmp, T, take_eq, true);
    __syncthreads();  // its last reads of s_tmp are done
    // packed (above T, equal to T) counts, scanned over the threads (whose
    // slots are in index order)
    int gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if ((cv >> j) & 1u) {
        gt += ck[j] > T;
        eq += ck[j] == T;
      }
    }
    const int cnt = gt | (eq << 16);
    const int incl = wave_incl_sum(cnt);
    if (lane == 63) s_tmp[wave] = static_cast<uint32_t>(incl);
    __syncthreads();
    int before = incl - cnt;
#pragma unroll
    for (int w = 0; w < W; ++w) before += w < wave ? static_cast<int>(s_tmp[w]) : 0;
    int g = before & 0xFFFF, e = before >> 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if ((cv >> j) & 1u) {
        const int32_t ix = s_cidx[tid * C + j];
        if (ck[j] > T) {
          s_sel[g + (e < take_eq ? e : take_eq)] = ix;
          ++g;
        } else if (ck[j] == T) {
          if (e < take_eq) s_sel[g + e] = ix;
          ++e;
        }
      }
    }
  } else if (!overflow) {
    uint32_t T;
    int take_eq;
    block_radix_select12<NT, NI>(key, valid, k, mn, mx, s_hist, s_tmp, T, take_eq);
    __syncthreads();  // its last reads of s_tmp are done
    // packed (above T, equal to T) counts per pass, scanned over the threads;
    // with 16 passes the per-pass prefixes are recomputed after the barriers
    // instead of kept live (32 keys per thread leave no registers for them)
    auto pass_count = [&](int r) {
      int gt = 0, eq = 0;
#pragma unroll
      for (int j = 2 * r; j < 2 * r + 2; ++j) {
        if ((valid >> j) & 1u) {
          gt += key[j] > T;
          eq += key[j] == T;
        }
      }
      return gt | (eq << 16);
    };
    int excl[kKeepExcl ? R : 1];  // within the wave
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int cnt = pass_count(r);
      const int incl = wave_incl_sum(cnt);
      if constexpr (kKeepExcl) excl[r] = incl - cnt;
      if (lane == 63) s_tmp[r * W + wave] = static_cast<uint32_t>(incl);
    }
    __syncthreads();
    if (wave == 0) {  // (pass, wave) totals -> exclusive offsets, in index order
      int carry = 0;
      for (int i0 = 0; i0 < R * W; i0 += 64) {
        const bool in = i0 + lane < R * W;
        const int v = in ? static_cast<int>(s_tmp[i0 + lane]) : 0;
        const int inc = wave_incl_sum(v);
        if (in) s_tmp[i0 + lane] = static_cast<uint32_t>(carry + inc - v);
        carry += __builtin_amdgcn_readlane(inc, 63);
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int ex;
      if constexpr (kKeepExcl) {
        ex = excl[r];
      } else {
        const int cnt = pass_count(r);
        ex = wave_incl_sum(cnt) - cnt;
      }
      const int before = static_cast<int>(s_tmp[r * W + wave]) + ex;
      int g = before & 0xFFFF, e = before >> 16;
      const int32_t list0 = ((r * NT + tid) >> 3) * kFiltList;
#pragma unroll
      for (int j = 2 * r; j < 2 * r + 2; ++j) {
        const int32_t ix = list0 + static_cast<int32_t>((idx8[j >> 2] >> (8 * (j & 3))) & 255u);
        if ((valid >> j) & 1u) {
          if (key[j] > T) {
            s_sel[g + (e < take_eq ? e : take_eq)] = ix;
            ++g;
          } else if (key[j] == T) {
            if (e < take_eq) s_sel[g + e] = ix;
            ++e;
          }
        }
      }
    }
  } else {
    // fallback: select over the whole pool, estimates recomputed per pass
    const u32x4_t qc = *reinterpret_cast<const u32x4_t*>(q_codes + pq * 16);
    const float fq = query_factor(q_fac, pq);
    const u32x4_t* kc = reinterpret_cast<const u32x4_t*>(codes_k) + pool * n;
    const uint32_t* kf = reinterpret_cast<const uint32_t*>(fac_k) + pool * n;
    auto key_at = [&](int64_t p) { return ordered_key_f(rabitq_estimate(qc, fq, kc[p], kf[p])); };
    SelectSmem sm{s_hist, s_tmp, reinterpret_cast<int*>(s_tmp + 2 * W)};
    uint32_t T;
    int take_eq;
    radix_select_stream<NT>(key_at, n, k, sm, T, take_eq);
    // ordered emit: positions in index order, ties at T by lowest index
    int emitted = 0, eq_seen = 0;
    for (int64_t c0 = 0; c0 < n; c0 += NT) {
      const int64_t p = c0 + tid;
      const uint32_t kp = p < n ? key_at(p) : 0u;
      const int is_eq = p < n && kp == T;
      int eq_total = 0;
      const int eq_b = eq_seen + Block<NT>::excl_scan(is_eq, reinterpret_cast<int*>(s_tmp), eq_total);
      const int sel = p < n && (kp > T || (is_eq && eq_b < take_eq));
      int sel_total = 0;
      const int pos = emitted + Block<NT>::excl_scan(sel, reinterpret_cast<int*>(s_tmp), sel_total);
      if (sel && pos < k) s_sel[pos] = static_cast<int32_t>(p);
      emitted += sel_total;
      eq_seen += eq_total;
      if (emitted >= k) break;
    }
  }
  __syncthreads();
  for (int i = tid; i < k; i += NT) out_cand[pq * k + i] = s_sel[i];

  // ---- exact rerank: 16-lane groups (one DPP row), lane l holds dims
  //      8l .. 8l+7; a pass covers 256 rows, a group's rows requested before
  //      any is used; the row sum halves by rotations 8, 4, 2, 1 (the same
  //      pairs as an xor butterfly, so the same sums) ----
  {
    const int l = tid & 15, grp = tid >> 4;
    constexpr int kGroups = NT / 16;
    constexpr int kRows = 4096 / NT;  // 256 rows per pass
    const u32x4_t qw = *reinterpret_cast<const u32x4_t*>(q + pq * kD + 8 * l);
    float qf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[e] = f16_to_f32(static_cast<uint16_t>(qw[e >> 1] >> (16 * (e & 1))));
    const uint16_t* kp = keys + pool * k_pool_stride;
    for (int c0 = 0; c0 < k; c0 += kRows * kGroups) {
      u32x4_t kw[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const int c = c0 + r * kGroups + grp;
        const int64_t ki = c < k ? static_cast<int64_t>(s_sel[c]) : -1;
        kw[r] = (ki >= 0 && ki < n) ? *reinterpret_cast<const u32x4_t*>(kp + ki * k_row_stride + 8 * l)
                                    : u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const int c = c0 + r * kGroups + grp;
        float sc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = qf[e] * f16_to_f32(static_cast<uint16_t>(kw[r][e >> 1] >> (16 * (e & 1))));
          sc = e == 0 ? pe : sc + pe;
        }
        sc = sc + __int_as_float(ZKV_ROR(__float_as_int(sc), 8));
        sc = sc + __int_as_float(ZKV_ROR(__float_as_int(sc), 4));
        sc = sc + __int_as_float(ZKV_ROR(__float_as_int(sc), 2));
        sc = sc + __int_as_float(ZKV_ROR(__float_as_int(sc), 1));
        if (c < k && l == 0) {
          s_score[c] = sc;
          // (score, slot) -> one key, larger = earlier: +-0 compare equal,
          // equal scores rank by slot (= by index)
          s_rkey[c] = (static_cast<uint64_t>(ordered_key_f(sc + 0.0f)) << 32) | (0xFFFFFFFFu - c);
        }
      }
    }
    if (tid == 0) s_rkey[k] = 0ull;  // pads an odd k's last pair (below every slot key)
  }
  __syncthreads();
  // ---- order: slot i goes to its rank, the number of larger slot keys.
  //      Groups of P lanes (a power of two <= 16, one DPP row at most) hold 4
  //      slots each; lane p of a group compares them with the 16-byte key
  //      pairs p, p + P, ... (adjacent lanes read adjacent pairs: no bank
  //      conflicts), and the group sums its counts by lane swizzles ----
  {
    const int groups = (k + 3) >> 2;
    int lp = 4;
    while (lp > 0 && (groups << lp) > NT) --lp;
    const int P = 1 << lp;
    const int g = tid >> lp, p = tid & (P - 1);
    const bool active = g < groups;
    const u32x4_t* rk = reinterpret_cast<const u32x4_t*>(s_rkey);
    uint64_t ki[4];
    {
      const int gg = active ? g : 0;
      const u32x4_t a = rk[2 * gg], b = rk[2 * gg + 1];
      ki[0] = a[0] | (static_cast<uint64_t>(a[1]) << 32);
      ki[1] = a[2] | (static_cast<uint64_t>(a[3]) << 32);
      ki[2] = b[0] | (static_cast<uint64_t>(b[1]) << 32);
      ki[3] = b[2] | (static_cast<uint64_t>(b[3]) << 32);
    }
    int rank[4] = {0, 0, 0, 0};
    const int pairs = (k + 1) >> 1;
    auto count = [&](const u32x4_t v) {
      const uint64_t k0 = v[0] | (static_cast<uint64_t>(v[1]) << 32);
      const uint64_t k1 = v[2] | (static_cast<uint64_t>(v[3]) << 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) rank[i] += static_cast<int>(k0 > ki[i]) + static_cast<int>(k1 > ki[i]);
    };
    int c = p;
    for (; c + 3 * P < pairs; c += 4 * P) {  // four pair reads in flight
      const u32x4_t v0 = rk[c], v1 = rk[c + P], v2 = rk[c + 2 * P], v3 = rk[c + 3 * P];
      count(v0);
      count(v1);
      count(v2);
      count(v3);
    }
    for (; c < pairs; c += P) count(rk[c]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (P > 1) rank[i] += swizzle_xor<1>(rank[i]);
      if (P > 2) rank[i] += swizzle_xor<2>(rank[i]);
      if (P > 4) rank[i] += swizzle_xor<4>(rank[i]);
      if (P > 8) rank[i] += swizzle_xor<8>(rank[i]);
    }
    if (active && p == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int slot = 4 * g + i;
        if (slot < k) {
          out_idx[pq * k + rank[i]] = s_sel[slot];
          out_score[pq * k + rank[i]] = s_score[slot];
        }
      }
    }
  }
}

int stage1_slice(int64_t n, int topk) {
  const int64_t small = 256 * kNI1;
  return (n + small - 1) / small * topk <= kMaxCand2 ? static_cast<int>(small) : 512 * kNI1;
}

struct SearchLayout {
  bool filter;
  int slice, n_slices;
  size_t q_codes, q_fac, tau, counts, cand_key, cand_idx, total;
};

SearchLayout search_layout(int pools, int queries, int64_t n, int topk) {
  SearchLayout L{};
  const int64_t pq = static_cast<int64_t>(pools) * queries;
  auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  L.filter = use_filter_path(n, topk);
  L.q_codes = 0;
  L.q_fac = up(pq * 16);
  L.tau = L.q_fac + up(pq * 4);
  size_t cand;
  if (L.filter) {
    // cand_key: the lists' 128-byte buckets
    L.slice = kFiltList;
    L.n_slices = static_cast<int>((n + kFiltList - 1) / kFiltList);
    L.counts = L.tau + up(pq * 4);
    L.cand_key = L.counts;
    L.cand_idx = L.cand_key;
    L.total = L.cand_key + up(static_cast<size_t>(pq) * L.n_slices * kBucketWords * 4);
    return L;
  } else {
    L.slice = stage1_slice(n, topk);
    L.n_slices = static_cast<int>((n + L.slice - 1) / L.slice);
    L.counts = L.tau;
    L.cand_key = L.tau;
    cand = static_cast<size_t>(pq) * L.n_slices * topk;
  }
  L.cand_idx = L.cand_key + up(cand * 4);
  L.total = L.cand_idx + up(cand * 4);
  return L;
}

int launch_encode(const uint16_t* x, int64_t row_stride, int64_t n, const float* signs, uint8_t* codes,
                  uint16_t* factors, hipStream_t stream) {
  if (n == 0) return ZKV_OK;
  const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
  rabitq_encode_kernel<<<blocks, 256, 0, stream>>>(x, row_stride, n, signs, codes, factors);
  return check_launch("rabitq_encode_kernel");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" int zkv_rabitq_encode(const uint16_t* x, int64_t row_stride, int64_t n, const float* signs,
                                 uint8_t* codes, uint16_t* factors, zkv_stream_t stream) {
  ZKV_REQUIRE(x && signs && codes && factors, "zkv_rabitq_encode: null pointer");
  ZKV_REQUIRE(n >= 0 && n <= (int64_t(1) << 31), "zkv_rabitq_encode: bad n=%lld", (long long)n);
  ZKV_REQUIRE(row_stride >= kD && row_stride % 8 == 0 && aligned16(x),
              "zkv_rabitq_encode: rows must be 16-byte aligned with stride >= 128 (got %lld)",
              (long long)row_stride);
  ZKV_REQUIRE(aligned16(codes) && (reinterpret_cast<uintptr_t>(factors) & 3u) == 0,
              "zkv_rabitq_encode: misaligned codes/factors");
  return launch_encode(x, row_stride, n, signs, codes, factors, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int zkv_rabitq_estimate(const uint8_t* codes_q, const uint16_t* factors_q,
                                   const uint8_t* codes_k, const uint16_t* factors_k, int pools,
                                   int queries, int64_t n, float* out, zkv_stream_t stream) {
  ZKV_REQUIRE(codes_q && factors_q && codes_k && factors_k && out, "zkv_rabitq_estimate: null pointer");
  ZKV_REQUIRE(pools > 0 && pools <= 65535 && queries > 0 && queries <= 65535 && n > 0 &&
                  n <= (int64_t(1) << 31),
              "zkv_rabitq_estimate: bad sizes pools=%d queries=%d n=%lld", pools, queries, (long long)n);
  ZKV_REQUIRE(aligned16(codes_q) && aligned16(codes_k), "zkv_rabitq_estimate: codes must be 16-byte aligned");
  dim3 grid(static_cast<unsigned>((n + 255) / 256), queries, pools);
  rabitq_estimate_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      codes_q, factors_q, codes_k, factors_k, n, queries, out);
  return check_launch("rabitq_estimate_kernel");
}

extern "C" size_t zkv_rabitq_search_workspace_size(int pools, int queries, int64_t n, int topk) {
  if (pools <= 0 || queries <= 0 || n <= 0 || topk <= 0) return 0;
  return search_layout(pools, queries, n, topk).total;
}

extern "C" int zkv_rabitq_search(const uint16_t* q, const uint16_t* keys, int64_t k_pool_stride,
                                 int64_t k_row_stride, const uint8_t* codes, const uint16_t* factors,
                                 const float* signs, int pools, int queries, int64_t n, int topk,
                                 int64_t* cand_idx, int64_t* final_idx, float* final_scores,
                                 void* workspace, size_t workspace_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(q && keys && codes && factors && signs && cand_idx && final_idx && final_scores && workspace,
              "zkv_rabitq_search: null pointer");
  ZKV_REQUIRE(pools > 0 && pools <= 65535 && queries > 0 && queries <= 65535,
              "zkv_rabitq_search: bad pools=%d queries=%d", pools, queries);
  ZKV_REQUIRE(n > 0 && n <= (int64_t(1) << 31) - 1, "zkv_rabitq_search: bad n=%lld", (long long)n);
  ZKV_REQUIRE(topk > 0 && topk <= kMaxTopk && topk <= n,
              "zkv_rabitq_search: topk=%d must be in [1, min(n=%lld, %d)]", topk, (long long)n, kMaxTopk);
  const SearchLayout L = search_layout(pools, queries, n, topk);
  ZKV_REQUIRE(L.filter || static_cast<int64_t>(L.n_slices) * topk <= kMaxCand2,
              "zkv_rabitq_search: %d slices of %d keys x topk %d exceed %d candidates per query",
              L.n_slices, L.slice, topk, kMaxCand2);
  ZKV_REQUIRE(workspace_bytes >= L.total, "zkv_rabitq_search: workspace of %zu bytes < %zu",
              workspace_bytes, L.total);
  ZKV_REQUIRE(k_row_stride >= kD && k_row_stride % 8 == 0 && k_pool_stride % 8 == 0 && aligned16(keys) &&
                  aligned16(q) && aligned16(codes) && aligned16(workspace),
              "zkv_rabitq_search: keys/q/codes must be 16-byte aligned rows (row stride %lld)",
              (long long)k_row_stride);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* q_codes = ws + L.q_codes;
  uint16_t* q_fac = reinterpret_cast<uint16_t*>(ws + L.q_fac);
  uint32_t* c_key = reinterpret_cast<uint32_t*>(ws + L.cand_key);
  int32_t* c_idx = reinterpret_cast<int32_t*>(ws + L.cand_idx);
  if (L.filter) {
    const FilterPlan f = filter_plan(n, topk);
    uint32_t* tau = reinterpret_cast<uint32_t*>(ws + L.tau);
    uint32_t* buckets = reinterpret_cast<uint32_t*>(ws + L.cand_key);
    rabitq_prep_kernel<<<dim3(queries, pools), kBigNT, 0, s>>>(q, signs, codes, factors, n, queries, f.s_count,
                                                                f.m, q_codes, q_fac, tau);
    int rc = check_launch("rabitq_prep_kernel");
    if (rc != ZKV_OK) return rc;
    rabitq_filter_kernel<<<dim3(L.n_slices, (queries + 63) / 64, pools), 256, 0, s>>>(
        q_codes, q_fac, tau, codes, factors, n, queries, L.n_slices, buckets);
    rc = check_launch("rabitq_filter_kernel");
    if (rc != ZKV_OK) return rc;
    const dim3 gs(queries, pools);
    const SelectShape sh = select_shape(n);
    switch (sh.nt * 100 + sh.passes) {
#define ZKV_SELECT(NT, R)                                                                                     \
  case NT * 100 + R:                                                                                          \
    rabitq_select_kernel<NT, R><<<gs, NT, 0, s>>>(buckets, L.n_slices, q_codes, q_fac, codes, factors, topk, \
                                                  q, keys, k_pool_stride, k_row_stride, n, queries,         \
                                                  cand_idx, final_idx, final_scores);                       \
    break;
      ZKV_SELECT(1024, 1)
      ZKV_SELECT(1024, 2)
      ZKV_SELECT(1024, 4)
      ZKV_SELECT(1024, 8)
      ZKV_SELECT(1024, 16)
#undef ZKV_SELECT
      default:
        return fail(ZKV_EINVAL, "zkv_rabitq_search: no select kernel for n=%lld", (long long)n);
    }
    return check_launch("rabitq_select_kernel");
  }
  int rc = launch_encode(q, kD, static_cast<int64_t>(pools) * queries, signs, q_codes, q_fac, s);
  if (rc != ZKV_OK) return rc;
  dim3 g1(L.n_slices, queries, pools);
  if (L.slice == 256 * kNI1)
    rabitq_stage1_kernel<256><<<g1, 256, 0, s>>>(q_codes, q_fac, codes, factors, n, queries, topk, c_key, c_idx);
  else
    rabitq_stage1_kernel<512><<<g1, 512, 0, s>>>(q_codes, q_fac, codes, factors, n, queries, topk, c_key, c_idx);
  rc = check_launch("rabitq_stage1_kernel");
  if (rc != ZKV_OK) return rc;
  dim3 g2(queries, pools);
  const int64_t n_last = n - static_cast<int64_t>(L.n_slices - 1) * L.slice;
  const int n_pad = n_last < topk ? topk - static_cast<int>(n_last) : 0;
  rabitq_stage2_kernel<<<g2, kNT2, 0, s>>>(c_key, c_idx, L.n_slices * topk, L.n_slices * topk - n_pad,
                                           topk, q, keys, k_pool_stride,
                                           k_row_stride, n, queries, cand_idx, final_idx, final_scores);
  return check_launch("rabitq_stage2_kernel");
}
