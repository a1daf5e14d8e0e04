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
// Block primitives for NT threads (multiple of 64)
// ----------------------------------------------------------------------------
template <int NT>
struct Block {
  static constexpr int kWaves = NT / 64;

  // exclusive prefix sum over threads (thread order) and the block total
  __device__ static int excl_scan(int v, int* s_tmp, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
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
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      mn = min(mn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mn), off)));
      mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), off)));
    }
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
// Stage 2: per (query, pool): top-k of the n_cand candidates (positions are in
// increasing index order), exact rerank, sort by (score desc, index asc).
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

  // exact rerank: 16-lane groups, lane l holds dims 8l .. 8l+7
  const int l = tid & 15;
  const u32x4_t qw = *reinterpret_cast<const u32x4_t*>(q + pq * kD + 8 * l);
  float qf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qf[e] = f16_to_f32(static_cast<uint16_t>(qw[e >> 1] >> (16 * (e & 1))));
  const uint16_t* kp = keys + pool * k_pool_stride;
  for (int c0 = 0; c0 < k; c0 += kNT2 / 16) {
    const int c = c0 + (tid >> 4);
    float s = 0.0f;
    // stage 1 always writes valid indices; a key row is read only for an
    // index inside the pool all the same
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
  for (int i = tid; i < P; i += kNT2)
    s_sort[i] = i < k ? (static_cast<uint64_t>(ordered_key_f(s_score[i] + 0.0f)) << 32) |
                            static_cast<uint64_t>(0xFFFFu - static_cast<uint32_t>(i))
                      : 0ull;
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int i = tid; i < P / 2; i += kNT2) {
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
  for (int i = tid; i < k; i += kNT2) {
    const int slot = static_cast<int>(0xFFFFu - static_cast<uint32_t>(s_sort[i] & 0xFFFFu));
    out_idx[pq * k + i] = s_sel[slot];
    out_score[pq * k + i] = s_score[slot];
  }
}

int stage1_slice(int64_t n, int topk) {
  const int64_t small = 256 * kNI1;
  return (n + small - 1) / small * topk <= kMaxCand2 ? static_cast<int>(small) : 512 * kNI1;
}

struct SearchLayout {
  int slice, n_slices;
  size_t q_codes, q_fac, cand_key, cand_idx, total;
};

SearchLayout search_layout(int pools, int queries, int64_t n, int topk) {
  SearchLayout L{};
  const int64_t pq = static_cast<int64_t>(pools) * queries;
  L.slice = stage1_slice(n, topk);
  L.n_slices = static_cast<int>((n + L.slice - 1) / L.slice);
  auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  L.q_codes = 0;
  L.q_fac = up(pq * 16);
  L.cand_key = L.q_fac + up(pq * 4);
  const size_t cand = static_cast<size_t>(pq) * L.n_slices * topk;
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
  ZKV_REQUIRE(static_cast<int64_t>(L.n_slices) * topk <= kMaxCand2,
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
