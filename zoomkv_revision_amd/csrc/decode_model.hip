// Model-side kernels of one decode step (the C5 counterpart of the reference
// runtime's layer_decode, Z/model_hub/LLM.py:208-251, with the rmsnorm /
// rope / silu pieces of Z/model_hub/qwen.py:493-604):
//
//  * decode_linear_kernel: y[m, n] = sum_k x[m, k] * w[n, k] for the few rows
//    m of a decode batch (M <= 16), bf16 in, fp32 accumulate, bf16 out, with
//    an optional RMSNorm of x on the way in and an optional epilogue
//    (residual add, or silu(gate) * up over the two halves of w).  The
//    weights are streamed once from HBM: a workgroup owns 16 output rows, its
//    waves split K, each k-block of 128 is four v_mfma_f32_16x16x32_bf16 with
//    the 16 weight rows as A and the (normalised) x rows, staged in LDS, as
//    the B columns.
//  * qk_norm_rope_kernel: per-head RMSNorm of q and k, rotate-half RoPE at
//    one position, and the k / v rows written straight into the cache.
//
// Rounding follows the torch restatement: every bf16 tensor of the
// reference is rounded (RNE) where the reference materialises it.
#include "zkv_common.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace zkv {
namespace {

typedef __bf16 bf16x8v_t __attribute__((ext_vector_type(8)));

constexpr int kLinKBlock = 128;  // four MFMA k-chunks of 32
constexpr int kLinMaxM = 16;     // MFMA B columns

enum LinearEpilogue : int { kEpiNone = 0, kEpiResidual = 1, kEpiSiluMul = 2 };

struct LinearParams {
  const uint16_t* x;  // [M, K] bf16, row stride x_ld
  int64_t x_ld;
  const uint16_t* w;  // [N, K] bf16, contiguous rows
  const uint16_t* norm_w;  // [K] bf16 or null
  float eps;
  const uint16_t* res;  // [M, N] bf16 (residual epilogue), row stride res_ld
  int64_t res_ld;
  void* out;  // [M, N] (or [M, N / 2] for silu * up), row stride out_ld
  int64_t out_ld;
  int M, K, N;
  int out_f32;
};

__device__ __forceinline__ float wave_sum(float v) {
  // butterfly over the 64 lanes (every lane ends with the total)
  v += __shfl_xor(v, 32);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

__device__ __forceinline__ void store_y(const LinearParams& p, int m, int n, float y) {
  if (p.out_f32)
    reinterpret_cast<float*>(p.out)[m * p.out_ld + n] = y;
  else
    reinterpret_cast<uint16_t*>(p.out)[m * p.out_ld + n] = f32_to_bf16_bits(y);
}

// Stages the M x K input rows into LDS (xs), RMS-normalised when kNorm:
// bf16(x * rsqrt(mean(x^2) + eps) * w).  red: M floats of scratch.
template <bool kNorm>
__device__ __forceinline__ void stage_x(const LinearParams& p, uint16_t* xs, float* red) {
  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int M = p.M, K = p.K;
  const int kv8 = K >> 3;  // 16-byte chunks per row
  if constexpr (kNorm) {
    // wave m' reduces rows m = m', m' + nw, ... (fixed order: deterministic)
    for (int m = wave; m < M; m += nw) {
      const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(p.x + m * p.x_ld);
      float ss = 0.0f;
      for (int i = lane; i < kv8; i += 64) {
        const u32x4_t v = xr[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = __uint_as_float(v[e] << 16), hi = __uint_as_float(v[e] & 0xFFFF0000u);
          ss = ss + lo * lo;
          ss = ss + hi * hi;
        }
      }
      // mean as the sum times 1/K (torch's mean), then rsqrt(mean + eps)
      ss = wave_sum(ss);
      if (lane == 0) red[m] = rsqrtf(ss * (1.0f / static_cast<float>(K)) + p.eps);
    }
    __syncthreads();
  }
  for (int i = tid; i < M * kv8; i += blockDim.x) {
    const int m = i / kv8, k8 = i - m * kv8;
    u32x4_t v = reinterpret_cast<const u32x4_t*>(p.x + m * p.x_ld)[k8];
    if constexpr (kNorm) {
      const float r = red[m];
      const u32x4_t wv = reinterpret_cast<const u32x4_t*>(p.norm_w)[k8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16r((__uint_as_float(v[e] << 16) * r) * __uint_as_float(wv[e] << 16));
        const float hi =
            bf16r((__uint_as_float(v[e] & 0xFFFF0000u) * r) * __uint_as_float(wv[e] & 0xFFFF0000u));
        v[e] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
      }
    }
    reinterpret_cast<u32x4_t*>(xs)[i] = v;
  }
  __syncthreads();
}

// One workgroup per tile of 16 output rows (silu * up: 8 gate rows and the 8
// matching up rows), NW waves splitting the K blocks.  Dynamic LDS: the M x K
// bf16 input rows, then NW x 64 x 4 fp32 partial tiles.
template <int kEpi, bool kNorm>
__global__ __launch_bounds__(1024) void decode_linear_kernel(const LinearParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);
  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int M = p.M, K = p.K;
  float* red = reinterpret_cast<float*>(lds + static_cast<size_t>(M) * K * 2);
  stage_x<kNorm>(p, xs, red);

  // ---- weight rows of this tile ----
  const int tile = blockIdx.x;
  int row;  // weight row of A row c (or -1 past N)
  if constexpr (kEpi == kEpiSiluMul) {
    const int half = p.N >> 1, j = tile * 8 + (c & 7);
    row = j < half ? (c < 8 ? j : half + j) : -1;
  } else {
    row = tile * 16 + c < p.N ? tile * 16 + c : -1;
  }
  const uint16_t* wr = p.w + static_cast<int64_t>(row < 0 ? 0 : row) * K;
  const bool col_ok = c < M;
  const uint16_t* xr = xs + (col_ok ? c : 0) * K;

  float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nkb = K / kLinKBlock;
  for (int kb = wave; kb < nkb; kb += nw) {
    u32x4_t a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = kb * kLinKBlock + 32 * j + 8 * g;
      a[j] = row >= 0 ? *reinterpret_cast<const u32x4_t*>(wr + k) : u32x4_t{0u, 0u, 0u, 0u};
      b[j] = col_ok ? *reinterpret_cast<const u32x4_t*>(xr + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v_t, a[j]),
                                                    __builtin_bit_cast(bf16x8v_t, b[j]), acc, 0, 0, 0);
  }

  // ---- sum the waves' partial tiles in wave order, then the epilogue ----
  reinterpret_cast<float4_t*>(red)[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  float4_t s = reinterpret_cast<const float4_t*>(red)[lane];
  for (int w = 1; w < nw; ++w) {
    const float4_t t = reinterpret_cast<const float4_t*>(red)[w * 64 + lane];
    s[0] += t[0], s[1] += t[1], s[2] += t[2], s[3] += t[3];
  }
  // lane (c, g) holds rows 4g + i of the tile for batch row c
  if constexpr (kEpi == kEpiSiluMul) {
    // gate rows sit in g < 2, the matching up rows 32 lanes higher
    float up[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      up[i] = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(s[i]), __float_as_uint(s[i]),
                                                               false, false)[1]);
    if (g >= 2 || !col_ok) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = tile * 8 + 4 * g + i;
      if (j >= (p.N >> 1)) continue;
      const float gt = bf16r(s[i]), u = bf16r(up[i]);
      const float act = bf16r(gt / (1.0f + expf(-gt)));
      store_y(p, c, j, bf16r(act * u));
    }
  } else {
    if (!col_ok) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = tile * 16 + 4 * g + i;
      if (n >= p.N) continue;
      float y = bf16r(s[i]);
      if constexpr (kEpi == kEpiResidual) y = bf16r(bf16_to_f32(p.res[c * p.res_ld + n]) + y);
      store_y(p, c, n, y);
    }
  }
}

// ---------------------------------------------------------------------------
// The same linear for M <= 4 input rows as a weight stream.  A unit of work
// is kR weight rows over all of K (silu * up: kR / 2 gate rows and the
// matching up rows); every wave takes units gw, gw + (waves in the grid), ...
// and walks their (unit, 512-element chunk) items with two items in flight:
// each item is kR loads of 1 KiB of one weight row (64 lanes x 16 B, whole
// cache lines, nontemporal) and, without a norm, the x rows' 16 B.  With the
// norm, the workgroup stages the normalised x rows in LDS once (the grid is
// at most a few workgroups per CU, so the staging is amortised over many
// units).  v_dot2_f32_bf16 accumulates w x x in fp32; at the unit's last
// chunk the lanes' partial sums are reduce-scattered with shuffles and the
// epilogue (that of decode_linear_kernel) runs by lane pairs.  Waves never
// wait for each other after the staging.  (The MFMA tile of
// decode_linear_kernel makes each load instruction touch 16 rows x 64 B and
// splits K over waves of a 16-row tile.)
// ---------------------------------------------------------------------------
constexpr int kGemvMaxM = 4;
constexpr int kGemvChunk = 512;  // elements of one row read by one wave instruction
constexpr int kGemvWaves = 4;

typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x2v_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2v_t, v); }

// (each dword named: a bit_cast of an indexed vector element in an unrolled
// loop compiled to four uses of element 0)
__device__ __forceinline__ float dot8(const u32x4_t w, const u32x4_t x, float acc) {
  const uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
  const uint32_t x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w0), as_bf16x2(x0), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w1), as_bf16x2(x1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w2), as_bf16x2(x2), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w3), as_bf16x2(x3), acc, false);
  return acc;
}

// One step of a reduce-scatter over the lanes: lanes whose `bit` is set keep
// the upper half of the N values, the others the lower half, each adding its
// partner's (lane ^ bit) copy of the half it keeps.
template <int N>
__device__ __forceinline__ void rs_step(const float (&v)[N], float (&o)[N / 2], int lane, int bit) {
  const bool hi = lane & bit;
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const float send = hi ? v[j] : v[j + N / 2];
    const float keep = hi ? v[j + N / 2] : v[j];
    o[j] = keep + __shfl_xor(send, bit);
  }
}

// The sum over the 64 lanes of value idx(lane) = lane >> (6 - log2 kV) of
// the kV per-lane values (lanes equal in the high bits hold copies).
template <int kV>
__device__ __forceinline__ float lane_reduce(const float (&acc)[kV], int lane) {
  float s;
  if constexpr (kV == 32) {
    float a[16], b[8], c[4], d[2], e[1];
    rs_step<32>(acc, a, lane, 32);
    rs_step<16>(a, b, lane, 16);
    rs_step<8>(b, c, lane, 8);
    rs_step<4>(c, d, lane, 4);
    rs_step<2>(d, e, lane, 2);
    s = e[0] + __shfl_xor(e[0], 1);
  } else if constexpr (kV == 16) {
    float a[8], b[4], c[2], d[1];
    rs_step<16>(acc, a, lane, 32);
    rs_step<8>(a, b, lane, 16);
    rs_step<4>(b, c, lane, 8);
    rs_step<2>(c, d, lane, 4);
    s = d[0] + __shfl_xor(d[0], 2);
    s = s + __shfl_xor(s, 1);
  } else {
    static_assert(kV == 8, "kV is 8, 16 or 32");
    float a[4], b[2], c[1];
    rs_step<8>(acc, a, lane, 32);
    rs_step<4>(a, b, lane, 16);
    rs_step<2>(b, c, lane, 8);
    s = c[0] + __shfl_xor(c[0], 4);
    s = s + __shfl_xor(s, 2);
    s = s + __shfl_xor(s, 1);
  }
  return s;
}

// kSplit: the narrow projections.  A unit is then worked by the whole
// workgroup, wave w taking chunks w, w + 4, ... (at least one each: the
// launcher uses it for K >= 4 chunks), and the waves' partial sums meet in
// LDS at the unit's end; the workgroups take units blockIdx.x, blockIdx.x +
// gridDim.x, ...
template <int kEpi, bool kNorm, int kR, int kD, bool kSplit>
__global__ __launch_bounds__(64 * kGemvWaves) void decode_stream_kernel(const LinearParams p, int n_units) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int kV = kR * kGemvMaxM;  // values per lane: acc[r * 4 + m]
  constexpr int kShift = kV == 32 ? 1 : (kV == 16 ? 2 : 3);
  float* rnorm = reinterpret_cast<float*>(lds);  // [4] norm factors
  float* red = rnorm + kGemvMaxM;                // kSplit: [waves][64] partial sums
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds + 16 + (kSplit ? kGemvWaves * 64 * 4 : 0));  // normalised x [M][K]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int M = p.M, K = p.K, N = p.N;
  const int n_chunks = (K + kGemvChunk - 1) / kGemvChunk;
  // this wave's units u0, u0 + du, ... and chunks c0, c0 + dc, ... (cnt per unit)
  const int u0 = kSplit ? blockIdx.x : blockIdx.x * kGemvWaves + wave;
  const int du = kSplit ? gridDim.x : gridDim.x * kGemvWaves;
  const int c0 = kSplit ? wave : 0, dc = kSplit ? kGemvWaves : 1;
  const int cnt = kSplit ? (n_chunks - wave + kGemvWaves - 1) / kGemvWaves : n_chunks;
  const int n_my = u0 < n_units ? (n_units - 1 - u0) / du + 1 : 0;
  const int n_items = n_my * cnt;
  constexpr int kXv = kGemvMaxM;  // the x rows' 16 B (no norm)

  auto unit_row = [&](int u, int r) {
    if constexpr (kEpi == kEpiSiluMul) {
      const int half = N >> 1, j = u * (kR / 2) + (r % (kR / 2));
      return j < half ? (r < kR / 2 ? j : half + j) : -1;
    } else {
      const int n = u * kR + r;
      return n < N ? n : -1;
    }
  };
  // item t of this wave: unit u0 + (t / cnt) du, chunk c0 + (t % cnt) dc
  auto load_item = [&](int t, u32x4_t (&wv)[kR], u32x4_t (&xv)[kXv]) {
    const int u = u0 + (t / cnt) * du, ci = c0 + (t % cnt) * dc;
    const int k = ci * kGemvChunk + 8 * lane;
    const bool ok = t < n_items && k < K;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int row = unit_row(u, r);
      wv[r] = ok && row >= 0 ? __builtin_nontemporal_load(
                                   reinterpret_cast<const u32x4_t*>(p.w + static_cast<int64_t>(row) * K + k))
                             : u32x4_t{0u, 0u, 0u, 0u};
    }
    if constexpr (!kNorm) {
#pragma unroll
      for (int m = 0; m < kGemvMaxM; ++m)
        xv[m] = ok && m < M ? *reinterpret_cast<const u32x4_t*>(p.x + m * p.x_ld + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  // kD register slots of items in flight
  u32x4_t wr[kD][kR], xr[kD][kXv];
#pragma unroll
  for (int d = 0; d < kD; ++d) load_item(d, wr[d], xr[d]);

  if constexpr (kNorm) {
    // wave m: the RMS factor of x row m; then the normalised rows to LDS
    // (the first items' weight loads are in flight)
    if (wave < M) {
      const u32x4_t* xrow = reinterpret_cast<const u32x4_t*>(p.x + wave * p.x_ld);
      float ss = 0.0f;
      for (int i = lane; i < (K >> 3); i += 64) {
        const u32x4_t v = xrow[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = __uint_as_float(v[e] << 16), hi = __uint_as_float(v[e] & 0xFFFF0000u);
          ss = ss + lo * lo;
          ss = ss + hi * hi;
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) rnorm[wave] = rsqrtf(ss * (1.0f / static_cast<float>(K)) + p.eps);
    }
    __syncthreads();
    for (int i = tid; i < M * (K >> 3); i += 64 * kGemvWaves) {
      const int m = i / (K >> 3), k8 = i - m * (K >> 3);
      u32x4_t v = reinterpret_cast<const u32x4_t*>(p.x + m * p.x_ld)[k8];
      const float r = rnorm[m];
      const u32x4_t wv = reinterpret_cast<const u32x4_t*>(p.norm_w)[k8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16r((__uint_as_float(v[e] << 16) * r) * __uint_as_float(wv[e] << 16));
        const float hi = bf16r((__uint_as_float(v[e] & 0xFFFF0000u) * r) * __uint_as_float(wv[e] & 0xFFFF0000u));
        v[e] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
      }
      reinterpret_cast<u32x4_t*>(xs)[i] = v;
    }
    __syncthreads();
  }

  float acc[kV];
#pragma unroll
  for (int j = 0; j < kV; ++j) acc[j] = 0.0f;
  auto step = [&](int t, const u32x4_t (&wv)[kR], const u32x4_t (&xv)[kXv]) {
    const int ci = c0 + (t % cnt) * dc;
    const int k = ci * kGemvChunk + 8 * lane;
    u32x4_t xm[kGemvMaxM];
#pragma unroll
    for (int m = 0; m < kGemvMaxM; ++m) {
      if constexpr (kNorm)
        xm[m] = m < M && k < K ? *reinterpret_cast<const u32x4_t*>(xs + m * K + k) : u32x4_t{0u, 0u, 0u, 0u};
      else
        xm[m] = xv[m];
    }
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
      for (int m = 0; m < kGemvMaxM; ++m) acc[r * kGemvMaxM + m] = dot8(wv[r], xm[m], acc[r * kGemvMaxM + m]);
    if (t % cnt != cnt - 1) return;
    // this wave's last chunk of the unit: sums over the lanes (and, split,
    // over the waves), epilogue, fresh accumulators
    const int u = u0 + (t / cnt) * du;
    float s = lane_reduce<kV>(acc, lane);
#pragma unroll
    for (int j = 0; j < kV; ++j) acc[j] = 0.0f;
    if constexpr (kSplit) {
      red[wave * 64 + lane] = s;
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 1; w < kGemvWaves; ++w) s += red[w * 64 + lane];
      }
      __syncthreads();  // red is free for the next unit
      if (wave != 0) return;
    }
    const int idx = lane >> kShift, r = idx / kGemvMaxM, m = idx % kGemvMaxM;
    const bool lead = (lane & ((1 << kShift) - 1)) == 0;
    const int row = unit_row(u, r);
    if constexpr (kEpi == kEpiSiluMul) {
      // the up row of gate row r sits kR / 2 rows (32 lanes) higher
      const float up = __shfl_xor(s, 32);
      if (lane >= 32 || !lead || m >= M || row < 0) return;
      const float gt = bf16r(s), uv = bf16r(up);
      const float act = bf16r(gt / (1.0f + expf(-gt)));
      store_y(p, m, row, bf16r(act * uv));
    } else {
      if (!lead || m >= M || row < 0) return;
      float y = bf16r(s);
      if constexpr (kEpi == kEpiResidual) y = bf16r(bf16_to_f32(p.res[m * p.res_ld + row]) + y);
      store_y(p, m, row, y);
    }
  };
  // slot d holds items d, d + kD, ...: refilled kD items ahead (every slot
  // index static)
  for (int t = 0; t < n_items; t += kD) {
#pragma unroll
    for (int d = 0; d < kD; ++d) {
      if (t + d < n_items) {
        step(t + d, wr[d], xr[d]);
        load_item(t + d + kD, wr[d], xr[d]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// q / k: per-head RMSNorm (bf16 out), then rotate-half RoPE at one position
// (bf16 out); v copied.  One wave per head of one batch row; lane l holds
// channels l and l + 64 (the two halves RoPE pairs).  Heads [0, hq) are q
// (to q_out), [hq, hq + hkv) k and [hq + hkv, hq + 2 hkv) v (to the cache).
// ---------------------------------------------------------------------------
struct QkParams {
  const uint16_t* qkv;  // [bs, (hq + 2 hkv) * 128] bf16, row stride qkv_ld
  int64_t qkv_ld;
  const uint16_t* q_norm;  // [128] bf16
  const uint16_t* k_norm;  // [128] bf16
  float eps;
  const float* cos;  // [64] fp32 (the position's row)
  const float* sin;
  uint16_t* q_out;  // [bs, hq, 128]
  uint16_t* k_dst;  // row of (b, h): k_dst + b * k_sb + h * k_sh
  int64_t k_sb, k_sh;
  uint16_t* v_dst;
  int64_t v_sb, v_sh;
  int bs, hq, hkv;
};

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const QkParams p) {
  const int heads = p.hq + 2 * p.hkv;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= p.bs * heads) return;
  const int b = item / heads, h = item - b * heads, lane = threadIdx.x & 63;
  const uint16_t* src = p.qkv + b * p.qkv_ld + h * 128;
  const float x1 = bf16_to_f32(src[lane]), x2 = bf16_to_f32(src[lane + 64]);
  if (h >= p.hq + p.hkv) {  // v: straight copy
    uint16_t* dst = p.v_dst + b * p.v_sb + (h - p.hq - p.hkv) * p.v_sh;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bool is_q = h < p.hq;
  const uint16_t* nw = is_q ? p.q_norm : p.k_norm;
  const float ss = wave_sum(x1 * x1 + x2 * x2);
  const float r = rsqrtf(ss * (1.0f / 128.0f) + p.eps);
  const float n1 = bf16r((x1 * r) * bf16_to_f32(nw[lane]));
  const float n2 = bf16r((x2 * r) * bf16_to_f32(nw[lane + 64]));
  const float cs = p.cos[lane], sn = p.sin[lane];
  const uint16_t y1 = f32_to_bf16_bits(n1 * cs - n2 * sn);
  const uint16_t y2 = f32_to_bf16_bits(n2 * cs + n1 * sn);
  uint16_t* dst = is_q ? p.q_out + (static_cast<int64_t>(b) * p.hq + h) * 128
                       : p.k_dst + b * p.k_sb + (h - p.hq) * p.k_sh;
  dst[lane] = y1;
  dst[lane + 64] = y2;
}

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" int zkv_decode_linear(const uint16_t* x, int64_t x_ld, int M, int K, const uint16_t* w, int N,
                                 const uint16_t* norm_w, float eps, const uint16_t* residual, int64_t res_ld,
                                 void* out, int64_t out_ld, int out_f32, int epilogue, zkv_stream_t stream) {
  ZKV_REQUIRE(x && w && out, "zkv_decode_linear: null pointer");
  ZKV_REQUIRE(M >= 1 && M <= kLinMaxM, "zkv_decode_linear: M=%d outside [1, %d]", M, kLinMaxM);
  ZKV_REQUIRE(K > 0 && K % kLinKBlock == 0, "zkv_decode_linear: K=%d is not a positive multiple of %d", K,
              kLinKBlock);
  ZKV_REQUIRE(N > 0, "zkv_decode_linear: N=%d", N);
  ZKV_REQUIRE(epilogue >= kEpiNone && epilogue <= kEpiSiluMul, "zkv_decode_linear: epilogue %d", epilogue);
  ZKV_REQUIRE(epilogue != kEpiResidual || residual, "zkv_decode_linear: residual epilogue without residual");
  ZKV_REQUIRE(epilogue != kEpiSiluMul || N % 2 == 0, "zkv_decode_linear: silu * up needs an even N (%d)", N);
  ZKV_REQUIRE(x_ld >= K && x_ld % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                  (norm_w == nullptr || (reinterpret_cast<uintptr_t>(norm_w) & 15) == 0),
              "zkv_decode_linear: x, w and the norm weight need 16-byte aligned rows");
  const size_t x_bytes = static_cast<size_t>(M) * K * 2;
  const int n_tiles = epilogue == kEpiSiluMul ? (N / 2 + 7) / 8 : (N + 15) / 16;
  // waves per workgroup: enough resident waves to keep the weight stream busy
  const int nkb = K / kLinKBlock;
  int nw = 1;
  while (nw < 16 && nw * 2 <= nkb && static_cast<int64_t>(n_tiles) * nw < 4096) nw *= 2;
  // and few enough k-blocks per wave that its loads overlap (the waves of a large N)
  while (nw < 16 && (nkb + nw - 1) / nw > 6) nw *= 2;
  const size_t lds = x_bytes + static_cast<size_t>(nw) * 64 * 16;
  ZKV_REQUIRE(lds <= 160 * 1024, "zkv_decode_linear: M x K = %d x %d needs %zu bytes of LDS (limit 160 KiB)", M,
              K, lds);
  LinearParams p{x, x_ld, w, norm_w, eps, residual, res_ld, out, out_ld, M, K, N, out_f32};
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (M <= kGemvMaxM && !getenv("ZKV_LINEAR_MFMA")) {
    // the weight stream: units of 8 rows for the wide projections, 4 or 2
    // for narrower ones (at least ~2048 units); a few workgroups per CU
    const int rows = epilogue == kEpiSiluMul ? N / 2 : N;
    const int n_chunks = (K + kGemvChunk - 1) / kGemvChunk;
    // narrow projections (fewer rows than ~2 units per wave of a full chip)
    // split K over the waves of a workgroup
    // (QKV, 6144 rows: 4 rows per unit 11.7 us, 2 rows 12.4; two or four
    // items in flight per wave: the same or slower at every projection)
    bool split = rows < 8192 && n_chunks >= kGemvWaves && !norm_w;
    int R = split ? 4 : (rows >= 16384 ? 8 : (rows >= 4096 ? 4 : 2));
    // ZKV_GEMV_SHAPE=R[,s] overrides the shape for tuning sweeps (s: split K)
    if (const char* e = getenv("ZKV_GEMV_SHAPE")) {
      int r = 0;
      char sp = 0;
      if (sscanf(e, "%d,%c", &r, &sp) >= 1 && (r == 2 || r == 4 || r == 8)) {
        R = r;
        split = sp == 's' && !norm_w && R == 4;
      }
    }
    const int per_unit = epilogue == kEpiSiluMul ? R / 2 : R;
    const int n_units = (rows + per_unit - 1) / per_unit;
    const int grid_g = std::max(1, std::min(split ? n_units : (n_units + kGemvWaves - 1) / kGemvWaves, 768));
    const size_t lds_g = 16 + (split ? kGemvWaves * 64 * 4 : 0) + (norm_w ? x_bytes : 0);
    ZKV_REQUIRE(lds_g <= 160 * 1024, "zkv_decode_linear: M x K = %d x %d needs %zu bytes of LDS", M, K, lds_g);
#define ZKV_GEMV(E, NORM, RR, D, SPLIT)                                                               \
  do {                                                                                                \
    static bool big_lds_set = false;                                                                  \
    if (lds_g > 64 * 1024 && !big_lds_set) {                                                          \
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_stream_kernel<E, NORM, RR, D, SPLIT>), \
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
        return fail(ZKV_EINVAL, "zkv_decode_linear: cannot raise the LDS limit to 160 KiB");          \
      big_lds_set = true;                                                                             \
    }                                                                                                 \
    decode_stream_kernel<E, NORM, RR, D, SPLIT><<<grid_g, 64 * kGemvWaves, lds_g, s>>>(p, n_units);   \
  } while (0)
#define ZKV_GEMV_R(E, NORM)                 \
  do {                                      \
    if (split)                              \
      ZKV_GEMV(E, NORM, 4, 2, true);        \
    else if (R == 8)                        \
      ZKV_GEMV(E, NORM, 8, 2, false);       \
    else if (R == 4)                        \
      ZKV_GEMV(E, NORM, 4, 2, false);       \
    else                                    \
      ZKV_GEMV(E, NORM, 2, 2, false);       \
  } while (0)
    if (norm_w) {
      if (epilogue == kEpiNone) ZKV_GEMV_R(kEpiNone, true);
      else if (epilogue == kEpiResidual) ZKV_GEMV_R(kEpiResidual, true);
      else ZKV_GEMV_R(kEpiSiluMul, true);
    } else {
      if (epilogue == kEpiNone) ZKV_GEMV_R(kEpiNone, false);
      else if (epilogue == kEpiResidual) ZKV_GEMV_R(kEpiResidual, false);
      else ZKV_GEMV_R(kEpiSiluMul, false);
    }
#undef ZKV_GEMV_R
#undef ZKV_GEMV
    return check_launch("decode_stream_kernel");
  }
  const dim3 grid(n_tiles), block(64 * nw);
  // dynamic LDS above 64 KiB has to be allowed per kernel (once)
#define ZKV_LIN(E, NORM)                                                                              \
  do {                                                                                                \
    static bool big_lds_set = false;                                                                  \
    if (lds > 64 * 1024 && !big_lds_set) {                                                            \
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_linear_kernel<E, NORM>),          \
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
        return fail(ZKV_EINVAL, "zkv_decode_linear: cannot raise the LDS limit to 160 KiB");          \
      big_lds_set = true;                                                                             \
    }                                                                                                 \
    decode_linear_kernel<E, NORM><<<grid, block, lds, s>>>(p);                                        \
  } while (0)
  if (norm_w) {
    if (epilogue == kEpiNone) ZKV_LIN(kEpiNone, true);
    else if (epilogue == kEpiResidual) ZKV_LIN(kEpiResidual, true);
    else ZKV_LIN(kEpiSiluMul, true);
  } else {
    if (epilogue == kEpiNone) ZKV_LIN(kEpiNone, false);
    else if (epilogue == kEpiResidual) ZKV_LIN(kEpiResidual, false);
    else ZKV_LIN(kEpiSiluMul, false);
  }
#undef ZKV_LIN
  return check_launch("decode_linear_kernel");
}

extern "C" int zkv_qk_norm_rope(const uint16_t* qkv, int64_t qkv_ld, int bs, int hq, int hkv,
                                const uint16_t* q_norm, const uint16_t* k_norm, float eps, const float* cos_row,
                                const float* sin_row, uint16_t* q_out, uint16_t* k_dst, int64_t k_sb,
                                int64_t k_sh, uint16_t* v_dst, int64_t v_sb, int64_t v_sh, zkv_stream_t stream) {
  ZKV_REQUIRE(qkv && q_norm && k_norm && cos_row && sin_row && q_out && k_dst && v_dst,
              "zkv_qk_norm_rope: null pointer");
  ZKV_REQUIRE(bs > 0 && hq > 0 && hkv > 0 && qkv_ld >= static_cast<int64_t>(hq + 2 * hkv) * 128,
              "zkv_qk_norm_rope: bad sizes bs=%d hq=%d hkv=%d qkv_ld=%lld", bs, hq, hkv,
              static_cast<long long>(qkv_ld));
  const QkParams p{qkv, qkv_ld, q_norm, k_norm, eps, cos_row, sin_row, q_out, k_dst, k_sb, k_sh,
                   v_dst, v_sb, v_sh, bs, hq, hkv};
  const int items = bs * (hq + 2 * hkv);
  qk_norm_rope_kernel<<<(items + 3) / 4, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(p);
  return check_launch("qk_norm_rope_kernel");
}
