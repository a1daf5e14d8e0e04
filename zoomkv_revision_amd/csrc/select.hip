// Page scoring and selection kernels (gfx950): Quest chunk upper bounds, exact
// top-k (with the fused LUT gather + skipped-tail concat), CDS density scores,
// the dense mask, the GQA-mean query and the KIVI stage-2 scorer.
//
// Bit-exactness: every fp32 reduction follows the reference kernel's order
// (cited per kernel), and bf16 rounding is RNE after every op as the
// reference's bf16 intrinsics do.
#include "zkv_common.hpp"

#include <cstdlib>
#include <type_traits>

namespace zkv {
namespace {

// ----------------------------------------------------------------------------
// Quest chunk score (Z/cache_hub/quest/quest_chunk_score.cu:31-103)
//   score = sum_d max(q_d * mn_d, q_d * mx_d); lane t of a 32-lane group sums
//   dims 4t..4t+3 left to right, then xor butterfly 16, 8, 4, 2, 1.
// Each 32-lane half of a wave64 scores 4 adjacent chunks per trip, issuing
// all their loads first (the valid flag is applied at the end), and the grid
// strides over all (b, kv, chunk).  HBM-bound: 512 B of metadata per chunk.
// ----------------------------------------------------------------------------
template <bool kFp16Meta>
__device__ __forceinline__ float meta_to_f32(uint16_t v) {
  if constexpr (kFp16Meta)
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  else
    return bf16_to_f32(v);
}

constexpr int kQuestUnroll = 4;  // chunks per 32-lane half per trip, loads issued together

template <bool kFp16Meta>
__global__ __launch_bounds__(256) void quest_score_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ cmin,
    const uint16_t* __restrict__ cmax, const uint8_t* __restrict__ valid, float* __restrict__ scores,
    int n_chunks, int n_max, int64_t total) {
  const int half = threadIdx.x >> 5;  // 8 halves of 32 lanes per block
  const int t = threadIdx.x & 31;
  constexpr int U = kQuestUnroll;
  for (int64_t item0 = (static_cast<int64_t>(blockIdx.x) * 8 + half) * U; item0 < total;
       item0 += static_cast<int64_t>(gridDim.x) * 8 * U) {
    u32x2_t qv[U], mv[U], xv[U];
    int64_t row[U];
    // all loads of the U chunks first (rows past the end re-read the last one)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t item = min(item0 + u, total - 1);
      const int64_t bh = item / n_chunks;
      const int chunk = static_cast<int>(item - bh * n_chunks);
      row[u] = bh * n_max + chunk;
      qv[u] = *reinterpret_cast<const u32x2_t*>(q + bh * 128 + 4 * t);
      mv[u] = *reinterpret_cast<const u32x2_t*>(cmin + row[u] * 128 + 4 * t);
      xv[u] = *reinterpret_cast<const u32x2_t*>(cmax + row[u] * 128 + 4 * t);
    }
    float sum[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float qq[4], mn[4], mx[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        qq[2 * i] = __uint_as_float(qv[u][i] << 16);
        qq[2 * i + 1] = __uint_as_float(qv[u][i] & 0xFFFF0000u);
        mn[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[u][i] & 0xFFFF));
        mn[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[u][i] >> 16));
        mx[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[u][i] & 0xFFFF));
        mx[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[u][i] >> 16));
      }
      float sm = fmaxf(qq[0] * mn[0], qq[0] * mx[0]);
      sm = sm + fmaxf(qq[1] * mn[1], qq[1] * mx[1]);
      sm = sm + fmaxf(qq[2] * mn[2], qq[2] * mx[2]);
      sm = sm + fmaxf(qq[3] * mn[3], qq[3] * mx[3]);
      sum[u] = sm;
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
#pragma unroll
      for (int u = 0; u < U; ++u) sum[u] = sum[u] + __shfl_xor(sum[u], off);
    if (t < U) {
      // lane u stores chunk u (every lane holds every sum after the butterfly)
      float out = sum[0];
      int64_t r = row[0];
#pragma unroll
      for (int u = 1; u < U; ++u)
        if (t == u) {
          out = sum[u];
          r = row[u];
        }
      const int64_t item = item0 + t;
      if (item < total) {
        if (valid != nullptr && !valid[r]) out = -INFINITY;
        scores[item] = out;
      }
    }
  }
}

// Quest bounds with the GQA-mean query formed in the same launch.  Block
// (x, bh) scores chunks [32x, 32x + 32) of row bh (8 halves of 32 lanes, 4
// chunks each, the quest_score_kernel lane order and sums).  Its metadata
// loads are issued first; meanwhile threads 0..127 form raw_q[bh] dim tid =
// bf16(sum_i q[b, h*group + i][tid] / group) in head order (gqa_mean_kernel's
// arithmetic) into LDS, and block 0 of the row stores it.
template <bool kFp16Meta, int U>
__global__ __launch_bounds__(256) void quest_gqa_kernel(
    const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh, int group, int kv,
    uint16_t* __restrict__ raw_q_out, const uint16_t* __restrict__ cmin, const uint16_t* __restrict__ cmax,
    const uint8_t* __restrict__ valid, float* __restrict__ scores, int n_chunks, int n_max) {
  __shared__ uint16_t s_q[128];
  const int half = threadIdx.x >> 5, t = threadIdx.x & 31;
  const int bh = blockIdx.y;
  const int c0 = (blockIdx.x * 8 + half) * U;
  u32x2_t mv[U], xv[U];
  int row[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int chunk = min(c0 + u, n_chunks - 1);  // past the end re-reads the last chunk
    row[u] = chunk;
    const int64_t off = (static_cast<int64_t>(bh) * n_max + chunk) * 128 + 4 * t;
    mv[u] = *reinterpret_cast<const u32x2_t*>(cmin + off);
    xv[u] = *reinterpret_cast<const u32x2_t*>(cmax + off);
  }
  if (threadIdx.x < 128) {
    const int b = bh / kv, h = bh - b * kv, d = threadIdx.x;
    const uint16_t* qp = q + b * q_sb + static_cast<int64_t>(h) * group * q_sh + d;
    constexpr int kRows = 8;  // head rows requested together, summed in head order
    uint16_t w[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) w[i] = qp[min(i, group - 1) * q_sh];
    float acc = bf16_to_f32(w[0]);
#pragma unroll
    for (int i = 1; i < kRows; ++i)
      if (i < group) acc = acc + bf16_to_f32(w[i]);
    for (int i = kRows; i < group; ++i) acc = acc + bf16_to_f32(qp[i * q_sh]);
    const uint16_t r = f32_to_bf16_bits(acc / static_cast<float>(group));
    s_q[d] = r;
    if (blockIdx.x == 0) raw_q_out[static_cast<int64_t>(bh) * 128 + d] = r;
  }
  __syncthreads();
  const u32x2_t qv = *reinterpret_cast<const u32x2_t*>(s_q + 4 * t);
  float qq[4];
  qq[0] = __uint_as_float(qv[0] << 16);
  qq[1] = __uint_as_float(qv[0] & 0xFFFF0000u);
  qq[2] = __uint_as_float(qv[1] << 16);
  qq[3] = __uint_as_float(qv[1] & 0xFFFF0000u);
  float sum[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float mn[4], mx[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      mn[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[u][i] & 0xFFFF));
      mn[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[u][i] >> 16));
      mx[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[u][i] & 0xFFFF));
      mx[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[u][i] >> 16));
    }
    float sm = fmaxf(qq[0] * mn[0], qq[0] * mx[0]);
    sm = sm + fmaxf(qq[1] * mn[1], qq[1] * mx[1]);
    sm = sm + fmaxf(qq[2] * mn[2], qq[2] * mx[2]);
    sm = sm + fmaxf(qq[3] * mn[3], qq[3] * mx[3]);
    sum[u] = sm;
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1)
#pragma unroll
    for (int u = 0; u < U; ++u) sum[u] = sum[u] + __shfl_xor(sum[u], off);
  if (t < U) {
    float out = sum[0];
    int r = row[0];
#pragma unroll
    for (int u = 1; u < U; ++u)
      if (t == u) {
        out = sum[u];
        r = row[u];
      }
    const int chunk = c0 + t;
    if (chunk < n_chunks) {
      const int64_t vr = static_cast<int64_t>(bh) * n_max + r;
      if (valid != nullptr && !valid[vr]) out = -INFINITY;
      scores[static_cast<int64_t>(bh) * n_chunks + chunk] = out;
    }
  }
}

// ----------------------------------------------------------------------------
// Exact top-k of a row (float_topk.cu:51-271 semantics, deterministic):
// radix select on order-preserving uint32 keys (4 rounds of 8 bits) finds the
// k-th largest key T exactly; then one ordered pass keeps every key > T and
// the lowest-index keys == T, writing them in increasing index order.
// No candidate buffer, so no overflow at any length (the reference drops
// candidates beyond 8192 per round, float_topk.cu:95).
// Optional: out = lut[idx] (float_topk_gather_concat.cu:109-114) and the
// skipped tail copied to out[k, k + sk).
// ----------------------------------------------------------------------------
constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;

// Optional second output of a top-k: a byte mask over the row's L slots, 1
// at every selected index (dense_mask_from_topk fused in; m == nullptr: none).
struct TopkMask {
  uint8_t* m;
  int64_t stride;
};

__device__ __forceinline__ uint32_t ordered_key(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int block_exclusive_count(bool flag, int* s_wave, int& total) {
  // exclusive rank of this thread's flag over the block (thread order), and
  // the block total; s_wave holds kTopkWaves ints
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t m = __ballot(flag);
  const int in_wave = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
  if (lane == 0) s_wave[wave] = __popcll(m);
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) {
    const int c = s_wave[w];
    before += (w < wave) ? c : 0;
    total += c;
  }
  __syncthreads();
  return before + in_wave;
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(
    const float* __restrict__ in, int64_t in_stride, int L, int k, int64_t* __restrict__ out,
    int64_t out_stride, const int64_t* __restrict__ lut, int64_t lut_stride,
    const int64_t* __restrict__ skipped, int64_t sk_stride, int sk_count, int64_t sentinel,
    const TopkMask mk) {
  __shared__ int s_hist[kTopkWaves][256];
  __shared__ int s_wave[kTopkWaves];
  __shared__ int s_bin, s_remain;
  const int row = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6;
  const float* x = in + row * in_stride;
  int64_t* o = out + row * out_stride;
  const int64_t* lrow = lut ? lut + row * lut_stride : nullptr;

  uint8_t* mrow = mk.m ? mk.m + row * mk.stride : nullptr;
  for (int i = tid; i < sk_count; i += kTopkThreads) o[k + i] = skipped[row * sk_stride + i];
  if (L <= k) {
    for (int i = tid; i < k; i += kTopkThreads) o[i] = (i < L) ? (lrow ? lrow[i] : i) : sentinel;
    if (mrow)
      for (int i = tid; i < L; i += kTopkThreads) mrow[i] = 1;
    return;
  }
  if (mrow)  // cleared here, set after the barriers below
    for (int i = tid; i < L; i += kTopkThreads) mrow[i] = 0;

  uint32_t prefix = 0, mask = 0;
  int remain = k;  // how many of the candidates matching (prefix, mask) to keep
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < kTopkWaves * 256; i += kTopkThreads) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < L; i += kTopkThreads) {
      const uint32_t key = ordered_key(x[i]);
      if ((key & mask) == prefix) atomicAdd(&s_hist[wave][(key >> shift) & 0xFF], 1);
    }
    __syncthreads();
    if (tid < 256) {
      int c = 0;
#pragma unroll
      for (int w = 0; w < kTopkWaves; ++w) c += s_hist[w][tid];
      s_hist[0][tid] = c;
    }
    __syncthreads();
    if (tid < 64) {
      // suffix counts over the 256 bins, 4 bins per lane, highest bins first
      int c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = s_hist[0][4 * tid + j];
      int lane_sum = c[0] + c[1] + c[2] + c[3];
      // inclusive suffix scan across lanes (lane 63 holds the top bins)
      int suf = lane_sum;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_down(suf, off);
        if (tid + off < 64) suf += v;
      }
      // bins above this lane's range: suf - lane_sum
      int above = suf - lane_sum;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const int at_or_above = above + c[j];
        if (at_or_above >= remain && above < remain) {
          s_bin = 4 * tid + j;
          s_remain = remain - above;
        }
        above = at_or_above;
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(s_bin) << shift;
    mask |= 0xFFu << shift;
    remain = s_remain;
    __syncthreads();
  }
  // prefix == T, remain = number of keys == T to keep (lowest indices first)
  const uint32_t T = prefix;
  int taken_eq = 0, written = 0;
  for (int base = 0; base < L; base += kTopkThreads) {
    const int i = base + tid;
    const uint32_t key = i < L ? ordered_key(x[i]) : 0u;
    const bool gt = i < L && key > T;
    const bool eq = i < L && key == T;
    int eq_total = 0;
    const int eq_rank = block_exclusive_count(eq, s_wave, eq_total);
    const bool sel = gt || (eq && taken_eq + eq_rank < remain);
    int sel_total = 0;
    const int pos = written + block_exclusive_count(sel, s_wave, sel_total);
    if (sel) {
      o[pos] = lrow ? lrow[i] : i;
      if (mrow) mrow[i] = 1;
    }
    taken_eq += eq_total;
    written += sel_total;
    if (written >= k) break;  // uniform across the block
  }
}

// ----------------------------------------------------------------------------
// The same selection for rows of at most 1024 * R elements with the row held
// in registers (thread t keeps indices t + 1024 j, j < R: coalesced loads,
// one read of the row for all four radix rounds).  The ordered output needs
// one scan: for each register row j a wave ballots its greater-than-T and
// equal-to-T bits; the (row j, wave w) counts, in index order j-major then
// w, are scanned once, giving every element its rank among the gt and the
// eq elements of lower index:  pos(i) = #gt below i + min(#eq below i, remain).
//
// Long rows with a small k (R >= 8, k <= 512) first narrow the row to a
// candidate list: tau = the m-th largest of 256 evenly spaced keys (top 16
// bits), with m set so that about 8k keys of the row are >= tau; the keys >=
// tau are compacted into LDS in index order.  When there are at least k of
// them (and no more than 4096) the k-th largest key of the row is >= tau, so
// every key of the top k, ties included, is a candidate and the selection
// over the candidates is the selection over the row; otherwise the row takes
// the full path.
// ----------------------------------------------------------------------------
constexpr int kTopkCand = 4096;
constexpr int kTopkSampledMaxK = 512;
constexpr int kTopkSample = 256;

__device__ __forceinline__ uint32_t ordered_key_bits(uint32_t b) {
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ordered_key(x) >= tau (tau != 0) on the raw bits b of x, as one unsigned
// compare: ((b - base) < lim) != inv.  For tau >= 2^31 (the key of a
// non-negative float) the passing bits are [tau - 2^31, 2^31); otherwise all
// bits except [2^32 - tau, 2^32) (the negative floats whose key is below
// tau).  Raw bits 0xFFFFFFFF (key 0) never pass.
struct TauTest {
  uint32_t base, lim;
  uint64_t inv;  // all ones when the compare result is inverted
};
__device__ __forceinline__ TauTest make_tau_test(uint32_t tau) {
  if (tau >= 0x80000000u) return {tau ^ 0x80000000u, 0x80000000u - (tau ^ 0x80000000u), 0ull};
  return {0u - tau, tau, ~0ull};
}

// Inclusive prefix sum over the 64 lanes of a wave: shifts by 1, 2, 4, 8
// within each row of 16 lanes, then lane 15 of a row added into the next row
// (rows 1 and 3) and lane 31 into rows 2 and 3 (DPP row_shr / row_bcast).
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return v;
}

// Per-(register row j, wave w) counts live at cnt[w * R + j]; their index
// order is j-major, then w.  wave_exclusive_scan replaces them, by one wave,
// with their exclusive prefix in that order and returns the total.
template <int R>
__device__ __forceinline__ uint32_t wave_exclusive_scan(uint32_t* cnt, int lane) {
  constexpr int N = R * kTopkWaves, kPer = N / 64;
  static_assert(N % 64 == 0, "whole entries per lane");
  uint32_t v[kPer];
  uint32_t sum = 0;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int idx = lane * kPer + e;  // (j, w) = (idx / 16, idx % 16)
    v[e] = cnt[(idx % kTopkWaves) * R + idx / kTopkWaves];
    sum += v[e];
  }
  const uint32_t inc = static_cast<uint32_t>(wave_inclusive_sum(static_cast<int>(sum)));
  uint32_t run = inc - sum;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int idx = lane * kPer + e;
    cnt[(idx % kTopkWaves) * R + idx / kTopkWaves] = run;
    run += v[e];
  }
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(inc), 63));
}

// A copy of a uniform value that the compiler cannot merge with other uses:
// the per-row bounds compares are then recomputed where they are used instead
// of being kept live (in scalar registers that spill) across the barriers.
__device__ __forceinline__ int opaque(int v) {
  v = __builtin_amdgcn_readfirstlane(v);
  asm volatile("" : "+s"(v));
  return v;
}

// Rank of this lane's bit among the set bits of a wave mask below it.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0)));
}

// Radix select over the n keys key[j] at list positions tid + 1024 j (later
// positions are ignored): returns T and remain such that the top k are the
// keys > T and the first `remain` keys == T in list order.  hist[0] must be
// zero on entry (both histograms are left dirty).  Each round: a block
// histogram of the next 8 bits, then wave 0 (lane l owns bins 252 - 4l ..
// 255 - 4l, so a prefix sum over lanes counts the keys in higher bins) finds
// the bin holding the remain-th key.  When the top k take every key of that
// bin, the rounds stop: T = the bin's lowest key value (prefix, low bits 0)
// and remain = the bin's count, which covers every key == T in it.
template <int R>
__device__ __forceinline__ uint32_t radix_select(const uint32_t (&key)[R], int n, int k, int (*hist)[256],
                                                 int* s_sel, int& remain) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  uint32_t prefix = 0, mask = 0;
  remain = k;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int shift = 24 - 8 * r;
    int* h = hist[r & 1];
    const int nr = opaque(n);
    // clear the other buffer (last read before the previous barrier) for the next round
    if (tid < 64) reinterpret_cast<int4*>(hist[(r + 1) & 1])[tid] = make_int4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const bool in = tid < nr - kTopkThreads * j && (key[j] & mask) == prefix;
      const int bin = (key[j] >> shift) & 0xFF;
      if (r == 0) {
        // Float keys share few top bytes, so most lanes of a wave hit one or
        // two bins: the two most common (by first lane) are added once per
        // wave, the remaining lanes add one each.
        uint64_t todo = __ballot(in);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          if (todo != 0) {
            const int lead = __builtin_ctzll(todo);
            const int b0 = __builtin_amdgcn_readlane(bin, lead);
            const uint64_t same = __ballot(bin == b0) & todo;
            if (lane == lead) atomicAdd(&h[b0], static_cast<int>(__popcll(same)));
            todo &= ~same;
          }
        }
        if ((todo >> lane) & 1ull) atomicAdd(&h[bin], 1);
      } else if (in) {
        atomicAdd(&h[bin], 1);
      }
    }
    __syncthreads();
    if (wave == 0) {
      const int4 c = reinterpret_cast<const int4*>(h)[63 - lane];
      const int lane_sum = c.x + c.y + c.z + c.w;
      int above = wave_inclusive_sum(lane_sum) - lane_sum;
      const int cb[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const int at_or_above = above + cb[j];
        if (at_or_above >= remain && above < remain) {
          s_sel[0] = 4 * (63 - lane) + j;
          s_sel[1] = remain - above;
          s_sel[2] = cb[j];
        }
        above = at_or_above;
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(s_sel[0]) << shift;
    mask |= 0xFFu << shift;
    remain = s_sel[1];
    if (remain == s_sel[2]) break;  // the whole bin is in the top k (uniform)
  }
  return prefix;
}

// Calls emit(pos, p) for every list position p < n in the top k (keys > T,
// then the first `remain` keys == T), pos = its rank in list order (< k).
template <int R, typename Emit>
__device__ __forceinline__ void ordered_emit(const uint32_t (&key)[R], int n, int k, uint32_t T, int remain,
                                             uint32_t* cnt, Emit&& emit) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  uint32_t mine = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const bool in_list = tid < n - kTopkThreads * j;
    const uint64_t gt = __ballot(in_list && key[j] > T), eq = __ballot(in_list && key[j] == T);
    const uint32_t c = static_cast<uint32_t>(__popcll(gt)) | (static_cast<uint32_t>(__popcll(eq)) << 16);
    mine = lane == j ? c : mine;
  }
  if (lane < R) cnt[wave * R + lane] = mine;
  __syncthreads();
  if (wave == 0) wave_exclusive_scan<R>(cnt, lane);
  __syncthreads();
  // the ballots are recomputed rather than kept live across the barriers
  const int n2 = opaque(n);
  const uint32_t T2 = static_cast<uint32_t>(opaque(static_cast<int>(T)));
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const bool in_list = tid < n2 - kTopkThreads * j;
    const bool is_gt = in_list && key[j] > T2, is_eq = in_list && key[j] == T2;
    const uint64_t gt = __ballot(is_gt), eq = __ballot(is_eq);
    if ((gt | eq) != 0) {
      const uint32_t pre = cnt[wave * R + j];
      const int gt_rank = static_cast<int>(pre & 0xFFFFu) + lanes_below(gt);
      const int eq_rank = static_cast<int>(pre >> 16) + lanes_below(eq);
      const int pos = gt_rank + min(eq_rank, remain);
      if ((is_gt || (is_eq && eq_rank < remain)) && pos < k) emit(pos, tid + kTopkThreads * j);
    }
  }
}

// The candidate path of a sampled row (see above); false when the number of
// keys >= tau is outside [k, kTopkCand] and the row must take the full path.
// bits[j]: raw float bits of row index tid + 1024 j, 0xFFFFFFFF past the row.
// The ballots are recomputed after the barrier rather than kept live.
template <int R>
__device__ __forceinline__ bool topk_from_candidates(const uint32_t (&bits)[R], int L, int k, const TauTest tt,
                                                     uint32_t* s_cnt, uint2* s_cand, int (*s_hist)[256],
                                                     int* s_sel, uint32_t* s_total, int64_t* o,
                                                     const int64_t* lrow, uint8_t* mrow) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int mine = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (kTopkThreads * j < L) {
      const uint64_t m = __ballot(bits[j] - tt.base < tt.lim) ^ tt.inv;
      mine = lane == j ? __popcll(m) : mine;
    }
  }
  if (lane < R) s_cnt[wave * R + lane] = static_cast<uint32_t>(mine);
  __syncthreads();
  if (wave == 0) {
    const uint32_t total = wave_exclusive_scan<R>(s_cnt, lane);
    if (lane == 0) *s_total = total;
  }
  __syncthreads();
  const int total = static_cast<int>(*s_total);
  if (total < k || total > kTopkCand) return false;
  // the ballots are recomputed rather than kept live across the barriers
  const int L2 = opaque(L);
  const uint32_t base2 = static_cast<uint32_t>(opaque(static_cast<int>(tt.base)));
  const uint32_t lim2 = static_cast<uint32_t>(opaque(static_cast<int>(tt.lim)));
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (kTopkThreads * j < L2) {
      const bool pass = bits[j] - base2 < lim2;
      const uint64_t m = __ballot(pass) ^ tt.inv;
      if (m != 0) {
        const int p = static_cast<int>(s_cnt[wave * R + j]) + lanes_below(m);
        if (pass != (tt.inv != 0) && p < kTopkCand)
          s_cand[p] = make_uint2(bits[j], static_cast<uint32_t>(tid + kTopkThreads * j));
      }
    }
  }
  __syncthreads();
  constexpr int kQ = kTopkCand / kTopkThreads;
  uint32_t ck[kQ];
#pragma unroll
  for (int q = 0; q < kQ; ++q)
    ck[q] = tid < total - kTopkThreads * q ? ordered_key_bits(s_cand[tid + kTopkThreads * q].x) : 0u;
  int remain;
  const uint32_t T = radix_select<kQ>(ck, total, k, s_hist, s_sel, remain);
  ordered_emit<kQ>(ck, total, k, T, remain, s_cnt, [&](int pos, int p) {
    const int i = static_cast<int>(s_cand[p].y);
    o[pos] = lrow ? lrow[i] : i;
    if (mrow) mrow[i] = 1;
  });
  return true;
}

template <int R>
__global__ __launch_bounds__(kTopkThreads) void topk_reg_kernel(
    const float* __restrict__ in, int64_t in_stride, int L, int k, int64_t* __restrict__ out,
    int64_t out_stride, const int64_t* __restrict__ lut, int64_t lut_stride,
    const int64_t* __restrict__ skipped, int64_t sk_stride, int sk_count, int64_t sentinel,
    const TopkMask mk) {
  constexpr bool kSampled = R >= 8;
  constexpr int kCand = kSampled ? kTopkCand : 1;
  static_assert(R % 4 == 0 && R * kTopkWaves >= 64, "register rows come in fours");
  static_assert(kTopkThreads * R <= 65536, "16-bit counts per (j, w) prefix");
  __shared__ __align__(16) int s_hist[2][256];
  __shared__ __align__(16) uint32_t s_cnt[R * kTopkWaves];  // [w][j] counts, then their exclusive prefix
  __shared__ uint2 s_cand[kCand];  // the sample keys, then (raw bits, index) of the candidates
  __shared__ int s_sel[3];
  __shared__ uint32_t s_tau, s_total;
  const int row = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* x = in + row * in_stride;
  int64_t* o = out + row * out_stride;
  const int64_t* lrow = lut ? lut + row * lut_stride : nullptr;

  uint8_t* mrow = mk.m ? mk.m + row * mk.stride : nullptr;
  for (int i = tid; i < sk_count; i += kTopkThreads) o[k + i] = skipped[row * sk_stride + i];
  if (L <= k) {
    for (int i = tid; i < k; i += kTopkThreads) o[i] = (i < L) ? (lrow ? lrow[i] : i) : sentinel;
    if (mrow)
      for (int i = tid; i < L; i += kTopkThreads) mrow[i] = 1;
    return;
  }
  if (mrow)  // cleared here, set after the barriers below
    for (int i = tid; i < L; i += kTopkThreads) mrow[i] = 0;
  // All loads are issued before any is used (addresses clamped into the row),
  // the sample first, and the threshold search runs while the row arrives.
  const bool sampled = kSampled && k <= kTopkSampledMaxK;
  float sample = 0.0f;
  if constexpr (kSampled) {
    sample = x[((tid % kTopkSample) * L) / kTopkSample];
    __builtin_amdgcn_sched_barrier(0);
  }
  float v[R];
#pragma unroll
  for (int j = 0; j < R; ++j) v[j] = x[kTopkThreads * j + min(tid, L - 1 - kTopkThreads * j)];
  // every thread stores its (possibly repeated) sample key, so the load is not sunk below the row loads
  if constexpr (kSampled) reinterpret_cast<uint32_t*>(s_cand)[tid] = ordered_key(sample);
  if (tid < 128) reinterpret_cast<int4*>(&s_hist[0][0])[tid] = make_int4(0, 0, 0, 0);
  __syncthreads();
  uint32_t tau = 0;
  if constexpr (kSampled) {
    if (sampled) {
      if (wave == 0) {
        constexpr int kPer = kTopkSample / 64;
        uint32_t sv[kPer];
#pragma unroll
        for (int e = 0; e < kPer; ++e) sv[e] = reinterpret_cast<const uint32_t*>(s_cand)[e * 64 + lane];
        const int target = min(8 * k, kTopkCand / 2);
        const int m = min(kTopkSample, max(1, (target * kTopkSample + L - 1) / L));
        uint32_t t = 0;
        for (int b = 31; b >= 16; --b) {
          const uint32_t c = t | (1u << b);
          int cnt = 0;
#pragma unroll
          for (int e = 0; e < kPer; ++e) cnt += __popcll(__ballot(sv[e] >= c));
          if (cnt >= m) t = c;
        }
        if (lane == 0) s_tau = t;
      }
      __syncthreads();
      tau = s_tau;
    }
  }
  uint32_t bits[R];
#pragma unroll
  for (int j = 0; j < R; ++j) bits[j] = tid < L - kTopkThreads * j ? __float_as_uint(v[j]) : ~0u;
  if constexpr (kSampled) {
    if (sampled && tau != 0) {
      if (topk_from_candidates<R>(bits, L, k, make_tau_test(tau), s_cnt, s_cand, s_hist, s_sel, &s_total, o,
                                  lrow, mrow))
        return;
    }
  }
  uint32_t key[R];
#pragma unroll
  for (int j = 0; j < R; ++j) key[j] = ordered_key_bits(bits[j]);
  int remain;
  const uint32_t T = radix_select<R>(key, L, k, s_hist, s_sel, remain);
  ordered_emit<R>(key, L, k, T, remain, s_cnt, [&](int pos, int i) {
    o[pos] = lrow ? lrow[i] : i;
    if (mrow) mrow[i] = 1;
  });
}

// ----------------------------------------------------------------------------
// GQA mean + Quest bounds + the row's top-k in one launch
// (S:1621-1626 + S:2223 + the float_topk_3d of S:2168-2190).  A 1024-thread
// block scores TR trips of 32 * kQuestUnroll chunks of one (b, kv) row (all
// trips' loads issued first) with the arithmetic of quest_gqa_kernel (so the
// scores are the same bits), stores them device-coherently (write-through)
// and counts itself in on the row's arrival slot.  The arrival is one
// fetch-and-add (the blocks of a row finish close together; compare-and-swap
// retries serialised them, 41 us against 27 at 64 rows x 2048 chunks), and TR
// is chosen so that the grid is one wave of blocks: each block waits for its
// stores' acknowledgement once (27 us with 1024 blocks, 20 with 512 of two
// trips).  The block that completes the row reads the row's scores back with
// device-coherent loads and runs topk_reg_kernel<4>'s radix select and
// ordered emit on them (the same indices, in increasing index order).
// ----------------------------------------------------------------------------
constexpr int kQuestTopkChunks = 32 * kQuestUnroll;  // chunks per 1024-thread block per trip
constexpr int kQuestTopkMaxL = 4 * kTopkThreads;       // rows up to 4096 chunks (4 registers)

template <bool kFp16Meta, int TR>
__global__ __launch_bounds__(kTopkThreads) void quest_topk_kernel(
    const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh, int group, int kv,
    uint16_t* __restrict__ raw_q_out, const uint16_t* __restrict__ cmin, const uint16_t* __restrict__ cmax,
    const uint8_t* __restrict__ valid, float* __restrict__ scores, int n_chunks, int n_max, int k,
    int64_t* __restrict__ out, int64_t out_stride, unsigned int* __restrict__ slots) {
  constexpr int U = kQuestUnroll;
  __shared__ uint16_t s_q[128];
  __shared__ __align__(16) int s_hist[2][256];
  __shared__ __align__(16) uint32_t s_cnt[4 * kTopkWaves];
  __shared__ int s_sel[3];
  __shared__ int s_last;
  const int tid = threadIdx.x, half = tid >> 5, t = tid & 31;
  const int bh = blockIdx.y;
  // trip r of this block covers chunks [(x TR + r) 128, +128); every trip's
  // loads are issued before any score is formed
  u32x2_t mv[TR][U], xv[TR][U];
#pragma unroll
  for (int r = 0; r < TR; ++r)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int chunk = min(((blockIdx.x * TR + r) * 32 + half) * U + u, n_chunks - 1);  // past the end re-reads
      const int64_t off = (static_cast<int64_t>(bh) * n_max + chunk) * 128 + 4 * t;
      mv[r][u] = *reinterpret_cast<const u32x2_t*>(cmin + off);
      xv[r][u] = *reinterpret_cast<const u32x2_t*>(cmax + off);
    }
  if (tid < 128) {
    const int b = bh / kv, h = bh - b * kv, d = tid;
    const uint16_t* qp = q + b * q_sb + static_cast<int64_t>(h) * group * q_sh + d;
    constexpr int kRows = 8;  // head rows requested together, summed in head order
    uint16_t w[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) w[i] = qp[min(i, group - 1) * q_sh];
    float acc = bf16_to_f32(w[0]);
#pragma unroll
    for (int i = 1; i < kRows; ++i)
      if (i < group) acc = acc + bf16_to_f32(w[i]);
    for (int i = kRows; i < group; ++i) acc = acc + bf16_to_f32(qp[i * q_sh]);
    const uint16_t r = f32_to_bf16_bits(acc / static_cast<float>(group));
    s_q[d] = r;
    if (blockIdx.x == 0) raw_q_out[static_cast<int64_t>(bh) * 128 + d] = r;
  }
  if (tid < 128) reinterpret_cast<int4*>(&s_hist[0][0])[tid] = make_int4(0, 0, 0, 0);
  __syncthreads();
  const u32x2_t qv = *reinterpret_cast<const u32x2_t*>(s_q + 4 * t);
  float qq[4];
  qq[0] = __uint_as_float(qv[0] << 16);
  qq[1] = __uint_as_float(qv[0] & 0xFFFF0000u);
  qq[2] = __uint_as_float(qv[1] << 16);
  qq[3] = __uint_as_float(qv[1] & 0xFFFF0000u);
  float* srow = scores + static_cast<int64_t>(bh) * n_chunks;
#pragma unroll
  for (int r = 0; r < TR; ++r) {
    const int c0 = ((blockIdx.x * TR + r) * 32 + half) * U;
    float sum[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float mn[4], mx[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        mn[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[r][u][i] & 0xFFFF));
        mn[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(mv[r][u][i] >> 16));
        mx[2 * i] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[r][u][i] & 0xFFFF));
        mx[2 * i + 1] = meta_to_f32<kFp16Meta>(static_cast<uint16_t>(xv[r][u][i] >> 16));
      }
      float sm = fmaxf(qq[0] * mn[0], qq[0] * mx[0]);
      sm = sm + fmaxf(qq[1] * mn[1], qq[1] * mx[1]);
      sm = sm + fmaxf(qq[2] * mn[2], qq[2] * mx[2]);
      sm = sm + fmaxf(qq[3] * mn[3], qq[3] * mx[3]);
      sum[u] = sm;
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
#pragma unroll
      for (int u = 0; u < U; ++u) sum[u] = sum[u] + __shfl_xor(sum[u], off);
    if (t < U) {
      float o = sum[0];
#pragma unroll
      for (int u = 1; u < U; ++u)
        if (t == u) o = sum[u];
      const int chunk = c0 + t;
      if (chunk < n_chunks) {
        if (valid != nullptr && !valid[static_cast<int64_t>(bh) * n_max + chunk]) o = -INFINITY;
        // device-coherent (write-through): the row's selecting block may run
        // on another XCD
        __hip_atomic_store(srow + chunk, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // this lane's score stores are device-visible, then one arrival per block
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) s_last = arrive_last_count(slots + bh, gridDim.x);
  __syncthreads();
  if (!s_last) return;

  // ---- the row's top-k: topk_reg_kernel<4> on the stored scores ----
  const int L = n_chunks, wave = tid >> 6;
  int64_t* o = out + static_cast<int64_t>(bh) * out_stride;
  if (L <= k) {
    for (int i = tid; i < k; i += kTopkThreads) o[i] = i < L ? i : -1;
    return;
  }
  constexpr int R = 4;
  float v[R];
#pragma unroll
  for (int j = 0; j < R; ++j)
    v[j] = __hip_atomic_load(srow + kTopkThreads * j + min(tid, L - 1 - kTopkThreads * j), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  uint32_t key[R];
#pragma unroll
  for (int j = 0; j < R; ++j)
    key[j] = ordered_key_bits(tid < L - kTopkThreads * j ? __float_as_uint(v[j]) : ~0u);
  (void)wave;
  int remain;
  const uint32_t T = radix_select<R>(key, L, k, s_hist, s_sel, remain);
  ordered_emit<R>(key, L, k, T, remain, s_cnt, [&](int pos, int i) { o[pos] = i; });
}

// ----------------------------------------------------------------------------
// Next-token sampling over the top-(k + W) window (Z/model_hub/LLM.py:63-139:
// temperature, top-k with ties at the k-th value kept, top-p keeping the token
// that crosses top_p, softmax, one multinomial draw), one launch per step.
// Block (x, row) takes the row's logits [x S, (x + 1) S), S = 8192, scaled as
// torch scales a CUDA tensor by a Python float (times the fp32 reciprocal),
// and stores its W' = k + W largest under the strict order (value desc, index
// asc) device-coherently: key bits << 32 | ~index.  The block that completes
// the row ranks the row's candidates in LDS (the row's first W' under the same
// order, sorted), and wave 0 holds the window, lane i its i-th largest:
//  * overflow: the last window value equals the k-th, so the tie group may
//    reach past the window; the host then draws over the whole vocabulary;
//  * top-k keeps the values >= the k-th; top-p (0 < p < 1) drops the tokens
//    after the first whose cumulative probability (summed in window order)
//    exceeds p;
//  * softmax as torch's warp softmax (max, exp of the difference, xor
//    butterfly sum over 64 lanes, division), then the draw of
//    torch.multinomial for one sample: the first index of the largest
//    p / e, e = the caller's Exp(1) row drawn from the generator.
// ----------------------------------------------------------------------------
constexpr int kSampleR = 8;
constexpr int kSampleSlice = kSampleR * kTopkThreads;  // logits per block
constexpr int kSampleMaxWindow = 64;                   // k + W: one wave holds the window
constexpr int kSampleMaxCand = 2 * kTopkThreads;       // slices x window ranked per row

__device__ __forceinline__ float wave_max_xor(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

// softmax over the 64 lanes (-inf lanes give 0)
__device__ __forceinline__ float wave_softmax(float x) {
  const float mx = wave_max_xor(x);
  const float e = expf(x - mx);
  return e / wave_sum_xor(e);
}

__global__ __launch_bounds__(kTopkThreads) void sample_window_kernel(
    const float* __restrict__ logits, int64_t ld, int vocab, float inv_t, int k, int win, float top_p,
    const float* __restrict__ expo, int64_t e_ld, uint64_t* __restrict__ cand, unsigned int* __restrict__ slots,
    int64_t* __restrict__ tokens, int32_t* __restrict__ overflow) {
  constexpr int R = kSampleR;
  __shared__ __align__(16) int s_hist[2][256];
  __shared__ __align__(16) uint32_t s_cnt[R * kTopkWaves];
  __shared__ int s_sel[3];
  __shared__ int s_last;
  __shared__ uint64_t s_c[kSampleMaxCand];
  __shared__ uint64_t s_win[kSampleMaxWindow];
  const int tid = threadIdx.x, row = blockIdx.y, nb = gridDim.x;
  const int x0 = blockIdx.x * kSampleSlice;
  const int L = min(kSampleSlice, vocab - x0);
  const float* x = logits + row * ld + x0;
  uint64_t* crow = cand + (static_cast<int64_t>(row) * nb + blockIdx.x) * win;
  auto put = [&](int pos, int p) {  // position p of the slice as candidate pos
    const uint64_t c = (static_cast<uint64_t>(ordered_key(x[p] * inv_t)) << 32) |
                       static_cast<uint32_t>(~static_cast<uint32_t>(x0 + p));
    __hip_atomic_store(crow + pos, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (L <= win) {
    for (int i = tid; i < win; i += kTopkThreads) {
      if (i < L) put(i, i);
      else __hip_atomic_store(crow + i, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    uint32_t key[R];
#pragma unroll
    for (int j = 0; j < R; ++j) key[j] = ordered_key(x[min(tid + kTopkThreads * j, L - 1)] * inv_t);
    if (tid < 128) reinterpret_cast<int4*>(&s_hist[0][0])[tid] = make_int4(0, 0, 0, 0);
    __syncthreads();
    int remain;
    const uint32_t T = radix_select<R>(key, L, win, s_hist, s_sel, remain);
    ordered_emit<R>(key, L, win, T, remain, s_cnt, put);
  }
  // this lane's candidate stores are device-visible, then one arrival per block
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) s_last = arrive_last_count(slots + row, nb);
  __syncthreads();
  if (!s_last) return;

  // ---- the row's window: the top `win` of its nb * win candidates ----
  // Candidate positions run in index order (slices in order, each slice's
  // candidates in index order), so the radix select's (key desc, position asc)
  // is (value desc, index asc).  The winners, emitted in position order, are
  // then ranked among themselves.
  constexpr int RC = 4;  // register rows of the radix helpers (positions past nc are ignored)
  static_assert(kSampleMaxCand <= RC * kTopkThreads, "candidates per row within the register rows");
  const int nc = nb * win;
  uint32_t ck[RC] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int h = 0; h < kSampleMaxCand / kTopkThreads; ++h) {
    const int i = tid + h * kTopkThreads;
    const uint64_t c = i < nc ? __hip_atomic_load(cand + static_cast<int64_t>(row) * nc + i, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : uint64_t{0};
    s_c[i] = c;
    ck[h] = static_cast<uint32_t>(c >> 32);
  }
  if (tid < 128) reinterpret_cast<int4*>(&s_hist[0][0])[tid] = make_int4(0, 0, 0, 0);
  __syncthreads();
  {
    int remain;
    const uint32_t T = radix_select<RC>(ck, nc, win, s_hist, s_sel, remain);
    ordered_emit<RC>(ck, nc, win, T, remain, s_cnt, [&](int pos, int p) { s_win[pos] = s_c[p]; });
  }
  __syncthreads();
  if (tid < win) {
    const uint64_t c = s_win[tid];
    int rank = 0;
    for (int j = 0; j < win; ++j) rank += s_win[j] > c ? 1 : 0;
    s_c[rank] = c;  // s_c is free again: the window in rank order
  }
  __syncthreads();
  if (tid >= 64) return;
  const int lane = tid;
  const bool in = lane < win;
  const uint64_t cw = in ? s_c[lane] : uint64_t{0};
  const uint32_t kb = static_cast<uint32_t>(cw >> 32);
  const float val = __uint_as_float((kb & 0x80000000u) ? (kb & 0x7FFFFFFFu) : ~kb);
  const int idx = static_cast<int>(~static_cast<uint32_t>(cw));
  const float kth = __shfl(val, k - 1), last = __shfl(val, win - 1);
  float w = in && !(val < kth) ? val : -INFINITY;
  if (top_p > 0.0f && top_p < 1.0f) {
    const float p = wave_softmax(w);
    float cum = 0.0f;  // p_0 + ... + p_lane, left to right
    for (int j = 0; j < win; ++j) {
      const float pj = __shfl(p, j);
      if (j <= lane) cum = cum + pj;
    }
    const float before = __shfl_up(cum, 1);
    if (lane >= 1 && before > top_p) w = -INFINITY;
  }
  const float prob = wave_softmax(w);
  const float e = expo[row * e_ld + (in ? idx : 0)];
  const float ratio = in ? prob / e : -INFINITY;
  const float best = wave_max_xor(ratio);
  int tok = in && ratio == best ? idx : vocab;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) tok = min(tok, __shfl_xor(tok, off));
  if (lane == 0) {
    tokens[row] = tok;
    overflow[row] = last == kth ? 1 : 0;
  }
}

// ----------------------------------------------------------------------------
// CDS density: centroid[chunk_id] . q (rerank_topk.cu:560-624): buf[t] = c[t]q[t]
// for t < 128, then buf[t] += buf[t+s], s = 64..1; invalid id -> -1e30.
// A wave scores kDensityItems slots (lane l starts with p[l] + p[l+64] of
// each), their loads issued together and their trees interleaved.  The tree
// steps read lane l + s without LDS: s = 32 and 16 by the gfx950 permlane
// swaps, s = 8, 4, 2, 1 by DPP row shifts (lanes >= s carry values that the
// later steps do not read).
// ----------------------------------------------------------------------------
constexpr int kDensityItems = 8;

// x[lane + 32] in lanes 0-31 / x[lane + 16] in lanes 0-15 (and 32-47).
__device__ __forceinline__ float from_lane_plus32(float x) {
  return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}
__device__ __forceinline__ float from_lane_plus16(float x) {
  return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}
// x[lane + n] within each row of 16 lanes (DPP row_shl:n)
template <int n>
__device__ __forceinline__ float from_lane_plus(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + n, 0xf, 0xf, false));
}

__global__ __launch_bounds__(256) void density_kernel(
    const int64_t* __restrict__ ids, int64_t id_sb, int64_t id_sh, const uint16_t* __restrict__ cent,
    int64_t c_sb, int64_t c_sh, int64_t c_sc, const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh,
    float* __restrict__ out, int64_t o_sb, int64_t o_sh, int kv, int nk, int n_chunks, int total) {
  constexpr int U = kDensityItems;
  const int lane = threadIdx.x & 63;
  const int item0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * U;
  if (item0 >= total) return;
  // consecutive items: (row bh, slot) advance with a wrap instead of a division each
  int bh = item0 / nk, slot = item0 - bh * nk;
  int bhs[U], slots[U];
  float v[U];
  bool ok[U];
  uint16_t c0[U], c1[U], q0[U], q1[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool in = item0 + u < total;
    bhs[u] = in ? bh : 0;
    slots[u] = in ? slot : 0;
    const int b = bhs[u] / kv, h = bhs[u] - (bhs[u] / kv) * kv;
    const int64_t cid = ids[b * id_sb + h * id_sh + slots[u]];
    ok[u] = cid >= 0 && cid < n_chunks;
    const uint16_t* c = cent + b * c_sb + h * c_sh + (ok[u] ? cid : 0) * c_sc;
    const uint16_t* qq = q + b * q_sb + h * q_sh;
    c0[u] = c[lane];
    c1[u] = c[lane + 64];
    q0[u] = qq[lane];
    q1[u] = qq[lane + 64];
    if (++slot == nk) slot = 0, ++bh;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float a = bf16_to_f32(c0[u]) * bf16_to_f32(q0[u]) + 0.0f;
    const float w = bf16_to_f32(c1[u]) * bf16_to_f32(q1[u]);
    v[u] = a + w;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus32(v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus16(v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus<8>(v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus<4>(v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus<2>(v[u]);
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = v[u] + from_lane_plus<1>(v[u]);
  if (lane == 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = bhs[u] / kv, h = bhs[u] - (bhs[u] / kv) * kv;
      if (item0 + u < total) out[b * o_sb + h * o_sh + slots[u]] = ok[u] ? v[u] : -1e30f;
    }
  }
}

// mask.fill_(False); mask.scatter_(2, positions, True) (rerank_topk.cu:926-954)
__global__ __launch_bounds__(256) void dense_mask_kernel(const int64_t* __restrict__ pos,
                                                         uint8_t* __restrict__ mask, int n_dense,
                                                         int nk) {
  const int row = blockIdx.x;
  uint8_t* m = mask + static_cast<int64_t>(row) * nk;
  for (int i = threadIdx.x; i < nk; i += blockDim.x) m[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n_dense; j += blockDim.x) {
    const int64_t p = pos[static_cast<int64_t>(row) * n_dense + j];
    if (p >= 0 && p < nk) m[p] = 1;
  }
}

// raw_q = bf16(sum_i q[group*h + i] / group), sum in head order (S:1621-1626)
__global__ __launch_bounds__(128) void gqa_mean_kernel(const uint16_t* __restrict__ q, int64_t q_sb,
                                                       int64_t q_sh, int kv, int group,
                                                       uint16_t* __restrict__ out) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const int b = bh / kv, h = bh % kv;
  const uint16_t* qp = q + b * q_sb + static_cast<int64_t>(h * group) * q_sh + d;
  float acc = bf16_to_f32(qp[0]);
  for (int i = 1; i < group; ++i) acc = acc + bf16_to_f32(qp[i * q_sh]);
  out[static_cast<int64_t>(bh) * 128 + d] = f32_to_bf16_bits(acc / static_cast<float>(group));
}

// ----------------------------------------------------------------------------
// KIVI stage-2 (kivi_qk_dot.cu:108-320): per selected chunk and token,
// k = bf16(bf16(code*scale) + mn), p = bf16(k*q), acc += p (fp32, d = 0..127),
// scale = bf16(bf16(mx - mn)/15); then a G-lane descending bitonic sort and
// keep dense_topk / sparse_topk per chunk, (-1e30, 0) elsewhere.
// One lane per token; G lanes per chunk; 256 threads per block.
// ----------------------------------------------------------------------------

// Value v of lane P of this lane's row of 16, for every lane of the row (DPP
// row_newbcast; it folds into the consuming v_mul / v_add).  The caller keeps
// all 16 lanes of a row active together.
template <int P>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + P, 0xF,
                                                            0xF, true));
}

// Channels 8P..8P+7 of one token: the scale, min and query of channel 8P+j sit
// in register j of lane P of the row, and reach every lane of the row by DPP.
template <int P>
struct QkRowDot {
  static __device__ __forceinline__ float run(float acc, const uint32_t (&words)[16], const float (&sc)[8],
                                              const float (&mn)[8], const float (&qv)[8]) {
    uint32_t lo = words[P] & 0x0F0F0F0Fu, hi = (words[P] >> 4) & 0x0F0F0F0Fu;
    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float code = static_cast<float>(((j & 1 ? hi : lo) >> (8 * (j >> 1))) & 0xFFu);
      const float kd = bf16r(bf16r(code * row_bcast<P>(sc[j])) + row_bcast<P>(mn[j]));
      acc = acc + bf16r(kd * row_bcast<P>(qv[j]));
    }
    return QkRowDot<P + 1>::run(acc, words, sc, mn, qv);
  }
};
template <>
struct QkRowDot<16> {
  static __device__ __forceinline__ float run(float acc, const uint32_t (&)[16], const float (&)[8],
                                              const float (&)[8], const float (&)[8]) {
    return acc;
  }
};

// 8 consecutive bf16 values as fp32; one 16-byte load when kVec (the caller
// has checked the address is 16-byte aligned).
template <bool kVec>
__device__ __forceinline__ void load8_bf16(const uint16_t* p, float (&out)[8]) {
  if constexpr (kVec) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(u[i] << 16);
      out[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = bf16_to_f32(p[i]);
  }
}

// Chunks of 16 tokens: one row of 16 lanes per chunk, no LDS.  Lane l of a
// row scores token l of the chunk and also loads channels 8l..8l+7 of the
// chunk's min / max and of the query, which the row shares through DPP.  Same
// arithmetic, in the same order, as kivi_qk_kernel.  Both kernels write
// lanes 0 .. out_w-1 of slot i at i * out_w (out_w = G: the reference's
// layout; less: only the kept lanes, the compact output).
template <int T, bool kVec>
__global__ __launch_bounds__(T) void kivi_qk_row_kernel(
    const int64_t* __restrict__ ids, int64_t id_sb, int64_t id_sh, const uint8_t* __restrict__ dmask,
    int64_t dm_sb, int64_t dm_sh, const int32_t* __restrict__ packed, int64_t pk_sb, int64_t pk_sh,
    int n_packed, const uint16_t* __restrict__ cmin, const uint16_t* __restrict__ cmax, int64_t cm_sb,
    int64_t cm_sh, int n_max, const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh,
    float* __restrict__ out_s, int64_t* __restrict__ out_i, int64_t o_sb, int64_t o_sh, int nk,
    int dense_topk, int sparse_topk, int out_w) {
  constexpr int G = 16, kChunks = T / G;
  const int b = blockIdx.z, h = blockIdx.y;
  const int local = threadIdx.x / G, lane = threadIdx.x % G;
  const int slot = blockIdx.x * kChunks + local;
  const bool valid_slot = slot < nk;  // the same for all 16 lanes of a row
  int64_t cid = 0;
  bool dense = false;
  if (valid_slot) {
    cid = ids[b * id_sb + h * id_sh + slot];
    dense = dmask[b * dm_sb + h * dm_sh + slot] != 0;
  }
  const bool in_range = cid >= 0 && cid < n_packed;
  uint32_t words[16];
  {
    const int32_t* w = packed + b * pk_sb + h * pk_sh + (valid_slot && in_range ? cid : 0) * (16 * G) + lane;
#pragma unroll
    for (int p = 0; p < 16; ++p) words[p] = static_cast<uint32_t>(w[p * G]);
  }
  float mn[8], mx[8], qv[8];
  load8_bf16<kVec>(q + b * q_sb + h * q_sh + 8 * lane, qv);
  if (valid_slot) {
    const int64_t mrow = (b * cm_sb + h * cm_sh) + (cid >= 0 && cid < n_max ? cid : 0) * 128 + 8 * lane;
    load8_bf16<kVec>(cmin + mrow, mn);
    load8_bf16<kVec>(cmax + mrow, mx);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) mn[j] = mx[j] = 0.0f;
  }
  float sc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sc[j] = kivi_scale(mn[j], mx[j]);
  // every lane runs the dot (all 16 lanes of a row must be active for DPP);
  // rows without a valid chunk discard it
  const float acc = QkRowDot<0>::run(0.0f, words, sc, mn, qv);
  float score = (valid_slot && in_range) ? acc : -1e30f;
  int token = static_cast<int>(cid) * G + lane;
#pragma unroll
  for (int k2 = 2; k2 <= G; k2 <<= 1) {
#pragma unroll
    for (int j = k2 >> 1; j >= 1; j >>= 1) {
      const float os = __shfl_xor(score, j);
      const int ot = __shfl_xor(token, j);
      const bool desc = (lane & k2) == 0;
      const bool lower = (lane & j) == 0;
      const bool swap = (desc == lower) ? (os > score) : (os < score);
      if (swap) {
        score = os;
        token = ot;
      }
    }
  }
  if (valid_slot && lane < out_w) {
    const int64_t oi = b * o_sb + h * o_sh + static_cast<int64_t>(slot) * out_w + lane;
    const int keep = dense ? dense_topk : sparse_topk;
    out_s[oi] = lane < keep ? score : -1e30f;
    out_i[oi] = lane < keep ? static_cast<int64_t>(token) : 0;
  }
}

template <int G, int T>
__global__ __launch_bounds__(T) void kivi_qk_kernel(
    const int64_t* __restrict__ ids, int64_t id_sb, int64_t id_sh, const uint8_t* __restrict__ dmask,
    int64_t dm_sb, int64_t dm_sh, const int32_t* __restrict__ packed, int64_t pk_sb, int64_t pk_sh,
    int n_packed, const uint16_t* __restrict__ cmin, const uint16_t* __restrict__ cmax, int64_t cm_sb,
    int64_t cm_sh, int n_max, const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_sh,
    float* __restrict__ out_s, int64_t* __restrict__ out_i, int64_t o_sb, int64_t o_sh, int nk,
    int dense_topk, int sparse_topk, int out_w) {
  constexpr int kChunks = T / G;
  // q is the same for every chunk of the block; the per-chunk rows are padded
  // by 4 floats so that the chunks of one wave read different LDS banks.
  __shared__ float s_q[128];
  __shared__ float s_mn[kChunks][132];
  __shared__ float s_sc[kChunks][132];
  const int b = blockIdx.z, h = blockIdx.y;
  const int local = threadIdx.x / G, lane = threadIdx.x % G;
  const int slot = blockIdx.x * kChunks + local;
  const bool valid_slot = slot < nk;
  int64_t cid = 0;
  bool dense = false;
  if (valid_slot) {
    cid = ids[b * id_sb + h * id_sh + slot];
    dense = dmask[b * dm_sb + h * dm_sh + slot] != 0;
  }
  const bool in_range = cid >= 0 && cid < n_packed;
  // the code words are loaded before the metadata so both latencies overlap
  uint32_t words[16];
  {
    const int32_t* w = packed + b * pk_sb + h * pk_sh + (valid_slot && in_range ? cid : 0) * (16 * G) + lane;
#pragma unroll
    for (int p = 0; p < 16; ++p) words[p] = static_cast<uint32_t>(w[p * G]);
  }
  for (int d = threadIdx.x; d < 128; d += T) s_q[d] = bf16_to_f32(q[b * q_sb + h * q_sh + d]);
  if (valid_slot) {
    const int64_t mrow = (b * cm_sb + h * cm_sh) + (cid >= 0 && cid < n_max ? cid : 0) * 128;
    for (int d = lane; d < 128; d += G) {
      const float mn = bf16_to_f32(cmin[mrow + d]);
      const float mx = bf16_to_f32(cmax[mrow + d]);
      s_mn[local][d] = mn;
      s_sc[local][d] = kivi_scale(mn, mx);
    }
  }
  __syncthreads();
  float score = -1e30f;
  int token = static_cast<int>(cid) * G + lane;
  if (valid_slot && in_range) {
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const uint32_t word = words[p];
      // nibbles 0, 2, 4, 6 (channels 8p, +2, +4, +6) in the bytes of lo,
      // nibbles 1, 3, 5, 7 in the bytes of hi: one byte-to-float each
      uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
      // (kept opaque so the byte extraction below stays v_cvt_f32_ubyteN
      // instead of being folded back into a 4-bit field extract per channel)
      asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = 8 * p + j;  // the sum stays sequential in d
        const float code = static_cast<float>(((j & 1 ? hi : lo) >> (8 * (j >> 1))) & 0xFFu);
        const float kd = bf16r(bf16r(code * s_sc[local][d]) + s_mn[local][d]);
        acc = acc + bf16r(kd * s_q[d]);
      }
    }
    score = acc;
  }
  // bitonic sort (descending) within the G lanes of this chunk (kivi_qk_dot.cu:286-303)
#pragma unroll
  for (int k2 = 2; k2 <= G; k2 <<= 1) {
#pragma unroll
    for (int j = k2 >> 1; j >= 1; j >>= 1) {
      const float os = __shfl_xor(score, j);
      const int ot = __shfl_xor(token, j);
      const bool desc = (lane & k2) == 0;
      const bool lower = (lane & j) == 0;
      const bool swap = (desc == lower) ? (os > score) : (os < score);
      if (swap) {
        score = os;
        token = ot;
      }
    }
  }
  if (valid_slot && lane < out_w) {
    const int64_t oi = b * o_sb + h * o_sh + static_cast<int64_t>(slot) * out_w + lane;
    const int keep = dense ? dense_topk : sparse_topk;
    out_s[oi] = lane < keep ? score : -1e30f;
    out_i[oi] = lane < keep ? static_cast<int64_t>(token) : 0;
  }
}

// ----------------------------------------------------------------------------
// Per-page fp16 min / max of bf16 keys (the Quest metadata of a paged cache,
// the fp16 counterpart of _compute_and_store_chunk_minmax's amin / amax,
// S:2025-2157).  min is rounded toward -inf and max toward +inf, so the
// Quest score stays an upper bound (every bf16 value inside fp16's normal
// range converts exactly).  Thread per channel, block per (page, kv, b).
// ----------------------------------------------------------------------------
__device__ __forceinline__ uint16_t f16_step(uint16_t h, bool up) {
  // next fp16 toward +inf (up) or -inf, for finite non-NaN h
  const bool neg = (h & 0x8000u) != 0;
  if ((h & 0x7FFFu) == 0) return up ? 0x0001u : 0x8001u;
  return static_cast<uint16_t>((neg == up) ? h - 1 : h + 1);
}

__device__ __forceinline__ uint16_t f16_round_dir(float x, bool up) {
  const _Float16 r = static_cast<_Float16>(x);
  const float rf = static_cast<float>(r);
  uint16_t h = __builtin_bit_cast(uint16_t, r);
  if (x != x) return h;
  if (up ? (rf < x) : (rf > x)) h = f16_step(h, up);
  return h;
}

__global__ __launch_bounds__(128) void page_minmax_f16_kernel(
    const uint16_t* __restrict__ keys, int64_t k_sb, int64_t k_sh, int64_t k_st, int page,
    int n_pages_max, uint16_t* __restrict__ pmin, uint16_t* __restrict__ pmax) {
  const int pg = blockIdx.x, h = blockIdx.y, b = blockIdx.z, ch = threadIdx.x;
  const uint16_t* k = keys + b * k_sb + h * k_sh + static_cast<int64_t>(pg) * page * k_st + ch;
  float mn = bf16_to_f32(k[0]), mx = mn;
  for (int t = 1; t < page; ++t) {
    const float v = bf16_to_f32(k[t * k_st]);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const int64_t o = ((static_cast<int64_t>(b) * gridDim.y + h) * n_pages_max + pg) * 128 + ch;
  pmin[o] = f16_round_dir(mn, false);
  pmax[o] = f16_round_dir(mx, true);
}

}  // namespace
}  // namespace zkv

using namespace zkv;

namespace zkv {
namespace {
// Chunks per 32-lane half of the fused GQA-mean Quest launch (loads issued
// together); ZKV_QUEST_UNROLL=4|8|16 overrides it for tuning sweeps.
int quest_gqa_unroll() {
  static int v = [] {
    int u = 4;
    if (const char* e = getenv("ZKV_QUEST_UNROLL")) u = atoi(e);
    return (u == 8 || u == 16) ? u : 4;
  }();
  return v;
}
}  // namespace
}  // namespace zkv

extern "C" int zkv_quest_chunk_score_gqa(const uint16_t* q, int64_t q_sb, int64_t q_sh, int hq,
                                         uint16_t* raw_q, const uint16_t* chunk_min,
                                         const uint16_t* chunk_max, int meta_fp16, float* scores, int bs,
                                         int kv, int n_chunks, int n_chunks_max, const uint8_t* valid,
                                         zkv_stream_t stream) {
  ZKV_REQUIRE(q && raw_q && chunk_min && chunk_max && scores, "zkv_quest_chunk_score_gqa: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0 && n_chunks >= 1 && n_chunks <= n_chunks_max &&
                  static_cast<int64_t>(bs) * kv <= 65535,
              "zkv_quest_chunk_score_gqa: bad sizes bs=%d hq=%d kv=%d n_chunks=%d n_chunks_max=%d", bs, hq,
              kv, n_chunks, n_chunks_max);
  auto s = reinterpret_cast<hipStream_t>(stream);
  auto launch = [&](auto u_tag) {
    constexpr int U = decltype(u_tag)::value;
    const dim3 grid((n_chunks + 8 * U - 1) / (8 * U), bs * kv);
    if (meta_fp16)
      quest_gqa_kernel<true, U><<<grid, 256, 0, s>>>(q, q_sb, q_sh, hq / kv, kv, raw_q, chunk_min, chunk_max,
                                                     valid, scores, n_chunks, n_chunks_max);
    else
      quest_gqa_kernel<false, U><<<grid, 256, 0, s>>>(q, q_sb, q_sh, hq / kv, kv, raw_q, chunk_min, chunk_max,
                                                      valid, scores, n_chunks, n_chunks_max);
  };
  const int u = quest_gqa_unroll();
  if (u == 16)
    launch(std::integral_constant<int, 16>{});
  else if (u == 8)
    launch(std::integral_constant<int, 8>{});
  else
    launch(std::integral_constant<int, 4>{});
  return check_launch("quest_gqa_kernel");
}

extern "C" int zkv_quest_chunk_topk_gqa(const uint16_t* q, int64_t q_sb, int64_t q_sh, int hq, uint16_t* raw_q,
                                        const uint16_t* chunk_min, const uint16_t* chunk_max, int meta_fp16,
                                        float* scores, int bs, int kv, int n_chunks, int n_chunks_max,
                                        const uint8_t* valid, int k, int64_t* out, int64_t out_stride,
                                        void* slots, size_t slots_bytes, zkv_stream_t stream) {
  ZKV_REQUIRE(q && raw_q && chunk_min && chunk_max && scores && out && slots,
              "zkv_quest_chunk_topk_gqa: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0 && n_chunks >= 1 && n_chunks <= n_chunks_max &&
                  n_chunks <= kQuestTopkMaxL && static_cast<int64_t>(bs) * kv <= 65535,
              "zkv_quest_chunk_topk_gqa: bad sizes bs=%d hq=%d kv=%d n_chunks=%d (at most %d) n_chunks_max=%d", bs,
              hq, kv, n_chunks, kQuestTopkMaxL, n_chunks_max);
  ZKV_REQUIRE(k >= 1 && out_stride >= k, "zkv_quest_chunk_topk_gqa: k=%d out_stride=%lld", k,
              static_cast<long long>(out_stride));
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(slots) & 3) == 0 && slots_bytes >= static_cast<size_t>(bs) * kv * 4,
              "zkv_quest_chunk_topk_gqa: slots need %zu bytes, 4-byte aligned (got %zu)",
              static_cast<size_t>(bs) * kv * 4, slots_bytes);
  auto s = reinterpret_cast<hipStream_t>(stream);
  auto* sl = static_cast<unsigned int*>(slots);
  // trips per block: the fewest that keep the grid within two 1024-thread
  // blocks per CU (one wave of blocks: each pays its store acknowledgement
  // and arrival once)
  const int rows = bs * kv;
  auto blocks_per_row = [&](int tr) { return (n_chunks + tr * kQuestTopkChunks - 1) / (tr * kQuestTopkChunks); };
  int tr = 1;
  while (tr < 4 && static_cast<int64_t>(rows) * blocks_per_row(tr) > 512) tr *= 2;
  if (const char* e = getenv("ZKV_QUEST_TRIPS")) tr = atoi(e) >= 4 ? 4 : (atoi(e) >= 2 ? 2 : 1);
  const dim3 grid(blocks_per_row(tr), rows);
  auto launch = [&](auto f16_tag, auto tr_tag) {
    constexpr bool F16 = decltype(f16_tag)::value;
    constexpr int TR = decltype(tr_tag)::value;
    quest_topk_kernel<F16, TR><<<grid, kTopkThreads, 0, s>>>(q, q_sb, q_sh, hq / kv, kv, raw_q, chunk_min,
                                                             chunk_max, valid, scores, n_chunks, n_chunks_max, k,
                                                             out, out_stride, sl);
  };
  auto by_trips = [&](auto f16_tag) {
    if (tr == 4) launch(f16_tag, std::integral_constant<int, 4>{});
    else if (tr == 2) launch(f16_tag, std::integral_constant<int, 2>{});
    else launch(f16_tag, std::integral_constant<int, 1>{});
  };
  if (meta_fp16) by_trips(std::true_type{});
  else by_trips(std::false_type{});
  return check_launch("quest_topk_kernel");
}

extern "C" int zkv_quest_chunk_score(const uint16_t* q, const uint16_t* chunk_min,
                                     const uint16_t* chunk_max, int meta_fp16, float* scores,
                                     int bs, int kv, int n_chunks, int n_chunks_max,
                                     const uint8_t* valid, zkv_stream_t stream) {
  ZKV_REQUIRE(q && chunk_min && chunk_max && scores, "zkv_quest_chunk_score: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && n_chunks >= 0 && n_chunks <= n_chunks_max,
              "zkv_quest_chunk_score: bad sizes bs=%d kv=%d n_chunks=%d n_chunks_max=%d", bs, kv,
              n_chunks, n_chunks_max);
  const int64_t total = static_cast<int64_t>(bs) * kv * n_chunks;
  if (total == 0) return ZKV_OK;
  const int64_t blocks64 = std::min<int64_t>((total + 8 * kQuestUnroll - 1) / (8 * kQuestUnroll), 8192);
  const int blocks = static_cast<int>(blocks64);
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (meta_fp16)
    quest_score_kernel<true><<<blocks, 256, 0, s>>>(q, chunk_min, chunk_max, valid, scores, n_chunks,
                                                    n_chunks_max, total);
  else
    quest_score_kernel<false><<<blocks, 256, 0, s>>>(q, chunk_min, chunk_max, valid, scores, n_chunks,
                                                     n_chunks_max, total);
  return check_launch("quest_score_kernel");
}

namespace {
int launch_topk(const float* scores, int64_t in_stride, int rows, int L, int k, int64_t* out, int64_t out_stride,
                const int64_t* lut, int64_t lut_stride, const int64_t* skipped, int64_t sk_stride, int sk_count,
                int64_t sentinel, const TopkMask mk, zkv_stream_t stream) {
  ZKV_REQUIRE(scores && out, "zkv_topk: null pointer");
  ZKV_REQUIRE(rows >= 0 && L >= 0 && k > 0, "zkv_topk: bad sizes rows=%d L=%d k=%d", rows, L, k);
  ZKV_REQUIRE(out_stride >= k + sk_count, "zkv_topk: out row of %lld < k + skipped = %d",
              static_cast<long long>(out_stride), k + sk_count);
  ZKV_REQUIRE(sk_count == 0 || skipped, "zkv_topk: null skipped");
  if (rows == 0) return ZKV_OK;
  auto s = reinterpret_cast<hipStream_t>(stream);
#define ZKV_TOPK_REG(R)                                                                          \
  topk_reg_kernel<R><<<rows, kTopkThreads, 0, s>>>(scores, in_stride, L, k, out, out_stride, lut, \
                                                   lut_stride, skipped, sk_stride, sk_count, sentinel, mk)
  if (L <= 4 * kTopkThreads)
    ZKV_TOPK_REG(4);
  else if (L <= 8 * kTopkThreads)
    ZKV_TOPK_REG(8);
  else if (L <= 16 * kTopkThreads)
    ZKV_TOPK_REG(16);
  else if (L <= 32 * kTopkThreads)
    ZKV_TOPK_REG(32);
  else
    topk_kernel<<<rows, kTopkThreads, 0, s>>>(scores, in_stride, L, k, out, out_stride, lut, lut_stride,
                                              skipped, sk_stride, sk_count, sentinel, mk);
#undef ZKV_TOPK_REG
  return check_launch("topk_kernel");
}
}  // namespace

extern "C" int zkv_topk(const float* scores, int64_t in_stride, int rows, int L, int k,
                        int64_t* out, int64_t out_stride, const int64_t* lut, int64_t lut_stride,
                        const int64_t* skipped, int64_t sk_stride, int sk_count, int64_t sentinel,
                        zkv_stream_t stream) {
  return launch_topk(scores, in_stride, rows, L, k, out, out_stride, lut, lut_stride, skipped, sk_stride,
                     sk_count, sentinel, TopkMask{nullptr, 0}, stream);
}

extern "C" int zkv_topk_dense_mask(const float* scores, int64_t in_stride, int rows, int L, int k,
                                   int64_t* out, int64_t out_stride, uint8_t* mask, int64_t mask_stride,
                                   zkv_stream_t stream) {
  ZKV_REQUIRE(mask && mask_stride >= L, "zkv_topk_dense_mask: null mask or row of %lld < L = %d",
              static_cast<long long>(mask_stride), L);
  return launch_topk(scores, in_stride, rows, L, k, out, out_stride, nullptr, 0, nullptr, 0, 0, -1,
                     TopkMask{mask, mask_stride}, stream);
}

extern "C" int zkv_chunk_density_scores(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                                        const uint16_t* centroids, int64_t c_sb, int64_t c_sh,
                                        int64_t c_sc, const uint16_t* raw_q, int64_t q_sb,
                                        int64_t q_sh, float* out, int64_t o_sb, int64_t o_sh,
                                        int bs, int kv, int nk, int n_chunks, zkv_stream_t stream) {
  ZKV_REQUIRE(chunk_ids && centroids && raw_q && out, "zkv_chunk_density_scores: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && nk >= 0, "zkv_chunk_density_scores: bad sizes");
  const int64_t total = static_cast<int64_t>(bs) * kv * nk;
  ZKV_REQUIRE(total < (int64_t{1} << 30), "zkv_chunk_density_scores: %lld slots exceed 2^30",
              static_cast<long long>(total));
  if (total == 0) return ZKV_OK;
  density_kernel<<<static_cast<int>((total + 4 * kDensityItems - 1) / (4 * kDensityItems)), 256, 0,
                   reinterpret_cast<hipStream_t>(stream)>>>(
      chunk_ids, id_sb, id_sh, centroids, c_sb, c_sh, c_sc, raw_q, q_sb, q_sh, out, o_sb, o_sh, kv, nk,
      n_chunks, static_cast<int>(total));
  return check_launch("density_kernel");
}

extern "C" int zkv_dense_mask_from_topk(const int64_t* positions, uint8_t* mask, int rows,
                                        int n_dense, int nk, zkv_stream_t stream) {
  ZKV_REQUIRE(positions && mask, "zkv_dense_mask_from_topk: null pointer");
  if (rows <= 0 || nk <= 0) return ZKV_OK;
  dense_mask_kernel<<<rows, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(positions, mask, n_dense, nk);
  return check_launch("dense_mask_kernel");
}

extern "C" int zkv_gqa_mean_query(const uint16_t* q, int64_t q_sb, int64_t q_sh, int bs, int hq,
                                  int kv, uint16_t* out, zkv_stream_t stream) {
  ZKV_REQUIRE(q && out, "zkv_gqa_mean_query: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq % kv == 0, "zkv_gqa_mean_query: bad heads hq=%d kv=%d", hq, kv);
  gqa_mean_kernel<<<bs * kv, 128, 0, reinterpret_cast<hipStream_t>(stream)>>>(q, q_sb, q_sh, kv,
                                                                              hq / kv, out);
  return check_launch("gqa_mean_kernel");
}

namespace {
int kivi_qk_launch(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh, const uint8_t* dense_mask,
                   int64_t dm_sb, int64_t dm_sh, const int32_t* packed_K, int64_t pk_sb, int64_t pk_sh,
                   int n_packed, const uint16_t* chunk_min, const uint16_t* chunk_max, int64_t cm_sb,
                   int64_t cm_sh, int n_chunks_max, const uint16_t* raw_q, int64_t q_sb, int64_t q_sh,
                   int dense_topk, int sparse_topk, int group_size, int out_width, float* out_scores,
                   int64_t* out_indices, int64_t o_sb, int64_t o_sh, int bs, int kv, int nk,
                   zkv_stream_t stream) {
  ZKV_REQUIRE(chunk_ids && dense_mask && packed_K && chunk_min && chunk_max && raw_q && out_scores &&
                  out_indices,
              "zkv_kivi_qk_dense_sparse: null pointer");
  ZKV_REQUIRE(group_size == 8 || group_size == 16,
              "kivi cuda kernel: group_size must be 8 or 16; got %d", group_size);
  ZKV_REQUIRE(dense_topk >= 1 && dense_topk <= group_size && sparse_topk >= 1 &&
                  sparse_topk <= group_size,
              "zkv_kivi_qk_dense_sparse: dense_topk=%d sparse_topk=%d out of [1, %d]", dense_topk,
              sparse_topk, group_size);
  ZKV_REQUIRE(out_width >= (dense_topk > sparse_topk ? dense_topk : sparse_topk) && out_width <= group_size,
              "zkv_kivi_qk_dense_sparse: out_width=%d outside [max(dense_topk, sparse_topk), %d]", out_width,
              group_size);
  ZKV_REQUIRE(bs > 0 && kv > 0 && nk >= 0, "zkv_kivi_qk_dense_sparse: bad sizes");
  if (nk == 0) return ZKV_OK;
  auto s = reinterpret_cast<hipStream_t>(stream);
#ifndef ZKV_KIVI_QK_THREADS
#define ZKV_KIVI_QK_THREADS 256
#endif
  constexpr int kT = ZKV_KIVI_QK_THREADS;  // threads per block: kT / G chunks
  if (group_size == 16) {
    // rows of 16 lanes, metadata and query in registers; 16-byte loads when
    // every metadata / query row starts 16-byte aligned
#ifndef ZKV_KIVI_QK_ROW_THREADS
#define ZKV_KIVI_QK_ROW_THREADS 256
#endif
    constexpr int kTr = ZKV_KIVI_QK_ROW_THREADS;
    dim3 grid((nk + kTr / 16 - 1) / (kTr / 16), kv, bs);
    const bool vec = ((reinterpret_cast<uintptr_t>(chunk_min) | reinterpret_cast<uintptr_t>(chunk_max) |
                       reinterpret_cast<uintptr_t>(raw_q)) & 15) == 0 &&
                     ((cm_sb | cm_sh | q_sb | q_sh) & 7) == 0;
#define ZKV_KIVI_QK_ROW(V)                                                                              \
  kivi_qk_row_kernel<kTr, V><<<grid, kTr, 0, s>>>(chunk_ids, id_sb, id_sh, dense_mask, dm_sb, dm_sh,      \
                                                packed_K, pk_sb, pk_sh, n_packed, chunk_min, chunk_max, \
                                                cm_sb, cm_sh, n_chunks_max, raw_q, q_sb, q_sh,          \
                                                out_scores, out_indices, o_sb, o_sh, nk, dense_topk,    \
                                                sparse_topk, out_width)
    if (vec)
      ZKV_KIVI_QK_ROW(true);
    else
      ZKV_KIVI_QK_ROW(false);
#undef ZKV_KIVI_QK_ROW
  } else {
    dim3 grid((nk + kT / 8 - 1) / (kT / 8), kv, bs);
    kivi_qk_kernel<8, kT><<<grid, kT, 0, s>>>(chunk_ids, id_sb, id_sh, dense_mask, dm_sb, dm_sh,
                                              packed_K, pk_sb, pk_sh, n_packed, chunk_min, chunk_max,
                                              cm_sb, cm_sh, n_chunks_max, raw_q, q_sb, q_sh, out_scores,
                                              out_indices, o_sb, o_sh, nk, dense_topk, sparse_topk,
                                              out_width);
  }
  return check_launch("kivi_qk_kernel");
}
}  // namespace

extern "C" int zkv_kivi_qk_dense_sparse(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                                        const uint8_t* dense_mask, int64_t dm_sb, int64_t dm_sh,
                                        const int32_t* packed_K, int64_t pk_sb, int64_t pk_sh,
                                        int n_packed, const uint16_t* chunk_min,
                                        const uint16_t* chunk_max, int64_t cm_sb, int64_t cm_sh,
                                        int n_chunks_max, const uint16_t* raw_q, int64_t q_sb,
                                        int64_t q_sh, int dense_topk, int sparse_topk,
                                        int group_size, float* out_scores, int64_t* out_indices,
                                        int64_t o_sb, int64_t o_sh, int bs, int kv, int nk,
                                        zkv_stream_t stream) {
  return kivi_qk_launch(chunk_ids, id_sb, id_sh, dense_mask, dm_sb, dm_sh, packed_K, pk_sb, pk_sh, n_packed,
                        chunk_min, chunk_max, cm_sb, cm_sh, n_chunks_max, raw_q, q_sb, q_sh, dense_topk,
                        sparse_topk, group_size, group_size, out_scores, out_indices, o_sb, o_sh, bs, kv, nk,
                        stream);
}

extern "C" int zkv_kivi_qk_dense_sparse_compact(const int64_t* chunk_ids, int64_t id_sb, int64_t id_sh,
                                                const uint8_t* dense_mask, int64_t dm_sb, int64_t dm_sh,
                                                const int32_t* packed_K, int64_t pk_sb, int64_t pk_sh,
                                                int n_packed, const uint16_t* chunk_min,
                                                const uint16_t* chunk_max, int64_t cm_sb, int64_t cm_sh,
                                                int n_chunks_max, const uint16_t* raw_q, int64_t q_sb,
                                                int64_t q_sh, int dense_topk, int sparse_topk,
                                                int group_size, int out_width, float* out_scores,
                                                int64_t* out_indices, int64_t o_sb, int64_t o_sh, int bs,
                                                int kv, int nk, zkv_stream_t stream) {
  return kivi_qk_launch(chunk_ids, id_sb, id_sh, dense_mask, dm_sb, dm_sh, packed_K, pk_sb, pk_sh, n_packed,
                        chunk_min, chunk_max, cm_sb, cm_sh, n_chunks_max, raw_q, q_sb, q_sh, dense_topk,
                        sparse_topk, group_size, out_width, out_scores, out_indices, o_sb, o_sh, bs, kv, nk,
                        stream);
}

namespace {
// the arrival counters lead the workspace: their place depends on bs only
size_t sample_slot_bytes(int bs) { return (static_cast<size_t>(bs) * 4 + 255) / 256 * 256; }
}  // namespace

extern "C" size_t zkv_sample_window_workspace_size(int bs, int vocab, int window) {
  if (bs <= 0 || vocab <= 0 || window <= 0) return 0;
  const size_t nb = (static_cast<size_t>(vocab) + kSampleSlice - 1) / kSampleSlice;
  return sample_slot_bytes(bs) + static_cast<size_t>(bs) * nb * window * 8;
}

extern "C" int zkv_sample_window(const float* logits, int64_t ld, int bs, int vocab, float inv_temperature,
                                 int top_k, int window, float top_p, const float* expo, int64_t expo_ld,
                                 int64_t* tokens, int32_t* overflow, void* workspace, size_t workspace_bytes,
                                 zkv_stream_t stream) {
  ZKV_REQUIRE(logits && expo && tokens && overflow && workspace, "zkv_sample_window: null pointer");
  ZKV_REQUIRE(bs > 0 && bs <= 65535 && vocab > 0 && ld >= vocab && expo_ld >= vocab,
              "zkv_sample_window: bad sizes bs=%d vocab=%d ld=%lld expo_ld=%lld", bs, vocab,
              static_cast<long long>(ld), static_cast<long long>(expo_ld));
  ZKV_REQUIRE(top_k >= 1 && window > top_k && window <= kSampleMaxWindow && window < vocab,
              "zkv_sample_window: need 1 <= top_k < window <= %d and window < vocab (top_k=%d window=%d vocab=%d)",
              kSampleMaxWindow, top_k, window, vocab);
  const int nb = (vocab + kSampleSlice - 1) / kSampleSlice;
  ZKV_REQUIRE(static_cast<int64_t>(nb) * window <= kSampleMaxCand,
              "zkv_sample_window: %d slices of %d logits x window %d exceed %d candidates per row", nb,
              kSampleSlice, window, kSampleMaxCand);
  const size_t need = zkv_sample_window_workspace_size(bs, vocab, window);
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0 && workspace_bytes >= need,
              "zkv_sample_window: workspace needs %zu bytes, 256-byte aligned (got %zu)", need, workspace_bytes);
  auto* slots = static_cast<unsigned int*>(workspace);
  auto* cand = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(workspace) + sample_slot_bytes(bs));
  sample_window_kernel<<<dim3(nb, bs), kTopkThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      logits, ld, vocab, inv_temperature, top_k, window, top_p, expo, expo_ld, cand, slots, tokens, overflow);
  return check_launch("sample_window_kernel");
}

extern "C" int zkv_page_minmax_f16(const uint16_t* keys, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                   int bs, int kv, int page_size, int n_pages, int n_pages_max,
                                   uint16_t* page_min, uint16_t* page_max, zkv_stream_t stream) {
  ZKV_REQUIRE(keys && page_min && page_max, "zkv_page_minmax_f16: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && kv <= 65535 && bs <= 65535 && page_size > 0 && n_pages >= 0 &&
                  n_pages <= n_pages_max,
              "zkv_page_minmax_f16: bad sizes bs=%d kv=%d page=%d n_pages=%d n_pages_max=%d", bs, kv,
              page_size, n_pages, n_pages_max);
  if (n_pages == 0) return ZKV_OK;
  page_minmax_f16_kernel<<<dim3(n_pages, kv, bs), 128, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      keys, k_sb, k_sh, k_st, page_size, n_pages_max, page_min, page_max);
  return check_launch("page_minmax_f16_kernel");
}
