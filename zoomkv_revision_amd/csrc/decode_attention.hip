// Fused 4-bit KV decode attention for gfx950 (MI355X).
//
// out[b, hq] = softmax(q[b, hq] . K[b, kv]^T * sm_scale) . V[b, kv], causal off,
// GQA: query heads hq = kv*gqa + c share KV head kv (the convention of
// flash_attn_with_kvcache at S:1742-1747 and of the GQA mean at S:1621-1626).
//
// K / V come from a Format Q cache (4-bit codes, fp16 scale / zero) plus a bf16
// residual window.  The work is HBM-bound (160 B per cached token per KV head
// against ~2 KFLOP), so the kernel is built to stream each 32-token tile from
// HBM exactly once for all `gqa` query heads:
//
//  * one wave64 per (context split, kv head, batch); each wave walks its
//    tiles with the next tile's 5 KiB already in flight (register double
//    buffer), and the launch has enough splits to give every CU several waves;
//  * nibbles become exact fp16 codes with two bit ops (0x6400|n = 1024+n,
//    0x4C00|n<<4 = 16+n/4) and one packed op, and are dequantized with one
//    v_pk_fma_f16 per pair: code*scale + zero;
//  * S^T[t, c] = sum_d Khat[t, d] q[c, d] and O^T[d, c] += sum_t Vhat[d, t] P[t, c]
//    run on the matrix cores as v_mfma_f32_16x16x32_f16 (query heads on the N
//    axis).  The Format Q word / metadata order is the MFMA operand order, so
//    the K-MFMA result lands in exactly the lanes the V-MFMA B operand needs:
//    no LDS round trip and no cross-lane shuffles except the softmax max/sum;
//  * online softmax in fp32 (base 2, log2(e)*sm_scale folded into q), with the
//    O rescale skipped when no running max moved;
//  * splits are merged by a second small kernel with the LSE rule of
//    lse_merge_torch (Z/cache_hub/lse_merge/lse_merge.py:79-119).
//
// MFMA 16x16x32 operand layout (lane l, c = l % 16, g = l / 16):
//   A: row c, k-slice g (8 halves);  B: k-slice g, column c;
//   D: rows 4g..4g+3, column c.
// K-MFMA: A = Khat (row = token c + 16m), B = q (column = query head c),
//   k-slice element e of dim block p = 4s + g is channel 8p + KSLOT[e],
//   KSLOT = (0,4,1,5,2,6,3,7).
// V-MFMA (one per j = 0..7): A = Vhat^T (row c = channel 8c + j), B = P,
//   k-slice element e of lane group g is token TAU[g][e] = 4g+e | 16+4g+e-4,
//   which is exactly where the K-MFMA left that token's score.
#include "zkv_common.hpp"

namespace zkv {
namespace {

constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;

struct AttnParams {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const int32_t* k_codes;
  const uint16_t* k_meta;
  const int32_t* v_codes;
  const uint16_t* v_meta;
  const uint16_t* k_res;
  const uint16_t* v_res;
  int g_cap, r_cap;
  int kv, gqa, n_groups, res_len, n_splits, tiles_per_split;
  float qscale;
  float* ws_o;   // [bs, kv, n_splits, gqa, 128]
  float* ws_ml;  // [bs, kv, n_splits, gqa, 2]
};

struct TileRaw {
  uint32_t kw[4][2];  // K words (dim block 4s+g, token c+16m)
  u32x4_t ks[4];      // K scale slots of dim block 4s+g
  u32x4_t kz[4];      // K zero slots
  u32x4_t vw[2];      // V words (octet g, channels 8c..8c+7)
  u32x4_t vs, vz;     // V scale / zero of octet g, channel group c/4
};

__device__ __forceinline__ u32x4_t ld16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

__device__ __forceinline__ void load_tile(const AttnParams& p, int64_t bh, int gi, int c, int g,
                                          TileRaw& r) {
  const int64_t tile = bh * p.g_cap + gi;
  const int32_t* kc = p.k_codes + tile * 512;
  const uint16_t* km = p.k_meta + tile * 256;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int blk = 4 * s + g;
#pragma unroll
    for (int m = 0; m < 2; ++m) r.kw[s][m] = static_cast<uint32_t>(kc[blk * 32 + c + 16 * m]);
    r.ks[s] = ld16(km + blk * 16);
    r.kz[s] = ld16(km + blk * 16 + 8);
  }
  const int32_t* vc = p.v_codes + tile * 512 + g * 128 + 8 * c;
  r.vw[0] = ld16(vc);
  r.vw[1] = ld16(vc + 4);
  const uint16_t* vm = p.v_meta + tile * 256 + ((c >> 2) * 4 + g) * 16;
  r.vs = ld16(vm);
  r.vz = ld16(vm + 8);
}

__device__ __forceinline__ half8_t dequant8(uint32_t w, const u32x4_t& sc, const u32x4_t& zr) {
  half2_t code[4];
  nibbles_to_half_pairs(w, code);
  half8_t a;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const half2_t x = __builtin_elementwise_fma(code[v], u32_as_half2(sc[v]), u32_as_half2(zr[v]));
    a[2 * v] = x[0];
    a[2 * v + 1] = x[1];
  }
  return a;
}

__device__ __forceinline__ float wave_max16(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_sum16(float x) {
  x = x + __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Online-softmax update for one tile: S holds the base-2 scores of tokens
// TAU[g][0..7] for query head c (masked tokens are -inf).  Returns P as the
// fp16 B operand of the V-MFMA and rescales O when a running max moved.
__device__ __forceinline__ half8_t softmax_step(const float4_t S[2], float& m_run, float& l_run,
                                                float4_t O[8]) {
  float sv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sv[i] = S[0][i];
    sv[4 + i] = S[1][i];
  }
  float mx = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
  mx = wave_max16(mx);
  const float m_new = fmaxf(m_run, mx);
  const float alpha = exp2f(m_run - m_new);
  m_run = m_new;
  half8_t pb;
  float ps = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pe = exp2f(sv[e] - m_new);
    ps += pe;
    pb[e] = static_cast<_Float16>(pe);
  }
  l_run = l_run * alpha + ps;
  if (__any(alpha != 1.0f)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) O[j] *= alpha;
  }
  return pb;
}

__global__ __launch_bounds__(64) void kivi4_attn_kernel(const AttnParams p) {
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int c = lane & 15, g = lane >> 4;
  const bool col_ok = c < p.gqa;
  const int64_t bh = static_cast<int64_t>(b) * p.kv + h;

  // ---- q as the K-MFMA B operand (element e of block 4s+g = channel 8(4s+g)+KSLOT[e]) ----
  half8_t qB[4];
  {
    const uint16_t* qp = p.q + b * p.q_sb + static_cast<int64_t>(h * p.gqa + (col_ok ? c : 0)) * p.q_sh;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t raw = ld16(qp + 8 * (4 * s + g));
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(raw[i] << 16);
        x[2 * i + 1] = __uint_as_float(raw[i] & 0xFFFF0000u);
      }
      constexpr int kslot[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
      for (int e = 0; e < 8; ++e) qB[s][e] = static_cast<_Float16>(col_ok ? x[kslot[e]] * p.qscale : 0.0f);
    }
  }

  float4_t O[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) O[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegBig, l_run = 0.0f;

  const int n_tiles = p.n_groups + (p.res_len + kTile - 1) / kTile;
  const int t0 = split * p.tiles_per_split;
  const int t1 = min(t0 + p.tiles_per_split, n_tiles);
  const int tq1 = min(t1, p.n_groups);  // quantized tiles are [t0, tq1)

  // ---- quantized tiles, next tile's raw data in flight ----
  if (t0 < tq1) {
    TileRaw cur;
    load_tile(p, bh, t0, c, g, cur);
    for (int t = t0; t < tq1; ++t) {
      TileRaw nxt;
      if (t + 1 < tq1) load_tile(p, bh, t + 1, c, g, nxt);
      float4_t S[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const half8_t a = dequant8(cur.kw[s][m], cur.ks[s], cur.kz[s]);
          S[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qB[s], S[m], 0, 0, 0);
        }
      }
      const half8_t pb = softmax_step(S, m_run, l_run, O);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const half8_t a = dequant8(cur.vw[j >> 2][j & 3], cur.vs, cur.vz);
        O[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, O[j], 0, 0, 0);
      }
      if (t + 1 < tq1) cur = nxt;
    }
  }

  // ---- bf16 residual tiles (at most r_cap / 32 of them, all in the last split) ----
  for (int t = max(t0, p.n_groups); t < t1; ++t) {
    const int base = (t - p.n_groups) * kTile;
    const int valid = min(kTile, p.res_len - base);
    const uint16_t* kr = p.k_res + (bh * p.r_cap + base) * 128;
    const uint16_t* vr = p.v_res + (bh * p.r_cap + base) * 128;
    float4_t S[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int tok = c + 16 * m;
        u32x4_t raw = {0u, 0u, 0u, 0u};
        if (tok < valid) raw = ld16(kr + tok * 128 + 8 * (4 * s + g));
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = __uint_as_float(raw[i] << 16);
          x[2 * i + 1] = __uint_as_float(raw[i] & 0xFFFF0000u);
        }
        constexpr int kslot[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        half8_t a;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = static_cast<_Float16>(x[kslot[e]]);
        S[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qB[s], S[m], 0, 0, 0);
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * g + i + 16 * m >= valid) S[m][i] = -INFINITY;
    const half8_t pb = softmax_step(S, m_run, l_run, O);
    // V^T operand: element e = token TAU[g][e], row c of M-tile j = channel 8c + j
    float vx[8][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = (e < 4) ? (4 * g + e) : (16 + 4 * g + e - 4);
      u32x4_t raw = {0u, 0u, 0u, 0u};
      if (tok < valid) raw = ld16(vr + tok * 128 + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vx[e][2 * i] = __uint_as_float(raw[i] << 16);
        vx[e][2 * i + 1] = __uint_as_float(raw[i] & 0xFFFF0000u);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half8_t a;
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = static_cast<_Float16>(vx[e][j]);
      O[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, O[j], 0, 0, 0);
    }
  }

  // ---- partial result of this split ----
  const float l_tot = wave_sum16(l_run);
  if (col_ok) {
    const int64_t row = (bh * p.n_splits + split) * p.gqa + c;
    float* o = p.ws_o + row * 128 + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // lane holds channels 8(4g+i)+j = 32g + 8i + j for j = 0..7
      *reinterpret_cast<float4_t*>(o + 8 * i) = float4_t{O[0][i], O[1][i], O[2][i], O[3][i]};
      *reinterpret_cast<float4_t*>(o + 8 * i + 4) = float4_t{O[4][i], O[5][i], O[6][i], O[7][i]};
    }
    if (g == 0) {
      p.ws_ml[row * 2] = m_run;
      p.ws_ml[row * 2 + 1] = l_tot;
    }
  }
}

// Merge the n_splits partials of every (b, query head) with the LSE rule.
__global__ __launch_bounds__(128) void kivi4_combine_kernel(const float* __restrict__ ws_o,
                                                            const float* __restrict__ ws_ml,
                                                            int kv, int gqa, int n_splits,
                                                            void* __restrict__ out, int out_f32) {
  const int bq = blockIdx.x;  // b * hq + hq_idx
  const int hq = kv * gqa;
  const int b = bq / hq, qh = bq % hq;
  const int h = qh / gqa, c = qh % gqa;
  const int d = threadIdx.x;
  const int64_t row0 = ((static_cast<int64_t>(b) * kv + h) * n_splits) * gqa + c;
  float mmax = kNegBig;
  for (int s = 0; s < n_splits; ++s) mmax = fmaxf(mmax, ws_ml[(row0 + s * gqa) * 2]);
  float num = 0.0f, den = 0.0f;
  for (int s = 0; s < n_splits; ++s) {
    const int64_t row = row0 + static_cast<int64_t>(s) * gqa;
    const float w = exp2f(ws_ml[row * 2] - mmax);
    den += w * ws_ml[row * 2 + 1];
    num += w * ws_o[row * 128 + d];
  }
  const float r = den > 0.0f ? num / den : 0.0f;
  const int64_t oi = static_cast<int64_t>(bq) * 128 + d;
  if (out_f32)
    reinterpret_cast<float*>(out)[oi] = r;
  else
    reinterpret_cast<uint16_t*>(out)[oi] = f32_to_bf16_bits(r);
}

struct SplitPlan {
  int n_splits, tiles_per_split;
};

SplitPlan plan_splits(int bs, int kv, int n_groups, int res_len, int n_splits) {
  const int n_tiles = n_groups + (res_len + kTile - 1) / kTile;
  int ns = n_splits;
  if (ns <= 0) {
    const int target = 2048;  // ~8 single-wave workgroups per CU on 256 CUs
    const int units = bs * kv;
    ns = (target + units - 1) / units;
  }
  ns = max(1, min(ns, max(n_tiles, 1)));
  const int per = (max(n_tiles, 1) + ns - 1) / ns;
  ns = (max(n_tiles, 1) + per - 1) / per;
  return {ns, per};
}

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" size_t zkv_kivi4_attention_workspace_size(int bs, int hq, int kv, int n_groups,
                                                     int res_len, int n_splits) {
  if (bs <= 0 || kv <= 0 || hq <= 0) return 0;
  const SplitPlan sp = plan_splits(bs, kv, n_groups, res_len, n_splits);
  return static_cast<size_t>(bs) * hq * sp.n_splits * (128 + 2) * sizeof(float);
}

extern "C" int zkv_kivi4_decode_attention(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                                          const int32_t* k_codes, const uint16_t* k_meta,
                                          const int32_t* v_codes, const uint16_t* v_meta, int g_cap,
                                          const uint16_t* k_res, const uint16_t* v_res, int r_cap,
                                          int bs, int hq, int kv, int n_groups, int res_len,
                                          float sm_scale, void* out, int out_f32, int n_splits,
                                          void* workspace, size_t workspace_bytes,
                                          zkv_stream_t stream) {
  ZKV_REQUIRE(q && out && workspace, "zkv_kivi4_decode_attention: null pointer");
  ZKV_REQUIRE(bs > 0 && kv > 0 && hq > 0 && hq % kv == 0,
              "zkv_kivi4_decode_attention: bad heads bs=%d hq=%d kv=%d", bs, hq, kv);
  const int gqa = hq / kv;
  ZKV_REQUIRE(gqa <= 16, "zkv_kivi4_decode_attention: at most 16 query heads per KV head; got %d", gqa);
  ZKV_REQUIRE(n_groups >= 0 && n_groups <= g_cap, "zkv_kivi4_decode_attention: n_groups=%d g_cap=%d",
              n_groups, g_cap);
  ZKV_REQUIRE(res_len >= 0 && res_len <= r_cap, "zkv_kivi4_decode_attention: res_len=%d r_cap=%d",
              res_len, r_cap);
  ZKV_REQUIRE(n_groups + res_len > 0, "zkv_kivi4_decode_attention: empty context");
  ZKV_REQUIRE(n_groups == 0 || (k_codes && k_meta && v_codes && v_meta),
              "zkv_kivi4_decode_attention: null cache pointer");
  ZKV_REQUIRE(res_len == 0 || (k_res && v_res), "zkv_kivi4_decode_attention: null residual pointer");
  ZKV_REQUIRE((q_sh % 8) == 0 && (q_sb % 8) == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0,
              "zkv_kivi4_decode_attention: q rows must be 16-byte aligned");
  const SplitPlan sp = plan_splits(bs, kv, n_groups, res_len, n_splits);
  const size_t need = static_cast<size_t>(bs) * hq * sp.n_splits * (128 + 2) * sizeof(float);
  if (workspace_bytes < need)
    return fail(ZKV_ESPACE, "zkv_kivi4_decode_attention: workspace %zu < %zu bytes", workspace_bytes, need);
  AttnParams p;
  p.q = q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.k_codes = k_codes;
  p.k_meta = k_meta;
  p.v_codes = v_codes;
  p.v_meta = v_meta;
  p.k_res = k_res;
  p.v_res = v_res;
  p.g_cap = g_cap;
  p.r_cap = r_cap;
  p.kv = kv;
  p.gqa = gqa;
  p.n_groups = n_groups;
  p.res_len = res_len;
  p.n_splits = sp.n_splits;
  p.tiles_per_split = sp.tiles_per_split;
  p.qscale = sm_scale * kLog2e;
  p.ws_o = reinterpret_cast<float*>(workspace);
  p.ws_ml = p.ws_o + static_cast<size_t>(bs) * hq * sp.n_splits * 128;
  auto s = reinterpret_cast<hipStream_t>(stream);
  kivi4_attn_kernel<<<dim3(sp.n_splits, kv, bs), 64, 0, s>>>(p);
  int rc = check_launch("kivi4_attn_kernel");
  if (rc) return rc;
  kivi4_combine_kernel<<<bs * hq, 128, 0, s>>>(p.ws_o, p.ws_ml, kv, gqa, sp.n_splits, out, out_f32);
  return check_launch("kivi4_combine_kernel");
}
