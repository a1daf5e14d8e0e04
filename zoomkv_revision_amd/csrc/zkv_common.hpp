// Shared helpers for the gfx950 ZoomKV decode-path kernels.
//
// Error convention of the C ABI: every entry point returns 0 on success and a
// nonzero ZKV_E* code on failure; the message of the last failure on the
// calling thread is available from zkv_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/zoomkv_gfx950.h"

namespace zkv {

// ---------------------------------------------------------------------------
// Host-side error reporting
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

#define ZKV_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::zkv::fail(ZKV_EINVAL, __VA_ARGS__);    \
  } while (0)

// ---------------------------------------------------------------------------
// Vector types
// ---------------------------------------------------------------------------
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Exact bf16 / fp16 arithmetic helpers (IEEE fp32 op, then RNE)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round an fp32 value to the nearest bfloat16, ties to even (NaN stays NaN).
// gfx950 does this in hardware (v_cvt_pk_bf16_f32); it agrees bit for bit
// with the integer form  u += 0x7fff + ((u >> 16) & 1), u >>= 16  on every
// finite input, fp32 subnormals included (built without denormal flushing).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

typedef float float2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// x rounded to bf16, as an fp32 value: one v_cvt_pk_bf16_f32 with x in the
// high half and +0 in the low half, whose 32-bit result is exactly the fp32
// encoding of bf16(x) (no shift or mask to unpack).
__device__ __forceinline__ float bf16r(float x) {
  const float2_t v = {0.0f, x};
  return __builtin_bit_cast(float, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float2_t bf16r2(float2_t x) { return float2_t{bf16r(x[0]), bf16r(x[1])}; }

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  _Float16 h = static_cast<_Float16>(x);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ half2_t u32_as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t half2_as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// bf16(1e-8): torch's clamp(min=1e-8) on a bf16 tensor compares against the
// scalar converted to bf16.
constexpr float kBf16OneEm8 = __builtin_bit_cast(float, 0x322C0000u);  // bf16(1e-8)

// Correctly rounded fp32 quotient x / b from r = 1 / b (itself correctly
// rounded): q = x r, then one fused multiply-add step with the exact
// remainder x - q b (Markstein's correction).  For bf16 values x and b with b,
// r and the quotient normal, the result is x / b bit for bit: the rounding
// depends only on the significands there, and every pair of bf16
// significands, and every bf16 x over b = 15, was checked against the IEEE
// division (tests/test_division_step.py).  Three VALU instructions against
// the ten of an IEEE division.
__device__ __forceinline__ float div_recip(float x, float b, float r) {
  const float q = x * r;
  return __builtin_fmaf(__builtin_fmaf(-q, b, x), r, q);
}

// x / 15 for a bf16 x: the multiply-add step where the quotient is normal
// and finite or x is a zero (kept with its sign: the step turns -0 into +0),
// the IEEE division otherwise (subnormal results, inf, NaN: a per-lane branch
// that ordinary inputs never take).
__device__ __forceinline__ float div15_bf16(float x) {
  constexpr float kRecip15 = 1.0f / 15.0f;  // correctly rounded by the compiler
  const float ax = fabsf(x);
  if ((ax >= 0x1p-120f && ax <= 0x1p127f) || ax == 0.0f) {
    const float q = div_recip(x, 15.0f, kRecip15);
    return ax == 0.0f ? x : q;
  }
  return x / 15.0f;
}

// One step of the KIVI bf16 ladder: integer code of x in [mn, mn + 15*scale].
//   scale = bf16(bf16(mx - mn) / 15); safe = max(scale, bf16(1e-8))
//   code  = rne(clamp(bf16(bf16(x - mn) / safe), 0, 15))
__device__ __forceinline__ float kivi_safe(float scale) { return fmaxf(scale, kBf16OneEm8); }

__device__ __forceinline__ uint32_t kivi_code(float x, float mn, float safe) {
  float d = bf16r(x - mn);
  float qv = bf16r(d / safe);
  qv = fminf(fmaxf(qv, 0.0f), 15.0f);
  return static_cast<uint32_t>(__builtin_rintf(qv));
}

// kivi_code with the division as div_recip(d, safe, r), r = 1 / safe, for a
// finite safe (the caller branches to kivi_code otherwise).  safe >= bf16(1e-8)
// and safe <= bf16max / 15 keep safe and r normal, and d = bf16(x - mn) <=
// bf16(mx - mn) is finite; where the quotient or the remainder leaves the
// normal range (d below ~2^-118) the quotient is below 2^-90 and both forms
// give code 0.
__device__ __forceinline__ uint32_t kivi_code_r(float x, float mn, float safe, float r) {
  float d = bf16r(x - mn);
  float qv = bf16r(div_recip(d, safe, r));
  qv = fminf(fmaxf(qv, 0.0f), 15.0f);
  return static_cast<uint32_t>(__builtin_rintf(qv));
}

__device__ __forceinline__ float kivi_scale(float mn, float mx) {
  return bf16r(div15_bf16(bf16r(mx - mn)));
}

// ---------------------------------------------------------------------------
// Nibble word -> four fp16 pairs holding the exact codes.
// Pair v (v = 0..3) holds (nibble v, nibble v + 4) as (lo, hi).
// 0x6400 | n is 1024 + n in fp16; 0x4C00 | (n << 4) is 16 + n / 4.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void nibbles_to_half_pairs(uint32_t w, half2_t out[4]) {
  const half2_t m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  const half2_t four = {(_Float16)4.0f, (_Float16)4.0f};
  const half2_t m64 = {(_Float16)-64.0f, (_Float16)-64.0f};
  const uint32_t w8 = w >> 8;
  half2_t a = u32_as_half2((w & 0x000F000Fu) | 0x64006400u);
  half2_t b = u32_as_half2((w & 0x00F000F0u) | 0x4C004C00u);
  half2_t c = u32_as_half2((w8 & 0x000F000Fu) | 0x64006400u);
  half2_t d = u32_as_half2((w8 & 0x00F000F0u) | 0x4C004C00u);
  out[0] = a + m1024;
  out[1] = __builtin_elementwise_fma(b, four, m64);
  out[2] = c + m1024;
  out[3] = __builtin_elementwise_fma(d, four, m64);
}

// ---------------------------------------------------------------------------
// In-launch arrival counts: the workgroups of one unit of work (the context
// splits of one (b, kv) attention) count themselves in on an 8-byte slot
// (epoch << 8) | count; the one that completes the count does the unit's
// final step.  A slot holding another epoch (an earlier launch, stale bytes)
// counts as empty, so slots need no zeroing; the last arrival leaves the
// count at 0 under its epoch, so a captured graph (which keeps its epoch)
// counts from 0 again on replay.  Epochs (next_epoch, host side, defined in
// decode_attention.hip) have bit 55 set and a random per-process base.
// ---------------------------------------------------------------------------
unsigned long long next_epoch();

// Called by one thread per arriving workgroup, after the workgroup's results
// are device-visible; true for the n-th arrival.  A slot still under another
// epoch is first claimed for this one (reset to count 0 by a compare-and-swap
// that only succeeds while the stale value is there: once any arrival has
// claimed it, the others see the epoch and stop); then every arrival counts
// itself in with one fetch-and-add.  At most three round trips per arrival
// however many arrive together (compare-and-swap counting retried once per
// competitor: 16 splits of one (b, kv) took up to 17 us to count in).
__device__ __forceinline__ bool arrive_last(unsigned long long* slot, unsigned long long epoch, int n) {
  const unsigned long long base = epoch << 8;
  unsigned long long cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while ((cur >> 8) != epoch &&
         !__hip_atomic_compare_exchange_strong(slot, &cur, base, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)) {
  }
  const unsigned long long old = __hip_atomic_fetch_add(slot, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = (old & 0xffull) == static_cast<unsigned long long>(n - 1);
  if (last) __hip_atomic_store(slot, base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// A plain arrival count for units with many workgroups (no compare-and-swap
// retries under contention): one fetch-and-add per workgroup on a slot that
// is 0 between launches; the n-th arrival finds n - 1, does the unit's final
// step and puts the slot back to 0.  Slots must be zeroed once before first
// use (a captured graph's replays leave them at 0 as well); launches that
// overlap on one slot race.
__device__ __forceinline__ bool arrive_last_count(unsigned int* slot, int n) {
  const unsigned int old = __hip_atomic_fetch_add(slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = old == static_cast<unsigned int>(n - 1);
  if (last) __hip_atomic_store(slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

}  // namespace zkv
