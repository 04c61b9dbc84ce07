// Shared helpers for the gfx950 kernels: element types, 16-byte vector
// loads/stores, conversions and the thread-local status message behind
// sah_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/shape_aware_hip.h"

namespace sah {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Host-side status reporting.
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_hip(hipError_t err, const char* what);

// ---------------------------------------------------------------------------
// Per-element-type traits: 8-wide vector type and fp32 conversions.
template <typename T>
struct Vec8;
template <>
struct Vec8<bf16> {
  typedef bf16x8 type;
  typedef bf16x4 half_type;
  typedef bf16x2 pair_type;
};
template <>
struct Vec8<f16> {
  typedef f16x8 type;
  typedef f16x4 half_type;
  typedef f16x2 pair_type;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }

// An fp32 result that a later narrowing to T must round as it stands.  For
// T = f16 the compiler would otherwise fold "fma in fp32, then round to f16"
// into v_fma_mix{lo,hi}_f16, which rounds the exact FMA result once and
// differs from rounding the fp32 result in rare cases; the empty register
// constraint keeps the two steps apart (no instruction is emitted), so every
// kernel that rounds a normalized row to f16 rounds it the same way.
template <typename T>
__device__ __forceinline__ float fp32_result(float v) {
  if constexpr (__is_same(T, f16)) asm volatile("" : "+v"(v));
  return v;
}

// Round-trip through the storage type (used where the reference rounds an
// intermediate to the model dtype, e.g. the residual stream).
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return to_f32(from_f32<T>(x));
}

// GELU(v) = v * Phi(v) with Phi(v) = erfc(-v / sqrt(2)) / 2.  erfc(z) for
// z >= 0 is the Chebyshev-fitted form of Numerical Recipes (Press et al.,
// 2nd ed., section 6.2, erfcc), fractional error below 1.2e-7 everywhere:
//   erfc(z) = t exp(-z^2 + P(t)),  t = 1 / (1 + z / 2),
//   P(t) = -1.26551223 + t (1.00002368 + t (0.37409196 + ... + t 0.17087277)).
// So Phi(v) = 1 - erfc(|v|/sqrt 2) / 2 for v >= 0 and erfc(|v|/sqrt 2) / 2 for
// v < 0; the negative side uses erfc directly (no cancellation in
// 1 + erf(v / sqrt 2)), and a bound on the RELATIVE error keeps the far
// negative tail accurate: in float32 (approximate reciprocal and exp2) the
// result is within 1.7e-5 relative of float64 exact GELU for v in [-10, 8]
// (measured on the CPU), far below half a bf16 ulp.  An absolute-error form
// (Abramowitz & Stegun 7.1.26, |erf error| <= 1.5e-7) was 1-2% off in
// relative terms below v = -5.
// Evaluated in log2 units with the constants folded: u = z sqrt(log2 e), so
// t = 1 / (1 + k_t u) and erfc(z) / 2 = t exp2(P'(t) - u^2), where P' is P
// times log2(e) with log2(1/2) added to its constant term.
__device__ __forceinline__ float gelu_exact(float v) {
  const float u = fabsf(v) * 8.493218003e-01f;  // |v| sqrt(log2(e) / 2)
  const float t = __builtin_amdgcn_rcpf(fmaf(4.162773056e-01f, u, 1.0f));
  float poly = fmaf(2.465172979e-01f, t, -1.186114945e+00f);
  poly = fmaf(poly, t, 2.147474464e+00f);
  poly = fmaf(poly, t, -1.637753152e+00f);
  poly = fmaf(poly, t, 4.023215817e-01f);
  poly = fmaf(poly, t, -2.687568603e-01f);
  poly = fmaf(poly, t, 1.396300565e-01f);
  poly = fmaf(poly, t, 5.397006155e-01f);
  poly = fmaf(poly, t, 1.442729204e+00f);
  poly = fmaf(poly, t, -2.825748218e+00f);
  const float half_erfc = t * __builtin_amdgcn_exp2f(fmaf(-u, u, poly));
  // v * Phi(v): v - v * erfc/2 for v >= 0, v * erfc/2 otherwise
  return v >= 0.0f ? fmaf(-v, half_erfc, v) : v * half_erfc;
}

// 16-byte global load/store of raw bits.
__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// Elementwise 8-wide conversion of 16 raw bytes holding eight 16-bit values.
template <typename T>
__device__ __forceinline__ void unpack8(u32x4 raw, float* out) {
  typedef typename Vec8<T>::type V;
  V v = __builtin_bit_cast(V, raw);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)v[i];
}
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* in) {
  typedef typename Vec8<T>::type V;
  V v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (T)in[i];
  return __builtin_bit_cast(u32x4, v);
}

// Row statistics across a wavefront (the fused norms).
// Merge Welford states of equal count across the wavefront (butterfly, so
// every lane ends with the row statistics), for G independent rows at once:
// each step's cross-lane exchanges of all G rows are issued together, so
// their latencies overlap.  Every row is merged exactly as with G = 1.
template <int G>
__device__ __forceinline__ void wave_welford_rows(float* mean, float* m2, float count) {
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) {
    float other_mean[G], other_m2[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      other_mean[g] = __shfl_xor(mean[g], offset);
      other_m2[g] = __shfl_xor(m2[g], offset);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float delta = other_mean[g] - mean[g];
      mean[g] = 0.5f * (mean[g] + other_mean[g]);
      m2[g] = m2[g] + other_m2[g] + delta * delta * (0.5f * count);
    }
    count *= 2.0f;
  }
}

__device__ __forceinline__ void wave_welford(float& mean, float& m2, float count) {
  wave_welford_rows<1>(&mean, &m2, count);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) v += __shfl_xor(v, offset);
  return v;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace sah
