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

// Round-trip through the storage type (used where the reference rounds an
// intermediate to the model dtype, e.g. the residual stream).
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return to_f32(from_f32<T>(x));
}

// GELU(v) = v * Phi(v) with Phi(v) = erfc(-v / sqrt(2)) / 2, and erfc(x) for
// x >= 0 from Abramowitz & Stegun 7.1.26:
//   erfc(x) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-x^2),
//   t = 1 / (1 + p x),  |erf error| <= 1.5e-7,
// so Phi(v) = 1 - erfc(|v|/sqrt 2) / 2 for v >= 0 and erfc(|v|/sqrt 2) / 2 for
// v < 0.  Using erfc directly on the negative side avoids the cancellation of
// 1 + erf(v / sqrt 2): against float64 exact GELU, the bf16 results of this
// form differ (by one ulp) on fewer elements than fp32 1 + erff(...) does
// (199 vs 404 of 200 000 N(0, 1.4) inputs, measured on the CPU), at about
// half the VALU work of a general-purpose erff (one reciprocal, one exp2).
__device__ __forceinline__ float gelu_exact(float v) {
  const float x = fabsf(v) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, x, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  const float e = __builtin_amdgcn_exp2f(x * (x * -1.4426950408889634f));
  const float half_erfc = 0.5f * (poly * t) * e;
  const float phi = v >= 0.0f ? 1.0f - half_erfc : half_erfc;
  return v * phi;
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
// every lane ends with the row statistics).
__device__ __forceinline__ void wave_welford(float& mean, float& m2, float count) {
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) {
    const float other_mean = __shfl_xor(mean, offset);
    const float other_m2 = __shfl_xor(m2, offset);
    const float delta = other_mean - mean;
    mean = 0.5f * (mean + other_mean);
    m2 = m2 + other_m2 + delta * delta * (0.5f * count);
    count *= 2.0f;
  }
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
