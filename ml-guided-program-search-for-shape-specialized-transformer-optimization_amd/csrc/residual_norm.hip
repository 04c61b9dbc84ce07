// Fused residual add + LayerNorm / RMSNorm for gfx950 (wave64).
//
// Semantics follow the reference's boundary (solution/transformer.py:1515-1644):
// the residual stream is rounded to its storage dtype before it is normalized
// (residual_add, solution/operators/norm/residual_add.py:28-39, then
// nn.LayerNorm with biased variance), and the mixed variant keeps an fp32
// stream with a 16-bit update exactly like
// solution/kernels/norm/triton_mixed_residual.py:41-76.
//
// Mapping: one wavefront per row, 16 bytes per lane per access, so a wave
// reads 1 KiB per load instruction with every lane's address contiguous.
// Rows narrower than one such pass (16-bit widths 128 and 256, fp32 width
// 128) use 4- or 8-byte accesses: VEC = width / 64 elements per lane.
// Each lane keeps its slice of the row in registers; statistics are a per-lane
// Welford state (count, mean, M2) merged across the 64 lanes with the
// pairwise (Chan et al.) update, so HBM is read exactly once per tensor.
// Algorithmic traffic per element: value + update read, residual + normalized
// written (8 B/element for an all-bf16 boundary).

#include "sah_common.hpp"

namespace sah {
namespace {

constexpr int kWave = 64;

template <typename T, int N>
struct VecIO {
  typedef T V __attribute__((ext_vector_type(N)));
  // Row data is read once: non-temporal loads (measured 25.5 -> 24.9 us for
  // 16384 x 1024 bf16 rows, 272 -> 268 us for 200000, outputs bitwise equal).
  static __device__ __forceinline__ void load(const T* p, float* out) {
    V v = __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = to_f32(v[i]);
  }
  static __device__ __forceinline__ void store(T* p, const float* in) {
    V v;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = from_f32<T>(in[i]);
    // Streaming store: rows are written once.  Measured on MI355X (bf16,
    // width 1024): 288 -> 277 us for 200000 rows, 27.4 -> 26.5 us for 16384.
    __builtin_nontemporal_store(v, reinterpret_cast<V*>(p));
  }
};


// TX: residual-stream dtype (value in, residual out); TU: update dtype;
// TY: normalized dtype; TP: weight/bias dtype.  ITERS * 64 * VEC == width.
// ONE_ROW: rows_per_wave == 1, compiled as straight-line code, so the affine
// parameters stay packed until they are used (55 instead of 77 VGPRs at width
// 1024 bf16: 8 instead of 6 waves per SIMD, 26.6 -> 25.6 us for 16384 rows).
template <typename TX, typename TU, typename TY, typename TP, int ITERS, bool HAS_RES, bool ONE_ROW,
          int VEC = 16 / sizeof(TX)>
__global__ __launch_bounds__(512) void norm_kernel(
    const TX* __restrict__ value, const TU* __restrict__ update,
    const TP* __restrict__ weight, const TP* __restrict__ bias,
    TX* __restrict__ residual, TY* __restrict__ normalized, int64_t rows,
    float eps, int rows_per_wave, int rms) {
  constexpr int WIDTH = ITERS * kWave * VEC;
  constexpr int N = ITERS * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int64_t first_row =
      ((int64_t)blockIdx.x * waves + wave) * (int64_t)rows_per_wave;

  // Affine parameters for this lane's columns (L2-resident across rows),
  // kept in their storage type and widened where they are used.  They are
  // loaded after the first row's HBM loads are issued, so those start first
  // (C3 shape, same box, alternating: 23.70 -> 23.63 us with one row per
  // wave of 4, 24.11 -> 23.93 us with 8).
  typedef typename VecIO<TP, VEC>::V VP;
  const bool has_w = weight != nullptr, has_b = bias != nullptr;
  VP w_raw[ITERS], b_raw[ITERS];

  for (int r = 0; r < (ONE_ROW ? 1 : rows_per_wave); ++r) {
    const int64_t row = first_row + r;
    if (row >= rows) return;  // wave-uniform
    const int64_t base = row * (int64_t)WIDTH;
    float v[N];
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
      const int col = (i * kWave + lane) * VEC;
      VecIO<TX, VEC>::load(value + base + col, v + i * VEC);
    }
    float u[HAS_RES ? N : 1];
    if constexpr (HAS_RES) {
#pragma unroll
      for (int i = 0; i < ITERS; ++i) {
        const int col = (i * kWave + lane) * VEC;
        VecIO<TU, VEC>::load(update + base + col, u + i * VEC);
      }
    }
    if (ONE_ROW || r == 0) {
#pragma unroll
      for (int i = 0; i < ITERS; ++i) {
        const int col = (i * kWave + lane) * VEC;
        if (has_w) w_raw[i] = *reinterpret_cast<const VP*>(weight + col);
        if (has_b) b_raw[i] = *reinterpret_cast<const VP*>(bias + col);
      }
    }
    if constexpr (HAS_RES) {
#pragma unroll
      for (int e = 0; e < N; ++e) v[e] = round_to<TX>(v[e] + u[e]);
#pragma unroll
      for (int i = 0; i < ITERS; ++i) {
        const int col = (i * kWave + lane) * VEC;
        VecIO<TX, VEC>::store(residual + base + col, v + i * VEC);
      }
    }

    float mean = 0.0f, rstd;
    if (!rms) {
      // Per-lane Welford state over this lane's N elements.
      float lane_mean = 0.0f;
#pragma unroll
      for (int e = 0; e < N; ++e) lane_mean += v[e];
      lane_mean *= (1.0f / N);
      float m2 = 0.0f;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float d = v[e] - lane_mean;
        m2 += d * d;
      }
      mean = lane_mean;
      wave_welford(mean, m2, (float)N);
      rstd = rsqrtf(m2 * (1.0f / WIDTH) + eps);
    } else {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < N; ++e) ss += v[e] * v[e];
      ss = wave_sum(ss);
      rstd = rsqrtf(ss * (1.0f / WIDTH) + eps);
    }

    float y[N];
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float we = has_w ? to_f32(w_raw[e / VEC][e % VEC]) : 1.0f;
      const float be = has_b ? to_f32(b_raw[e / VEC][e % VEC]) : 0.0f;
      y[e] = fp32_result<TY>((v[e] - mean) * rstd * we + be);
    }
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
      const int col = (i * kWave + lane) * VEC;
      VecIO<TY, VEC>::store(normalized + base + col, y + i * VEC);
    }
  }
}

size_t dtype_size(int dtype) {
  switch (dtype) {
    case SAH_DTYPE_F32:
      return 4;
    case SAH_DTYPE_F16:
    case SAH_DTYPE_BF16:
      return 2;
    default:
      return 0;
  }
}

struct NormArgs {
  const void* value;
  const void* update;
  const void* weight;
  const void* bias;
  void* residual;
  void* normalized;
  int64_t rows;
  int64_t width;
  float eps;
  int norm_kind;
  int block_rows;
  int num_warps;
  hipStream_t stream;
};

template <typename TX, typename TU, typename TY, typename TP, bool HAS_RES, int NARROW>
int launch_narrow(const NormArgs& a) {
  const int rows_per_wave = a.block_rows / a.num_warps;
  const int64_t grid = ceil_div(a.rows, a.block_rows);
  if (grid > INT32_MAX) return fail(SAH_ERR_UNSUPPORTED, "too many rows");
  const dim3 block(a.num_warps * kWave);
  if (rows_per_wave == 1)
    hipLaunchKernelGGL((norm_kernel<TX, TU, TY, TP, 1, HAS_RES, true, NARROW>), dim3(grid), block, 0,
                       a.stream, static_cast<const TX*>(a.value), static_cast<const TU*>(a.update),
                       static_cast<const TP*>(a.weight), static_cast<const TP*>(a.bias),
                       static_cast<TX*>(a.residual), static_cast<TY*>(a.normalized), a.rows, a.eps,
                       rows_per_wave, a.norm_kind);
  else
    hipLaunchKernelGGL((norm_kernel<TX, TU, TY, TP, 1, HAS_RES, false, NARROW>), dim3(grid), block, 0,
                       a.stream, static_cast<const TX*>(a.value), static_cast<const TU*>(a.update),
                       static_cast<const TP*>(a.weight), static_cast<const TP*>(a.bias),
                       static_cast<TX*>(a.residual), static_cast<TY*>(a.normalized), a.rows, a.eps,
                       rows_per_wave, a.norm_kind);
  return check_hip(hipGetLastError(), "norm kernel launch");
}

template <typename TX, typename TU, typename TY, typename TP, bool HAS_RES>
int launch_typed(const NormArgs& a) {
  constexpr int VEC = 16 / sizeof(TX);
  const int64_t per_iter = (int64_t)kWave * VEC;
  // Narrow rows: one access of width / 64 elements per lane.
  if (a.width == 128) return launch_narrow<TX, TU, TY, TP, HAS_RES, 2>(a);
  if (a.width == 256 && VEC == 8) return launch_narrow<TX, TU, TY, TP, HAS_RES, 4>(a);
  if (a.width % per_iter != 0) {
    return fail(SAH_ERR_UNSUPPORTED, "norm width %lld is 128, %sor a multiple of %lld",
                (long long)a.width, VEC == 8 ? "256 " : "", (long long)per_iter);
  }
  const int64_t iters = a.width / per_iter;
  const int rows_per_wave = a.block_rows / a.num_warps;
  const int64_t grid = ceil_div(a.rows, a.block_rows);
  if (grid > INT32_MAX) return fail(SAH_ERR_UNSUPPORTED, "too many rows");
  const dim3 block(a.num_warps * kWave);
  const TX* value = static_cast<const TX*>(a.value);
  const TU* update = static_cast<const TU*>(a.update);
  const TP* weight = static_cast<const TP*>(a.weight);
  const TP* bias = static_cast<const TP*>(a.bias);
  TX* residual = static_cast<TX*>(a.residual);
  TY* normalized = static_cast<TY*>(a.normalized);
#define SAH_NORM_CASE(IT)                                                        \
  case IT:                                                                       \
    if (rows_per_wave == 1)                                                      \
      hipLaunchKernelGGL((norm_kernel<TX, TU, TY, TP, IT, HAS_RES, true>),       \
                         dim3(grid), block, 0, a.stream, value, update, weight,  \
                         bias, residual, normalized, a.rows, a.eps,              \
                         rows_per_wave, a.norm_kind);                            \
    else                                                                         \
      hipLaunchKernelGGL((norm_kernel<TX, TU, TY, TP, IT, HAS_RES, false>),      \
                         dim3(grid), block, 0, a.stream, value, update, weight,  \
                         bias, residual, normalized, a.rows, a.eps,              \
                         rows_per_wave, a.norm_kind);                            \
    break;
  switch (iters) {
    SAH_NORM_CASE(1)
    SAH_NORM_CASE(2)
    SAH_NORM_CASE(4)
    SAH_NORM_CASE(8)
    SAH_NORM_CASE(16)
    default:
      return fail(SAH_ERR_UNSUPPORTED,
                  "norm width %lld not implemented (supported: 128, %s%lld x {1,2,4,8,16})",
                  (long long)a.width, VEC == 8 ? "256, " : "", (long long)per_iter);
  }
#undef SAH_NORM_CASE
  return check_hip(hipGetLastError(), "norm kernel launch");
}

template <typename TX, typename TU, typename TY, bool HAS_RES>
int launch_params(const NormArgs& a, int param_dtype, int value_dtype) {
  if (param_dtype == SAH_DTYPE_F32) return launch_typed<TX, TU, TY, float, HAS_RES>(a);
  if (param_dtype == value_dtype) return launch_typed<TX, TU, TY, TX, HAS_RES>(a);
  return fail(SAH_ERR_UNSUPPORTED, "param dtype must be f32 or the value dtype");
}

int validate_common(const NormArgs& a, bool has_res, int value_dtype,
                    int normalized_dtype, int param_dtype) {
  if (a.value == nullptr || a.normalized == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "value and normalized must be non-null");
  if (has_res && (a.update == nullptr || a.residual == nullptr))
    return fail(SAH_ERR_INVALID_ARGUMENT, "update and residual must be non-null");
  if (a.rows < 0 || a.width <= 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "rows must be >= 0 and width > 0");
  if (a.norm_kind != SAH_NORM_LAYER && a.norm_kind != SAH_NORM_RMS)
    return fail(SAH_ERR_INVALID_ARGUMENT, "unknown norm kind %d", a.norm_kind);
  if (!(a.num_warps == 1 || a.num_warps == 2 || a.num_warps == 4 || a.num_warps == 8))
    return fail(SAH_ERR_UNSUPPORTED, "num_warps must be 1, 2, 4 or 8");
  if (a.block_rows <= 0 || a.block_rows % a.num_warps != 0 || a.block_rows > 64)
    return fail(SAH_ERR_UNSUPPORTED,
                "block_rows must be a positive multiple of num_warps and <= 64");
  if (!(a.eps >= 0.0f)) return fail(SAH_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  if (dtype_size(value_dtype) == 0 || dtype_size(normalized_dtype) == 0 ||
      dtype_size(param_dtype) == 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "unknown dtype code");
  const void* ptrs[] = {a.value, a.update, a.weight, a.bias, a.residual, a.normalized};
  for (const void* p : ptrs) {
    if (p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15u) != 0)
      return fail(SAH_ERR_INVALID_ARGUMENT, "all tensors must be 16-byte aligned");
  }
  return SAH_OK;
}

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_residual_norm(const void* value, const void* update,
                                 const void* weight, const void* bias,
                                 void* residual, void* normalized, int64_t rows,
                                 int64_t width, float eps, int value_dtype,
                                 int update_dtype, int normalized_dtype,
                                 int param_dtype, int norm_kind, int block_rows,
                                 int num_warps, sah_stream_t stream) {
  NormArgs a{value, update, weight, bias, residual, normalized, rows, width, eps,
             norm_kind, block_rows, num_warps, reinterpret_cast<hipStream_t>(stream)};
  int status = validate_common(a, true, value_dtype, normalized_dtype, param_dtype);
  if (status != SAH_OK) return status;
  if (dtype_size(update_dtype) == 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "unknown update dtype code");
  if (rows == 0) return SAH_OK;
  const int v = value_dtype, u = update_dtype, y = normalized_dtype, p = param_dtype;
  if (v == SAH_DTYPE_BF16 && u == SAH_DTYPE_BF16 && y == SAH_DTYPE_BF16)
    return launch_params<bf16, bf16, bf16, true>(a, p, v);
  if (v == SAH_DTYPE_F16 && u == SAH_DTYPE_F16 && y == SAH_DTYPE_F16)
    return launch_params<f16, f16, f16, true>(a, p, v);
  if (v == SAH_DTYPE_F32 && p == SAH_DTYPE_F32) {
    if (u == SAH_DTYPE_F32 && y == SAH_DTYPE_F32)
      return launch_typed<float, float, float, float, true>(a);
    if (u == SAH_DTYPE_F16 && y == SAH_DTYPE_F16)
      return launch_typed<float, f16, f16, float, true>(a);
    if (u == SAH_DTYPE_F16 && y == SAH_DTYPE_F32)
      return launch_typed<float, f16, float, float, true>(a);
    if (u == SAH_DTYPE_BF16 && y == SAH_DTYPE_BF16)
      return launch_typed<float, bf16, bf16, float, true>(a);
    if (u == SAH_DTYPE_BF16 && y == SAH_DTYPE_F32)
      return launch_typed<float, bf16, float, float, true>(a);
  }
  return fail(SAH_ERR_UNSUPPORTED,
              "residual norm dtype combination (value=%d, update=%d, normalized=%d, "
              "param=%d) is not implemented",
              v, u, y, p);
}

extern "C" int sah_norm(const void* value, const void* weight, const void* bias,
                        void* normalized, int64_t rows, int64_t width, float eps,
                        int value_dtype, int normalized_dtype, int param_dtype,
                        int norm_kind, int block_rows, int num_warps,
                        sah_stream_t stream) {
  NormArgs a{value, nullptr, weight, bias, nullptr, normalized, rows, width, eps,
             norm_kind, block_rows, num_warps, reinterpret_cast<hipStream_t>(stream)};
  int status = validate_common(a, false, value_dtype, normalized_dtype, param_dtype);
  if (status != SAH_OK) return status;
  if (rows == 0) return SAH_OK;
  const int v = value_dtype, y = normalized_dtype, p = param_dtype;
  if (v == SAH_DTYPE_BF16 && y == SAH_DTYPE_BF16)
    return launch_params<bf16, bf16, bf16, false>(a, p, v);
  if (v == SAH_DTYPE_F16 && y == SAH_DTYPE_F16)
    return launch_params<f16, f16, f16, false>(a, p, v);
  if (v == SAH_DTYPE_F32 && p == SAH_DTYPE_F32) {
    if (y == SAH_DTYPE_F32) return launch_typed<float, float, float, float, false>(a);
    if (y == SAH_DTYPE_F16) return launch_typed<float, float, f16, float, false>(a);
    if (y == SAH_DTYPE_BF16) return launch_typed<float, float, bf16, float, false>(a);
  }
  return fail(SAH_ERR_UNSUPPORTED,
              "norm dtype combination (value=%d, normalized=%d, param=%d) is not "
              "implemented",
              v, y, p);
}
