// Whole FFN fused through its residual add and LayerNorm / RMSNorm, for
// gfx950 (CDNA4): the hidden activation and the branch update never reach
// HBM.
//
// Same contract as the reference's fused MLP boundary
// (solution/kernels/boundary/triton_ffn_residual_norm.py:44-135), on this
// build's 16-bit residual stream:
//   hidden     = round_to(T, GELU(x W1^T + b1))   fp32 accumulation, exact GELU
//   update     = round_to(T, hidden W2^T + b2)
//   residual   = round_to(T, value + update)
//   normalized = round_to(T, norm(residual) * gamma + beta)
// with the hidden rounded to the stream dtype before W2 consumes it and the
// update rounded before it is added, the two rounding points the reference
// keeps explicit (:91-94, :101-104) and the unfused path has.  The reference
// serves D = F = 128; this kernel takes D in {128, 256} and any F that is a
// multiple of 64.
//
// MI355X formulation:
//  * One workgroup of 4 wavefronts owns 64 rows; its x block stays in LDS.
//    The FFN width is streamed in chunks of 64 hidden units: each chunk's
//    W1 rows and W2 columns are staged in LDS, wave w forms one 32 x 32 block
//    of the hidden chunk (hidden^T = W1 x^T with v_mfma_f32_32x32x16, so
//    every lane's accumulator column is one row), adds the bias, applies the
//    exact GELU, rounds and stores it to LDS; then every wave accumulates its
//    D/4 output columns of all 64 rows (update^T = W2 hidden^T) in registers
//    across the chunks.
//  * Epilogue: bias, one rounding, the update tile staged in the dead x
//    block; then one wave per row adds the residual and normalizes with the
//    fused norm kernel's narrow-row mapping (lane l holds columns
//    l * D/64 .. + D/64 - 1) and arithmetic (per-lane Welford state merged
//    across the wavefront, statistics over the rounded residual), so for a
//    given update the residual and normalized rows equal sah_residual_norm's.

#include <cmath>

#include "sah_common.hpp"

namespace sah {
namespace {

constexpr int kMlpWaves = 4;
constexpr int kMlpThreads = kMlpWaves * 64;
constexpr int kMlpRows = 64;   // rows per workgroup
constexpr int kMlpChunk = 64;  // hidden units per chunk

struct MlpNormParams {
  const void* x;       // [rows][D], row stride x_ld
  const void* w1;      // [F][D]
  const void* b1;      // [F] or null
  const void* w2;      // [D][F]
  const void* b2;      // [D] or null
  const void* value;   // [rows][D] residual stream in
  const void* gamma;   // [D] or null (1)
  const void* beta;    // [D] or null (0)
  void* residual;      // [rows][D]
  void* normalized;    // [rows][D]
  int64_t rows, x_ld;
  int f;
  float eps;
  int rms;
};

__device__ __forceinline__ f32x16 mlp_mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mlp_mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <typename T, int N>
struct NarrowVec {
  typedef T V __attribute__((ext_vector_type(N)));
};

template <typename T, int D>
__global__ __launch_bounds__(kMlpThreads) void mlp_norm_kernel(MlpNormParams p) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec8<T>::half_type V4;
  constexpr int XR = D + 8;           // x / W1 / update row (elements): 16-byte pad
  constexpr int HR = kMlpChunk + 8;   // hidden / W2 row (elements)
  constexpr int KS = D / 16;          // MFMA slices of the first product
  constexpr int NBW = D / 128;        // 32-column blocks of the update per wave
  constexpr int DC = D / 8;           // 16-byte chunks per D-long row
  constexpr int EPL = D / 64;         // residual / norm elements per lane
  static_assert(D == 128 || D == 256, "the x block and one chunk of W1 and W2 stay in LDS");

  __shared__ __attribute__((aligned(16))) T x_lds[kMlpRows][XR];
  __shared__ __attribute__((aligned(16))) T w1_lds[kMlpChunk][XR];
  __shared__ __attribute__((aligned(16))) T w2_lds[D][HR];
  __shared__ __attribute__((aligned(16))) T h_lds[kMlpRows][HR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.x * kMlpRows;
  const int F = p.f;

  const T* xg = static_cast<const T*>(p.x);
  const T* w1g = static_cast<const T*>(p.w1);
  const T* w2g = static_cast<const T*>(p.w2);
  const T* b1g = static_cast<const T*>(p.b1);
  const T* b2g = static_cast<const T*>(p.b2);

  // ---- x block: 64 rows x D, rows past the end read as zero.
#pragma unroll
  for (int i = 0; i < kMlpRows * DC / kMlpThreads; ++i) {
    const int c = tid + kMlpThreads * i;
    const int row = c / DC;
    const int kc = (c % DC) * 8;
    const int64_t m = m0 + row;
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (m < p.rows) raw = load16(xg + m * p.x_ld + kc);
    *reinterpret_cast<u32x4*>(&x_lds[row][kc]) = raw;
  }

  // update^T accumulators: block (i, j) = output columns n0w + 32 i .., rows 32 j ..
  const int n0w = wave * (D / kMlpWaves);
  f32x16 acc[NBW][2];
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // This wave's block of each hidden chunk: hidden units 32 hb .., rows 32 rb ..
  const int hb = wave >> 1;
  const int rb = wave & 1;

  for (int f0 = 0; f0 < F; f0 += kMlpChunk) {
    // ---- stage the chunk: W1 rows f0 .. f0 + 63 (64 x D) and the chunk's
    // 64 columns of every W2 row (D x 64).
#pragma unroll
    for (int i = 0; i < kMlpChunk * DC / kMlpThreads; ++i) {
      const int c = tid + kMlpThreads * i;
      const int row = c / DC;
      const int kc = (c % DC) * 8;
      *reinterpret_cast<u32x4*>(&w1_lds[row][kc]) = load16(w1g + (int64_t)(f0 + row) * D + kc);
    }
#pragma unroll
    for (int i = 0; i < D * (kMlpChunk / 8) / kMlpThreads; ++i) {
      const int c = tid + kMlpThreads * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 8;
      *reinterpret_cast<u32x4*>(&w2_lds[row][kc]) = load16(w2g + (int64_t)row * F + f0 + kc);
    }
    __syncthreads();

    // ---- hidden^T block = W1 x^T, then bias, exact GELU, one rounding.
    f32x16 hacc = {};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const V8 a = *reinterpret_cast<const V8*>(&w1_lds[32 * hb + l32][16 * s + 8 * half]);
      const V8 b = *reinterpret_cast<const V8*>(&x_lds[32 * rb + l32][16 * s + 8 * half]);
      hacc = mlp_mfma32(a, b, hacc);
    }
    // Register r holds hidden unit 32 hb + 8 (r / 4) + 4 half + r % 4 of row 32 rb + l32.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int hl = 32 * hb + 8 * g + 4 * half;
      float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b1g != nullptr) {
        const V4 raw = *reinterpret_cast<const V4*>(b1g + f0 + hl);
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = to_f32(raw[q]);
      }
      V4 out;
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = from_f32<T>(gelu_exact(hacc[4 * g + q] + bv[q]));
      *reinterpret_cast<V4*>(&h_lds[32 * rb + l32][hl]) = out;
    }
    __syncthreads();

    // ---- update^T += W2[:, chunk] hidden^T.
#pragma unroll
    for (int s = 0; s < kMlpChunk / 16; ++s) {
      V8 hf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        hf[j] = *reinterpret_cast<const V8*>(&h_lds[32 * j + l32][16 * s + 8 * half]);
#pragma unroll
      for (int i = 0; i < NBW; ++i) {
        const V8 a = *reinterpret_cast<const V8*>(&w2_lds[n0w + 32 * i + l32][16 * s + 8 * half]);
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mlp_mfma32(a, hf[j], acc[i][j]);
      }
    }
    __syncthreads();  // the next chunk overwrites W1, W2 and the hidden block
  }

  // ---- update = round(acc + b2), staged in the x block (dead after the last
  // chunk; the loop ended with a barrier).  Register r of acc[i][j] is column
  // n0w + 32 i + 8 (r / 4) + 4 half + r % 4 of row 32 j + l32.
  T(*u_lds)[XR] = x_lds;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0w + 32 * i + 8 * g + 4 * half;
      float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b2g != nullptr) {
        const V4 raw = *reinterpret_cast<const V4*>(b2g + n);
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = to_f32(raw[q]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        V4 out;
#pragma unroll
        for (int q = 0; q < 4; ++q) out[q] = from_f32<T>(acc[i][j][4 * g + q] + bv[q]);
        *reinterpret_cast<V4*>(&u_lds[32 * j + l32][n]) = out;
      }
    }
  }
  __syncthreads();

  // ---- residual add + norm, one wave per row, lane l on columns l * EPL ...
  typedef typename NarrowVec<T, EPL>::V VN;
  const int col = lane * EPL;
  const T* gamma = static_cast<const T*>(p.gamma);
  const T* beta = static_cast<const T*>(p.beta);
  float w[EPL], b[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    w[e] = gamma != nullptr ? to_f32(gamma[col + e]) : 1.0f;
    b[e] = beta != nullptr ? to_f32(beta[col + e]) : 0.0f;
  }
  const T* vg = static_cast<const T*>(p.value);
  T* rg = static_cast<T*>(p.residual);
  T* yg = static_cast<T*>(p.normalized);
  for (int rr = wave; rr < kMlpRows; rr += kMlpWaves) {
    const int64_t m = m0 + rr;
    if (m >= p.rows) break;  // wave-uniform
    const int64_t base = m * (int64_t)D + col;
    const VN vin = *reinterpret_cast<const VN*>(vg + base);
    const VN uin = *reinterpret_cast<const VN*>(&u_lds[rr][col]);
    float v[EPL];
    VN rout;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      v[e] = round_to<T>(to_f32(vin[e]) + to_f32(uin[e]));
      rout[e] = from_f32<T>(v[e]);
    }
    *reinterpret_cast<VN*>(rg + base) = rout;
    float mean = 0.0f, rstd;
    if (!p.rms) {
      float lane_mean = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) lane_mean += v[e];
      lane_mean *= (1.0f / EPL);
      float m2 = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float d = v[e] - lane_mean;
        m2 += d * d;
      }
      mean = lane_mean;
      wave_welford(mean, m2, (float)EPL);
      rstd = rsqrtf(m2 * (1.0f / D) + p.eps);
    } else {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) ss += v[e] * v[e];
      ss = wave_sum(ss);
      rstd = rsqrtf(ss * (1.0f / D) + p.eps);
    }
    VN yout;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      yout[e] = from_f32<T>(fp32_result<T>((v[e] - mean) * rstd * w[e] + b[e]));
    *reinterpret_cast<VN*>(yg + base) = yout;
  }
}

template <typename T, int D>
int launch_mlp_norm(const MlpNormParams& prm, hipStream_t stream) {
  const int64_t blocks = (prm.rows + kMlpRows - 1) / kMlpRows;
  hipLaunchKernelGGL((mlp_norm_kernel<T, D>), dim3((unsigned)blocks), dim3(kMlpThreads), 0, stream, prm);
  return check_hip(hipGetLastError(), "MLP residual norm kernel launch");
}

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_mlp_residual_norm_launch_supported(int64_t width, int block_rows, int num_warps) {
  return (width == 128 || width == 256) && block_rows == kMlpRows && num_warps == kMlpWaves;
}

extern "C" int sah_mlp_residual_norm(const void* x, const void* w1, const void* b1, const void* w2,
                                     const void* b2, const void* value, const void* gamma,
                                     const void* beta, void* residual, void* normalized,
                                     int64_t rows, int64_t width, int64_t ffn,
                                     int64_t x_row_stride, float eps, int dtype, int norm_kind,
                                     int block_rows, int num_warps, sah_stream_t stream) {
  if (!sah_mlp_residual_norm_launch_supported(width, block_rows, num_warps))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_mlp_residual_norm: (width %lld, block_rows %d, num_warps %d) is not implemented "
                "(width 128 or 256, 64 rows, 4 waves)",
                (long long)width, block_rows, num_warps);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16)
    return fail(SAH_ERR_UNSUPPORTED, "sah_mlp_residual_norm: dtype %d is not bf16 or f16", dtype);
  if (norm_kind != SAH_NORM_LAYER && norm_kind != SAH_NORM_RMS)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_mlp_residual_norm: unknown norm kind %d", norm_kind);
  if (rows < 0 || ffn <= 0 || ffn % kMlpChunk != 0 || ffn > (1 << 20))
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_mlp_residual_norm: rows must be >= 0 and ffn a positive multiple of %d "
                "(at most 2^20); got rows %lld, ffn %lld",
                kMlpChunk, (long long)rows, (long long)ffn);
  if (x_row_stride < width || x_row_stride % 8 != 0)
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_mlp_residual_norm: x row stride %lld must cover the width and be a multiple of 8",
                (long long)x_row_stride);
  if (!(std::isfinite(eps) && eps >= 0.0f))
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_mlp_residual_norm: eps must be finite and >= 0");
  if (rows == 0) return SAH_OK;
  if (x == nullptr || w1 == nullptr || w2 == nullptr || value == nullptr || residual == nullptr ||
      normalized == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_mlp_residual_norm: null tensor pointer");
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w2) || !aligned16(value) || !aligned16(residual) ||
      !aligned16(normalized) || (gamma != nullptr && !aligned16(gamma)) ||
      (beta != nullptr && !aligned16(beta)) ||
      (b1 != nullptr && (reinterpret_cast<uintptr_t>(b1) & 7u) != 0) ||
      (b2 != nullptr && (reinterpret_cast<uintptr_t>(b2) & 7u) != 0))
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_mlp_residual_norm: tensors must be 16-byte aligned, biases 8-byte");
  if (ceil_div(rows, kMlpRows) > INT32_MAX)
    return fail(SAH_ERR_UNSUPPORTED, "sah_mlp_residual_norm: %lld rows is too many", (long long)rows);

  MlpNormParams prm = {};
  prm.x = x;
  prm.w1 = w1;
  prm.b1 = b1;
  prm.w2 = w2;
  prm.b2 = b2;
  prm.value = value;
  prm.gamma = gamma;
  prm.beta = beta;
  prm.residual = residual;
  prm.normalized = normalized;
  prm.rows = rows;
  prm.x_ld = x_row_stride;
  prm.f = (int)ffn;
  prm.eps = eps;
  prm.rms = norm_kind == SAH_NORM_RMS;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == SAH_DTYPE_BF16)
    return width == 128 ? launch_mlp_norm<bf16, 128>(prm, s) : launch_mlp_norm<bf16, 256>(prm, s);
  return width == 128 ? launch_mlp_norm<f16, 128>(prm, s) : launch_mlp_norm<f16, 256>(prm, s);
}
