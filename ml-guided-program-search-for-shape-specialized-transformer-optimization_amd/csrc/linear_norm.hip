// Linear + residual add + LayerNorm / RMSNorm boundary for gfx950 (CDNA4).
//
// Same contract as the reference's fused linear boundary
// (solution/kernels/boundary/triton_linear_residual_norm.py:34-109): the
// branch update of a block (the attention output projection, or the FFN
// output projection) never reaches HBM.
//   update     = round_to(T, x W^T + b)          fp32 accumulation, bias in fp32
//   residual   = round_to(T, value + update)
//   normalized = round_to(T, norm(residual) * gamma + beta)
// The update is rounded to the stream dtype before it is added, as the
// reference rounds it to its fp16 branch dtype (:88-90) and as the unfused
// path does (the projection's output, then sah_residual_norm); the residual
// and norm arithmetic are those of csrc/residual_norm.hip.
//
// MI355X formulation:
//  * One workgroup (8 wavefronts) owns BM = 65536 / D whole rows, so the row
//    statistics never leave the workgroup.  Wave w computes output columns
//    [w D/8, (w+1) D/8) of all BM rows: 8 accumulator blocks of 32 x 32
//    (v_mfma_f32_32x32x16, computed transposed: update^T = W x^T).
//  * W is read straight from global memory (L2: W is at most a few MB and is
//    shared by every workgroup) into the MFMA A operand: each wave reads a
//    disjoint slice, so staging it in LDS would buy no reuse.  Within each
//    64-wide K step the K order is permuted (MFMA slice kk, lane half h takes
//    k = 32 h + 8 kk .. +7) so every lane reads 64 contiguous bytes of its W
//    row per step; x uses the same permutation when its fragments are read
//    from LDS.  The W fragments of step s+1 are loaded into the registers of
//    step s right after their MFMAs issue.
//  * x (shared by all 8 waves) goes through a double-buffered LDS stage
//    (rows padded by 16 bytes: conflict-free 16-byte operand reads), one
//    barrier per K step.
//  * Epilogue: bias, one rounding, the bf16/fp16 update tile staged in the
//    same LDS; then every wave normalizes whole rows exactly like the fused
//    norm kernel (16-byte accesses, per-lane Welford state merged across the
//    wavefront), reading the residual input and writing the residual and the
//    normalized rows once.

#include <cmath>

#include "sah_common.hpp"

namespace sah {
namespace {

constexpr int kLnWaves = 8;
constexpr int kLnThreads = kLnWaves * 64;
constexpr int kLnBK = 64;
constexpr int kLnXRow = kLnBK + 8;  // LDS x row (elements), 16-byte pad

struct LinearNormParams {
  const void* x;       // [rows][K], row stride x_ld
  const void* w;       // [D][K], contiguous
  const void* bias;    // [D] or null
  const void* value;   // [rows][D] residual stream in
  const void* gamma;   // [D] or null (1)
  const void* beta;    // [D] or null (0)
  void* residual;      // [rows][D]
  void* normalized;    // [rows][D]
  int64_t rows, x_ld;
  int k;
  float eps;
  int rms;
};

__device__ __forceinline__ f32x16 ln_mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 ln_mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int D>
struct LnShape {
  static constexpr int BM = 65536 / D;          // rows per workgroup
  static constexpr int COLS = D / kLnWaves;     // output columns per wave
  static constexpr int NB = COLS / 32;          // column blocks per wave
  static constexpr int MB = BM / 32;            // row blocks
  static constexpr int XCPT = BM * (kLnBK / 8) / kLnThreads;  // x chunks per thread and step
  static constexpr int UROW = D + 8;            // LDS update row (elements)
  static_assert(NB * MB == 8, "eight accumulator blocks per wave");
  static_assert(XCPT >= 1, "every thread stages x");
};

template <typename T, int D>
__global__ __launch_bounds__(kLnThreads) void linear_norm_kernel(LinearNormParams p) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec8<T>::half_type V4;
  typedef LnShape<D> S;
  constexpr int BM = S::BM, NB = S::NB, MB = S::MB;

  constexpr size_t kXBytes = 2ull * BM * kLnXRow * sizeof(T);
  constexpr size_t kUBytes = (size_t)BM * S::UROW * sizeof(T);
  __shared__ __attribute__((aligned(16))) unsigned char smem[kXBytes > kUBytes ? kXBytes : kUBytes];
  T(*x_lds)[BM][kLnXRow] = reinterpret_cast<T(*)[BM][kLnXRow]>(smem);
  T(*u_lds)[S::UROW] = reinterpret_cast<T(*)[S::UROW]>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int n0w = wave * S::COLS;

  const T* xg = static_cast<const T*>(p.x);
  const T* wg = static_cast<const T*>(p.w);

  // ---- x staging: XCPT chunks of 16 bytes per thread and K step.
  u32x4 x_pref[S::XCPT];
  auto load_x = [&](int k0) {
#pragma unroll
    for (int i = 0; i < S::XCPT; ++i) {
      const int c = tid + kLnThreads * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 8;
      const int64_t m = m0 + row;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (m < p.rows) raw = load16(xg + m * p.x_ld + k0 + kc);
      x_pref[i] = raw;
    }
  };
  auto store_x = [&](int stage) {
#pragma unroll
    for (int i = 0; i < S::XCPT; ++i) {
      const int c = tid + kLnThreads * i;
      *reinterpret_cast<u32x4*>(&x_lds[stage][c >> 3][(c & 7) * 8]) = x_pref[i];
    }
  };
  // ---- W fragments: block i, MFMA slice kk of the step at k0.
  const T* w_rows = wg + (int64_t)(n0w + l32) * p.k + 32 * half;
  V8 wf[NB][4];
  auto load_w = [&](int k0, int kk) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
      wf[i][kk] = __builtin_bit_cast(V8, load16(w_rows + (int64_t)(32 * i) * p.k + k0 + 8 * kk));
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int steps = p.k / kLnBK;
  load_x(0);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) load_w(0, kk);
  store_x(0);
  __syncthreads();

  for (int s = 0; s < steps; ++s) {
    const int stage = s & 1;
    const bool has_next = s + 1 < steps;
    if (has_next) load_x((s + 1) * kLnBK);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      V8 xf[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j)
        xf[j] = *reinterpret_cast<const V8*>(&x_lds[stage][32 * j + l32][32 * half + 8 * kk]);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = ln_mfma32(wf[i][kk], xf[j], acc[i][j]);
      if (has_next) load_w((s + 1) * kLnBK, kk);
    }
    if (has_next) store_x(stage ^ 1);
    __syncthreads();
  }

  // ---- update = round(acc + bias), staged in LDS (the x stages are dead:
  // the loop ended with a barrier).  Register r of acc[i][j] is column
  // 32 i + 8 (r / 4) + 4 half + r % 4 of the wave's slab, row 32 j + l32.
  const T* bg = static_cast<const T*>(p.bias);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0w + 32 * i + 8 * g + 4 * half;
      float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bg != nullptr) {
        const V4 raw = *reinterpret_cast<const V4*>(bg + n);
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = to_f32(raw[q]);
      }
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        V4 out;
#pragma unroll
        for (int q = 0; q < 4; ++q) out[q] = from_f32<T>(acc[i][j][4 * g + q] + bv[q]);
        *reinterpret_cast<V4*>(&u_lds[32 * j + l32][n]) = out;
      }
    }
  }
  __syncthreads();

  // ---- residual add + norm, one wave per row (the fused norm kernel's
  // arithmetic and lane-to-column mapping).
  constexpr int ITERS = D / 512;
  constexpr int N = ITERS * 8;
  const T* gamma = static_cast<const T*>(p.gamma);
  const T* beta = static_cast<const T*>(p.beta);
  float w[N], b[N];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int col = (it * 64 + lane) * 8;
    if (gamma != nullptr) {
      unpack8<T>(load16(gamma + col), w + it * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) w[it * 8 + e] = 1.0f;
    }
    if (beta != nullptr) {
      unpack8<T>(load16(beta + col), b + it * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) b[it * 8 + e] = 0.0f;
    }
  }
  const T* vg = static_cast<const T*>(p.value);
  T* rg = static_cast<T*>(p.residual);
  T* yg = static_cast<T*>(p.normalized);
  for (int rr = wave; rr < BM; rr += kLnWaves) {
    const int64_t m = m0 + rr;
    if (m >= p.rows) break;  // wave-uniform
    const int64_t base = m * (int64_t)D;
    float v[N];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int col = (it * 64 + lane) * 8;
      float u[8];
      unpack8<T>(load16(vg + base + col), v + it * 8);
      unpack8<T>(*reinterpret_cast<const u32x4*>(&u_lds[rr][col]), u);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[it * 8 + e] = round_to<T>(v[it * 8 + e] + u[e]);
      store16(rg + base + col, pack8<T>(v + it * 8));
    }
    float mean = 0.0f, rstd;
    if (!p.rms) {
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
      rstd = rsqrtf(m2 * (1.0f / D) + p.eps);
    } else {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < N; ++e) ss += v[e] * v[e];
      ss = wave_sum(ss);
      rstd = rsqrtf(ss * (1.0f / D) + p.eps);
    }
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int col = (it * 64 + lane) * 8;
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        y[e] = fp32_result<T>((v[it * 8 + e] - mean) * rstd * w[it * 8 + e] + b[it * 8 + e]);
      store16(yg + base + col, pack8<T>(y));
    }
  }
}

template <typename T, int D>
int launch_linear_norm(const LinearNormParams& prm, hipStream_t stream) {
  const int64_t blocks = (prm.rows + LnShape<D>::BM - 1) / LnShape<D>::BM;
  hipLaunchKernelGGL((linear_norm_kernel<T, D>), dim3((unsigned)blocks), dim3(kLnThreads), 0, stream, prm);
  return check_hip(hipGetLastError(), "linear residual norm kernel launch");
}

template <typename T>
int dispatch_linear_norm(const LinearNormParams& prm, int64_t width, hipStream_t stream) {
  switch (width) {
    case 512: return launch_linear_norm<T, 512>(prm, stream);
    default: return launch_linear_norm<T, 1024>(prm, stream);
  }
}

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_linear_residual_norm_launch_supported(int64_t width, int block_rows, int num_warps) {
  return (width == 512 || width == 1024) && (int64_t)block_rows * width == 65536 && num_warps == kLnWaves;
}

extern "C" int sah_linear_residual_norm(const void* x, const void* weight, const void* bias,
                                        const void* value, const void* gamma, const void* beta,
                                        void* residual, void* normalized, int64_t rows,
                                        int64_t in_features, int64_t width, int64_t x_row_stride,
                                        float eps, int dtype, int norm_kind, int block_rows,
                                        int num_warps, sah_stream_t stream) {
  if (!sah_linear_residual_norm_launch_supported(width, block_rows, num_warps))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_linear_residual_norm: width %lld with (block_rows %d, num_warps %d) is not "
                "implemented (width 512 or 1024, block_rows = 65536 / width, 8 wavefronts)",
                (long long)width, block_rows, num_warps);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16)
    return fail(SAH_ERR_UNSUPPORTED, "sah_linear_residual_norm: dtype %d is not bf16 or f16", dtype);
  if (norm_kind != SAH_NORM_LAYER && norm_kind != SAH_NORM_RMS)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear_residual_norm: unknown norm kind %d", norm_kind);
  if (rows < 0 || in_features <= 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear_residual_norm: bad sizes rows=%lld in=%lld",
                (long long)rows, (long long)in_features);
  if (in_features % kLnBK != 0 || in_features > (1 << 20))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_linear_residual_norm: in_features must be a multiple of %d (got %lld)", kLnBK,
                (long long)in_features);
  if (x_row_stride < in_features || x_row_stride % 8 != 0)
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_linear_residual_norm: x row stride %lld must cover in_features and be a "
                "multiple of 8",
                (long long)x_row_stride);
  if (!(eps >= 0.0f))
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear_residual_norm: eps must be >= 0");
  if (rows == 0) return SAH_OK;
  if (x == nullptr || weight == nullptr || value == nullptr || residual == nullptr || normalized == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear_residual_norm: null tensor pointer");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(value) || !aligned16(residual) ||
      !aligned16(normalized) || (gamma != nullptr && !aligned16(gamma)) ||
      (beta != nullptr && !aligned16(beta)) ||
      (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 7u) != 0))
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_linear_residual_norm: tensors must be 16-byte aligned (bias 8-byte)");
  const int64_t blocks = (rows + block_rows - 1) / block_rows;
  if (blocks > INT32_MAX)
    return fail(SAH_ERR_UNSUPPORTED, "sah_linear_residual_norm: %lld rows is too many", (long long)rows);

  LinearNormParams prm = {};
  prm.x = x;
  prm.w = weight;
  prm.bias = bias;
  prm.value = value;
  prm.gamma = gamma;
  prm.beta = beta;
  prm.residual = residual;
  prm.normalized = normalized;
  prm.rows = rows;
  prm.x_ld = x_row_stride;
  prm.k = (int)in_features;
  prm.eps = eps;
  prm.rms = norm_kind == SAH_NORM_RMS;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return dtype == SAH_DTYPE_BF16 ? dispatch_linear_norm<bf16>(prm, width, s)
                                 : dispatch_linear_norm<f16>(prm, width, s);
}
