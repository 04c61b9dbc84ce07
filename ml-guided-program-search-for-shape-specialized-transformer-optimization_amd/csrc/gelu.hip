// Exact GELU over a contiguous 16-bit tensor, for gfx950 (CDNA4).
//
// Same contract as the reference's elementwise FFN activation
// (solution/kernels/ffn/triton_exact_gelu.py:50-118): y = GELU(x) with
// GELU(v) = 0.5 v (1 + erf(v / sqrt(2))) evaluated in fp32 and one rounding
// to the output dtype.  The activation itself is gelu_exact() of
// sah_common.hpp (erfc form, no cancellation on the negative side).
//
// HBM-bound: 2 bytes read and 2 written per element.  A workgroup of
// num_warps wavefronts covers block_size elements; every thread issues all of
// its 16-byte loads before the first store (CPT chunks in flight), and the
// input may be the output (each thread reads its chunks before writing them).

#include "sah_common.hpp"

namespace sah {
namespace {

template <typename T, int CPT>
__global__ __launch_bounds__(512) void gelu_kernel(const T* x, T* y, int64_t n) {
  typedef typename Vec8<T>::type V8;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x * CPT * 8;
  u32x4 raw[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int64_t idx = first + ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    raw[c] = (u32x4){0u, 0u, 0u, 0u};
    if (idx + 8 <= n) raw[c] = load16(x + idx);
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int64_t idx = first + ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    if (idx + 8 <= n) {
      V8 v = __builtin_bit_cast(V8, raw[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = from_f32<T>(gelu_exact(to_f32(v[e])));
      store16(y + idx, __builtin_bit_cast(u32x4, v));
    } else if (idx < n) {  // the ragged end: fewer than 8 elements left
      for (int64_t e = idx; e < n; ++e) y[e] = from_f32<T>(gelu_exact(to_f32(x[e])));
    }
  }
}

template <typename T, int CPT>
int launch_gelu(const void* x, void* y, int64_t n, int threads, hipStream_t stream) {
  const int64_t per_block = (int64_t)threads * CPT * 8;
  const int64_t blocks = (n + per_block - 1) / per_block;
  hipLaunchKernelGGL((gelu_kernel<T, CPT>), dim3((unsigned)blocks), dim3(threads), 0, stream,
                     static_cast<const T*>(x), static_cast<T*>(y), n);
  return check_hip(hipGetLastError(), "gelu kernel launch");
}

template <typename T>
int dispatch_gelu(const void* x, void* y, int64_t n, int threads, int cpt, hipStream_t stream) {
  switch (cpt) {
    case 1: return launch_gelu<T, 1>(x, y, n, threads, stream);
    case 2: return launch_gelu<T, 2>(x, y, n, threads, stream);
    case 4: return launch_gelu<T, 4>(x, y, n, threads, stream);
    default: return launch_gelu<T, 8>(x, y, n, threads, stream);
  }
}

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_gelu_launch_supported(int block_size, int num_warps) {
  if (num_warps != 1 && num_warps != 2 && num_warps != 4 && num_warps != 8) return 0;
  const int per_pass = num_warps * 64 * 8;  // elements of one 16-byte chunk per thread
  if (block_size < per_pass || block_size % per_pass != 0) return 0;
  const int cpt = block_size / per_pass;
  return cpt == 1 || cpt == 2 || cpt == 4 || cpt == 8;
}

extern "C" int sah_gelu(const void* x, void* y, int64_t n, int dtype, int block_size, int num_warps,
                        sah_stream_t stream) {
  if (!sah_gelu_launch_supported(block_size, num_warps))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_gelu: block_size %d with %d wavefronts is not implemented "
                "(block_size = 512 x num_warps x {1, 2, 4, 8})",
                block_size, num_warps);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16)
    return fail(SAH_ERR_UNSUPPORTED, "sah_gelu: dtype %d is not bf16 or f16", dtype);
  if (n < 0) return fail(SAH_ERR_INVALID_ARGUMENT, "sah_gelu: negative element count %lld", (long long)n);
  if (n == 0) return SAH_OK;
  if (x == nullptr || y == nullptr) return fail(SAH_ERR_INVALID_ARGUMENT, "sah_gelu: null tensor pointer");
  if (!aligned16(x) || !aligned16(y))
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_gelu: x and y must be 16-byte aligned");
  const int threads = num_warps * 64;
  const int cpt = block_size / (threads * 8);
  const int64_t blocks = (n + block_size - 1) / block_size;
  if (blocks > 0x7fffffffLL)
    return fail(SAH_ERR_UNSUPPORTED, "sah_gelu: %lld elements need too many workgroups", (long long)n);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return dtype == SAH_DTYPE_BF16 ? dispatch_gelu<bf16>(x, y, n, threads, cpt, s)
                                 : dispatch_gelu<f16>(x, y, n, threads, cpt, s);
}
