// Linear layer with a fused bias + exact-GELU epilogue, for gfx950 (CDNA4).
//
// Same contract as the reference's fused FFN input projection
// (solution/kernels/ffn/triton_linear_exact_gelu.py:69-137):
//   y = GELU(x W^T + b),  GELU(v) = 0.5 v (1 + erf(v / sqrt(2)))
// with fp32 accumulation, the bias added in fp32, the activation evaluated in
// fp32 and one rounding to the output dtype.  With the activation switched off
// the same kernel is a plain Linear (bias optional).
//
// MI355X formulation:
//  * 256 x 256 output tile per workgroup of 8 wavefronts (2 x 4), each wave
//    owning 128 rows x 64 columns; K advances 64 at a time through a
//    double-buffered LDS stage (rows padded by 16 bytes, conflict-free 16-byte
//    operand reads) with one barrier per K step.
//  * The product is computed transposed, Y^T = W X^T, with
//    v_mfma_f32_32x32x16_{bf16,f16}: both operands are 16-byte row chunks of
//    the row-major x and W tiles, and every lane's accumulator column is one
//    output row holding runs of 4 consecutive output columns, so the epilogue
//    packs them into 8-byte LDS writes and the tile leaves through LDS as
//    fully coalesced 16-byte stores.
//  * Workgroup ids are remapped so that each XCD (ids are dealt round-robin
//    over the 8 XCDs) works on a contiguous run of tiles: the x rows of a
//    run's tiles are shared in that XCD's L2.
//
// The same GEMM with a head-major epilogue is the packed QKV projection of the
// reference's native-layout path (solution/kernels/projection/
// triton_qkv_layout.py:60-115): x [B*S, D] times the packed [3D, D] weight,
// bias added in fp32, one rounding, and every output column scattered
// straight into query / key / value as [B, H, S, head_dim] (no [B, S, 3D]
// intermediate).  The value may instead be written seq-contiguous,
// [B, H, head_dim, v_ld], for consumers that want V^T (the attention kernel
// reads the [B, H, S, head_dim] value as given).
//
// With a LayerNorm prologue (sah_norm_qkv_projection) the projection also
// fuses the model's first LayerNorm, the reference's initial-norm / QKV fusion
// (solution/kernels/projection/triton_shape07_initial_norm_qkv.py:67-140):
// a row-statistics kernel first forms each row's fp32 mean and 1/std into a
// workspace (8 bytes per row; one wavefront per row with the lane mapping,
// per-lane Welford state and pairwise merge of the fused norm kernel, so the
// statistics are those of sah_norm bit for bit), then the projection
// normalizes x as each K step is staged into LDS, rounding the normalized
// row to the model dtype before the MFMAs as the unfused boundary rounds its
// output.  The normalized rows never reach HBM.  (Forming the statistics
// inside the projection instead makes each of the 3 d_model / 256 column
// tiles of a row block re-read the whole block before its first MFMA.)

#include <cmath>

#include "sah_common.hpp"

namespace sah {
namespace {

constexpr int kBM = 256;              // output rows per workgroup
constexpr int kBN = 256;              // output columns per workgroup
constexpr int kBK = 64;               // K per stage
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRow = kBK + 8;         // LDS operand row (elements), 16-byte pad
constexpr int kOutRow = kBN + 8;      // LDS output staging row (elements)

// Epilogues: row-major y (optionally through exact GELU), or the head-major
// Q / K / V scatter.
constexpr int kEpiRows = 0;
constexpr int kEpiRowsGelu = 1;
constexpr int kEpiHeads = 2;

struct LinearParams {
  const void* x;     // [rows][K], row stride x_ld
  const void* w;     // [N][K], contiguous
  const void* bias;  // [N] or null, same dtype as x
  void* y;           // [rows][N], row stride y_ld (row-major epilogues)
  int64_t rows, x_ld, y_ld;
  int n, k;
  int tiles_n, num_tiles;
  // Head-major epilogue: output columns [0, D) -> q, [D, 2D) -> k,
  // [2D, 3D) -> v, column c of a block -> head c / head_dim, element
  // c % head_dim; row r -> token (r / seq_len, r % seq_len).
  void* q;
  void* kk;
  void* v;
  int64_t v_ld;      // seq stride of a seq-contiguous value
  int seq_len, heads, head_dim, d_model;
  int v_seq_major;   // value as [B][H][head_dim][v_ld] instead of [B][H][S][head_dim]
  int seq_aligned;   // seq_len % 8 == 0: 8-token runs never cross a sequence
  // LayerNorm on the x rows: weight / bias [K] in the x dtype and each
  // row's (mean, 1/std).
  const void* ln_w;
  const void* ln_b;
  const float2* ln_stats;
};

// Row statistics of G rows of K = ITERS * 512 elements by one wavefront,
// exactly as the fused norm kernel forms them: lane l holds elements
// (i * 64 + l) * 8 .. + 7 of a row, a per-lane mean then M2, merged across
// the wave.
template <typename T, int ITERS, int G>
__device__ __forceinline__ void group_stats(const u32x4 (*raw)[ITERS], float eps, float2* out) {
  constexpr int N = ITERS * 8;
  float mean[G], m2[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v[N];
#pragma unroll
    for (int i = 0; i < ITERS; ++i) unpack8<T>(raw[g][i], v + 8 * i);
    float lane_mean = 0.0f;
#pragma unroll
    for (int e = 0; e < N; ++e) lane_mean += v[e];
    lane_mean *= (1.0f / N);
    float lane_m2 = 0.0f;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float d = v[e] - lane_mean;
      lane_m2 += d * d;
    }
    mean[g] = lane_mean;
    m2[g] = lane_m2;
  }
  wave_welford_rows<G>(mean, m2, (float)N);
#pragma unroll
  for (int g = 0; g < G; ++g) out[g] = make_float2(mean[g], rsqrtf(m2[g] * (1.0f / (N * 64)) + eps));
}

// (mean, 1/std) of every row of x [rows][K] into stats[rows]: wavefront w
// of a workgroup owns G consecutive rows, loads all of them, then forms their
// statistics together (the row loads and the cross-lane merges of the G
// rows overlap).
constexpr int kStatsWaves = 4;
template <typename T, int ITERS>
__global__ __launch_bounds__(kStatsWaves * 64) void row_stats_kernel(const T* x, int64_t x_ld,
                                                                      int64_t rows, float eps,
                                                                      float2* stats) {
  constexpr int G = 16 / ITERS;  // 64 VGPRs of row data per lane
  const int lane = threadIdx.x & 63;
  const int64_t first = ((int64_t)blockIdx.x * kStatsWaves + (threadIdx.x >> 6)) * G;
  if (first >= rows) return;  // wave-uniform; the kernel has no barrier
  u32x4 raw[G][ITERS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    // rows past the end read the group's first row (in bounds), never stored
    const T* rp = x + (first + g < rows ? first + g : first) * x_ld;
#pragma unroll
    for (int i = 0; i < ITERS; ++i) raw[g][i] = load16(rp + (i * 64 + lane) * 8);
  }
  float2 st[G];
  group_stats<T, ITERS, G>(raw, eps, st);
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (first + g < rows) stats[first + g] = st[g];
  }
}

template <typename T, int ITERS>
int launch_row_stats(const T* x, int64_t x_ld, int64_t rows, float eps, float2* stats,
                     hipStream_t stream) {
  constexpr int64_t rows_per_block = kStatsWaves * (16 / ITERS);
  const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((row_stats_kernel<T, ITERS>), dim3((unsigned)blocks), dim3(kStatsWaves * 64), 0,
                     stream, x, x_ld, rows, eps, stats);
  return check_hip(hipGetLastError(), "row statistics kernel launch");
}

template <typename T>
int row_stats(const void* x, int64_t x_ld, int64_t rows, int64_t k, float eps, float2* stats,
              hipStream_t stream) {
  const T* xt = static_cast<const T*>(x);
  switch (k) {
    case 512: return launch_row_stats<T, 1>(xt, x_ld, rows, eps, stats, stream);
    case 1024: return launch_row_stats<T, 2>(xt, x_ld, rows, eps, stats, stream);
    case 2048: return launch_row_stats<T, 4>(xt, x_ld, rows, eps, stats, stream);
    default: return launch_row_stats<T, 8>(xt, x_ld, rows, eps, stats, stream);
  }
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <typename T, int EPI, bool LN = false>
__global__ __launch_bounds__(kThreads) void linear_kernel(LinearParams p) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec8<T>::half_type V4;
  constexpr bool GELU = EPI == kEpiRowsGelu;

  // Two operand stages of x and W rows; after the K loop the same bytes hold
  // the output tile.
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * 2 * kBM * kRow * sizeof(T)];
  T(*x_lds)[kBM][kRow] = reinterpret_cast<T(*)[kBM][kRow]>(smem);
  T(*w_lds)[kBN][kRow] = reinterpret_cast<T(*)[kBN][kRow]>(smem + 2 * kBM * kRow * sizeof(T));
  T(*y_lds)[kOutRow] = reinterpret_cast<T(*)[kOutRow]>(smem);
  static_assert(kBM * kOutRow * sizeof(T) <= sizeof(smem), "output staging must fit");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const int wave_m = wave >> 2;  // 128-row slab
  const int wave_n = wave & 3;   // 64-column slab

  // ---- workgroup id -> tile, contiguous runs per XCD.
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int local = bid >> 3;
  const int per = p.num_tiles >> 3;
  const int rem = p.num_tiles & 7;
  const int logical =
      xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int tile_m = logical / p.tiles_n;
  const int tile_n = logical - tile_m * p.tiles_n;
  const int64_t m0 = (int64_t)tile_m * kBM;
  const int n0 = tile_n * kBN;

  const T* xg = static_cast<const T*>(p.x);
  const T* wg = static_cast<const T*>(p.w);

  // ---- LayerNorm: the (mean, 1/std) of the 4 rows this thread stages.
  float ln_mean[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ln_rstd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (LN) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + ((tid + kThreads * i) >> 3);
      if (m < p.rows) {
        const float2 st = p.ln_stats[m];
        ln_mean[i] = st.x;
        ln_rstd[i] = st.y;
      }
    }
  }
  const T* lnw = static_cast<const T*>(p.ln_w);
  const T* lnb = static_cast<const T*>(p.ln_b);

  // ---- staging: 4 chunks of 16 bytes of x and of W per thread and K step.
  // Chunk c = tid + kThreads * i is row c / 8, elements 8 (c % 8) .. + 7
  // (the same 8 columns for all four chunks of a thread).
  u32x4 x_pref[4], w_pref[4];
  u32x4 lnw_pref = {0u, 0u, 0u, 0u}, lnb_pref = {0u, 0u, 0u, 0u};
  auto load_step = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 8;
      const int64_t m = m0 + row;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (m < p.rows) raw = load16(xg + m * p.x_ld + k0 + kc);
      x_pref[i] = raw;
      w_pref[i] = load16(wg + (int64_t)(n0 + row) * p.k + k0 + kc);
    }
    if constexpr (LN) {
      const int kc = (tid & 7) * 8;
      lnw_pref = load16(lnw + k0 + kc);
      lnb_pref = load16(lnb + k0 + kc);
    }
  };
  auto store_step = [&](int stage) {
    float lw[8], lb[8];
    if constexpr (LN) {
      unpack8<T>(lnw_pref, lw);
      unpack8<T>(lnb_pref, lb);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 8;
      u32x4 xs = x_pref[i];
      if constexpr (LN) {
        // the fused norm kernel's expression, rounded to T from fp32 as it does
        float v[8], y[8];
        unpack8<T>(xs, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = fp32_result<T>((v[e] - ln_mean[i]) * ln_rstd[i] * lw[e] + lb[e]);
        xs = pack8<T>(y);
      }
      *reinterpret_cast<u32x4*>(&x_lds[stage][row][kc]) = xs;
      *reinterpret_cast<u32x4*>(&w_lds[stage][row][kc]) = w_pref[i];
    }
  };

  // acc[i][j]: Y^T block of 32 columns (i) x 32 rows (j); lane = one row.
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int steps = p.k / kBK;
  load_step(0);
  store_step(0);
  __syncthreads();

  for (int s = 0; s < steps; ++s) {
    const int stage = s & 1;
    const bool has_next = s + 1 < steps;
    if (has_next) load_step((s + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      V8 wf[2], xf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        wf[i] = *reinterpret_cast<const V8*>(&w_lds[stage][wave_n * 64 + 32 * i + l32][16 * kk + 8 * half]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xf[j] = *reinterpret_cast<const V8*>(&x_lds[stage][wave_m * 128 + 32 * j + l32][16 * kk + 8 * half]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(wf[i], xf[j], acc[i][j]);
    }
    if (has_next) store_step(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue: bias, activation, one rounding; stage the tile in LDS.
  // Accumulator register r of acc[i][j] holds output column
  // 32 i + 8 (r / 4) + 4 half + r % 4 (within the wave's slab) of row 32 j + l32.
  const T* bg = static_cast<const T*>(p.bias);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n_l = wave_n * 64 + 32 * i + 8 * g + 4 * half;
      float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bg != nullptr) {
        const V4 raw = *reinterpret_cast<const V4*>(bg + n0 + n_l);
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = to_f32(raw[q]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        V4 out;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v = acc[i][j][4 * g + q] + bv[q];
          if (GELU) v = gelu_exact(v);
          out[q] = from_f32<T>(v);
        }
        *reinterpret_cast<V4*>(&y_lds[wave_m * 128 + 32 * j + l32][n_l]) = out;
      }
    }
  }
  __syncthreads();

  constexpr int kChunks = (kBM * kBN / 8) / kThreads;  // 16-byte chunks per thread
  if constexpr (EPI != kEpiHeads) {
    // ---- coalesced 16-byte stores of the valid rows.
    T* yg = static_cast<T*>(p.y);
#pragma unroll
    for (int s2 = 0; s2 < kChunks; ++s2) {
      const int c = tid + kThreads * s2;
      const int row = c >> 5;          // 32 chunks of 8 elements per row
      const int col = (c & 31) * 8;
      const int64_t m = m0 + row;
      if (m < p.rows) store16(yg + m * p.y_ld + n0 + col, *reinterpret_cast<const u32x4*>(&y_lds[row][col]));
    }
  } else {
    // ---- head-major scatter.  d_model is a multiple of kBN, so the whole
    // tile belongs to one of q / k / v.  Token indices fit in 32 bits (the
    // host checks rows < 2^31).
    const int which = n0 / p.d_model;
    const int c0 = n0 - which * p.d_model;
    T* dst = static_cast<T*>(which == 0 ? p.q : which == 1 ? p.kk : p.v);
    const unsigned seq = (unsigned)p.seq_len;
    const int hd = p.head_dim;
    if (which != 2 || !p.v_seq_major) {
      // [B][H][S][hd]: a 16-byte chunk is 8 consecutive elements of one head
      // (head_dim is a multiple of 8).
#pragma unroll 4
      for (int s2 = 0; s2 < kChunks; ++s2) {
        const int c = tid + kThreads * s2;
        const int row = c >> 5;
        const int col = (c & 31) * 8;
        const int64_t m = m0 + row;
        if (m >= p.rows) continue;
        const unsigned b = (unsigned)m / seq;
        const unsigned s = (unsigned)m - b * seq;
        const int within = c0 + col;
        const int head = within / hd;
        const int e = within - head * hd;
        T* out = dst + (((int64_t)b * p.heads + head) * (int64_t)seq + s) * hd + e;
        store16(out, *reinterpret_cast<const u32x4*>(&y_lds[row][col]));
      }
    } else {
      // [B][H][hd][v_ld]: a 16-byte chunk is 8 consecutive tokens of one
      // column, read down an LDS column (consecutive lanes take consecutive
      // columns: conflict-free).
#pragma unroll 4
      for (int s2 = 0; s2 < kChunks; ++s2) {
        const int c = tid + kThreads * s2;
        const int col = c & (kBN - 1);
        const int row0 = (c >> 8) * 8;
        const int64_t m = m0 + row0;
        if (m >= p.rows) continue;
        const int within = c0 + col;
        const int head = within / hd;
        const int e = within - head * hd;
        if (p.seq_aligned && m + 8 <= p.rows) {
          const unsigned b = (unsigned)m / seq;
          const unsigned s = (unsigned)m - b * seq;
          V8 run;
#pragma unroll
          for (int t = 0; t < 8; ++t) run[t] = y_lds[row0 + t][col];
          T* out = dst + (((int64_t)b * p.heads + head) * hd + e) * p.v_ld + s;
          store16(out, __builtin_bit_cast(u32x4, run));
        } else {
          for (int t = 0; t < 8 && m + t < p.rows; ++t) {
            const unsigned b = (unsigned)(m + t) / seq;
            const unsigned s = (unsigned)(m + t) - b * seq;
            dst[(((int64_t)b * p.heads + head) * hd + e) * p.v_ld + s] = y_lds[row0 + t][col];
          }
        }
      }
    }
  }
}

template <typename T, int EPI, bool LN = false>
int launch_linear(const LinearParams& prm, hipStream_t stream) {
  hipLaunchKernelGGL((linear_kernel<T, EPI, LN>), dim3(prm.num_tiles), dim3(kThreads), 0, stream, prm);
  return check_hip(hipGetLastError(), "linear kernel launch");
}

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_linear_launch_supported(int block_m, int block_n, int block_k, int num_warps,
                                           int num_stages) {
  return block_m == kBM && block_n == kBN && block_k == kBK && num_warps == kWaves && num_stages == 2;
}

extern "C" int sah_linear(const void* x, const void* weight, const void* bias, void* y,
                          int64_t rows, int64_t in_features, int64_t out_features,
                          int64_t x_row_stride, int64_t y_row_stride, int dtype, int activation,
                          int block_m, int block_n, int block_k, int num_warps, int num_stages,
                          sah_stream_t stream) {
  if (!sah_linear_launch_supported(block_m, block_n, block_k, num_warps, num_stages))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_linear: launch (%d, %d, %d, %d, %d) is not implemented (256, 256, 64, 8, 2)",
                block_m, block_n, block_k, num_warps, num_stages);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16)
    return fail(SAH_ERR_UNSUPPORTED, "sah_linear: dtype %d is not bf16 or f16", dtype);
  if (activation != SAH_ACTIVATION_NONE && activation != SAH_ACTIVATION_GELU_EXACT)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear: unknown activation %d", activation);
  if (rows < 0 || in_features <= 0 || out_features <= 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear: bad sizes rows=%lld in=%lld out=%lld",
                (long long)rows, (long long)in_features, (long long)out_features);
  if (in_features % kBK != 0 || out_features % kBN != 0 || in_features > (1 << 20) ||
      out_features > (1 << 20))
    return fail(SAH_ERR_UNSUPPORTED,
                "sah_linear: in_features must be a multiple of %d and out_features of %d "
                "(got %lld, %lld)",
                kBK, kBN, (long long)in_features, (long long)out_features);
  if (x_row_stride < in_features || y_row_stride < out_features || x_row_stride % 8 != 0 ||
      y_row_stride % 8 != 0)
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_linear: row strides must cover the row and be multiples of 8 elements "
                "(x %lld, y %lld)",
                (long long)x_row_stride, (long long)y_row_stride);
  if (rows == 0) return SAH_OK;
  if (x == nullptr || weight == nullptr || y == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "sah_linear: null tensor pointer");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(y) ||
      (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 7u) != 0))
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_linear: x, weight and y must be 16-byte aligned, bias 8-byte aligned");
  const int64_t tiles_m = (rows + kBM - 1) / kBM;
  const int64_t tiles_n = out_features / kBN;
  if (tiles_m * tiles_n > INT32_MAX)
    return fail(SAH_ERR_UNSUPPORTED, "sah_linear: %lld rows is too many", (long long)rows);

  LinearParams prm = {};
  prm.x = x;
  prm.w = weight;
  prm.bias = bias;
  prm.y = y;
  prm.rows = rows;
  prm.x_ld = x_row_stride;
  prm.y_ld = y_row_stride;
  prm.n = (int)out_features;
  prm.k = (int)in_features;
  prm.tiles_n = (int)tiles_n;
  prm.num_tiles = (int)(tiles_m * tiles_n);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool gelu = activation == SAH_ACTIVATION_GELU_EXACT;
  if (dtype == SAH_DTYPE_BF16)
    return gelu ? launch_linear<bf16, kEpiRowsGelu>(prm, s) : launch_linear<bf16, kEpiRows>(prm, s);
  return gelu ? launch_linear<f16, kEpiRowsGelu>(prm, s) : launch_linear<f16, kEpiRows>(prm, s);
}

extern "C" int sah_qkv_launch_supported(int block_m, int block_n, int block_k, int num_warps) {
  return block_m == kBM && block_n == kBN && block_k == kBK && num_warps == kWaves;
}

namespace {
int qkv_projection(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
                   const void* weight, const void* bias, void* query, void* key, void* value,
                   int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads,
                   int64_t x_row_stride, int value_layout, int64_t value_seq_stride, int dtype,
                   int block_m, int block_n, int block_k, int num_warps, void* workspace,
                   size_t workspace_bytes, sah_stream_t stream) {
  const bool ln = ln_weight != nullptr || ln_bias != nullptr;
  const char* entry = ln ? "sah_norm_qkv_projection" : "sah_qkv_projection";
  if (!sah_qkv_launch_supported(block_m, block_n, block_k, num_warps))
    return fail(SAH_ERR_UNSUPPORTED, "%s: launch (%d, %d, %d, %d) is not implemented (256, 256, 64, 8)",
                entry, block_m, block_n, block_k, num_warps);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16)
    return fail(SAH_ERR_UNSUPPORTED, "%s: dtype %d is not bf16 or f16", entry, dtype);
  if (value_layout != SAH_QKV_VALUE_BHSD && value_layout != SAH_QKV_VALUE_SEQ_MAJOR)
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: unknown value layout %d", entry, value_layout);
  if (batch < 0 || seq_len <= 0 || d_model <= 0 || heads <= 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: bad sizes batch=%lld seq_len=%lld d_model=%lld heads=%lld",
                entry, (long long)batch, (long long)seq_len, (long long)d_model, (long long)heads);
  if (d_model % kBN != 0 || d_model > (1 << 18) || d_model % heads != 0 || (d_model / heads) % 8 != 0)
    return fail(SAH_ERR_UNSUPPORTED, "%s: d_model must be a multiple of %d (at most 2^18) and split "
                "into heads of a multiple of 8 elements (got d_model %lld, %lld heads)",
                entry, kBN, (long long)d_model, (long long)heads);
  if (x_row_stride < d_model || x_row_stride % 8 != 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: x row stride %lld must cover d_model and be a multiple of 8",
                entry, (long long)x_row_stride);
  if (value_layout == SAH_QKV_VALUE_SEQ_MAJOR && (value_seq_stride < seq_len || value_seq_stride % 8 != 0))
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: value seq stride %lld must cover seq_len %lld and be a "
                "multiple of 8", entry, (long long)value_seq_stride, (long long)seq_len);
  if (ln) {
    if (ln_weight == nullptr || ln_bias == nullptr)
      return fail(SAH_ERR_INVALID_ARGUMENT, "%s: LayerNorm weight and bias are both required", entry);
    if (!aligned16(ln_weight) || !aligned16(ln_bias))
      return fail(SAH_ERR_INVALID_ARGUMENT, "%s: LayerNorm weight and bias must be 16-byte aligned",
                  entry);
    if (!(std::isfinite(ln_eps) && ln_eps >= 0.0f))
      return fail(SAH_ERR_INVALID_ARGUMENT, "%s: eps must be finite and non-negative", entry);
    if (d_model != 512 && d_model != 1024 && d_model != 2048 && d_model != 4096)
      return fail(SAH_ERR_UNSUPPORTED, "%s: d_model must be 512, 1024, 2048 or 4096 (got %lld)", entry,
                  (long long)d_model);
  }
  if (batch == 0) return SAH_OK;
  if (seq_len > INT32_MAX || batch > INT32_MAX / seq_len)
    return fail(SAH_ERR_UNSUPPORTED, "%s: batch x seq_len must be below 2^31", entry);
  if (x == nullptr || weight == nullptr || query == nullptr || key == nullptr || value == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", entry);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(query) || !aligned16(key) || !aligned16(value) ||
      (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 7u) != 0))
    return fail(SAH_ERR_INVALID_ARGUMENT, "%s: x, weight, query, key and value must be 16-byte aligned, "
                "bias 8-byte aligned", entry);
  const int64_t rows = batch * seq_len;
  if (ln) {
    const size_t need = sah_norm_qkv_workspace_bytes(batch, seq_len);
    if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
      return fail(SAH_ERR_WORKSPACE, "%s: needs a 16-byte aligned workspace of %zu bytes (got %zu)", entry,
                  need, workspace == nullptr ? (size_t)0 : workspace_bytes);
  }
  const int64_t tiles_m = (rows + kBM - 1) / kBM;
  const int64_t tiles_n = 3 * d_model / kBN;

  LinearParams prm = {};
  prm.ln_w = ln_weight;
  prm.ln_b = ln_bias;
  prm.ln_stats = static_cast<const float2*>(workspace);
  prm.x = x;
  prm.w = weight;
  prm.bias = bias;
  prm.rows = rows;
  prm.x_ld = x_row_stride;
  prm.n = (int)(3 * d_model);
  prm.k = (int)d_model;
  prm.tiles_n = (int)tiles_n;
  prm.num_tiles = (int)(tiles_m * tiles_n);
  prm.q = query;
  prm.kk = key;
  prm.v = value;
  prm.v_ld = value_layout == SAH_QKV_VALUE_SEQ_MAJOR ? value_seq_stride : 0;
  prm.seq_len = (int)seq_len;
  prm.heads = (int)heads;
  prm.head_dim = (int)(d_model / heads);
  prm.d_model = (int)d_model;
  prm.v_seq_major = value_layout == SAH_QKV_VALUE_SEQ_MAJOR;
  prm.seq_aligned = seq_len % 8 == 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (ln) {
    float2* stats = static_cast<float2*>(workspace);
    const int status = dtype == SAH_DTYPE_BF16 ? row_stats<bf16>(x, x_row_stride, rows, d_model, ln_eps, stats, s)
                                               : row_stats<f16>(x, x_row_stride, rows, d_model, ln_eps, stats, s);
    if (status != SAH_OK) return status;
    return dtype == SAH_DTYPE_BF16 ? launch_linear<bf16, kEpiHeads, true>(prm, s)
                                   : launch_linear<f16, kEpiHeads, true>(prm, s);
  }
  return dtype == SAH_DTYPE_BF16 ? launch_linear<bf16, kEpiHeads>(prm, s)
                                 : launch_linear<f16, kEpiHeads>(prm, s);
}
}  // namespace

extern "C" int sah_qkv_projection(const void* x, const void* weight, const void* bias, void* query,
                                  void* key, void* value, int64_t batch, int64_t seq_len,
                                  int64_t d_model, int64_t heads, int64_t x_row_stride,
                                  int value_layout, int64_t value_seq_stride, int dtype,
                                  int block_m, int block_n, int block_k, int num_warps,
                                  sah_stream_t stream) {
  return qkv_projection(x, nullptr, nullptr, 0.0f, weight, bias, query, key, value, batch, seq_len,
                        d_model, heads, x_row_stride, value_layout, value_seq_stride, dtype, block_m,
                        block_n, block_k, num_warps, nullptr, 0, stream);
}

extern "C" size_t sah_norm_qkv_workspace_bytes(int64_t batch, int64_t seq_len) {
  if (batch <= 0 || seq_len <= 0 || batch > INT64_MAX / 8 / seq_len) return 0;
  return (size_t)(batch * seq_len) * sizeof(float2);
}

extern "C" int sah_norm_qkv_projection(const void* x, const void* ln_weight, const void* ln_bias,
                                       float ln_eps, const void* weight, const void* bias,
                                       void* query, void* key, void* value, int64_t batch,
                                       int64_t seq_len, int64_t d_model, int64_t heads,
                                       int64_t x_row_stride, int value_layout,
                                       int64_t value_seq_stride, int dtype, int block_m,
                                       int block_n, int block_k, int num_warps,
                                       void* workspace, size_t workspace_bytes,
                                       sah_stream_t stream) {
  if (ln_weight == nullptr || ln_bias == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "sah_norm_qkv_projection: LayerNorm weight and bias are both required");
  return qkv_projection(x, ln_weight, ln_bias, ln_eps, weight, bias, query, key, value, batch,
                        seq_len, d_model, heads, x_row_stride, value_layout, value_seq_stride,
                        dtype, block_m, block_n, block_k, num_warps, workspace, workspace_bytes,
                        stream);
}
