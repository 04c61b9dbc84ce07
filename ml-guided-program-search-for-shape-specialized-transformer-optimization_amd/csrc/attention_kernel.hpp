// attn_fwd_kernel (the plain and scaled-key causal attention kernels) and
// the device helpers it uses, shared by attention_fwd.hip (host code, the
// plain-path instantiations and the other kernels) and attention_scaled.hip
// (the scaled-key-path instantiations, compiled with their own scheduler).
// Everything here has internal linkage: each translation unit instantiates
// only the kernels it launches or hands out.

#pragma once

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "sah_common.hpp"

namespace sah {
namespace {

constexpr int kHeadDim = 64;
constexpr int kBlockN = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kPad = 8;                   // 16-byte row padding in LDS
constexpr int kKRow = kHeadDim + kPad;    // K tile row (elements)
// V tiles stay key-major in LDS: 64 key rows of 128 bytes, each row's 16-byte
// chunks permuted by v_ring_swizzle (below), in the direct-to-LDS ring and in
// the register-staged buffers alike.
constexpr int kVTileBytes = kBlockN * kHeadDim * 2;
constexpr float kLog2e = 1.4426950408889634f;
// The plain kernel raises a row's softmax shift only when a tile maximum
// exceeds it by more than this many powers of two (probabilities then stay
// below 256, far inside the fp32 accumulators and the 16-bit P range).  On
// N(0,1) data that cuts the O rescales from ~1 in 6 tiles to about one per
// row; measured 40.50 -> 40.20 ms on the long-sequence chunk and 1.69 ->
// 1.61 ms at B16 H32 S4096.
constexpr float kLazyShift = 8.0f;
// The tile maximum is formed only for rows whose score bound
// c * |q| * max|k| over the tile exceeds the current shift by more than this
// many powers of two.  Every other row's probabilities stay below 2^kSafeExp:
// for bf16 P (the fp32 exponent range) 2^64, far from overflow even summed
// over 2^31 keys in fp32; for fp16 P 2^15, below the fp16 maximum of 65504.
template <typename T>
constexpr float safe_exponent() {
  return std::is_same<T, f16>::value ? 15.0f : 64.0f;
}
// Scaled-key path (plain kernel, with the key-norm pre-pass).  The pre-pass
// also writes every key multiplied by c and rounded to fp16 (11-bit mantissa),
// and a block of query rows whose largest c |q| max|k| is at most this bound
// (over the keys it reads) runs its tiles on the fp16 MFMA with Q in fp16:
// the MFMA then yields the log2-domain score c q.k itself, and since every
// such score lies in [-bound, bound], P = exp2(score) needs neither a shift
// nor a row maximum (bf16 P: 2^32 is far inside the fp32 exponent range; fp16
// P: 2^15 < 65504).  Softmax is shift-invariant; only the point where P is
// rounded to 16 bits moves.  Rounding P to bf16 has the same relative error at
// any exponent; fp16 P below 2^-14 is subnormal and keeps an absolute error
// of 2^-25, at most 2^-10 relative at the smallest P of 2^-15.  Rounding c k
// to fp16 (unit roundoff 2^-11) moves a score by at most 2^-11 c |q| |k| in
// log2 units: 2^-6 at the bf16 bound, up to 1.1% on one P when the 64
// roundings of a key all lean the same way against q, about 0.1% for
// roundings of random sign.  The official bf16 order rounds the score itself
// to bf16 (2^-9 relative), four times that bound at the same scores.
// Blocks with a larger bound (large-magnitude inputs, an outlier key or
// query) keep the shifted path on the original keys.
template <typename T>
constexpr float scaled_key_bound() {
  return std::is_same<T, f16>::value ? 15.0f : 32.0f;
}
// |q| and c max|k| must also stay below this for the fp16 operands: no
// overflow, and fp16 subnormals of the other operand contribute at most
// 8 * 4096 * 2^-25 = 2^-10 to a score.
constexpr float kScaledKeyMaxNorm = 4096.0f;
// The path is chosen per block of this many query rows (a multiple of every
// plain launch's block_m), from that block's largest |q| and the largest |k|
// of the keys it reads, so every launch takes the same path for a row and the
// results stay independent of the launch.
constexpr int kScaledKeyRows = 512;
// Sequences at least this long get the preparation launch (norm tables and
// fp16 scaled keys, one extra read of Q and K) and with it the scaled-key
// path.  Measured on MI355X, bf16, preparation included, same box with the
// two thresholds alternating: the C4 forward (B16 H32 S4096, two layers)
// 13.11/13.13 -> 12.92/12.96 ms with the path from 4096 keys on; at B8 H16
// S2048 the attention operator 82.3 -> 99.4 us, where the preparation costs
// more than the cheaper tiles save.
constexpr int64_t kKeyNormMinSeq = 4096;

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;  // [B][H][S][64], head_dim stride 1, key stride v_ss
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_ss;
  int seq_len;
  int heads;
  int num_q_tiles;
  int num_blocks;
  int head_group;  // > 0: heads per issue group on one XCD (batch*heads % 8 == 0)
  // c = |scale| * log2(e) > 0 (log2(e) for scale 0).  Every Q dword is loaded
  // as (raw & q_and) ^ q_xor: the identity for scale > 0, the sign flip of
  // both 16-bit halves for scale < 0 (so c * (-q).k = scale * log2(e) * q.k),
  // and zero for scale 0 (every visible key then weighs the same, as in
  // softmax(0 * s)).  The kernels' running maximum of raw scores relies on
  // c > 0.
  float c;
  uint32_t q_and, q_xor;
  // Largest key norm of every 64-key tile, [batch*heads][key_tiles]
  // (long_prepare_kernel), for the plain kernel's score bound; null when the
  // host skips that pre-pass (short sequences), and then every tile forms
  // its row maximum.
  const float* knorm;
  int key_tiles;
  // Keys times c in fp16, [batch*heads][key_tiles * 64][64] (rows past the
  // sequence never read), written by the pre-pass; null without it.
  const f16* kc;
  // Largest |k| and largest |q| of every block of kScaledKeyRows rows,
  // [batch*heads][num_row_blocks] each; set with kc.
  const float* kblock;
  const float* qblock;
  int num_row_blocks;
};

// Workgroup id -> (batch*head, query tile).  With head_group G > 0, XCD x
// (ids x, x + 8, ...) owns heads x, x + 8, x + 16, ... (k of them) and issues
// them in groups of G: tile nq-1 of every head of the group, then tile nq-2,
// and so on (the last group may be smaller).  With G = 0 (batch*heads not a
// multiple of 8) each XCD takes a contiguous range of head-major ids, longest
// tile of each head first.  Both are bijections onto the grid.
__device__ __forceinline__ void tile_of(const AttnParams& p, int& bh, int& q_tile) {
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int local = bid >> 3;
  const int nq = p.num_q_tiles;
  if (p.head_group > 0) {
    const int k = p.num_blocks / (8 * nq);
    const int span = p.head_group * nq;
    const int group = local / span;
    const int r = local - group * span;
    const int size = min(p.head_group, k - group * p.head_group);
    const int rank = r / size;
    bh = xcd + 8 * (group * p.head_group + (r - rank * size));
    q_tile = nq - 1 - rank;
  } else {
    const int nb = p.num_blocks;
    const int per = nb >> 3;
    const int rem = nb & 7;
    const int logical =
        xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    bh = logical / nq;
    q_tile = nq - 1 - (logical - bh * nq);
  }
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float dot2_sum(bf16x2 p, float acc) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(p, one, acc, false);
}
__device__ __forceinline__ float dot2_sum(f16x2 p, float acc) {
  const f16x2 one = {(f16)1.0f, (f16)1.0f};
  return __builtin_amdgcn_fdot2(p, one, acc, false);
}

// Row of the K tile that MFMA A-row i reads: bits 2 and 3 exchanged.
__device__ __forceinline__ int k_row_for(int i) {
  return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// Load 8 consecutive elements starting at `src` (element index `first` of a
// row of `limit` valid elements); elements at or past `limit` read as zero.
template <typename T>
__device__ __forceinline__ u32x4 load8_guarded(const T* src, int64_t first,
                                               int64_t limit) {
  if (first + 8 <= limit) return load16(src);
  typedef typename Vec8<T>::type V;
  V v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (first + e < limit) ? src[e] : (T)0.0f;
  return __builtin_bit_cast(u32x4, v);
}

// Buffer resource over the bytes from `base` on (raw, unchecked range), and
// a 16-byte load at a 32-bit byte offset from it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}

// Direct-to-LDS tile ring (scaled-key path): tile rows of 128 bytes, chunk c
// (8 elements) of row r in 16-byte slot c ^ ring_swizzle(r).  The swizzle
// keeps the operand reads of every 8- and 16-lane group on distinct slots
// (rows 0..15 in the order the score and PV reads visit them).
__device__ __forceinline__ int ring_swizzle(int r) {
  return ((r >> 1) & 1) | (((r ^ (r >> 2)) & 1) << 1) | (((r ^ (r >> 3)) & 1) << 2);
}
// Chunk swizzle of a key-major V tile in LDS: logical chunk c of key row r
// sits in slot c ^ v_ring_swizzle(r).  A transposed read of a 16-lane group
// covers four consecutive key rows and two adjacent chunks of each; the
// swizzle puts those eight chunks in eight distinct slots (distinct banks;
// measured: no bank conflicts, where 160-byte padded rows without the
// swizzle conflicted).
__device__ __forceinline__ int v_ring_swizzle(int r) { return 2 * (r & 3); }
// Byte offset, inside a V tile, of this lane's first transposed read of the
// PV operand for head_dim block d (add 16 u * 128 for keys 16 u .., and 512
// for the second read, four key rows further): key row
// 8 (lane / 32) + (lane / 4) % 4, head_dim column 32 d + 16 ((lane / 16) % 2)
// + 4 (lane % 4).
__device__ __forceinline__ uint32_t v_tr_offset(int lane, int d) {
  const int row = 8 * (lane >> 5) + ((lane >> 2) & 3);
  const int col = 32 * d + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int chunk = (2 * col) >> 4;
  return (uint32_t)(row * 128 + ((chunk ^ v_ring_swizzle(row)) << 4) + ((2 * col) & 15));
}
// Byte offset of chunk c8 / 8 of key row `row` in a V tile.
__device__ __forceinline__ uint32_t v_store_offset(int row, int c8) {
  return (uint32_t)(row * 128 + (((c8 >> 3) ^ v_ring_swizzle(row)) << 4));
}

// ds_read_b64_tr_b16: lane l of each 16-lane group receives element l % 4 of
// the 8 bytes addressed by lanes 4 e + l / 4 of its group, e = 0..3.  When
// lane j of the group addresses key row kb + j / 4 at head_dim column
// d0 + 4 (j % 4), lane l therefore receives V[kb .. kb + 3][d0 + l]: four
// consecutive keys of one head_dim column, the transposed operand.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  auto q = (__attribute__((address_space(3))) v4s*)(const_cast<void*>(p));
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(q));
}
// The eight keys of a PV A-operand fragment: two transposed reads, four key
// rows apart.
template <typename V8>
__device__ __forceinline__ V8 lds_read_tr16_pair(const void* lo, const void* hi) {
  const u32x2 a = lds_read_tr16(lo);
  const u32x2 b = lds_read_tr16(hi);
  return __builtin_bit_cast(V8, u32x4{a[0], a[1], b[0], b[1]});
}

// One 16-byte direct-to-LDS load per lane: lane i's bytes from
// base + offset land at LDS byte lds + 16 i (base and lds wave-uniform,
// moved to scalar registers here).  Written as assembly so the compiler does
// not treat it as an LDS write (it would wait for it before every LDS read);
// the tile loop waits for it explicitly.
__device__ __forceinline__ void dma16(const void* base, uint32_t offset, uint32_t lds) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t sbase = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(offset), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// s_waitcnt with at most n vector-memory operations outstanding (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left open).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Cross-half reductions: lanes l and l^32 hold the two key halves of one
// query row.  v_permlane32_swap exchanges the halves of two registers; the max
// (or sum) of the two results is the cross-half value in every lane, whichever
// half each register received.
// The max is one v_max_f32 written as assembly: through fmaxf the compiler
// first quiets both swapped values (two more v_max_f32), since it cannot see
// that a lane move keeps them canonical.
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(r[0])), "v"(__uint_as_float(r[1])));
  return m;
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// PATH: kPathAll runs every workgroup on the shifted path (no scaled keys);
// with the scaled keys, kPathScaled runs the workgroups that qualify for the
// scaled-key path and kPathShifted the others, as two launches over the same
// grid (each kernel keeps one copy of the tile loop: both copies in one
// kernel raised its register use past the 4-wave-per-SIMD budget).
constexpr int kPathAll = 0;
constexpr int kPathScaled = 1;
constexpr int kPathShifted = 2;

// Wavefronts per SIMD the kernel must keep (the second __launch_bounds__
// argument; 4 waves per SIMD means <= 128 VGPRs): the double-buffered 8-wave,
// 32-rows-per-wave instantiations (the long-sequence launch), and the 4-wave,
// 32-rows-per-wave instantiations of the shifted paths (128-row tiles; four
// workgroups per CU instead of three).  Their scaled-key twins and the
// single-buffered 8-wave ones would spill under it and are left unbounded.
template <typename T, int QG, int STAGES, int WAVES, int PATH>
constexpr int attn_min_waves_per_simd() {
  return (QG == 1 && ((WAVES == 8 && STAGES == 2) || (WAVES == 4 && PATH != kPathScaled))) ? 4 : 1;
}

template <typename T, int QG, int STAGES, int WAVES, int PATH>
__global__ __launch_bounds__(WAVES * 64, (attn_min_waves_per_simd<T, QG, STAGES, WAVES, PATH>())) void attn_fwd_kernel(AttnParams p) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec8<T>::half_type V4;
  typedef typename Vec8<T>::pair_type V2;
  constexpr int BM = WAVES * 32 * QG;
  constexpr int NT = WAVES * 64;             // threads
  constexpr int CPT = (kBlockN * 8) / NT;    // 16-byte chunks of a tile per thread

  // The scaled-key path of the 8-wave launches (32 or 64 rows per wave)
  // stages K and V by direct-to-LDS loads into a ring of three tiles (two
  // in flight while one is read); the other kernels use padded double
  // buffers filled through registers.
  constexpr bool kDma = PATH == kPathScaled && STAGES == 2 && WAVES == 8;
  constexpr int kRing = 3;
  constexpr int kRingStage = 2 * kBlockN * kHeadDim * (int)sizeof(T);  // K then V, 16 KiB
  __shared__ __attribute__((aligned(16))) T k_lds[kDma ? 1 : STAGES][kDma ? 1 : kBlockN][kDma ? 8 : kKRow];
  __shared__ __attribute__((aligned(16))) unsigned char v_lds[kDma ? 1 : STAGES][kDma ? 16 : kVTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char ring[kDma ? kRing * kRingStage : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave index in a scalar register on the scaled-key path, so its per-tile
  // wave conditions are scalar compares; the other paths keep it in a VGPR
  // (a scalar copy there raised their register use with no measured gain).
  const int wave = (PATH == kPathScaled) ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  int bh, q_tile;
  tile_of(p, bh, q_tile);
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const int S = p.seq_len;

  const T* qbase = static_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh;
  const T* kbase = static_cast<const T*>(p.k) + b * p.k_sb + h * p.k_sh;
  const T* vbase = static_cast<const T*>(p.v) + b * p.v_sb + h * p.v_sh;
  T* obase = static_cast<T*>(p.o) + b * p.o_sb + (int64_t)h * kHeadDim;

  const int q0 = q_tile * BM;
  const int wq0 = q0 + wave * 32 * QG;                 // first query of this wave
  // Last valid query of this wave; -1 when the wave has none (skips every tile).
  const int wq_last = (wq0 < S) ? min(wq0 + 32 * QG, S) - 1 : -1;
  const int key_end = min(q0 + BM, S);
  const int n_tiles = (key_end + kBlockN - 1) / kBlockN;

  // ---- scaled-key path: taken by the block of kScaledKeyRows query rows
  // that holds this workgroup's rows when c max|q| max|k| <= scaled_key_bound
  // over the block's rows and the keys they read (and both operands fit fp16
  // comfortably).  Every wave forms the same exact maxima, so the workgroup
  // returns as a whole or not at all, before it loads anything else.
  constexpr bool SCALED = PATH == kPathScaled;
  if constexpr (PATH != kPathAll) {  // the host launches these only with the tables
    // The block's rows read keys [0, its end): key blocks 0 .. blk.
    const int blk = q0 / kScaledKeyRows;
    typedef const __attribute__((address_space(1))) float* TableFloats;
    TableFloats kblock = (TableFloats)p.kblock + (int64_t)bh * p.num_row_blocks;
    const float qmax = ((TableFloats)p.qblock)[(int64_t)bh * p.num_row_blocks + blk];
    float kmax = 0.0f;
    for (int t = lane; t <= blk; t += 64) kmax = fmaxf(kmax, kblock[t]);
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, offset));
    const float c = p.c;
    const bool scaled = kmax * c <= kScaledKeyMaxNorm && qmax <= kScaledKeyMaxNorm &&
                        qmax * c * kmax <= scaled_key_bound<T>();
    if (scaled != SCALED) return;
    __builtin_amdgcn_sched_barrier(0);  // keep the loads below after the exit
  }

  // ---- Q^T operands (B operand of S^T = K Q^T), kept in registers; the
  // sign fold of a non-positive scale is skipped (uniform branch) otherwise.
  const bool q_transform = p.q_and != 0xffffffffu || p.q_xor != 0u;
  V8 qop[QG][4];
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    const int qi = wq0 + g * 32 + l32;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (qi < S) raw = load16(qbase + (int64_t)qi * p.q_ss + 16 * s + 8 * half);
      if (q_transform) raw = (raw & p.q_and) ^ p.q_xor;
      qop[g][s] = __builtin_bit_cast(V8, raw);
    }
  }
  // c * |q| per row: the score bound of a tile is qnc * (its largest |k|).
  float qnc[QG];
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (float)qop[g][s][e];
        ss = fmaf(x, x, ss);
      }
    qnc[g] = sqrtf(half_swap_sum(ss)) * p.c;
  }

  // Key source: the keys as given, or the pre-pass's fp16 keys times c on the
  // scaled-key path.
  const T* kb = SCALED ? reinterpret_cast<const T*>(p.kc) + (int64_t)bh * p.key_tiles * kBlockN * kHeadDim
                       : kbase;
  const int64_t kss = SCALED ? (int64_t)kHeadDim : p.k_ss;

  const int a_row = k_row_for(l32);

  // ---- cooperative tile loader: CPT x 16 B of K and of V per thread (both
  // key-major: 64 key rows of 128 bytes).  Full tiles are read as buffer
  // loads: a tile base in scalar registers plus this thread's 32-bit byte
  // offset inside the tile (the host keeps 64 rows of K and of V within
  // 2^31 bytes).
  uint32_t k_off[CPT], v_off[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int chunk = tid + NT * i;
    const int row = chunk >> 3;
    const int c8 = (chunk & 7) * 8;
    k_off[i] = (uint32_t)(((int64_t)row * kss + c8) * (int64_t)sizeof(T));
    v_off[i] = (uint32_t)(((int64_t)row * p.v_ss + c8) * (int64_t)sizeof(T));
  }
  u32x4 k_pref[CPT], v_pref[CPT];
  auto load_tile = [&](int tile) {
    const int k0 = tile * kBlockN;
    if (k0 + kBlockN <= S) {  // tile-uniform: every key of the tile exists
      const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kb + (int64_t)k0 * kss);
      const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vbase + (int64_t)k0 * p.v_ss);
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        k_pref[i] = buffer_load16(kr, k_off[i]);
        v_pref[i] = buffer_load16(vr, v_off[i]);
      }
    } else {
      const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kb + (int64_t)k0 * kss);
      const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vbase + (int64_t)k0 * p.v_ss);
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int row = (tid + NT * i) >> 3;
        u32x4 kraw = {0u, 0u, 0u, 0u}, vraw = {0u, 0u, 0u, 0u};
        if (k0 + row < S) {  // rows past the sequence stay zero
          kraw = buffer_load16(kr, k_off[i]);
          vraw = buffer_load16(vr, v_off[i]);
        }
        k_pref[i] = kraw;
        v_pref[i] = vraw;
      }
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int chunk = tid + NT * i;
      const int row = chunk >> 3;
      const int c8 = (chunk & 7) * 8;
      *reinterpret_cast<u32x4*>(&k_lds[stage][row][c8]) = k_pref[i];
      *reinterpret_cast<u32x4*>(&v_lds[stage][v_store_offset(row, c8)]) = v_pref[i];
    }
  };

  // Ring loader (kDma): the 16 bytes of lane l of wave w land at tile row
  // dr = 8 w + l / 8, slot l % 8, so they carry logical chunk
  // (l % 8) ^ ring_swizzle(dr) of key row dr of K and
  // (l % 8) ^ v_ring_swizzle(dr) of key row dr of V.
  const int dr = wave * 8 + (lane >> 3);
  const int dc = (lane & 7) ^ ring_swizzle(dr);
  const int dcv = (lane & 7) ^ v_ring_swizzle(dr);
  const uint32_t k_ring_off = (uint32_t)(((int64_t)dr * kss + 8 * dc) * (int64_t)sizeof(T));
  const uint32_t v_ring_off = (uint32_t)(((int64_t)dr * p.v_ss + 8 * dcv) * (int64_t)sizeof(T));
  const uint32_t ring_lds =
      (uint32_t)(uintptr_t)((__attribute__((address_space(3))) unsigned char*)ring);
  // Fills ring stage `stage` with tile `tile`; returns whether it issued
  // direct-to-LDS loads (two per lane).  A tile that reaches past the
  // sequence goes through registers, zero-filled, into the same slots.
  auto fill_ring = [&](int tile, int stage) -> bool {
    const int k0 = tile * kBlockN;
    const T* kt = kb + (int64_t)k0 * kss;
    const T* vt = vbase + (int64_t)k0 * p.v_ss;
    const uint32_t dst = ring_lds + stage * kRingStage + wave * 1024;
    if (k0 + kBlockN <= S) {
      dma16(kt, k_ring_off, dst);
      dma16(vt, v_ring_off, dst + kRingStage / 2);
      return true;
    }
    u32x4 kraw = {0u, 0u, 0u, 0u}, vraw = {0u, 0u, 0u, 0u};
    if (k0 + dr < S) {  // rows past the sequence stay zero
      kraw = buffer_load16(tile_rsrc(kt), k_ring_off);
      vraw = buffer_load16(tile_rsrc(vt), v_ring_off);
    }
    unsigned char* slot = ring + stage * kRingStage + wave * 1024 + lane * 16;
    *reinterpret_cast<u32x4*>(slot) = kraw;
    *reinterpret_cast<u32x4*>(slot + kRingStage / 2) = vraw;
    return false;
  };
  // Operand fragments.  K: rows 32 t + a_row, chunk 2 s + half (one 16-byte
  // read).  V: the PV A operand (head_dim rows 32 d + l32, keys 16 u + 8 half
  // .. + 7) from the key-major V tile by two transposed reads (v_tr_offset).
  // The in-tile byte offsets are kept for the whole loop, so every operand
  // read is one register plus an immediate (stage, subtile, second read).
  uint32_t k_ring_at[4], v_at[2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    k_ring_at[i] = (uint32_t)(a_row * 128 + (((2 * i + half) ^ ring_swizzle(a_row)) << 4));
#pragma unroll
  for (int d = 0; d < 2; ++d) v_at[d] = v_tr_offset(lane, d);
  auto k_frag = [&](int stage, int t, int s) -> V8 {
    if constexpr (kDma)
      return *reinterpret_cast<const V8*>(ring + stage * kRingStage + 32 * t * 128 + k_ring_at[s]);
    else
      return *reinterpret_cast<const V8*>(&k_lds[stage][32 * t + a_row][16 * s + 8 * half]);
  };
  auto v_frag = [&](int stage, int d, int u) -> V8 {
    const unsigned char* tile = kDma ? ring + stage * kRingStage + kRingStage / 2 : &v_lds[stage][0];
    const unsigned char* at = tile + 16 * u * 128 + v_at[d];
    return lds_read_tr16_pair<V8>(at, at + 4 * 128);
  };

  // ---- running state (lane-local: query l32 of each group).
  f32x16 acc[QG][2];
  float m_run[QG], l_run[QG];
  // Scaled-key path: the row sums run on the matrix cores.  Read as the B
  // operand of a 16x16x32 product, a P^T fragment holds, in lane 16 kg + n,
  // the 8 probabilities of query n + 16 (kg % 2) for keys 8 (kg / 2) .. of
  // its 16-key slice; A = `ones` (row 0 ones for kg even, row 1 for kg odd)
  // makes C[0][n] and C[1][n] the slice sums of queries n and n + 16, which
  // accumulate over the slices into lanes 0..15 of rsum.
  f32x4 rsum[QG];
  V8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)0.0f;
  if constexpr (SCALED) {
    const bool one_lane = (lane == 0 || lane == 32 || lane == 17 || lane == 49);
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = one_lane ? (T)1.0f : (T)0.0f;
  }
#pragma unroll
  for (int g = 0; g < QG; ++g) rsum[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][d][r] = 0.0f;
  }
  const float c = p.c;
  // The key-norm table exists only with the preparation pass, whose blocks
  // run kPathScaled or kPathShifted; the host sets knorm and kc together, so
  // a kPathAll launch never has it and drops the per-tile bound check.
  const bool bounded = PATH != kPathAll && p.knorm != nullptr;  // uniform
  // Global address space spelled out: the table entry of the next tile is
  // then a scalar load (uniform address, read-only).  Left to inference the
  // compiler emitted a flat load here, whose completion every later LDS wait
  // of the loop also waited for (6% slower on the long-sequence chunk).
  typedef const __attribute__((address_space(1))) float* GlobalFloats;
  GlobalFloats knorm = bounded ? (GlobalFloats)p.knorm + (int64_t)bh * p.key_tiles : nullptr;

  if constexpr (SCALED && !std::is_same<T, f16>::value) {
    // Q in fp16 (kept in the same registers): exact for |q| <= 4096 down to
    // the fp16 normal range.
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f16x8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (f16)(float)qop[g][s][e];
        qop[g][s] = __builtin_bit_cast(V8, h);
      }
  }

  bool ring_next = false;  // the next ring tile was issued as direct-to-LDS loads
  if constexpr (kDma) {
    fill_ring(0, 0);
    ring_next = n_tiles > 1 && fill_ring(1, 1);
  } else {
    load_tile(0);
    store_tile(0);
    __syncthreads();
  }
  float kn_next = bounded ? knorm[0] : 0.0f;

  // Tile loop.  On the scaled-key path it runs two tiles per iteration with
  // two LDS stages, or three with the ring (the inner loop is unrolled), so
  // each copy's stage is a constant and the LDS operand reads and stores use
  // immediate offsets; the other paths keep one tile per iteration (two
  // copies of their larger state spill).
  constexpr int kStep = kDma ? kRing : ((STAGES == 2 && PATH == kPathScaled) ? 2 : 1);
  for (int j0 = 0; j0 < n_tiles; j0 += kStep) {
#pragma unroll
    for (int u = 0; u < kStep; ++u) {
      const int j = j0 + u;
      if (kStep > 1 && j >= n_tiles) break;
      const int stage = (kStep > 1) ? u : ((STAGES == 2) ? (j & 1) : 0);
      const bool has_next = j + 1 < n_tiles;
      if constexpr (kDma) {
        // Tile j has landed once only the next tile's loads (if it was
        // issued to the ring) remain; the barrier then also retires every
        // wave's reads of the stage refilled below (tile j - 1's).
        if (ring_next)
          wait_vmcnt<2>();
        else
          wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xc07f & ~(0xF << 8));  // lgkmcnt(0): register-path stores
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // From here on ring_next describes tile j + 2, the next wait's.
        ring_next = j + 2 < n_tiles && fill_ring(j + 2, (u + 2) % kRing);
      } else {
        if (has_next) load_tile(j + 1);
      }
      const float kn = kn_next;
      if (bounded && has_next) kn_next = knorm[j + 1];
      const int k0 = j * kBlockN;

      if (k0 <= wq_last) {  // wave-uniform: skip tiles entirely above this wave's rows
        // S^T[key][query] for 2 subtiles of 32 keys; on the scaled-key path
        // both operands hold fp16 bits and the result is c q.k.
        f32x16 sacc[QG][2];
#pragma unroll
        for (int g = 0; g < QG; ++g)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[g][t][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const V8 a = k_frag(stage, t, s);
#pragma unroll
            for (int g = 0; g < QG; ++g)
              if constexpr (SCALED)
                sacc[g][t] = mfma32(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, qop[g][s]),
                                    sacc[g][t]);
              else
                sacc[g][t] = mfma32(a, qop[g][s], sacc[g][t]);
          }
        }

        // Scaled-key path: the wave's exponential phase runs at raised
        // priority, so among the waves of a SIMD the one converting scores
        // to P issues first and the next MFMAs find their operands sooner
        // (priority during the MFMA phases instead measured 3.8% slower).
        if constexpr (SCALED) __builtin_amdgcn_s_setprio(1);
        // Causal mask: only tiles that reach past this wave's first query.
        // Element r of subtile t is key k0 + 32 t + 16 (r / 8) + 8 half + r % 8;
        // it is masked when that exceeds the lane's query, i.e. when the
        // constant 32 t + 16 (r / 8) + r % 8 exceeds qi - k0 - 8 half (one
        // compare against an immediate per element).
        if (k0 + kBlockN - 1 > wq0) {
#pragma unroll
          for (int g = 0; g < QG; ++g) {
            const int lim = wq0 + 32 * g + l32 - k0 - 8 * half;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; ++r)
                if (32 * t + 16 * (r >> 3) + (r & 7) > lim) sacc[g][t][r] = -INFINITY;
          }
        }

        V8 pb[QG][4];
#pragma unroll
        for (int g = 0; g < QG; ++g) {
          float lsum = l_run[g];
          if constexpr (SCALED) {
            // P = exp2(c q.k): every score lies within the bound, no shift.
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int t = u >> 1;
              const int rb = (u & 1) * 8;
              V8 pk;
#pragma unroll
              for (int e = 0; e < 8; e += 2) {
                V2 pair;
                pair[0] = (T)__builtin_amdgcn_exp2f(sacc[g][t][rb + e]);
                pair[1] = (T)__builtin_amdgcn_exp2f(sacc[g][t][rb + e + 1]);
                pk[e] = pair[0];
                pk[e + 1] = pair[1];
              }
              pb[g][u] = pk;
              rsum[g] = mfma16(ones, pk, rsum[g]);
            }
          } else {
            // Rows whose bound keeps every probability below 2^safe_exponent skip the
            // tile maximum.  Rows that need it move their shift up to the tile
            // maximum only when that exceeds it by more than kLazyShift (log2
            // units), so the O rescale is rare.  Both decisions are per row, so
            // results do not depend on the launch.
            const bool need = !bounded || qnc[g] * kn - m_run[g] * c > safe_exponent<T>();
            if (__any(need)) {
              // From -inf the chain compiles to v_max3 only (starting from an
              // element, the compiler quiets the first two operands first).
              float mx = -INFINITY;
#pragma unroll
              for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[g][t][r]);
              mx = half_swap_max(mx);
              const bool grow = need && (mx - m_run[g]) * c > kLazyShift;
              if (__any(grow)) {
                const float m_new = grow ? mx : m_run[g];
                const float alpha = exp2f((m_run[g] - m_new) * c);
                lsum *= alpha;
#pragma unroll
                for (int d = 0; d < 2; ++d)
#pragma unroll
                  for (int r = 0; r < 16; ++r) acc[g][d][r] *= alpha;
                m_run[g] = m_new;
              }
            }
            const float mc = m_run[g] * c;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int t = u >> 1;
              const int rb = (u & 1) * 8;
              V8 pk;
#pragma unroll
              for (int e = 0; e < 8; e += 2) {
                V2 pair;
                pair[0] = (T)__builtin_amdgcn_exp2f(fmaf(sacc[g][t][rb + e], c, -mc));
                pair[1] = (T)__builtin_amdgcn_exp2f(fmaf(sacc[g][t][rb + e + 1], c, -mc));
                lsum = dot2_sum(pair, lsum);
                pk[e] = pair[0];
                pk[e + 1] = pair[1];
              }
              pb[g][u] = pk;
            }
          }
          l_run[g] = lsum;
        }

        if constexpr (SCALED) __builtin_amdgcn_s_setprio(0);
        // O^T[dh][query] += V^T[dh][keys] P^T[keys][query]
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const V8 a = v_frag(stage, d, u);
#pragma unroll
            for (int g = 0; g < QG; ++g) acc[g][d] = mfma32(a, pb[g][u], acc[g][d]);
          }
        }
      }

      if (!kDma && has_next) {
        if (STAGES == 1) __syncthreads();  // everyone done reading the single buffer
        store_tile(STAGES == 2 ? ((j + 1) & 1) : 0);
        __syncthreads();
      }
    }
  }

  // ---- normalize and write [B, S, H*64].
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    const int qi = wq0 + 32 * g + l32;
    float l_tot;
    if constexpr (SCALED) {
      const float lo = __shfl(rsum[g][0], l32 & 15);
      const float hi = __shfl(rsum[g][1], l32 & 15);
      l_tot = l32 < 16 ? lo : hi;
    } else {
      l_tot = half_swap_sum(l_run[g]);
    }
    if (qi >= S) continue;
    const float inv = 1.0f / l_tot;
    T* orow = obase + (int64_t)qi * p.o_ss;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        V4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = (T)(acc[g][d][4 * a4 + e] * inv);
        *reinterpret_cast<V4*>(orow + 32 * d + 8 * a4 + 4 * half) = out;
      }
  }
}

}  // namespace
}  // namespace sah
