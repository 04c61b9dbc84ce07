// Causal attention forward, head_dim 64, for gfx950 (CDNA4, wave64, MFMA).
//
// Same contract as the reference's streaming kernel
// (solution/shape14/triton_streaming_dh64.py:69-190): softmax(Q K^T * scale +
// causal mask) V with an online (running max / running sum) softmax in fp32,
// P rounded to the input dtype before the PV product, the S x S score matrix
// never materialized, and the result written straight into [B, S, H*64].
//
// MI355X formulation (not a translation of the Triton program):
//  * Each wavefront owns 32*QG query rows; a workgroup is 4 or 8 waves
//    sharing K and V tiles of 64 keys staged in LDS (double buffered).
//  * The score tile is computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_{bf16,f16}: the B operand (Q^T) stays in registers for
//    the whole kernel and every lane's accumulator column is ONE query row, so
//    the softmax max and sum are in-lane reductions plus one swap between the
//    two half-waves.  All 64 lanes' statistics are lane-local, which also makes
//    the O rescale lane-local.
//  * K rows are read from LDS in an order with index bits 2 and 3 exchanged.
//    That makes a lane's S^T registers cover 8 consecutive keys per half-wave,
//    which is exactly the k-slice the next MFMA needs, so P^T goes from the
//    score accumulator to the B operand of O^T = V^T P^T without any lane
//    exchange (one packed fp32->16-bit conversion per pair).
//  * V is read key-major as the caller hands it over ([B, H, S, 64], any key
//    stride, e.g. the packed QKV view) and staged in LDS like K; the PV
//    A operand (V^T rows) comes out of LDS through ds_read_b64_tr_b16, the
//    gfx950 transposed read, so no V^T copy is made.  A caller's
//    seq-contiguous V^T is copied key-major first (transpose_vt_kernel).
//    On the scaled-key path the 8-wave launch stages K and V by
//    direct-to-LDS loads into a three-tile ring.
//  * The kernel template is in attention_kernel.hpp; this file instantiates
//    the plain path and holds the host code, attention_scaled.hip the
//    scaled-key path.
//  * Lazy softmax shift (plain kernel): a row's shift m rises to the tile
//    maximum only when that exceeds m by more than 2^8 in probability, so
//    the O rescale by exp(m_old - m_new) is rare and is skipped when no row
//    of the wave moved (rows that did not move scale by exactly 1).  Softmax
//    is invariant to the shift; only where P is rounded differs.
//  * Grid: one workgroup per (batch*head, query tile).  The hardware deals
//    workgroup ids round-robin over the 8 XCDs; ids are remapped so that all
//    tiles of a head land on one XCD (its L2 keeps the head's K and V) and
//    each XCD issues its heads in groups: within a group, longest (last)
//    query tiles first across the group's heads.  The host sizes the groups
//    to about two rounds of resident workgroups (see head_group_for), which
//    balances the causal triangle when a head has few query tiles.

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "attention_kernel.hpp"

namespace sah {

// The scaled-key-path instantiations of attn_fwd_kernel live in
// attention_scaled.hip; this returns one of them (bf16 or fp16, 4 or 8
// waves, 32 or 64 query rows per wave, 1 or 2 LDS stages).
const void* scaled_path_kernel(bool bf16_type, int waves, int qg, int num_stages);

namespace {

// Software-pipelined variant (num_stages == 3): the score MFMAs of the next
// tile run while the current tile's exponentials are on the VALU, and the PV
// MFMAs of the current tile run while the next tile's row maximum is formed.
// Measured on gfx950, VALU work hides under MFMA execution far better when the
// same wavefront interleaves the two than when another wavefront on the SIMD
// supplies it, so the overlap is built into each wavefront's instruction
// stream rather than left to occupancy.
//
// Iteration j of a wave (tiles 0..w_tiles-1), with S^T(j) already scaled and
// shifted in registers (s * c - m_j * c, masked entries -inf):
//   phase A: MFMA S^T(j+1) = K(j+1) Q^T       ||  P(j) = exp2(S^T(j)), pack,
//                                                  row sum
//   phase B: MFMA O^T += V^T(j) P^T(j)          ||  mask S^T(j+1) if diagonal,
//                                                  row max, m_{j+1}, shift
//                                                  S^T(j+1) by m_{j+1}
//   then, only if some row raised its maximum, O and l are rescaled by
//   exp2((m_j - m_{j+1}) c) (after PV(j), which was computed at m_j).
// Two score buffers alternate (the loop is unrolled by two so that no
// register copies are needed).  The workgroup-level loop keeps K(j+1) and
// V(j) in LDS during iteration j (two stages each) and prefetches K(j+2) and
// V(j+1) through registers, with one barrier per iteration.
//
// QG query groups of 32 rows per wave would share every K and V^T fragment
// read from LDS; only QG = 1 is launched: with two groups the double-buffered
// scores need more registers than two waves per SIMD allow, and at one wave
// per SIMD the kernel measured slower than the plain 64-row kernel.
template <typename T, int QG>
__global__ __launch_bounds__(kThreads, QG == 1 ? 2 : 1) void attn_fwd_pipelined_kernel(AttnParams p) {
  typedef typename Vec8<T>::type V8;
  typedef typename Vec8<T>::half_type V4;
  typedef typename Vec8<T>::pair_type V2;
  constexpr int BM = kWaves * 32 * QG;

  __shared__ __attribute__((aligned(16))) T k_lds[2][kBlockN][kKRow];
  __shared__ __attribute__((aligned(16))) unsigned char v_lds[2][kVTileBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
  const int wq0 = q0 + wave * 32 * QG;
  const int wq_last = (wq0 < S) ? min(wq0 + 32 * QG, S) - 1 : -1;
  const int key_end = min(q0 + BM, S);
  const int n_tiles = (key_end + kBlockN - 1) / kBlockN;
  // Tiles this wave computes: [0, w_tiles); tiles from j_mask on need the mask.
  const int w_tiles = wq_last < 0 ? 0 : wq_last / kBlockN + 1;
  const int j_mask = wq0 / kBlockN;

  const bool q_transform = p.q_and != 0xffffffffu || p.q_xor != 0u;
  V8 qop[QG][4];
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    const int qi = wq0 + 32 * g + l32;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (qi < S) raw = load16(qbase + (int64_t)qi * p.q_ss + 16 * s + 8 * half);
      if (q_transform) raw = (raw & p.q_and) ^ p.q_xor;
      qop[g][s] = __builtin_bit_cast(V8, raw);
    }
  }

  // ---- cooperative loads: 2 x 16 B of a K tile / a V tile per thread (both
  // key-major).
  u32x4 k_pref[2], v_pref[2];
  auto load_k = [&](int tile) {
    const int k0 = tile * kBlockN;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int chunk = tid + kThreads * i;
      const int key = k0 + (chunk >> 3);
      const int c8 = (chunk & 7) * 8;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (key < S) raw = load16(kbase + (int64_t)key * p.k_ss + c8);
      k_pref[i] = raw;
    }
  };
  auto load_v = [&](int tile) {
    const int k0 = tile * kBlockN;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int chunk = tid + kThreads * i;
      const int key = k0 + (chunk >> 3);
      const int c8 = (chunk & 7) * 8;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (key < S) raw = load16(vbase + (int64_t)key * p.v_ss + c8);
      v_pref[i] = raw;
    }
  };
  auto store_k = [&](int tile) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int chunk = tid + kThreads * i;
      *reinterpret_cast<u32x4*>(&k_lds[tile & 1][chunk >> 3][(chunk & 7) * 8]) = k_pref[i];
    }
  };
  auto store_v = [&](int tile) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int chunk = tid + kThreads * i;
      *reinterpret_cast<u32x4*>(&v_lds[tile & 1][v_store_offset(chunk >> 3, (chunk & 7) * 8)]) = v_pref[i];
    }
  };

  f32x16 acc[QG][2];
#pragma unroll
  for (int g = 0; g < QG; ++g)
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][d][r] = 0.0f;
  float m_run[QG], l_run[QG];
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
  }
  const float c = p.c;
  const int a_row = k_row_for(l32);
  // Transposed V reads (see attn_fwd_kernel): in-tile byte offsets.
  const uint32_t v_at[2] = {v_tr_offset(lane, 0), v_tr_offset(lane, 1)};

  // S^T(j) = K(j) Q^T (raw scores) for every group; each K fragment feeds QG MFMAs.
  auto scores = [&](int j, f32x16 (*s)[2]) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const V8 ka =
            *reinterpret_cast<const V8*>(&k_lds[j & 1][32 * t + a_row][16 * u + 8 * half]);
#pragma unroll
        for (int g = 0; g < QG; ++g)
          s[g][t] = mfma32(ka, qop[g][u], u == 0 ? f32x16{} : s[g][t]);
      }
  };
  // Keys above the lane's query row of group g -> -inf.
  auto mask = [&](f32x16* s, int g, int k0) {
    const int qi = wq0 + 32 * g + l32;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * t + 16 * (r >> 3) + 8 * half + (r & 7);
        if (key > qi) s[t][r] = -INFINITY;
      }
  };
  // Row maximum of raw scores (four independent partial maxima), new running
  // max, and the in-place shift s -> s * c - m_new * c.  Returns
  // exp2((m_old - m_new) c).
  auto shift = [&](f32x16* s, int g) -> float {
    float pm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = q >> 1, rb = (q & 1) * 8;
      pm[q] = s[t][rb];
#pragma unroll
      for (int r = 1; r < 8; ++r) pm[q] = fmaxf(pm[q], s[t][rb + r]);
    }
    const float mx = half_swap_max(fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3])));
    const float m_new = fmaxf(m_run[g], mx);
    const float alpha = __builtin_amdgcn_exp2f((m_run[g] - m_new) * c);
    m_run[g] = m_new;
    const float mc = m_new * c;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = fmaf(s[t][r], c, -mc);
    return alpha;
  };
  // P(j) = exp2 of the shifted scores, rounded to T and packed as the B
  // operand of the PV MFMA; returns the row sum of the rounded values.
  auto exponentiate = [&](const f32x16* s, V8* pb) -> float {
    float lsum = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = u >> 1;
      const int rb = (u & 1) * 8;
      V8 pk;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        V2 pair;
        pair[0] = (T)__builtin_amdgcn_exp2f(s[t][rb + e]);
        pair[1] = (T)__builtin_amdgcn_exp2f(s[t][rb + e + 1]);
        lsum = dot2_sum(pair, lsum);
        pk[e] = pair[0];
        pk[e + 1] = pair[1];
      }
      pb[u] = pk;
    }
    return lsum;
  };
  // O^T += V^T(j) P^T(j) for every group; each V^T fragment (read transposed
  // from the key-major V tile) feeds QG MFMAs.
  auto pv = [&](int j, V8 (*pb)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const V8 va =
            lds_read_tr16_pair<V8>(&v_lds[j & 1][16 * u * 128 + v_at[d]],
                                   &v_lds[j & 1][16 * u * 128 + 512 + v_at[d]]);
#pragma unroll
        for (int g = 0; g < QG; ++g) acc[g][d] = mfma32(va, pb[g][u], acc[g][d]);
      }
  };
  auto rescale = [&](float alpha, int g) {
    l_run[g] *= alpha;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[g][d][r] *= alpha;
    }
  };

  // Workgroup-level end of iteration j: K(j+2) and V(j+1) go from the
  // prefetch registers into the stages that held K(j) and V(j-1).
  auto advance = [&](int j) {
    const bool v_next = j + 1 < n_tiles;
    if (j + 2 < n_tiles) store_k(j + 2);
    if (v_next) {
      store_v(j + 1);
      __syncthreads();
    }
  };
  auto prefetch = [&](int j) {
    if (j + 2 < n_tiles) load_k(j + 2);
    if (j + 1 < n_tiles) load_v(j + 1);
  };
  // Steady-state iteration (tiles j and j+1 both unmasked for every wave):
  // no branch between the MFMA groups and the VALU work they overlap.
  auto steady = [&](int j, f32x16 (*cur)[2], f32x16 (*nxt)[2]) {
    prefetch(j);
    V8 pb[QG][4];
    scores(j + 1, nxt);
#pragma unroll
    for (int g = 0; g < QG; ++g) l_run[g] += exponentiate(cur[g], pb[g]);
    pv(j, pb);
    float alpha[QG];
#pragma unroll
    for (int g = 0; g < QG; ++g) alpha[g] = shift(nxt[g], g);
#pragma unroll
    for (int g = 0; g < QG; ++g) rescale(alpha[g], g);
    advance(j);
  };

  // ---- prologue: K(0), K(1), V(0) in LDS; S^T(0) shifted.
  load_k(0);
  store_k(0);
  if (n_tiles > 1) load_k(1);
  load_v(0);
  if (n_tiles > 1) store_k(1);
  store_v(0);
  __syncthreads();

  // Every wave forms S^T(0), also one without rows (zero queries): the
  // steady iterations below run on all four waves.
  f32x16 s_a[QG][2], s_b[QG][2];
  scores(0, s_a);
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    if (j_mask == 0) mask(s_a[g], g, 0);
    (void)shift(s_a[g], g);  // m_run was -inf: nothing to rescale
  }
  // Stage 0 of K is rewritten (with K(2)) at the end of iteration 0: every
  // wave must have read K(0) first.
  __syncthreads();

  // Iterations [0, j_steady) are steady for all four waves: the workgroup's
  // first diagonal tile is q0 / 64 and every wave computes at least up to it.
  // Waves without rows (past the sequence end) run them on zero queries and
  // write nothing.
  const int j_steady = max(q0 / kBlockN - 1, 0);
  int j = 0;
  for (; j + 1 < j_steady; j += 2) {
    steady(j, s_a, s_b);
    steady(j + 1, s_b, s_a);
  }
  if (j < j_steady) {
    steady(j, s_a, s_b);
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int t = 0; t < 2; ++t) s_a[g][t] = s_b[g][t];
    ++j;
  }
  // Remaining iterations (diagonal tiles, ragged end): not pipelined; tile j+1
  // is computed into the same buffer after P(j) has been formed.
  for (; j < n_tiles; ++j) {
    prefetch(j);
    if (j < w_tiles) {
      V8 pb[QG][4];
#pragma unroll
      for (int g = 0; g < QG; ++g) l_run[g] += exponentiate(s_a[g], pb[g]);
      pv(j, pb);
      if (j + 1 < w_tiles) {
        scores(j + 1, s_a);
#pragma unroll
        for (int g = 0; g < QG; ++g) {
          if (j + 1 >= j_mask) mask(s_a[g], g, (j + 1) * kBlockN);
          rescale(shift(s_a[g], g), g);
        }
      }
    }
    advance(j);
  }

#pragma unroll
  for (int g = 0; g < QG; ++g) {
    const int qi = wq0 + 32 * g + l32;
    const float l_tot = half_swap_sum(l_run[g]);
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

// fp32 causal attention (the reference's fp32 portable path, e.g. BASELINE's
// CPU configuration run on the GPU): scores, softmax and PV all in fp32 on
// the VALU, P kept in fp32 (the input dtype, so the reference's rounding of P
// is the identity).  One workgroup per (batch*head, 64-query tile); four
// lanes per query row, each owning 16 of a K/V tile's 64 keys: it forms those
// 16 scores with full 64-element dot products, shares the tile maximum with
// its three partners (two xor shuffles), and accumulates P V over its keys
// into a private 64-wide O row.  The partners' O rows and sums are added once
// at the end.  K and V tiles (64 x 64 fp32, head_dim-contiguous) are staged
// through LDS; every lane of a quarter reads the same K/V row (broadcast).
struct AttnF32Params {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_ss;
  int seq_len;
  int heads;
  float c;  // |scale| log2(e), > 0
  uint32_t q_and, q_xor;
};

__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(AttnF32Params p) {
  constexpr int kRows = 64;
  __shared__ __attribute__((aligned(16))) float k_lds[kBlockN][kHeadDim + 4];
  __shared__ __attribute__((aligned(16))) float v_lds[kBlockN][kHeadDim + 4];
  const int tid = threadIdx.x;
  const int row = tid >> 2;      // query row within the tile
  const int quarter = tid & 3;   // keys [16*quarter, 16*quarter + 16) of each tile
  const int bh = blockIdx.y;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const int S = p.seq_len;
  const int qi = blockIdx.x * kRows + row;
  const float* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)min(qi, S - 1) * p.q_ss;
  const float* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + h * p.v_sh;

  float q[kHeadDim];
#pragma unroll
  for (int d = 0; d < kHeadDim; d += 4) {
    u32x4 raw = load16(qrow + d);
    raw = (raw & p.q_and) ^ p.q_xor;
    const f32x4 f = __builtin_bit_cast(f32x4, raw);
    q[d] = f[0];
    q[d + 1] = f[1];
    q[d + 2] = f[2];
    q[d + 3] = f[3];
  }
  float o[kHeadDim];
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) o[d] = 0.0f;
  float m_run = -INFINITY, l_part = 0.0f;
  const float c = p.c;
  const int last_query = min(blockIdx.x * kRows + kRows, S) - 1;
  const int n_tiles = last_query / kBlockN + 1;

  for (int j = 0; j < n_tiles; ++j) {
    const int k0 = j * kBlockN;
    __syncthreads();  // the previous tile is no longer read
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int chunk = tid + 256 * i;  // 1024 float4 chunks per 64 x 64 tile
      const int key = chunk >> 4;
      const int c4 = (chunk & 15) * 4;
      u32x4 kraw = {0u, 0u, 0u, 0u}, vraw = {0u, 0u, 0u, 0u};
      if (k0 + key < S) {
        kraw = load16(kbase + (int64_t)(k0 + key) * p.k_ss + c4);
        vraw = load16(vbase + (int64_t)(k0 + key) * p.v_ss + c4);
      }
      *reinterpret_cast<u32x4*>(&k_lds[key][c4]) = kraw;
      *reinterpret_cast<u32x4*>(&v_lds[key][c4]) = vraw;
    }
    __syncthreads();
    float sc[16];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = 16 * quarter + e;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < kHeadDim; d += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(&k_lds[key][d]);
        dot = fmaf(q[d], kv[0], dot);
        dot = fmaf(q[d + 1], kv[1], dot);
        dot = fmaf(q[d + 2], kv[2], dot);
        dot = fmaf(q[d + 3], kv[3], dot);
      }
      sc[e] = (k0 + key <= qi) ? dot : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    // Rows past the sequence end (qi >= S) see every key and stay finite.
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int d = 0; d < kHeadDim; ++d) o[d] *= alpha;
    const float mc = m_new * c;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = __builtin_amdgcn_exp2f(fmaf(sc[e], c, -mc));
      l_part += pe;
      const int key = 16 * quarter + e;
#pragma unroll
      for (int d = 0; d < kHeadDim; d += 4) {
        const f32x4 vv = *reinterpret_cast<const f32x4*>(&v_lds[key][d]);
        o[d] = fmaf(pe, vv[0], o[d]);
        o[d + 1] = fmaf(pe, vv[1], o[d + 1]);
        o[d + 2] = fmaf(pe, vv[2], o[d + 2]);
        o[d + 3] = fmaf(pe, vv[3], o[d + 3]);
      }
    }
  }
  // The four partners share m_run, so their partial sums add directly.
  l_part += __shfl_xor(l_part, 1);
  l_part += __shfl_xor(l_part, 2);
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) {
    o[d] += __shfl_xor(o[d], 1);
    o[d] += __shfl_xor(o[d], 2);
  }
  if (qi >= S) return;
  const float inv = 1.0f / l_part;
  float* orow = p.o + b * p.o_sb + (int64_t)qi * p.o_ss + (int64_t)h * kHeadDim + 16 * quarter;
#pragma unroll
  for (int d = 0; d < 16; d += 4) {
    f32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // o[16 * quarter + d + e], with a compile-time index per quarter
      float value = 0.0f;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        if (qq == quarter) value = o[16 * qq + d + e];
      out[e] = value * inv;
    }
    store16(orow + d, __builtin_bit_cast(u32x4, out));
  }
}

// Long-sequence preparation of one block of kScaledKeyRows rows of one
// (batch, head), one launch for the whole attention call:
//  * K: the largest |k| of every 64-key tile (knorm) and of the block
//    (kblock), and every key times c rounded to fp16 (kc, [batch*heads]
//    [key_tiles * 64][64]; rows past the sequence are not written);
//  * Q: the largest |q| of the block (qblock; 0 when zero_q: the queries of a
//    zero scale, which the attention reads as zero).
// Wave w takes tiles 2w and 2w + 1 of the block for K and Q: eight lanes per
// row with 16 bytes each, so reads and fp16 writes are contiguous runs; fp32
// sums of squares.  V is not touched: the attention kernels read it as given.
struct PrepParams {
  const void* k;
  const void* q;
  float* knorm;
  float* kblock;
  float* qblock;
  f16* kc;
  int64_t k_sb, k_sh, k_ss, q_sb, q_sh, q_ss;
  float c;
  int zero_q;
  int heads, seq_len, key_tiles, num_row_blocks;
};

// Sum over the eight lanes of one row (lanes 8 r .. 8 r + 7) in every one of
// them, by DPP moves: neighbour pairs, then pairs of pairs, then the mirrored
// half-row, the order of a butterfly over lane bits 0, 1, 2 (each add is
// commutative, so every lane holds the same bits).
__device__ __forceinline__ float row8_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));  // lane ^ 1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));  // lane ^ 2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false)); // 7 - lane
  return x;
}

// Sum of squares of the eight 16-bit values in `raw`, fp32, in element order.
template <typename T>
__device__ __forceinline__ float chunk_sq(u32x4 raw) {
  float f[8];
  unpack8<T>(raw, f);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = fmaf(f[e], f[e], s);
  return s;
}

// Largest squared row norm of a 64-row tile held as raw[i] = 16 bytes of row
// 8 i + lane / 8 (chunk lane % 8), rows at or past `valid` excluded; the
// result is in every lane.
template <typename T>
__device__ __forceinline__ float tile_max_sq(const u32x4 (&raw)[8], int valid, int lane) {
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float ss2 = row8_sum(chunk_sq<T>(raw[i]));
    if (8 * i + (lane >> 3) < valid) mx = fmaxf(mx, ss2);
  }
#pragma unroll
  for (int offset = 32; offset >= 8; offset >>= 1) mx = fmaxf(mx, __shfl_xor(mx, offset));
  return mx;
}

template <typename T>
__global__ __launch_bounds__(256) void long_prepare_kernel(PrepParams pp) {
  __shared__ float red[2][4];
  const int blk = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / pp.heads;
  const int h = bh - b * pp.heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int kTilesPerBlock = kScaledKeyRows / 64;
  const int t0 = blk * kTilesPerBlock;
  const int t_end = min(t0 + kTilesPerBlock, pp.key_tiles);
  const int S = pp.seq_len;

  const T* kbase = static_cast<const T*>(pp.k) + b * pp.k_sb + h * pp.k_sh;
  const T* qbase = static_cast<const T*>(pp.q) + b * pp.q_sb + h * pp.q_sh;
  f16* kc = pp.kc + (int64_t)bh * pp.key_tiles * 64 * kHeadDim;
  const int c8 = (lane & 7) * 8;

  // Every load of the wave's two K tiles and two Q tiles is issued before
  // any is used: rows past the sequence (and tiles past the block's end)
  // read row S - 1 instead, and are left out of the maxima and the stores.
  u32x4 kraw[2][8], qraw[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min((t0 + 2 * wave + j) * 64 + 8 * i + (lane >> 3), S - 1);
      kraw[j][i] = load16(kbase + (int64_t)row * pp.k_ss + c8);
    }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min((t0 + 2 * wave + j) * 64 + 8 * i + (lane >> 3), S - 1);
      qraw[j][i] = load16(qbase + (int64_t)row * pp.q_ss + c8);
    }

  // A tile past the block's end lies past the sequence (t_end < t0 + 8 only
  // for the last block), so it has no valid rows: it adds 0 to the maxima and
  // writes nothing.
  float kmax = 0.0f, qmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = t0 + 2 * wave + j;
    const int valid = S - t * 64;  // rows of the tile inside the sequence
    // Keys times c, rounded once to fp16 (fp32 product, then fp16).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + (lane >> 3);
      if (r < valid) {
        float f[8];
        unpack8<T>(kraw[j][i], f);
        f16x8 scaled;
#pragma unroll
        for (int e = 0; e < 8; ++e) scaled[e] = (f16)fp32_result<f16>(f[e] * pp.c);
        store16(kc + (int64_t)(t * 64 + r) * kHeadDim + c8, __builtin_bit_cast(u32x4, scaled));
      }
    }
    const float km = tile_max_sq<T>(kraw[j], valid, lane);
    const float qm = tile_max_sq<T>(qraw[j], valid, lane);
    if (lane == 0 && t < t_end) pp.knorm[(int64_t)bh * pp.key_tiles + t] = sqrtf(km);
    kmax = fmaxf(kmax, km);
    qmax = fmaxf(qmax, qm);
  }
  if (lane == 0) {
    red[0][wave] = kmax;
    red[1][wave] = qmax;
  }
  __syncthreads();
  if (tid == 0) {
    const float k4 = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float q4 = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    pp.kblock[(int64_t)bh * pp.num_row_blocks + blk] = sqrtf(k4);
    pp.qblock[(int64_t)bh * pp.num_row_blocks + blk] = pp.zero_q ? 0.0f : sqrtf(q4);
  }
}

// A seq-contiguous V^T [B, H, 64, >=S] (seq stride 1, head_dim stride
// vt_sd) -> V [B, H, S, 64] contiguous, the key-major layout the attention
// kernels read.  One workgroup per 64 keys; keys at or past S are neither
// read nor written.
template <typename T>
__global__ __launch_bounds__(256) void transpose_vt_kernel(
    const T* __restrict__ vt, T* __restrict__ v, int64_t vt_sb, int64_t vt_sh,
    int64_t vt_sd, int heads, int seq_len) {
  typedef typename Vec8<T>::type V8;
  __shared__ T tile[kHeadDim][64 + 2];  // [head_dim][key]
  const int bh = blockIdx.y;
  const int b = bh / heads;
  const int h = bh - b * heads;
  const int k0 = blockIdx.x * 64;
  const T* src = vt + b * vt_sb + h * vt_sh;
  T* dst = v + (int64_t)bh * seq_len * kHeadDim;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int chunk = tid + 256 * i;
    const int d = chunk >> 3;
    const int c8 = (chunk & 7) * 8;
    const V8 vals = __builtin_bit_cast(
        V8, load8_guarded<T>(src + (int64_t)d * vt_sd + k0 + c8, (int64_t)k0 + c8, seq_len));
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[d][c8 + e] = vals[e];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int chunk = tid + 256 * i;
    const int row = chunk >> 3;
    const int c8 = (chunk & 7) * 8;
    if (k0 + row >= seq_len) continue;
    V8 vals;
#pragma unroll
    for (int e = 0; e < 8; ++e) vals[e] = tile[c8 + e][row];
    store16(dst + (int64_t)(k0 + row) * kHeadDim + c8, __builtin_bit_cast(u32x4, vals));
  }
}

int64_t padded_seq(int64_t seq_len) { return ceil_div(seq_len, 64) * 64; }

bool launch_supported(int block_m, int block_n, int num_warps, int num_stages) {
  if (block_n != kBlockN || (num_warps != 4 && num_warps != 8)) return false;
  if (num_stages == 3) return block_m == 128 && num_warps == 4;  // software-pipelined kernel
  if (num_stages != 1 && num_stages != 2) return false;
  // 32 or 64 query rows per wave.
  return block_m == 32 * num_warps || block_m == 64 * num_warps;
}

template <typename T, int WAVES, int PATH>
const void* plain_kernel(int qg, int num_stages) {
  if (qg == 1)
    return num_stages == 2 ? reinterpret_cast<const void*>(&attn_fwd_kernel<T, 1, 2, WAVES, PATH>)
                           : reinterpret_cast<const void*>(&attn_fwd_kernel<T, 1, 1, WAVES, PATH>);
  return num_stages == 2 ? reinterpret_cast<const void*>(&attn_fwd_kernel<T, 2, 2, WAVES, PATH>)
                         : reinterpret_cast<const void*>(&attn_fwd_kernel<T, 2, 1, WAVES, PATH>);
}

template <typename T, int WAVES>
const void* plain_kernel_path(int qg, int num_stages, int path) {
  if (path == kPathScaled) return scaled_path_kernel(std::is_same<T, bf16>::value, WAVES, qg, num_stages);
  if (path == kPathShifted) return plain_kernel<T, WAVES, kPathShifted>(qg, num_stages);
  return plain_kernel<T, WAVES, kPathAll>(qg, num_stages);
}

// Workgroups of `kernel` that fit on one CU at once (registers, LDS, waves),
// cached per kernel in a fixed table (the library has fewer attention
// kernels than slots; a kernel past the table is queried every time); 0 when
// the runtime cannot say.
int resident_per_cu(const void* kernel, int threads) {
  struct Slot {
    const void* kernel;
    int blocks;
  };
  static std::mutex mutex;
  static Slot cache[32] = {};
  std::lock_guard<std::mutex> lock(mutex);
  for (const Slot& slot : cache)
    if (slot.kernel == kernel) return slot.blocks;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    blocks = 0;
  }
  for (Slot& slot : cache)
    if (slot.kernel == nullptr) {
      slot = {kernel, blocks};
      break;
    }
  return blocks;
}

// Heads per issue group (see tile_of).  Each XCD holds slots = CUs/8 x
// resident workgroups at once; groups of about 2 x slots workgroups let the
// longest tiles of a group start first while the group stays small enough to
// keep its heads' K and V in the XCD's L2.  Measured on MI355X (bf16):
// B8 H16 S2048 0.150 -> 0.110 ms (256/64/8/2), B16 H32 S4096 1.74 -> 1.53 ms,
// B4 H16 S8192 0.82 -> 0.69 ms; long sequences (hundreds of tiles per head)
// get one head per group, the plain head-major order.  The CU count of the
// current device is used; the order never changes results.
int head_group_for(int64_t batch_heads, int64_t q_tiles, const void* kernel, int threads) {
  if (batch_heads % 8 != 0) return 0;
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int64_t slots = (int64_t)resident_per_cu(kernel, threads) * (cus / 8);
  if (slots <= 0) return 0;
  const int64_t heads_per_xcd = batch_heads / 8;
  const int64_t groups = std::max<int64_t>(1, (heads_per_xcd * q_tiles + slots) / (2 * slots));
  return (int)ceil_div(heads_per_xcd, groups);
}

template <typename T>
int launch_attention(AttnParams prm, int block_m, int num_warps, int num_stages,
                     hipStream_t stream) {
  const int64_t batch_heads = prm.num_blocks / prm.num_q_tiles;
  const void* kernel;
  int threads;
  if (num_stages == 3) {
    kernel = reinterpret_cast<const void*>(&attn_fwd_pipelined_kernel<T, 1>);
    threads = kThreads;
  } else {
    const int qg = block_m / (32 * num_warps);
    if (prm.kc != nullptr) {
      // The scaled-key workgroups, then the others, over the same grid.
      threads = num_warps * 64;
      for (int path : {kPathScaled, kPathShifted}) {
        kernel = num_warps == 8 ? plain_kernel_path<T, 8>(qg, num_stages, path)
                                : plain_kernel_path<T, 4>(qg, num_stages, path);
        prm.head_group = head_group_for(batch_heads, prm.num_q_tiles, kernel, threads);
        void* args[] = {&prm};
        const int status =
            check_hip(hipLaunchKernel(kernel, dim3(prm.num_blocks), dim3(threads), args, 0, stream),
                      "attention kernel launch");
        if (status != SAH_OK) return status;
      }
      return SAH_OK;
    }
    kernel = num_warps == 8 ? plain_kernel_path<T, 8>(qg, num_stages, kPathAll)
                            : plain_kernel_path<T, 4>(qg, num_stages, kPathAll);
    threads = num_warps * 64;
  }
  prm.head_group = head_group_for(batch_heads, prm.num_q_tiles, kernel, threads);
  void* args[] = {&prm};
  return check_hip(hipLaunchKernel(kernel, dim3(prm.num_blocks), dim3(threads), args, 0, stream),
                   "attention kernel launch");
}

template <typename T>
int launch_transpose_vt(const void* vt, void* v, int64_t batch, int64_t heads,
                        int64_t seq_len, int64_t vt_sb, int64_t vt_sh, int64_t vt_sd,
                        hipStream_t stream) {
  const dim3 grid((unsigned)ceil_div(seq_len, 64), (unsigned)(batch * heads)), block(256);
  hipLaunchKernelGGL((transpose_vt_kernel<T>), grid, block, 0, stream,
                     static_cast<const T*>(vt), static_cast<T*>(v), vt_sb, vt_sh, vt_sd,
                     (int)heads, (int)seq_len);
  return check_hip(hipGetLastError(), "V^T transpose launch");
}

template <typename T>
int launch_long_prepare(const PrepParams& pp, int64_t batch_heads, hipStream_t stream) {
  const dim3 grid((unsigned)pp.num_row_blocks, (unsigned)batch_heads), block(256);
  hipLaunchKernelGGL((long_prepare_kernel<T>), grid, block, 0, stream, pp);
  return check_hip(hipGetLastError(), "long-sequence preparation launch");
}

// Bytes of the per-tile key-norm table, rounded up to 256; 0 for sequences
// that run without it.
size_t key_norm_bytes(int64_t batch, int64_t heads, int64_t seq_len) {
  if (seq_len < kKeyNormMinSeq) return 0;
  return (size_t)ceil_div(batch * heads * ceil_div(seq_len, 64) * (int64_t)sizeof(float), 256) * 256;
}

// Bytes of the two per-block tables (largest |k|, largest |q| of every block
// of kScaledKeyRows rows), rounded up to 256; 0 without the key-norm table.
size_t row_block_bytes(int64_t batch, int64_t heads, int64_t seq_len) {
  if (seq_len < kKeyNormMinSeq) return 0;
  return (size_t)ceil_div(2 * batch * heads * ceil_div(seq_len, kScaledKeyRows) * (int64_t)sizeof(float), 256) * 256;
}

// Bytes of the scaled fp16 keys that go with the table (64-key tiles of 64
// elements); 0 for sequences that run without it.
size_t scaled_key_bytes(int64_t batch, int64_t heads, int64_t seq_len) {
  if (seq_len < kKeyNormMinSeq) return 0;
  return (size_t)batch * (size_t)heads * (size_t)padded_seq(seq_len) * kHeadDim * sizeof(f16);
}

// The regions of one call's workspace, in order: the three norm tables and
// the fp16 scaled keys when the call runs the preparation launch, then a
// key-major copy of V when the caller hands over a seq-contiguous V^T (the
// kernels read a head_dim-contiguous V as given).
struct WorkspaceLayout {
  size_t norm = 0, block = 0, kc = 0, vcopy = 0;
  size_t total() const { return norm + block + kc + vcopy; }
};

// `prepared`: the call runs the preparation launch (long sequences on the
// plain kernel).  Without it the plain kernel takes the shifted path for
// every workgroup, as below 4096 keys, and needs no tables.
WorkspaceLayout workspace_layout(int64_t batch, int64_t heads, int64_t seq_len,
                                 int64_t v_stride_d, int dtype, bool prepared) {
  WorkspaceLayout layout;
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || dtype == SAH_DTYPE_F32) return layout;
  if (prepared) {
    layout.norm = key_norm_bytes(batch, heads, seq_len);
    layout.block = row_block_bytes(batch, heads, seq_len);
    layout.kc = scaled_key_bytes(batch, heads, seq_len);
  }
  if (v_stride_d != 1)
    layout.vcopy = (size_t)batch * (size_t)heads * (size_t)seq_len * (size_t)kHeadDim * 2;
  return layout;
}

// Whether a call may run the preparation launch: a long sequence on the
// plain kernel (the pipelined kernel, num_stages 3, keeps the exact running
// maximum and never reads the tables).
bool prepares(int64_t seq_len, int num_stages, int dtype) {
  return seq_len >= kKeyNormMinSeq && num_stages != 3 && dtype != SAH_DTYPE_F32;
}

int run_attention(
    const void* query, const void* key, const void* value, void* output, int64_t batch,
    int64_t heads, int64_t seq_len, int64_t head_dim, int64_t q_stride_b,
    int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h,
    int64_t k_stride_s, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t v_stride_d, int64_t o_stride_b, int64_t o_stride_s, float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages, void* workspace,
    size_t workspace_bytes, bool allow_prepare, hipStream_t stream);

}  // namespace
}  // namespace sah

using namespace sah;

extern "C" int sah_causal_attention_launch_supported(int block_m, int block_n,
                                                     int num_warps, int num_stages) {
  return launch_supported(block_m, block_n, num_warps, num_stages) ? 1 : 0;
}

extern "C" size_t sah_causal_attention_workspace_bytes(int64_t batch, int64_t heads,
                                                       int64_t seq_len, int64_t head_dim,
                                                       int64_t v_stride_s,
                                                       int64_t v_stride_d, int dtype) {
  (void)head_dim;
  (void)v_stride_s;
  // The largest need over the launches (the plain launches; the pipelined
  // launch, num_stages 3, needs at most the V copy).  The fp32 kernel reads K
  // and V as given.
  return workspace_layout(batch, heads, seq_len, v_stride_d, dtype,
                          prepares(seq_len, 2, dtype)).total();
}

extern "C" int sah_causal_attention_bsd(
    const void* query, const void* key, const void* value, void* output, int64_t batch,
    int64_t heads, int64_t seq_len, int64_t head_dim, int64_t q_stride_b,
    int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h,
    int64_t k_stride_s, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t v_stride_d, int64_t o_stride_b, int64_t o_stride_s, float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages, void* workspace,
    size_t workspace_bytes, sah_stream_t stream_handle) {
  return run_attention(query, key, value, output, batch, heads, seq_len, head_dim, q_stride_b,
                       q_stride_h, q_stride_s, k_stride_b, k_stride_h, k_stride_s, v_stride_b,
                       v_stride_h, v_stride_s, v_stride_d, o_stride_b, o_stride_s, scale, dtype,
                       block_m, block_n, num_warps, num_stages, workspace, workspace_bytes,
                       /*allow_prepare=*/true, reinterpret_cast<hipStream_t>(stream_handle));
}

namespace sah {
namespace {

int run_attention(
    const void* query, const void* key, const void* value, void* output, int64_t batch,
    int64_t heads, int64_t seq_len, int64_t head_dim, int64_t q_stride_b,
    int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h,
    int64_t k_stride_s, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t v_stride_d, int64_t o_stride_b, int64_t o_stride_s, float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages, void* workspace,
    size_t workspace_bytes, bool allow_prepare, hipStream_t stream) {
  if (query == nullptr || key == nullptr || value == nullptr || output == nullptr)
    return fail(SAH_ERR_INVALID_ARGUMENT, "attention tensors must be non-null");
  if (head_dim != kHeadDim)
    return fail(SAH_ERR_UNSUPPORTED, "head_dim must be 64 (got %lld)", (long long)head_dim);
  if (dtype != SAH_DTYPE_BF16 && dtype != SAH_DTYPE_F16 && dtype != SAH_DTYPE_F32)
    return fail(SAH_ERR_UNSUPPORTED, "attention dtype must be bf16, f16 or f32");
  if (!launch_supported(block_m, block_n, num_warps, num_stages))
    return fail(SAH_ERR_UNSUPPORTED,
                "attention launch (block_m=%d, block_n=%d, num_warps=%d, "
                "num_stages=%d) is not implemented",
                block_m, block_n, num_warps, num_stages);
  if (batch < 0 || heads <= 0 || seq_len < 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "invalid attention sizes");
  if (batch == 0 || seq_len == 0) return SAH_OK;
  if (seq_len > (int64_t)1 << 30 || batch * heads > (int64_t)1 << 30)
    return fail(SAH_ERR_UNSUPPORTED, "attention sizes exceed the 32-bit tile indexing");
  if (!std::isfinite(scale)) return fail(SAH_ERR_INVALID_ARGUMENT, "scale must be finite");

  // Q and K: 16-byte rows.
  const int64_t vec = (dtype == SAH_DTYPE_F32) ? 4 : 8;  // elements per 16 bytes
  const int64_t qk_strides[] = {q_stride_b, q_stride_h, q_stride_s,
                                k_stride_b, k_stride_h, k_stride_s};
  for (int64_t s : qk_strides)
    if (s % vec != 0)
      return fail(SAH_ERR_INVALID_ARGUMENT,
                  "query/key strides must be multiples of 16 bytes");
  if (!aligned16(query) || !aligned16(key) || !aligned16(output))
    return fail(SAH_ERR_INVALID_ARGUMENT, "query/key/output must be 16-byte aligned");
  if (o_stride_b % 4 != 0 || o_stride_s % 4 != 0)
    return fail(SAH_ERR_INVALID_ARGUMENT, "output strides must be multiples of 4");

  AttnParams prm;
  prm.q = query;
  prm.k = key;
  prm.o = output;
  prm.q_sb = q_stride_b;
  prm.q_sh = q_stride_h;
  prm.q_ss = q_stride_s;
  prm.k_sb = k_stride_b;
  prm.k_sh = k_stride_h;
  prm.k_ss = k_stride_s;
  prm.o_sb = o_stride_b;
  prm.o_ss = o_stride_s;
  prm.seq_len = (int)seq_len;
  prm.heads = (int)heads;
  // The kernels take c = |scale| log2(e) > 0 and fold the sign of the scale
  // into the query (see AttnParams), so any finite scale is exact: negating a
  // bf16/fp16 value is exact, and the MFMA sums of negated products are the
  // negated sums.
  if (scale > 0.0f) {
    prm.c = scale * kLog2e;
    prm.q_and = 0xffffffffu;
    prm.q_xor = 0u;
  } else if (scale < 0.0f) {
    prm.c = -scale * kLog2e;
    prm.q_and = 0xffffffffu;
    prm.q_xor = 0x80008000u;
  } else {
    prm.c = kLog2e;
    prm.q_and = 0u;
    prm.q_xor = 0u;
  }
  if (!(prm.c > 0.0f) || !std::isfinite(prm.c))
    return fail(SAH_ERR_INVALID_ARGUMENT, "scale * log2(e) must be a finite nonzero float");
  if (dtype == SAH_DTYPE_F32) {
    // fp32: one kernel for every launch (the launch was validated above and
    // does not change results), V read head_dim-contiguous as given.
    if (v_stride_d != 1)
      return fail(SAH_ERR_UNSUPPORTED, "fp32 attention needs a head_dim-contiguous value");
    if (!aligned16(value) || v_stride_b % 4 || v_stride_h % 4 || v_stride_s % 4)
      return fail(SAH_ERR_INVALID_ARGUMENT,
                  "value must be 16-byte aligned with strides multiple of 4");
    if (batch * heads > 65535)
      return fail(SAH_ERR_UNSUPPORTED, "fp32 attention takes at most 65535 batch*heads");
    AttnF32Params fp;
    fp.q = static_cast<const float*>(query);
    fp.k = static_cast<const float*>(key);
    fp.v = static_cast<const float*>(value);
    fp.o = static_cast<float*>(output);
    fp.q_sb = q_stride_b;
    fp.q_sh = q_stride_h;
    fp.q_ss = q_stride_s;
    fp.k_sb = k_stride_b;
    fp.k_sh = k_stride_h;
    fp.k_ss = k_stride_s;
    fp.v_sb = v_stride_b;
    fp.v_sh = v_stride_h;
    fp.v_ss = v_stride_s;
    fp.o_sb = o_stride_b;
    fp.o_ss = o_stride_s;
    fp.seq_len = (int)seq_len;
    fp.heads = (int)heads;
    fp.c = prm.c;
    fp.q_and = prm.q_and;
    fp.q_xor = prm.q_xor != 0u ? 0x80000000u : 0u;
    hipLaunchKernelGGL(attn_fwd_f32_kernel, dim3((unsigned)ceil_div(seq_len, 64), (unsigned)(batch * heads)),
                       dim3(256), 0, stream, fp);
    return check_hip(hipGetLastError(), "fp32 attention launch");
  }
  const int64_t q_tiles = ceil_div(seq_len, block_m);
  const int64_t blocks = q_tiles * batch * heads;
  if (blocks > INT32_MAX) return fail(SAH_ERR_UNSUPPORTED, "too many attention tiles");
  prm.num_q_tiles = (int)q_tiles;
  prm.num_blocks = (int)blocks;

  // Workspace: the per-tile key-norm table, the per-block key and query norm
  // tables and the fp16 scaled keys (long sequences on the plain kernel),
  // then, for a seq-contiguous V^T, its key-major copy.
  const bool prepared = allow_prepare && prepares(seq_len, num_stages, dtype);
  const WorkspaceLayout layout =
      workspace_layout(batch, heads, seq_len, v_stride_d, dtype, prepared);
  const size_t need = layout.total();
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(SAH_ERR_WORKSPACE, "attention needs %zu workspace bytes, got %zu", need,
                workspace_bytes);
  if (need > 0 && !aligned16(workspace))
    return fail(SAH_ERR_INVALID_ARGUMENT, "attention workspace must be 16-byte aligned");
  // The preparation and V-copy launches put batch * heads on the grid's y axis.
  if ((prepared || layout.vcopy > 0) && batch * heads > 65535)
    return fail(SAH_ERR_UNSUPPORTED,
                "attention with %s takes at most 65535 batch*heads (got %lld)",
                prepared ? "the long-sequence preparation" : "a seq-contiguous value",
                (long long)(batch * heads));
  const size_t norm_bytes = layout.norm;
  const size_t block_bytes = layout.block;
  const size_t kc_bytes = layout.kc;
  unsigned char* base = static_cast<unsigned char*>(workspace);
  void* vcopy_space = layout.vcopy > 0 ? base + norm_bytes + block_bytes + kc_bytes : nullptr;
  int status = SAH_OK;
  prm.knorm = nullptr;
  prm.kblock = nullptr;
  prm.qblock = nullptr;
  prm.kc = nullptr;
  prm.key_tiles = (int)ceil_div(seq_len, 64);
  prm.num_row_blocks = (int)ceil_div(seq_len, kScaledKeyRows);
  if (v_stride_d == 1) {
    if (!aligned16(value) || v_stride_b % 8 || v_stride_h % 8 || v_stride_s % 8)
      return fail(SAH_ERR_INVALID_ARGUMENT,
                  "value must be 16-byte aligned with strides multiple of 8");
  } else if (v_stride_s == 1) {
    if (!aligned16(value) || v_stride_b % 8 || v_stride_h % 8 || v_stride_d % 8)
      return fail(SAH_ERR_INVALID_ARGUMENT,
                  "seq-contiguous value must be 16-byte aligned with strides multiple of 8");
  } else {
    return fail(SAH_ERR_INVALID_ARGUMENT,
                "value needs a unit stride on the head_dim or the seq axis");
  }
  // The tile loaders address 64 key rows of K and of V at 32-bit byte
  // offsets from a per-tile base: both row strides must be non-negative and
  // 64 rows must span less than 2^31 bytes.
  const int64_t v_row_stride = (v_stride_d == 1) ? v_stride_s : kHeadDim;
  if (k_stride_s < 0 || v_row_stride < 0 || k_stride_s >= ((int64_t)1 << 24) ||
      v_row_stride >= ((int64_t)1 << 24))
    return fail(SAH_ERR_UNSUPPORTED,
                "key/value row strides must lie in [0, 2^24) elements (32-bit tile offsets)");
  // Long sequences (the plain kernel): one preparation launch writes the
  // norm tables and the fp16 scaled keys.
  if (prepared) {
    PrepParams pp;
    pp.k = key;
    pp.q = query;
    pp.knorm = reinterpret_cast<float*>(base);
    pp.kblock = reinterpret_cast<float*>(base + norm_bytes);
    pp.qblock = pp.kblock + batch * heads * prm.num_row_blocks;
    pp.kc = reinterpret_cast<f16*>(base + norm_bytes + block_bytes);
    pp.k_sb = k_stride_b;
    pp.k_sh = k_stride_h;
    pp.k_ss = k_stride_s;
    pp.q_sb = q_stride_b;
    pp.q_sh = q_stride_h;
    pp.q_ss = q_stride_s;
    pp.c = prm.c;
    pp.zero_q = prm.q_and == 0u ? 1 : 0;
    pp.heads = (int)heads;
    pp.seq_len = (int)seq_len;
    pp.key_tiles = prm.key_tiles;
    pp.num_row_blocks = prm.num_row_blocks;
    status = (dtype == SAH_DTYPE_BF16) ? launch_long_prepare<bf16>(pp, batch * heads, stream)
                                       : launch_long_prepare<f16>(pp, batch * heads, stream);
    if (status != SAH_OK) return status;
    prm.knorm = pp.knorm;
    prm.kblock = pp.kblock;
    prm.qblock = pp.qblock;
    prm.kc = pp.kc;
  }
  if (v_stride_d == 1) {
    // The reference layout (head_dim-contiguous, any key stride): read as
    // given, transposed on the way from LDS into the PV operand.
    prm.v = value;
    prm.v_sb = v_stride_b;
    prm.v_sh = v_stride_h;
    prm.v_ss = v_stride_s;
  } else {
    // A seq-contiguous V^T: copied key-major into the workspace first.
    status = (dtype == SAH_DTYPE_BF16)
                 ? launch_transpose_vt<bf16>(value, vcopy_space, batch, heads, seq_len,
                                             v_stride_b, v_stride_h, v_stride_d, stream)
                 : launch_transpose_vt<f16>(value, vcopy_space, batch, heads, seq_len,
                                            v_stride_b, v_stride_h, v_stride_d, stream);
    if (status != SAH_OK) return status;
    prm.v = vcopy_space;
    prm.v_sb = heads * seq_len * kHeadDim;
    prm.v_sh = seq_len * kHeadDim;
    prm.v_ss = kHeadDim;
  }
  return (dtype == SAH_DTYPE_BF16)
             ? launch_attention<bf16>(prm, block_m, num_warps, num_stages, stream)
             : launch_attention<f16>(prm, block_m, num_warps, num_stages, stream);
}

}  // namespace
}  // namespace sah

// ---------------------------------------------------------------------------
// Variant of sah_causal_attention_bsd for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops): the
// workspace (norm tables, fp16 scaled keys, the key-major copy of a
// seq-contiguous V^T) lives in this
// file-scope device array, of which each GPU holds its own copy for the life
// of the process.
// Kernel arguments need its device address, which differs per GPU and is
// looked up once per device with hipGetSymbolAddress; the array's name is
// only a host-side stand-in and is never passed to a kernel.
static __device__ __align__(256) unsigned char scratch[SAH_ATTENTION_STATIC_WORKSPACE_BYTES];

namespace sah {
namespace {

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device, or null on failure
// (the status is then in sah_last_error()).
void* scratch_address() {
  static std::mutex mutex;
  static void* address[kMaxDevices] = {};
  int device = 0;
  if (check_hip(hipGetDevice(&device), "hipGetDevice") != SAH_OK) return nullptr;
  if (device < 0 || device >= kMaxDevices) {
    fail(SAH_ERR_UNSUPPORTED, "device ordinal %d exceeds the static workspace table", device);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mutex);
  if (address[device] == nullptr) {
    void* ptr = nullptr;
    if (check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "static workspace lookup") != SAH_OK)
      return nullptr;
    address[device] = ptr;
  }
  return address[device];
}

}  // namespace
}  // namespace sah

extern "C" int sah_causal_attention_bsd_static_workspace(
    const void* query, const void* key, const void* value, void* output, int64_t batch,
    int64_t heads, int64_t seq_len, int64_t head_dim, int64_t q_stride_b,
    int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h,
    int64_t k_stride_s, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t v_stride_d, int64_t o_stride_b, int64_t o_stride_s, float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages, sah_stream_t stream) {
  // The whole call when its workspace fits the array.  Otherwise the call
  // runs in chunks of heads of one batch row whose workspace fits: heads are
  // independent and every head takes the same path (the path is chosen per
  // head from its own tables), so the chunks give bitwise the result of one
  // call.  The prepared layout is kept when one head's fits; otherwise every
  // chunk runs the shifted path without preparation, as below 4096 keys.
  constexpr size_t kLimit = (size_t)SAH_ATTENTION_STATIC_WORKSPACE_BYTES;
  const hipStream_t hip_stream = reinterpret_cast<hipStream_t>(stream);
  bool prepare = prepares(seq_len, num_stages, dtype);
  auto need_for = [&](int64_t b, int64_t h, bool prep) {
    return workspace_layout(b, h, seq_len, v_stride_d, dtype, prep).total();
  };
  int64_t chunk_heads = heads;
  const bool whole = need_for(batch, heads, prepare) <= kLimit;
  if (!whole) {
    if (prepare && need_for(1, 1, true) > kLimit) prepare = false;
    // The most heads whose workspace fits (it grows with the head count).
    int64_t lo = 0, hi = heads;
    while (lo < hi) {
      const int64_t mid = lo + (hi - lo + 1) / 2;
      if (need_for(1, mid, prepare) <= kLimit)
        lo = mid;
      else
        hi = mid - 1;
    }
    chunk_heads = lo;
    if (chunk_heads == 0)
      return fail(SAH_ERR_WORKSPACE,
                  "attention needs %zu workspace bytes for one head, above the static workspace of "
                  "%zu bytes; use sah_causal_attention_bsd with a caller-provided workspace",
                  need_for(1, 1, prepare), kLimit);
  }
  const size_t need = need_for(whole ? batch : 1, chunk_heads, prepare);
  void* workspace = nullptr;
  if (need > 0) {
    workspace = scratch_address();
    if (workspace == nullptr) return SAH_ERR_HIP;
  }
  if (whole)
    return run_attention(query, key, value, output, batch, heads, seq_len, head_dim, q_stride_b,
                         q_stride_h, q_stride_s, k_stride_b, k_stride_h, k_stride_s, v_stride_b,
                         v_stride_h, v_stride_s, v_stride_d, o_stride_b, o_stride_s, scale, dtype,
                         block_m, block_n, num_warps, num_stages, workspace, need > 0 ? kLimit : 0,
                         prepare, hip_stream);
  // Element size of the 16-bit dtypes (fp32 calls need no workspace and
  // never reach here).
  const int64_t es = 2;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t h0 = 0; h0 < heads; h0 += chunk_heads) {
      const int64_t hn = std::min(chunk_heads, heads - h0);
      const char* q = static_cast<const char*>(query) + es * (b * q_stride_b + h0 * q_stride_h);
      const char* k = static_cast<const char*>(key) + es * (b * k_stride_b + h0 * k_stride_h);
      const char* v = static_cast<const char*>(value) + es * (b * v_stride_b + h0 * v_stride_h);
      char* o = static_cast<char*>(output) + es * (b * o_stride_b + h0 * head_dim);
      const int status = run_attention(
          q, k, v, o, 1, hn, seq_len, head_dim, q_stride_b, q_stride_h, q_stride_s, k_stride_b,
          k_stride_h, k_stride_s, v_stride_b, v_stride_h, v_stride_s, v_stride_d, o_stride_b,
          o_stride_s, scale, dtype, block_m, block_n, num_warps, num_stages, workspace,
          need > 0 ? kLimit : 0, prepare, hip_stream);
      if (status != SAH_OK) return status;
    }
  return SAH_OK;
}
