// nn-scored edge attention: an edge MLP produces one score per edge, online
// softmax over each destination row weights a gathered value field.
//
// Reference: tg.nn.trace'd score networks (python/tiga/compiler/
// nn_capture.py:1-33: a linear chain of nn.Linear and component-wise
// activations over concatenated per-edge field gathers) evaluated by the
// row-centric fused tile of compiler/edge_nn_attention.py:1-20 and
// interop/torch/message_passing.py:2372-2577; semantics of
// _evaluate_reference + reduce_online_softmax (message_passing.py:2848-2894,
// reducer_oracle.py:60-137).
//
// MI355X design: the score network is evaluated edge-parallel, one edge per
// lane, so every lane does useful work whatever the row degrees; its inputs
// are gathered straight from the field tables (no [E, K] tensor) and its
// weights, uniform across the wave, are read through the scalar cache into
// scalar registers that feed the FMAs directly.  Every layer is zero-padded
// to a common width W (16, 24, 32 or 64) on the host, which keeps every
// register index compile-time; the real widths bound the loops through
// uniform branches.  The softmax and the value gather are
// separate row passes (segment softmax here, the weighted CSR sum of
// tgx_sum.hip for the values), which adds 8 bytes per edge (score, weight)
// to a gather of 4 F bytes per edge.
//
// Backward: segment softmax backward per row (ds = a (da - <a, da>)), then
// the per-edge MLP backward replays the chain, back-propagates ds, writes the
// per-edge gradients of every input segment (reduced per source row over the
// transposed CSR and per destination row over the CSR by the caller) and
// sums the weight and bias gradients (sum over edges of dz_l (x) a_l) in the
// same pass: the hidden layers' on fp32 MFMA, from rows each wave stages in
// LDS, the one-output last layer's (ds a) in per-lane registers; per-block
// partial sums are added in a fixed order, so every gradient is
// deterministic and nothing per layer and edge goes to HBM.
#include <hip/hip_runtime.h>

#include <atomic>
#include <type_traits>

#include "tgx_nn_common.h"
#include "tgx_profile.h"

// Built twice: here the public entry points, and as tgx_nn_math.hip
// (TGX_NN_MATH 1) the tgx_edge_mlp_*_math functions they call for chains
// that use exp, log, abs, sin, cos, a power or LayerNorm (the segment
// softmax entry points are built here only).
// Each tier is also split by column index type, so the halves compile in
// parallel: built directly, this file holds the int32_t kernels and the
// entry points; tgx_nn_i64.hip (and tgx_nn_math_i64.hip) build it with
// TGX_NN_INDEX 64 for the int64_t kernels alone.
#ifndef TGX_NN_INDEX
#define TGX_NN_INDEX 32
#endif

#if TGX_NN_MATH
#define TGX_NN_ENTRY(name) int name##_math
#define TGX_TO_MATH(mlp, call)
#else
#define TGX_NN_ENTRY(name) extern "C" int name
#define TGX_TO_MATH(mlp, call) \
  if (tgx::mlp::uses_math_tier(mlp)) return call
#endif

namespace tgx {
namespace {

using namespace mlp;

// Occupancy targets (blocks of 256 per CU, i.e. waves per SIMD): left to
// itself the register allocator spends registers on scheduling freedom and
// lands just above a step (one fewer wave per SIMD).
template <int W, int L>
constexpr int fwd_blocks_per_cu() { return W <= 32 ? (L <= 2 ? 6 : 5) : 3; }
// The kernels with the second set of functions and LayerNorm hold more
// per lane (LayerNorm sums, the larger switch): one wave per SIMD fewer
// keeps them from spilling.
template <int W, int L>
constexpr int bwd_blocks_per_cu() {
  constexpr int n = W == 16 ? 3 : W == 24 ? (L <= 2 ? 3 : 2) : (L <= 2 ? 2 : 1);
  return TGX_NN_MATH && n > 1 ? n - 1 : n;
}

template <typename I, int W, int L>
__global__ __launch_bounds__(256, (fwd_blocks_per_cu<W, L>())) void edge_mlp_fwd_kernel(const I* __restrict__ col,
                                                           const int32_t* __restrict__ dst,
                                                           int64_t n_edges, MlpView m,
                                                           float* __restrict__ scores) {
  cfloat* wg = scalar_weights(m.w);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_edges) return;
  float a[W], z[W];
  gather_inputs<I, W>(m, e, col, dst, a);
  const int nw = layer_stride<W>(m);
#pragma unroll
  for (int l = 0; l + 1 < L; ++l) {
    linear<W>(wg + l * nw, a, z, m.n_out[l], m.nb_in[l]);
    norm_layer<W>(m, l, wg + l * nw, z);
    activate_all<W>(z, a, m.act[l], m.param[l], m.param2[l], m.nb_in[l + 1],
                    m.n_out[l]);
  }
  scores[e] = linear_out1<W>(wg + (L - 1) * nw, a, m.nb_in[L - 1]);
}

// The last layer's input per edge (the activation after layer L - 2, or the
// gathered input when L = 1): hidden[e][0..hw).
template <typename I, int W, int L>
__global__ __launch_bounds__(256) void edge_mlp_hidden_kernel(const I* __restrict__ col,
                                                              const int32_t* __restrict__ dst,
                                                              int64_t n_edges, MlpView m,
                                                              float* __restrict__ hidden,
                                                              int hw) {
  cfloat* wg = scalar_weights(m.w);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_edges) return;
  float a[W], z[W];
  gather_inputs<I, W>(m, e, col, dst, a);
  const int nw = layer_stride<W>(m);
#pragma unroll
  for (int l = 0; l + 1 < L; ++l) {
    linear<W>(wg + l * nw, a, z, m.n_out[l], m.nb_in[l]);
    norm_layer<W>(m, l, wg + l * nw, z);
    activate_all<W>(z, a, m.act[l], m.param[l], m.param2[l], m.nb_in[l + 1],
                    m.n_out[l]);
  }
  float* out = hidden + e * hw;
#pragma unroll
  for (int k = 0; k < W; ++k)
    if (k < hw) out[k] = a[k];
}

// ---- weight gradients on fp32 MFMA ------------------------------------------
//
// dW_l = sum over edges of dz_l[e] (x) a_l[e] (pre-activation gradient times
// layer input) is a [W x E] x [E x W] product.  Each wave stages the rows of
// its edges in LDS (32 edges per round, row stride W + 4 floats) and feeds
// them to fp32 MFMA, which takes exact fp32 products and fp32 sums like
// v_fma_f32:
//   W = 16: v_mfma_f32_16x16x4_f32, lane l gives G[4s + l/16][l%16] (A
//           operand, G^T) and A[4s + l/16][l%16] (B operand);
//           D[o][i]: i = l%16, o = 4(l/16) + q for accumulator q.
//   W = 32, 64: v_mfma_f32_32x32x2_f32 per 32 x 32 tile, lane l gives row
//           2s + l/32, column l%32 (+32 per tile); D[o][i]: i = l%32,
//           o = 8(q/4) + 4(l/32) + q%4.
// The bias gradient (the column sums of G) is summed from the same reads.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Staging row stride: 24-wide layers use the 32-wide MFMA tiles, their
// columns 24..31 staying zero.
template <int W>
constexpr int mlp_ld() { return (W == 24 ? 32 : W) + 4; }

template <int W>
struct OuterAcc {
  static constexpr int kTiles = W == 64 ? 4 : 1;
  using Tile = typename std::conditional<W == 16, f32x4, f32x16>::type;
  Tile c[kTiles];
  float b[W == 64 ? 2 : 1];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < kTiles; ++t) c[t] = Tile{};
#pragma unroll
    for (int t = 0; t < (W == 64 ? 2 : 1); ++t) b[t] = 0.f;
  }
};

// acc += G^T A over the 32 staged rows of this wave.
template <int W>
__device__ __forceinline__ void outer_accumulate(const float* sg, const float* sa,
                                                 OuterAcc<W>& acc) {
  constexpr int LD = mlp_ld<W>();
  const int l = lane_id();
  if constexpr (W == 16) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int at = (4 * s + l / 16) * LD + l % 16;
      const float g = sg[at], a = sa[at];
      acc.b[0] += g;
      acc.c[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(g, a, acc.c[0], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int at = (2 * s + l / 32) * LD + l % 32;
      const float g0 = sg[at], a0 = sa[at];
      acc.b[0] += g0;
      acc.c[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(g0, a0, acc.c[0], 0, 0, 0);
      if constexpr (W == 64) {
        const float g1 = sg[at + 32], a1 = sa[at + 32];
        acc.b[1] += g1;
        acc.c[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(g0, a1, acc.c[1], 0, 0, 0);
        acc.c[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(g1, a0, acc.c[2], 0, 0, 0);
        acc.c[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(g1, a1, acc.c[3], 0, 0, 0);
      }
    }
  }
}

#if TGX_NN_MATH
// The diagonal of the wave's accumulated W x W block and its column sums:
// red[i] = acc[i][i], red[W + i] = b[i] (a LayerNorm's d gamma, d beta).
template <int W>
__device__ __forceinline__ void outer_store_norm(const OuterAcc<W>& acc, float* red) {
  static_assert(W <= 32, "normalized layers are at most 32 wide");
  const int l = lane_id();
  if constexpr (W == 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (4 * (l / 16) + q == l % 16) red[l % 16] = acc.c[0][q];
    float b = acc.b[0];
    b += __shfl_xor(b, 16, 64);
    b += __shfl_xor(b, 32, 64);
    if (l < 16) red[W + l] = b;
  } else {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int o = 8 * (q / 4) + 4 * (l / 32) + q % 4, i = l % 32;
      if (o == i && i < W) red[i] = acc.c[0][q];
    }
    const float b = acc.b[0] + __shfl_xor(acc.b[0], 32, 64);
    if (l < W) red[W + l] = b;
  }
}
#endif

// Orders this wave's LDS accesses around an exchange between its lanes: a
// wave's LDS instructions execute in issue order, so only the compiler has
// to be kept from moving accesses across (rocPRIM's wave_barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stage this wave's (G, A) rows and add G^T A to acc: lanes 0..31 first,
// then lanes 32..63, through the wave's own LDS region (no block barrier:
// the waves of a block progress independently).
template <int W>
__device__ __forceinline__ void outer_layer(float* sg, float* sa, const float (&g)[W],
                                            const float (&a)[W], OuterAcc<W>& acc) {
  constexpr int LD = mlp_ld<W>();
  const int l = lane_id();
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    if ((l >> 5) == round) {
      float* pg = sg + (l & 31) * LD;
      float* pa = sa + (l & 31) * LD;
#pragma unroll
      for (int k = 0; k < W; k += 4) {
        *reinterpret_cast<f32x4*>(pg + k) = f32x4{g[k], g[k + 1], g[k + 2], g[k + 3]};
        *reinterpret_cast<f32x4*>(pa + k) = f32x4{a[k], a[k + 1], a[k + 2], a[k + 3]};
      }
    }
    wave_lds_sync();
    outer_accumulate<W>(sg, sa, acc);
    wave_lds_sync();
  }
}

// The wave's accumulated [W x W | W] block, written row-major into red.
template <int W>
__device__ __forceinline__ void outer_store(const OuterAcc<W>& acc, float* red) {
  const int l = lane_id();
  if constexpr (W == 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(4 * (l / 16) + q) * W + l % 16] = acc.c[0][q];
    float b = acc.b[0];
    b += __shfl_xor(b, 16, 64);
    b += __shfl_xor(b, 32, 64);
    if (l < 16) red[W * W + l] = b;
  } else {
#pragma unroll
    for (int t = 0; t < OuterAcc<W>::kTiles; ++t) {
      const int ro = 32 * (t >> 1), ci = 32 * (t & 1);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int o = ro + 8 * (q / 4) + 4 * (l / 32) + q % 4, i = ci + l % 32;
        if (W != 24 || (o < W && i < W)) red[o * W + i] = acc.c[t][q];
      }
    }
#pragma unroll
    for (int t = 0; t < (W == 64 ? 2 : 1); ++t) {
      const float b = acc.b[t] + __shfl_xor(acc.b[t], 32, 64);
      if (l < (W == 24 ? 24 : 32)) red[W * W + 32 * t + l] = b;
    }
  }
}

// Per-edge backward of the score chain plus the weight-gradient sums.  ds_e
// arrives from the softmax backward.  Each block walks a contiguous range of
// edges in steps of 256 (one edge per lane), replays the chain, back-
// propagates ds, writes the input gradient of every segment per edge
// (dseg[s][e][:width_s]) and accumulates dW_l, db_l for every layer on MFMA;
// the block's sums go to partial[block] (n_layers x [W*W | W]) in a fixed
// order.
//
// SEED: the gradient at the last layer's input is given per destination row
// (seed[dst[e]][0..hw), the edge-network sum's backward) instead of coming
// from a one-output last layer; the last layer's sums then stay zero.
// ACT >= 0: every hidden layer's activation is that code, fixed at compile
// time (the runtime switch and its branches are gone: 0.362 -> 0.340 ms on
// the nn step's LeakyReLU chain); -1 reads m.act per layer.
template <typename I, int W, int L, bool SEED, int ACT = -1>
__global__ __launch_bounds__(256, (bwd_blocks_per_cu<W, L>())) void edge_mlp_bwd_kernel(
    const I* __restrict__ col, const int32_t* __restrict__ dst, int64_t n_edges, int64_t chunk,
    MlpView m_arg, const float* __restrict__ dscore, float* __restrict__ partial,
    const float* __restrict__ seed, int hw) {
  constexpr int NW = W * W + W;
  constexpr int LD = mlp_ld<W>();
  constexpr int SW = 2 * 32 * LD;  // one wave's staging: G rows | A rows
  static_assert(SW >= NW, "a wave's staging holds one layer's block");
  __shared__ __align__(16) float stage[4 * SW];
  cfloat* const w_all = scalar_weights(m_arg.w);
  const int wave = threadIdx.x >> 6;
  float* sg = stage + wave * SW;
  float* sa = sg + 32 * LD;
  if constexpr (W == 24) {
    // Staging columns 24..35 are never written by the rounds: zero once.
    for (int i = threadIdx.x; i < 4 * SW; i += 256) stage[i] = 0.f;
    __syncthreads();
  }
  OuterAcc<W> acc[L > 1 ? L - 1 : 1];   // the hidden layers' sums
  float last_w[W];   // this lane's sum of ds a for the last layer, and of ds
  float last_b = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) last_w[i] = 0.f;
#pragma unroll
  for (int l = 0; l < (L > 1 ? L - 1 : 1); ++l) acc[l].zero();
#if TGX_NN_MATH
  // LayerNorm parameter sums of the hidden layers: sum dy (x) x_hat, whose
  // diagonal is d gamma, and sum dy = d beta, on the same MFMA path.
  OuterAcc<W> acc_n[L > 1 ? L - 1 : 1];
#pragma unroll
  for (int l = 0; l < (L > 1 ? L - 1 : 1); ++l) acc_n[l].zero();
#endif
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t e1 = e0 + chunk < n_edges ? e0 + chunk : n_edges;
  // Each step's source and destination row ids are loaded one step ahead.
  int64_t next_src = 0, next_dst = 0;
  if (e0 + threadIdx.x < e1) {
    next_src = col[e0 + threadIdx.x];
    next_dst = dst[e0 + threadIdx.x];
  }
  for (int64_t base = e0; base < e1; base += 256) {
    // The weights are reloaded (scalar-cache hits) and the network's shape
    // fields re-read in every step: hoisted out of the loop, the weights and
    // the tile guards derived from the shape would all be live at once and
    // spill.
    cfloat* wg = opaque(w_all);
    MlpView m = m_arg;
    launder(m);
    const int nw = layer_stride<W>(m);
    const int64_t e = base + threadIdx.x;
    const bool valid = e < e1;
    float x[W];                        // gathered input (layer 0's input)
    // Pre-activations of the hidden layers (x_hat for a normalized layer,
    // with 1 / sqrt(var + eps) in rstd).
    float z[L > 1 ? L - 1 : 1][W];
#if TGX_NN_MATH
    float rstd[L > 1 ? L - 1 : 1];
#endif
    // The activation's input of hidden layer l: z[l], or gamma x_hat + beta.
    auto act_input = [&](auto lc, float (&y)[W]) TGX_INLINE_LAMBDA {
      constexpr int l = decltype(lc)::value;
#if TGX_NN_MATH
      if (m.norm[l]) {
        norm_affine<W>(wg + l * nw + W * W + W, z[l], y);
        return;
      }
#endif
#pragma unroll
      for (int k = 0; k < W; ++k) y[k] = z[l][k];
    };
    const int64_t cur_dst = next_dst;
    const int64_t cur_src = next_src;
    if (valid) {
      gather_rows<W>(m, e, next_src, next_dst, x);
    } else {
#pragma unroll
      for (int k = 0; k < W; ++k) x[k] = 0.f;
    }
    if (e + 256 < e1) {
      next_src = col[e + 256];
      next_dst = dst[e + 256];
    }
    {
      float a[W];
#pragma unroll
      for (int k = 0; k < W; ++k) a[k] = x[k];
      static_for<L - 1>([&](auto lc) TGX_INLINE_LAMBDA {
        constexpr int l = decltype(lc)::value;
        linear<W>(wg + l * nw, a, z[l], m.n_out[l], m.nb_in[l]);
#if TGX_NN_MATH
        if (m.norm[l]) rstd[l] = norm_rows<W>(z[l], m.n_out[l], m.eps[l]);
#endif
        float y[W];
        act_input(lc, y);
        activate_all<W>(y, a, ACT >= 0 ? ACT : m.act[l], m.param[l], m.param2[l], m.nb_in[l + 1],
                        m.n_out[l]);
      });
    }
    // Input of layer l: x, or the activation of z[l-1].
    auto layer_input = [&](auto lc, float (&a)[W]) TGX_INLINE_LAMBDA {
      constexpr int l = decltype(lc)::value;
      if constexpr (l == 0) {
#pragma unroll
        for (int k = 0; k < W; ++k) a[k] = x[k];
      } else {
        float y[W];
        act_input(std::integral_constant<int, l - 1>{}, y);
        activate_all<W>(y, a, ACT >= 0 ? ACT : m.act[l - 1], m.param[l - 1], m.param2[l - 1], m.nb_in[l],
                        m.n_out[l - 1]);
      }
    };
    float g[W];
    float alpha = 0.f;   // attention backward: the edge's recomputed weight
    if constexpr (SEED) {
      // The gradient at the last layer's input, gathered from the edge's row.
      const float* q = seed + cur_dst * hw;
#pragma unroll
      for (int k = 0; k < W; ++k) g[k] = (valid && k < hw) ? q[k] : 0.f;
    } else {
      // Last layer: one output, gradient ds (0 on lanes past the range):
      // read, or formed here from the replayed score (attention backward
      // from the saved logsumexp).
      cfloat* wl = wg + (L - 1) * nw;
      float a[W];
      layer_input(std::integral_constant<int, L - 1>{}, a);
      float ds = 0.f;
      if (m.att_lse != nullptr) {
        if (valid)
          ds = attention_score_grad(m, e, cur_dst, cur_src,
                                    linear_out1<W>(wl, a, m.nb_in[L - 1]), alpha);
      } else if (valid) {
        ds = dscore[e];
      }
      // One output row: its gradient ds a is summed per lane (an MFMA outer
      // product would spend a 32 x 32 tile on it).
      last_b += ds;
#pragma unroll
      for (int c = 0; c < W / 8; ++c)
        if (2 * c < m.nb_in[L - 1])
#pragma unroll
          for (int j = 0; j < 8; ++j) last_w[8 * c + j] = fmaf(ds, a[8 * c + j], last_w[8 * c + j]);
      linear_t_out1<W>(wl, ds, g, m.nb_in[L - 1]);   // d a[L-1] = ds w
    }
    static_for<L - 1>([&](auto kc) TGX_INLINE_LAMBDA {
      constexpr int l = L - 2 - decltype(kc)::value;
      float dzl[W];
      {
        float y[W];
        act_input(std::integral_constant<int, l>{}, y);
        activate_grad_all<W>(y, g, dzl, ACT >= 0 ? ACT : m.act[l], m.param[l], m.param2[l], m.nb_in[l + 1],
                             m.n_out[l]);
      }
#if TGX_NN_MATH
      if (m.norm[l]) {
        // dzl is the gradient at y here: the gamma and beta sums, then the
        // gradient at z through the normalization.
        outer_layer<W>(sg, sa, dzl, z[l], acc_n[l]);
        norm_rows_grad<W>(wg + l * nw + W * W + W, z[l], dzl, m.n_out[l], rstd[l]);
      }
#endif
#pragma unroll
      for (int o = 0; o < W; ++o) pin(dzl[o]);
      {
        float a[W];
        layer_input(std::integral_constant<int, l>{}, a);
        outer_layer<W>(sg, sa, dzl, a, acc[l]);
      }
      // d a[l] = W_l^T dz.
      linear_t<W>(wg + l * nw, dzl, g, m.n_out[l], m.nb_in[l]);
    });
    // g = d x: split per segment.
    if (valid) scatter_segments<W>(m, e, g, alpha, cur_dst);
  }
  // Block sums, layer by layer: each wave's block into its staging region,
  // then the four added in wave order.
  const int nwb = layer_stride<W>(m_arg);
  float* out = partial + static_cast<int64_t>(blockIdx.x) * L * nwb;
#pragma unroll
  for (int l = 0; l < L; ++l) {
    if (l == L - 1) {
      // The last layer: the wave's lanes summed by a butterfly, then the
      // [W x W | W] block with only row 0 and bias 0 nonzero.
      const int lane = lane_id();
#pragma unroll
      for (int i = 0; i < W; ++i)
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) last_w[i] += __shfl_xor(last_w[i], d, 64);
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) last_b += __shfl_xor(last_b, d, 64);
      for (int idx = lane; idx < NW; idx += 64) sg[idx] = 0.f;
      wave_lds_sync();
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < W; ++i) sg[i] = last_w[i];
        sg[W * W] = last_b;
      }
    } else {
      outer_store<W>(acc[l], sg);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < NW; idx += 256)
      out[l * nwb + idx] = (stage[idx] + stage[SW + idx]) + (stage[2 * SW + idx] + stage[3 * SW + idx]);
    __syncthreads();
#if TGX_NN_MATH
    if (nwb > NW) {
      // [d gamma | d beta] after the layer's block (zero for the last layer).
      if (l + 1 < L) outer_store_norm<W>(acc_n[l < L - 1 ? l : 0], sg);
      __syncthreads();
      for (int idx = threadIdx.x; idx < 2 * W; idx += 256)
        out[l * nwb + NW + idx] =
            l + 1 < L ? (stage[idx] + stage[SW + idx]) + (stage[2 * SW + idx] + stage[3 * SW + idx])
                      : 0.f;
      __syncthreads();
    }
#endif
  }
}

// Segment softmax kernels: each wave takes four consecutive rows.  When
// the longest of them has at most 16 edges, each row gets a 16-lane slot
// (one edge per lane, the whole wave at once); at most 32, the rows go
// two at a time in 32-lane slots; longer, one at a time over the whole
// wave.  fn(row, slot width, lane in slot) runs for every row of the group
// (rows past n_rows included, with no edges) on all lanes of its slot.
constexpr int kSoftmaxRowsPerWave = 4;

template <typename I, typename Fn>
__device__ __forceinline__ void softmax_row_groups(const I* row_ptr, int64_t n_rows, Fn&& fn) {
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kSoftmaxRowsPerWave;
  if (row0 >= n_rows) return;   // wave-uniform
  const int lane = lane_id();
  const int64_t r = row0 + (lane & 3);
  const int64_t len =
      r < n_rows ? static_cast<int64_t>(row_ptr[r + 1]) - static_cast<int64_t>(row_ptr[r]) : 0;
  int longest = static_cast<int>(len < 64 ? len : 64);
  longest = max(longest, __shfl_xor(longest, 1, 64));
  longest = max(longest, __shfl_xor(longest, 2, 64));
  longest = uniform(longest);
  if (longest <= 16) {
    fn(row0 + (lane >> 4), std::integral_constant<int, 16>{}, lane & 15);
  } else if (longest <= 32) {
    for (int h = 0; h < 2; ++h) fn(row0 + 2 * h + (lane >> 5), std::integral_constant<int, 32>{},
                                   lane & 31);
  } else {
    for (int q = 0; q < kSoftmaxRowsPerWave; ++q)
      fn(row0 + q, std::integral_constant<int, 64>{}, lane);
  }
}

// alpha_e = exp(s_e - m) / l over one row in a slot of S lanes, lse = m +
// log l (-inf and no weights for an empty row).  exp(s - m) / l rather than
// exp(s - lse): s - m is exact (two nearby fp32 values), while lse carries
// the rounding of a large score (about 6e-5 at 1000, the reference's
// overflow test).  A row of at most S edges keeps its scores in registers.
template <int S, typename Score>
__device__ __forceinline__ void softmax_row(int64_t row, bool has, int64_t e0, int64_t e1,
                                            int hl, Score&& score, float* __restrict__ alpha,
                                            float* __restrict__ lse) {
  const int64_t len = e1 - e0;
  float m, l;
  if (len <= S) {
    const bool on = hl < len;
    const float sc = on ? score(e0 + hl) : kNegInf;
    m = group_max<S>(sc);
    const float p = on ? __expf(sc - m) : 0.f;
    l = group_sum<S>(p);
    if (on) alpha[e0 + hl] = p * (1.f / l);
  } else {
    m = kNegInf;
    for (int64_t e = e0 + hl; e < e1; e += S) m = fmaxf(m, score(e));
    m = group_max<S>(m);
    l = 0.f;
    for (int64_t e = e0 + hl; e < e1; e += S) l += __expf(score(e) - m);
    l = group_sum<S>(l);
    const float inv = 1.f / l;
    for (int64_t e = e0 + hl; e < e1; e += S) alpha[e] = __expf(score(e) - m) * inv;
  }
  if (has && hl == 0) lse[row] = len > 0 ? m + __logf(l) : kNegInf;
}

// Scores stored per edge.
template <typename I>
__global__ __launch_bounds__(256) void segment_softmax_fwd_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, const float* __restrict__ scores,
    float* __restrict__ alpha, float* __restrict__ lse) {
  softmax_row_groups(row_ptr, n_rows, [&](int64_t row, auto slot, int hl) {
    const bool has = row < n_rows;
    const int64_t e0 = has ? static_cast<int64_t>(row_ptr[row]) : 0;
    const int64_t e1 = has ? static_cast<int64_t>(row_ptr[row + 1]) : 0;
    softmax_row<decltype(slot)::value>(row, has, e0, e1, hl,
                                       [&](int64_t e) { return scores[e]; }, alpha, lse);
  });
}

// The same with the scores read where a field lives: role 0 a source-node
// table read through col[e], role 1 a destination-node table (one score per
// row), role 2 one score per edge; each multiplied by `scale`.  This is the
// reference's stable-weighted row tile over a raw per-edge score
// (Translate.cpp:3004-3450, reducer_oracle.py:60-137) minus the value sum.
template <typename I, int ROLE>
__device__ __forceinline__ float role_score(const float* scores, const I* col, int64_t e,
                                            int64_t row, float scale) {
  if constexpr (ROLE == 0) return scale * scores[static_cast<int64_t>(col[e])];
  if constexpr (ROLE == 1) return scale * scores[row];
  return scale * scores[e];
}

template <typename I, int ROLE>
__global__ __launch_bounds__(256) void segment_softmax_gather_kernel(
    const I* __restrict__ row_ptr, const I* __restrict__ col, int64_t n_rows,
    const float* __restrict__ scores, float scale, float* __restrict__ alpha,
    float* __restrict__ lse) {
  softmax_row_groups(row_ptr, n_rows, [&](int64_t row, auto slot, int hl) {
    const bool has = row < n_rows;
    const int64_t e0 = has ? static_cast<int64_t>(row_ptr[row]) : 0;
    const int64_t e1 = has ? static_cast<int64_t>(row_ptr[row + 1]) : 0;
    softmax_row<decltype(slot)::value>(
        row, has, e0, e1, hl,
        [&](int64_t e) { return role_score<I, ROLE>(scores, col, e, row, scale); }, alpha, lse);
  });
}

// The segment softmax and the weighted sum of the value rows in one pass
// (the reference's row-centric tile: per row only (m, l) and the output,
// compiler/edge_nn_attention.py:127-338, reducer_oracle.py:60-137):
// out[i] = sum_e alpha_e value[col[e]], value rows of F <= FV floats.  Each
// lane forms its edges' weights, multiplies them into its running sums of
// the gathered rows, and the slot adds the lanes' sums.  alpha may be null.
template <int S, int FV, typename I, typename Score>
__device__ __forceinline__ void softmax_sum_row(int64_t row, bool has, int64_t e0, int64_t e1,
                                                int hl, Score&& score, const I* col,
                                                const float* __restrict__ value, int F,
                                                float* __restrict__ alpha,
                                                float* __restrict__ lse,
                                                float* __restrict__ out) {
  const int64_t len = e1 - e0;
  float m, l;
  float acc[FV];
#pragma unroll
  for (int k = 0; k < FV; ++k) acc[k] = 0.f;
  // Rows of exactly FV (a multiple of 4) floats are read as 16-byte vectors
  // (the caller passes a 16-byte aligned table).
  const bool vec = FV % 4 == 0 && F == FV;
  auto load_row = [&](int64_t e, float (&v)[FV]) {
    const float* src = value + static_cast<int64_t>(col[e]) * F;
    if (vec) {
#pragma unroll
      for (int k = 0; k < FV; k += 4) {
        const f32x4 q = *reinterpret_cast<const f32x4*>(src + k);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[k + r] = q[r];
      }
    } else {
#pragma unroll
      for (int k = 0; k < FV; ++k) v[k] = k < F ? src[k] : 0.f;
    }
  };
  auto add_row = [&](int64_t e, float a) {
    float v[FV];
    load_row(e, v);
#pragma unroll
    for (int k = 0; k < FV; ++k) acc[k] = fmaf(a, v[k], acc[k]);
  };
  if (len <= S) {
    // The row's value rows are requested with its scores, before the
    // reductions that form the weights.
    const bool on = hl < len;
    float v[FV];
    const float sc = on ? score(e0 + hl) : kNegInf;
    if (on) load_row(e0 + hl, v);
    m = group_max<S>(sc);
    const float p = on ? __expf(sc - m) : 0.f;
    l = group_sum<S>(p);
    if (on) {
      const float a = p * (1.f / l);
      if (alpha) alpha[e0 + hl] = a;
#pragma unroll
      for (int k = 0; k < FV; ++k) acc[k] = a * v[k];
    }
  } else {
    m = kNegInf;
    for (int64_t e = e0 + hl; e < e1; e += S) m = fmaxf(m, score(e));
    m = group_max<S>(m);
    l = 0.f;
    for (int64_t e = e0 + hl; e < e1; e += S) l += __expf(score(e) - m);
    l = group_sum<S>(l);
    const float inv = 1.f / l;
    for (int64_t e = e0 + hl; e < e1; e += S) {
      const float a = __expf(score(e) - m) * inv;
      if (alpha) alpha[e] = a;
      add_row(e, a);
    }
  }
#pragma unroll
  for (int k = 0; k < FV; ++k)
    if (k < F) acc[k] = group_sum<S>(acc[k]);
  if (has && hl == 0) {
    lse[row] = len > 0 ? m + __logf(l) : kNegInf;
#pragma unroll
    for (int k = 0; k < FV; ++k)
      if (k < F) out[row * F + k] = acc[k];
  }
}

template <typename I, int ROLE, int FV>
__global__ __launch_bounds__(256) void segment_softmax_sum_kernel(
    const I* __restrict__ row_ptr, const I* __restrict__ col, int64_t n_rows,
    const float* __restrict__ scores, float scale, const float* __restrict__ value, int F,
    float* __restrict__ alpha, float* __restrict__ lse, float* __restrict__ out) {
  softmax_row_groups(row_ptr, n_rows, [&](int64_t row, auto slot, int hl) {
    const bool has = row < n_rows;
    const int64_t e0 = has ? static_cast<int64_t>(row_ptr[row]) : 0;
    const int64_t e1 = has ? static_cast<int64_t>(row_ptr[row + 1]) : 0;
    softmax_sum_row<decltype(slot)::value, FV>(
        row, has, e0, e1, hl,
        [&](int64_t e) { return role_score<I, ROLE>(scores, col, e, row, scale); }, col, value,
        F, alpha, lse, out);
  });
}

// ds_e = alpha_e (dalpha_e - sum_row alpha dalpha).
template <typename I>
__global__ __launch_bounds__(256) void segment_softmax_bwd_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, const float* __restrict__ alpha,
    const float* __restrict__ dalpha, float* __restrict__ dscore) {
  softmax_row_groups(row_ptr, n_rows, [&](int64_t row, auto slot, int hl) {
    constexpr int S = decltype(slot)::value;
    const bool has = row < n_rows;
    const int64_t e0 = has ? static_cast<int64_t>(row_ptr[row]) : 0;
    const int64_t e1 = has ? static_cast<int64_t>(row_ptr[row + 1]) : 0;
    if (e1 - e0 <= S) {
      const bool on = hl < e1 - e0;
      const float al = on ? alpha[e0 + hl] : 0.f;
      const float da = on ? dalpha[e0 + hl] : 0.f;
      const float d = group_sum<S>(al * da);
      if (on) dscore[e0 + hl] = al * (da - d);
    } else {
      float d = 0.f;
      for (int64_t e = e0 + hl; e < e1; e += S) d += alpha[e] * dalpha[e];
      d = group_sum<S>(d);
      for (int64_t e = e0 + hl; e < e1; e += S) dscore[e] = alpha[e] * (dalpha[e] - d);
    }
  });
}

// out[c] = sum over rows r of p[r][c] in a fixed order, two levels: block
// (column block, slice) sums a contiguous range of rows with coalesced
// reads, then one thread per column adds the kColSlices slice sums.
constexpr int kColSlices = 16;

__global__ __launch_bounds__(256) void colsum_slice_kernel(const float* __restrict__ p,
                                                           int64_t rows, int n,
                                                           float* __restrict__ slices) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= n) return;
  const int64_t per = (rows + kColSlices - 1) / kColSlices;
  const int64_t r0 = blockIdx.y * per;
  const int64_t r1 = r0 + per < rows ? r0 + per : rows;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int64_t r = r0;
  for (; r + 4 <= r1; r += 4) {
    s0 += p[(r + 0) * n + c];
    s1 += p[(r + 1) * n + c];
    s2 += p[(r + 2) * n + c];
    s3 += p[(r + 3) * n + c];
  }
  for (; r < r1; ++r) s0 += p[r * n + c];
  slices[static_cast<int64_t>(blockIdx.y) * n + c] = (s0 + s1) + (s2 + s3);
}

// n_slices = 0 writes zeros (no reads).
__global__ __launch_bounds__(256) void colsum_final_kernel(const float* __restrict__ slices,
                                                           int n_slices, int n,
                                                           float* __restrict__ out) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= n) return;
  float s = 0.f;
  for (int k = 0; k < n_slices; ++k) s += slices[static_cast<int64_t>(k) * n + c];
  out[c] = s;
}

// Persistent backward grid: as many blocks as the device holds at once
// (`resident`, from the occupancy query of the kernel), chunks of whole
// 256-edge steps.
int mlp_bwd_blocks(int64_t n_edges, int64_t resident, int64_t* chunk) {
  int64_t c = ceil_div(n_edges, resident > 0 ? resident : 1);
  c = align_up(static_cast<size_t>(c < 256 ? 256 : c), 256);
  *chunk = c;
  return static_cast<int>(ceil_div(n_edges, c));
}

// need_data: the segment rows are read (some edge exists); with no edges an
// empty field may come with a null pointer.
int check_mlp(const tgx_edge_mlp* mlp, MlpView* view, bool need_data) {
  TGX_REQUIRE(mlp, "null mlp");
  TGX_REQUIRE(mlp->n_layers >= 1 && mlp->n_layers <= kMaxLayers, "1 to %d linear layers",
              kMaxLayers);
  TGX_REQUIRE(mlp->width == 16 || mlp->width == 24 || mlp->width == 32 || mlp->width == 64,
              "padded width must be 16, 24, 32 or 64");
  TGX_REQUIRE(mlp->n_segments >= 1 && mlp->n_segments <= kMaxSegments,
              "1 to %d input segments", kMaxSegments);
  TGX_REQUIRE(mlp->weights_dev, "null weights");
  int in_width = 0;
  for (int s = 0; s < mlp->n_segments; ++s) {
    TGX_REQUIRE(mlp->seg_role[s] >= TGX_ROLE_SRC && mlp->seg_role[s] <= TGX_ROLE_EDGE,
                "bad segment role");
    TGX_REQUIRE(mlp->seg_width[s] > 0 && mlp->seg_stride[s] >= mlp->seg_width[s] &&
                    (mlp->seg_dev[s] || !need_data),
                "bad segment %d", s);
    in_width += mlp->seg_width[s];
  }
  TGX_REQUIRE(in_width <= mlp->width, "inputs (%d) exceed the padded width", in_width);
  for (int l = 0; l + 1 < mlp->n_layers; ++l)
    TGX_REQUIRE(mlp->act[l] >= TGX_ACT_IDENTITY &&
                    mlp->act[l] <= (TGX_NN_MATH ? TGX_ACT_POW : TGX_ACT_HARDSWISH),
                "bad activation code");
  MlpView v{};
  v.att_fold = -1;
  v.n_layers = mlp->n_layers;
  v.in_width = in_width;
  int n_in = in_width;
  for (int l = 0; l < kMaxLayers; ++l) {
    int n_out = mlp->width;
    if (l < mlp->n_layers && mlp->out_width[l] != 0) n_out = mlp->out_width[l];
    if (l + 1 == mlp->n_layers) TGX_REQUIRE(n_out == 1 || mlp->out_width[l] == 0,
                                            "the last layer has one output");
    TGX_REQUIRE(n_out >= 1 && n_out <= mlp->width, "layer %d output width %d outside 1..%d", l,
                n_out, mlp->width);
    v.n_out[l] = n_out;
    v.nb_in[l] = (n_in + 3) / 4;
    n_in = n_out;
  }
  for (int l = 0; l < kMaxLayers; ++l) {
    v.act[l] = l + 1 < mlp->n_layers ? mlp->act[l] : TGX_ACT_IDENTITY;
    v.param[l] = mlp->act_param[l];
    v.param2[l] = mlp->act_param2[l];
    v.norm[l] = 0;
    v.eps[l] = 0.f;
    if (l < mlp->n_layers && mlp->norm[l]) {
      TGX_REQUIRE(TGX_NN_MATH, "internal: a normalized chain on the kernels without LayerNorm");
      TGX_REQUIRE(l + 1 < mlp->n_layers, "the last layer cannot be normalized");
      TGX_REQUIRE(mlp->width <= 32, "normalized layers need a padded width of at most 32");
      TGX_REQUIRE(mlp->norm_eps[l] >= 0.f && mlp->norm_eps[l] <= 1e30f,
                  "norm_eps must be finite and >= 0");
      TGX_REQUIRE(v.n_out[l] >= 1, "empty normalized layer");
      v.norm[l] = 1;
      v.eps[l] = mlp->norm_eps[l];
    }
  }
  v.nw = block_floats(mlp);
  v.w = mlp->weights_dev;
  v.n_seg = mlp->n_segments;
  int k = 0;
  for (int s = 0; s < kMaxSegments; ++s) {
    const bool on = s < mlp->n_segments;
    v.role[s] = on ? mlp->seg_role[s] : TGX_ROLE_EDGE;
    v.width[s] = on ? mlp->seg_width[s] : 0;
    v.stride[s] = on ? mlp->seg_stride[s] : 0;
    v.ptr[s] = on ? mlp->seg_dev[s] : nullptr;
    v.grad[s] = nullptr;
    v.off[s] = k;
    if (on) k += mlp->seg_width[s];
  }
  *view = v;
  return TGX_OK;
}

template <typename I, int W>
void launch_fwd(int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                float* scores, hipStream_t s) {
  const int64_t blocks = ceil_div(E, 256);
  if constexpr (!TGX_NN_MATH)   // one layer: no function, never the second set
    if (L == 1) edge_mlp_fwd_kernel<I, W, 1><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
  if (L == 2) edge_mlp_fwd_kernel<I, W, 2><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
  if (L == 3) edge_mlp_fwd_kernel<I, W, 3><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
}

#if TGX_NN_INDEX == 64
// Blocks of edge_mlp_bwd_kernel<int64_t, W, L> resident on the current
// device at once: per CU, the smaller of what the 160 KB of LDS and the 512
// registers per SIMD lane allow (each 256-thread block puts one wave on each
// of the CU's four SIMDs), from the kernel's attributes; the larger of that
// and the runtime's occupancy query.  The int64 instance sizes int32 launches
// too: the workspace query has no index width, and it must size the partial
// buffer for the same grid the launch uses.  No block waits for another, so a
// grid larger than what is resident only costs a second round of blocks.
template <int W, int L>
int64_t bwd_resident_blocks() {
  // Per device, computed once; concurrent first calls compute the same value.
  static std::atomic<int64_t> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int64_t known = cached[dev].load(std::memory_order_relaxed);
  if (known == 0) {
    const void* fn = reinterpret_cast<const void*>(edge_mlp_bwd_kernel<int64_t, W, L, false>);
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess)
      per_cu = 0;
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, fn) == hipSuccess && attr.numRegs > 0) {
      const int regs = (attr.numRegs + 7) / 8 * 8;
      const int by_regs = 512 / regs;
      const int by_lds = attr.sharedSizeBytes > 0
                             ? static_cast<int>((160 * 1024) / attr.sharedSizeBytes)
                             : by_regs;
      const int mine = by_regs < by_lds ? by_regs : by_lds;
      if (mine > per_cu) per_cu = mine;
    }
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    known = static_cast<int64_t>(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    cached[dev].store(known, std::memory_order_relaxed);
  }
  return known;
}

int64_t resident_blocks_any(int W, int L) {
  if constexpr (!TGX_NN_MATH) {
    if (L == 1)
      return W == 16 ? bwd_resident_blocks<16, 1>()
                     : W == 24 ? bwd_resident_blocks<24, 1>() : bwd_resident_blocks<32, 1>();
  }
  if (W == 16) return L <= 2 ? bwd_resident_blocks<16, 2>() : bwd_resident_blocks<16, 3>();
  if (W == 24) return L <= 2 ? bwd_resident_blocks<24, 2>() : bwd_resident_blocks<24, 3>();
  return L <= 2 ? bwd_resident_blocks<32, 2>() : bwd_resident_blocks<32, 3>();
}
#endif

template <typename I, int W, bool SEED>
void launch_bwd(int L, const I* col, const int32_t* dst, int64_t E, int blocks, int64_t chunk,
                const MlpView& v, const float* ds, float* partial, const float* seed, int hw,
                hipStream_t s) {
  if constexpr (!TGX_NN_MATH && !SEED) {
    // Chains whose hidden layers all use LeakyReLU (the reference's GAT
    // score network) or all ReLU take a kernel built for that activation.
    bool leaky = L >= 2, relu = L >= 2;
    for (int l = 0; l + 1 < L; ++l) {
      leaky = leaky && v.act[l] == TGX_ACT_LEAKY_RELU;
      relu = relu && v.act[l] == TGX_ACT_RELU;
    }
    if (leaky) {
      if (L == 2)
        edge_mlp_bwd_kernel<I, W, 2, SEED, TGX_ACT_LEAKY_RELU><<<blocks, 256, 0, s>>>(
            col, dst, E, chunk, v, ds, partial, seed, hw);
      else
        edge_mlp_bwd_kernel<I, W, 3, SEED, TGX_ACT_LEAKY_RELU><<<blocks, 256, 0, s>>>(
            col, dst, E, chunk, v, ds, partial, seed, hw);
      return;
    }
    if (relu) {
      if (L == 2)
        edge_mlp_bwd_kernel<I, W, 2, SEED, TGX_ACT_RELU><<<blocks, 256, 0, s>>>(
            col, dst, E, chunk, v, ds, partial, seed, hw);
      else
        edge_mlp_bwd_kernel<I, W, 3, SEED, TGX_ACT_RELU><<<blocks, 256, 0, s>>>(
            col, dst, E, chunk, v, ds, partial, seed, hw);
      return;
    }
  }
  if constexpr (!TGX_NN_MATH)
    if (L == 1)
      edge_mlp_bwd_kernel<I, W, 1, SEED><<<blocks, 256, 0, s>>>(col, dst, E, chunk, v, ds,
                                                                partial, seed, hw);
  if (L == 2)
    edge_mlp_bwd_kernel<I, W, 2, SEED><<<blocks, 256, 0, s>>>(col, dst, E, chunk, v, ds,
                                                              partial, seed, hw);
  if (L == 3)
    edge_mlp_bwd_kernel<I, W, 3, SEED><<<blocks, 256, 0, s>>>(col, dst, E, chunk, v, ds,
                                                              partial, seed, hw);
}

template <typename I, int W>
void launch_hidden(int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                   float* hidden, int hw, hipStream_t s) {
  const int64_t blocks = ceil_div(E, 256);
  if constexpr (!TGX_NN_MATH)
    if (L == 1) edge_mlp_hidden_kernel<I, W, 1><<<blocks, 256, 0, s>>>(col, dst, E, v, hidden, hw);
  if (L == 2) edge_mlp_hidden_kernel<I, W, 2><<<blocks, 256, 0, s>>>(col, dst, E, v, hidden, hw);
  if (L == 3) edge_mlp_hidden_kernel<I, W, 3><<<blocks, 256, 0, s>>>(col, dst, E, v, hidden, hw);
}

template <typename I>
void dispatch_fwd(int W, int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                  float* scores, hipStream_t s) {
  if (W == 16) launch_fwd<I, 16>(L, col, dst, E, v, scores, s);
  if (W == 24) launch_fwd<I, 24>(L, col, dst, E, v, scores, s);
  if (W == 32) launch_fwd<I, 32>(L, col, dst, E, v, scores, s);
  if (W == 64) launch_fwd<I, 64>(L, col, dst, E, v, scores, s);
}

template <typename I, bool SEED = false>
void dispatch_bwd(int W, int L, const I* col, const int32_t* dst, int64_t E, int blocks,
                  int64_t chunk, const MlpView& v, const float* ds, float* partial,
                  hipStream_t s, const float* seed = nullptr, int hw = 0) {
  if (W == 16) launch_bwd<I, 16, SEED>(L, col, dst, E, blocks, chunk, v, ds, partial, seed, hw, s);
  if (W == 24) launch_bwd<I, 24, SEED>(L, col, dst, E, blocks, chunk, v, ds, partial, seed, hw, s);
  if (W == 32) launch_bwd<I, 32, SEED>(L, col, dst, E, blocks, chunk, v, ds, partial, seed, hw, s);
}

template <typename I>
void dispatch_hidden(int W, int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                     float* hidden, int hw, hipStream_t s) {
  if (W == 16) launch_hidden<I, 16>(L, col, dst, E, v, hidden, hw, s);
  if (W == 24) launch_hidden<I, 24>(L, col, dst, E, v, hidden, hw, s);
  if (W == 32) launch_hidden<I, 32>(L, col, dst, E, v, hidden, hw, s);
}

// Width of the last layer's input: the previous layer's real output, or the
// concatenated input of a one-layer network.
[[maybe_unused]] int last_input_width(const tgx_edge_mlp* mlp, const MlpView& v) {
  return mlp->n_layers > 1 ? v.n_out[mlp->n_layers - 2] : v.in_width;
}

}  // namespace

// The launches for this build's column index type (declared in
// tgx_nn_common.h).
namespace mlp {
using IndexT = std::conditional<TGX_NN_INDEX == 64, int64_t, int32_t>::type;

void TGX_TIER(mlp_fwd)(int W, int L, const IndexT* col, const int32_t* dst, int64_t E,
                       const MlpView& v, float* scores, hipStream_t s) {
  dispatch_fwd(W, L, col, dst, E, v, scores, s);
}

void TGX_TIER(mlp_hidden)(int W, int L, const IndexT* col, const int32_t* dst, int64_t E,
                          const MlpView& v, float* hidden, int hw, hipStream_t s) {
  dispatch_hidden(W, L, col, dst, E, v, hidden, hw, s);
}

void TGX_TIER(mlp_bwd)(bool seeded, int W, int L, const IndexT* col, const int32_t* dst,
                       int64_t E, int blocks, int64_t chunk, const MlpView& v, const float* ds,
                       float* partial, const float* seed, int hw, hipStream_t s) {
  if (seeded)
    dispatch_bwd<IndexT, true>(W, L, col, dst, E, blocks, chunk, v, ds, partial, s, seed, hw);
  else
    dispatch_bwd<IndexT, false>(W, L, col, dst, E, blocks, chunk, v, ds, partial, s);
}

#if TGX_NN_INDEX == 64
int64_t TGX_TIER(mlp_bwd_resident)(int W, int L) { return resident_blocks_any(W, L); }
#endif
}  // namespace mlp
}  // namespace tgx

#if TGX_NN_INDEX == 32

using namespace tgx;

TGX_NN_ENTRY(tgx_edge_mlp_scores)(const void* col, const int32_t* dst_index, int idx_bits,
                                  int64_t n_edges, const tgx_edge_mlp* mlp, float* scores,
                                  void* stream) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_scores_math(col, dst_index, idx_bits, n_edges, mlp, scores,
                                            stream));
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  if (n_edges == 0) return TGX_OK;
  TGX_REQUIRE(col && dst_index && scores, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("edge_mlp_fwd_kernel", s);
  if (idx_bits == 32)
    tgx::mlp::TGX_TIER(mlp_fwd)(mlp->width, mlp->n_layers, static_cast<const int32_t*>(col),
                                dst_index, n_edges, v, scores, s);
  else
    tgx::mlp::TGX_TIER(mlp_fwd)(mlp->width, mlp->n_layers, static_cast<const int64_t*>(col),
                                dst_index, n_edges, v, scores, s);
  TGX_LAUNCHED("edge_mlp_fwd_kernel");
  return TGX_OK;
}

TGX_NN_ENTRY(tgx_edge_mlp_backward_workspace)(int64_t n_edges, const tgx_edge_mlp* mlp,
                                              size_t* bytes) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_backward_workspace_math(n_edges, mlp, bytes));
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  const int64_t n = static_cast<int64_t>(mlp->n_layers) * block_floats(mlp);
  int64_t chunk = 0;
  const int blocks = n_edges == 0 ? 0
                     : mlp->width == 64
                         ? TGX_TIER(outer_blocks)(n_edges, &chunk)
                         : mlp_bwd_blocks(n_edges, tgx::mlp::TGX_TIER(mlp_bwd_resident)(mlp->width, mlp->n_layers),
                                          &chunk);
  size_t planes = 0;
  if (mlp->width == 64)
    planes = 2 * align_up(static_cast<size_t>(mlp->n_layers) * n_edges * 64 * sizeof(float));
  *bytes = align_up(static_cast<size_t>(blocks) * n * sizeof(float)) +
           align_up(static_cast<size_t>(kColSlices) * n * sizeof(float)) + planes;
  return TGX_OK;
}

namespace {

// The backward of a one-output chain for a checked view `v`: the score
// gradients come from dscore, or are formed per edge from v's attention
// fields (dscore null).
int mlp_backward_body(const void* col, const int32_t* dst_index, int idx_bits, int64_t n_edges,
                      const tgx_edge_mlp* mlp, MlpView& v, const float* dscore,
                      float* dweights, float* const* dseg, void* workspace,
                      size_t workspace_bytes, void* stream) {
  TGX_REQUIRE(dweights && dseg, "null pointer");
  const int n = mlp->n_layers * block_floats(mlp);
  hipStream_t s = as_stream(stream);
  if (n_edges == 0) {
    // Zero sums, written by a kernel rather than a memset.
    colsum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(nullptr, 0, n, dweights);
    TGX_LAUNCHED("colsum_final_kernel");
    return TGX_OK;
  }
  TGX_REQUIRE(col && dst_index && (dscore || v.att_lse) && workspace, "null pointer");
  for (int k = 0; k < mlp->n_segments; ++k) {
    TGX_REQUIRE(dseg[k], "null gradient for segment %d", k);
    v.grad[k] = dseg[k];
  }
  size_t need = 0;
  TGX_REQUIRE(TGX_TIER(tgx_edge_mlp_backward_workspace)(n_edges, mlp, &need) == TGX_OK &&
                  workspace_bytes >= need,
              "workspace too small");
  int64_t chunk = 0;
  const int blocks =
      mlp->width == 64
          ? TGX_TIER(outer_blocks)(n_edges, &chunk)
          : mlp_bwd_blocks(n_edges, tgx::mlp::TGX_TIER(mlp_bwd_resident)(mlp->width, mlp->n_layers), &chunk);
  const size_t part_bytes = align_up(static_cast<size_t>(blocks) * n * sizeof(float));
  const size_t slice_bytes = align_up(static_cast<size_t>(kColSlices) * n * sizeof(float));
  float* partial = static_cast<float*>(workspace);
  float* slices = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes);
  if (mlp->width == 64) {
    const size_t plane = align_up(static_cast<size_t>(mlp->n_layers) * n_edges * 64 * sizeof(float));
    float* acts = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes + slice_bytes);
    float* dz = reinterpret_cast<float*>(reinterpret_cast<char*>(acts) + plane);
    const int st = tgx::mlp::TGX_TIER(planes_backward)(mlp->n_layers, idx_bits, col, dst_index,
                                                       n_edges, v, dscore, acts, dz, blocks,
                                                       chunk, partial, s);
    if (st != TGX_OK) return st;
  } else {
    TGX_PROFILE("edge_mlp_bwd_kernel", s);
    if (idx_bits == 32)
      tgx::mlp::TGX_TIER(mlp_bwd)(false, mlp->width, mlp->n_layers,
                                  static_cast<const int32_t*>(col), dst_index, n_edges, blocks,
                                  chunk, v, dscore, partial, nullptr, 0, s);
    else
      tgx::mlp::TGX_TIER(mlp_bwd)(false, mlp->width, mlp->n_layers,
                                  static_cast<const int64_t*>(col), dst_index, n_edges, blocks,
                                  chunk, v, dscore, partial, nullptr, 0, s);
    TGX_LAUNCHED("edge_mlp_bwd_kernel");
  }
  {
    TGX_PROFILE("colsum_kernels", s);
    colsum_slice_kernel<<<dim3(ceil_div(n, 256), kColSlices), 256, 0, s>>>(partial, blocks,
                                                                           n, slices);
    TGX_LAUNCHED("colsum_slice_kernel");
    colsum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(slices, kColSlices, n, dweights);
    TGX_LAUNCHED("colsum_final_kernel");
  }
  return TGX_OK;
}

}  // namespace

TGX_NN_ENTRY(tgx_edge_mlp_backward)(const void* col, const int32_t* dst_index, int idx_bits,
                                    int64_t n_edges, const tgx_edge_mlp* mlp,
                                    const float* dscore, float* dweights, float* const* dseg,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_backward_math(col, dst_index, idx_bits, n_edges, mlp, dscore,
                                              dweights, dseg, workspace, workspace_bytes,
                                              stream));
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  const int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(n_edges == 0 || dscore, "null pointer");
  return mlp_backward_body(col, dst_index, idx_bits, n_edges, mlp, v, dscore, dweights, dseg,
                           workspace, workspace_bytes, stream);
}

TGX_NN_ENTRY(tgx_edge_mlp_attention_backward)(
    const void* col, const int32_t* dst_index, int idx_bits, int64_t n_edges,
    const tgx_edge_mlp* mlp, const float* lse, const float* out, const float* dout,
    const float* value, int32_t value_width, float* alpha, int fold_segment, float* dweights,
    float* const* dseg, void* workspace, size_t workspace_bytes, void* stream) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_attention_backward_math(
                       col, dst_index, idx_bits, n_edges, mlp, lse, out, dout, value,
                       value_width, alpha, fold_segment, dweights, dseg, workspace,
                       workspace_bytes, stream));
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  TGX_REQUIRE(value_width >= 1, "value_width must be >= 1");
  MlpView v;
  const int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(fold_segment >= -1 && fold_segment < mlp->n_segments,
              "fold_segment must be -1 or a segment index");
  if (fold_segment >= 0)
    TGX_REQUIRE(mlp->seg_width[fold_segment] == value_width,
                "the folded segment's width (%d) must equal value_width (%d)",
                mlp->seg_width[fold_segment], value_width);
  if (n_edges > 0) {
    TGX_REQUIRE(lse && out && dout && value, "null pointer");
    if (value_width % 4 == 0)
      TGX_REQUIRE(reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(dout) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(value) % 16 == 0,
                  "out, dout and value rows of a multiple of 4 floats need 16-byte alignment");
  }
  v.att_lse = lse;
  v.att_out = out;
  v.att_dout = dout;
  v.att_value = value;
  v.att_alpha = alpha;
  v.att_width = value_width;
  v.att_fold = fold_segment;
  return mlp_backward_body(col, dst_index, idx_bits, n_edges, mlp, v, nullptr, dweights, dseg,
                           workspace, workspace_bytes, stream);
}

#if !TGX_NN_MATH
extern "C" int tgx_segment_softmax_fwd(const void* row_ptr, int idx_bits, int64_t n_rows,
                                       const float* scores, float* alpha, float* lse,
                                       void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0, "negative size");
  if (n_rows == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && lse, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("segment_softmax_fwd_kernel", s);
  if (idx_bits == 32)
    segment_softmax_fwd_kernel<<<ceil_div(n_rows, 4 * kSoftmaxRowsPerWave), 256, 0, s>>>(
        static_cast<const int32_t*>(row_ptr), n_rows, scores, alpha, lse);
  else
    segment_softmax_fwd_kernel<<<ceil_div(n_rows, 4 * kSoftmaxRowsPerWave), 256, 0, s>>>(
        static_cast<const int64_t*>(row_ptr), n_rows, scores, alpha, lse);
  TGX_LAUNCHED("segment_softmax_fwd_kernel");
  return TGX_OK;
}

namespace tgx {
namespace {
template <typename I>
void launch_gather_softmax(const I* row_ptr, const I* col, int64_t n_rows,
                           const float* scores, int role, float scale, float* alpha,
                           float* lse, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>(ceil_div(n_rows, 4 * kSoftmaxRowsPerWave));
  if (role == TGX_ROLE_SRC)
    segment_softmax_gather_kernel<I, 0><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                               scale, alpha, lse);
  else if (role == TGX_ROLE_DST)
    segment_softmax_gather_kernel<I, 1><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                               scale, alpha, lse);
  else
    segment_softmax_gather_kernel<I, 2><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                               scale, alpha, lse);
}
}  // namespace
}  // namespace tgx

extern "C" int tgx_segment_softmax_gather_fwd(const void* row_ptr, const void* col,
                                              int idx_bits, int64_t n_rows,
                                              const float* scores, int role, float scale,
                                              float* alpha, float* lse, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0, "negative size");
  TGX_REQUIRE(role == TGX_ROLE_SRC || role == TGX_ROLE_DST || role == TGX_ROLE_EDGE,
              "role must be TGX_ROLE_SRC, TGX_ROLE_DST or TGX_ROLE_EDGE");
  if (n_rows == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && lse, "null pointer");
  TGX_REQUIRE(role != TGX_ROLE_SRC || col, "source-role scores need col");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("segment_softmax_gather_kernel", s);
  if (idx_bits == 32)
    launch_gather_softmax(static_cast<const int32_t*>(row_ptr), static_cast<const int32_t*>(col),
                          n_rows, scores, role, scale, alpha, lse, s);
  else
    launch_gather_softmax(static_cast<const int64_t*>(row_ptr), static_cast<const int64_t*>(col),
                          n_rows, scores, role, scale, alpha, lse, s);
  TGX_LAUNCHED("segment_softmax_gather_kernel");
  return TGX_OK;
}

namespace tgx {
namespace {
template <typename I, int ROLE>
void launch_softmax_sum(const I* row_ptr, const I* col, int64_t n_rows, const float* scores,
                        float scale, const float* value, int F, float* alpha, float* lse,
                        float* out, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>(ceil_div(n_rows, 4 * kSoftmaxRowsPerWave));
  if (F == 1)
    segment_softmax_sum_kernel<I, ROLE, 1><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                                   scale, value, F, alpha, lse,
                                                                   out);
  else if (F <= 2)
    segment_softmax_sum_kernel<I, ROLE, 2><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                                   scale, value, F, alpha, lse,
                                                                   out);
  else if (F <= 4)
    segment_softmax_sum_kernel<I, ROLE, 4><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                                   scale, value, F, alpha, lse,
                                                                   out);
  else
    segment_softmax_sum_kernel<I, ROLE, 8><<<blocks, 256, 0, s>>>(row_ptr, col, n_rows, scores,
                                                                   scale, value, F, alpha, lse,
                                                                   out);
}

template <typename I>
void launch_softmax_sum_role(const I* row_ptr, const I* col, int64_t n_rows,
                             const float* scores, int role, float scale, const float* value,
                             int F, float* alpha, float* lse, float* out, hipStream_t s) {
  if (role == TGX_ROLE_SRC)
    launch_softmax_sum<I, 0>(row_ptr, col, n_rows, scores, scale, value, F, alpha, lse, out, s);
  else if (role == TGX_ROLE_DST)
    launch_softmax_sum<I, 1>(row_ptr, col, n_rows, scores, scale, value, F, alpha, lse, out, s);
  else
    launch_softmax_sum<I, 2>(row_ptr, col, n_rows, scores, scale, value, F, alpha, lse, out, s);
}
}  // namespace
}  // namespace tgx

extern "C" int tgx_segment_softmax_sum_fwd(const void* row_ptr, const void* col, int idx_bits,
                                           int64_t n_rows, const float* scores, int role,
                                           float scale, const float* value, int F,
                                           float* alpha, float* lse, float* out,
                                           void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0, "negative size");
  TGX_REQUIRE(role == TGX_ROLE_SRC || role == TGX_ROLE_DST || role == TGX_ROLE_EDGE,
              "role must be TGX_ROLE_SRC, TGX_ROLE_DST or TGX_ROLE_EDGE");
  if (F < 1 || F > 8) {
    set_error("the fused softmax sum takes value rows of 1 to 8 floats (got %d)", F);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE((F != 4 && F != 8) || reinterpret_cast<uintptr_t>(value) % 16 == 0,
              "value rows of 4 or 8 floats need a 16-byte aligned table");
  if (n_rows == 0) return TGX_OK;
  // col, scores and value are read only for rows with edges.
  TGX_REQUIRE(row_ptr && lse && out, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("segment_softmax_sum_kernel", s);
  if (idx_bits == 32)
    launch_softmax_sum_role(static_cast<const int32_t*>(row_ptr),
                            static_cast<const int32_t*>(col), n_rows, scores, role, scale, value,
                            F, alpha, lse, out, s);
  else
    launch_softmax_sum_role(static_cast<const int64_t*>(row_ptr),
                            static_cast<const int64_t*>(col), n_rows, scores, role, scale, value,
                            F, alpha, lse, out, s);
  TGX_LAUNCHED("segment_softmax_sum_kernel");
  return TGX_OK;
}

extern "C" int tgx_segment_softmax_bwd(const void* row_ptr, int idx_bits, int64_t n_rows,
                                       const float* alpha, const float* dalpha, float* dscore,
                                       void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0, "negative size");
  if (n_rows == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("segment_softmax_bwd_kernel", s);
  if (idx_bits == 32)
    segment_softmax_bwd_kernel<<<ceil_div(n_rows, 4 * kSoftmaxRowsPerWave), 256, 0, s>>>(
        static_cast<const int32_t*>(row_ptr), n_rows, alpha, dalpha, dscore);
  else
    segment_softmax_bwd_kernel<<<ceil_div(n_rows, 4 * kSoftmaxRowsPerWave), 256, 0, s>>>(
        static_cast<const int64_t*>(row_ptr), n_rows, alpha, dalpha, dscore);
  TGX_LAUNCHED("segment_softmax_bwd_kernel");
  return TGX_OK;
}

#endif  // !TGX_NN_MATH

TGX_NN_ENTRY(tgx_edge_mlp_hidden)(const void* col, const int32_t* dst_index, int idx_bits,
                                  int64_t n_edges, const tgx_edge_mlp* mlp, float* hidden,
                                  int32_t hidden_width, void* stream) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_hidden_math(col, dst_index, idx_bits, n_edges, mlp, hidden,
                                            hidden_width, stream));
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  if (mlp->width == 64) {
    set_error("edge-network sums support padded widths 16, 24 and 32");
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(hidden_width == last_input_width(mlp, v),
              "hidden_width %d is not the last layer's input width %d", hidden_width,
              last_input_width(mlp, v));
  if (n_edges == 0) return TGX_OK;
  TGX_REQUIRE(col && dst_index && hidden, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("edge_mlp_hidden_kernel", s);
  if (idx_bits == 32)
    tgx::mlp::TGX_TIER(mlp_hidden)(mlp->width, mlp->n_layers, static_cast<const int32_t*>(col),
                                   dst_index, n_edges, v, hidden, hidden_width, s);
  else
    tgx::mlp::TGX_TIER(mlp_hidden)(mlp->width, mlp->n_layers, static_cast<const int64_t*>(col),
                                   dst_index, n_edges, v, hidden, hidden_width, s);
  TGX_LAUNCHED("edge_mlp_hidden_kernel");
  return TGX_OK;
}

TGX_NN_ENTRY(tgx_edge_mlp_backward_seeded)(const void* col, const int32_t* dst_index,
                                           int idx_bits, int64_t n_edges,
                                           const tgx_edge_mlp* mlp, const float* seed,
                                           int32_t seed_width, float* dweights,
                                           float* const* dseg, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  TGX_TO_MATH(mlp, tgx_edge_mlp_backward_seeded_math(col, dst_index, idx_bits, n_edges, mlp, seed,
                                                     seed_width, dweights, dseg, workspace,
                                                     workspace_bytes, stream));
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v, n_edges > 0);
  if (st != TGX_OK) return st;
  if (mlp->width == 64) {
    set_error("edge-network sums support padded widths 16, 24 and 32");
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(seed_width == last_input_width(mlp, v),
              "seed_width %d is not the last layer's input width %d", seed_width,
              last_input_width(mlp, v));
  TGX_REQUIRE(dweights && dseg, "null pointer");
  const int n = mlp->n_layers * block_floats(mlp);
  hipStream_t s = as_stream(stream);
  if (n_edges == 0) {
    colsum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(nullptr, 0, n, dweights);
    TGX_LAUNCHED("colsum_final_kernel");
    return TGX_OK;
  }
  TGX_REQUIRE(col && dst_index && seed && workspace, "null pointer");
  for (int k = 0; k < mlp->n_segments; ++k) {
    TGX_REQUIRE(dseg[k], "null gradient for segment %d", k);
    v.grad[k] = dseg[k];
  }
  size_t need = 0;
  TGX_REQUIRE(TGX_TIER(tgx_edge_mlp_backward_workspace)(n_edges, mlp, &need) == TGX_OK &&
                  workspace_bytes >= need,
              "workspace too small");
  int64_t chunk = 0;
  const int blocks = mlp_bwd_blocks(n_edges, tgx::mlp::TGX_TIER(mlp_bwd_resident)(mlp->width, mlp->n_layers), &chunk);
  const size_t part_bytes = align_up(static_cast<size_t>(blocks) * n * sizeof(float));
  float* partial = static_cast<float*>(workspace);
  float* slices = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes);
  {
    TGX_PROFILE("edge_mlp_bwd_seeded_kernel", s);
    if (idx_bits == 32)
      tgx::mlp::TGX_TIER(mlp_bwd)(true, mlp->width, mlp->n_layers,
                                  static_cast<const int32_t*>(col), dst_index, n_edges, blocks,
                                  chunk, v, nullptr, partial, seed, seed_width, s);
    else
      tgx::mlp::TGX_TIER(mlp_bwd)(true, mlp->width, mlp->n_layers,
                                  static_cast<const int64_t*>(col), dst_index, n_edges, blocks,
                                  chunk, v, nullptr, partial, seed, seed_width, s);
    TGX_LAUNCHED("edge_mlp_bwd_seeded_kernel");
  }
  {
    TGX_PROFILE("colsum_kernels", s);
    colsum_slice_kernel<<<dim3(ceil_div(n, 256), kColSlices), 256, 0, s>>>(partial, blocks,
                                                                           n, slices);
    TGX_LAUNCHED("colsum_slice_kernel");
    colsum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(slices, kColSlices, n, dweights);
    TGX_LAUNCHED("colsum_final_kernel");
  }
  return TGX_OK;
}

#endif  // TGX_NN_INDEX == 32
