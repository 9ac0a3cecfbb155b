// 64-wide score networks: the backward in two passes (the fused form of
// tgx_nn.hip would need up to 192 live accumulator registers per lane).
// The per-edge pass replays the chain and writes every layer's input and
// pre-activation gradient to workspace planes; outer_sum_kernel then sums
// their products per block, and tgx_nn.hip's column sums add the blocks in a
// fixed order.
#include <hip/hip_runtime.h>

#include "tgx_nn_common.h"
#include "tgx_profile.h"

namespace tgx {
namespace mlp {
namespace {

// The 64-wide chain's backward in two passes (its fused form would need 192
// live accumulator registers per lane for three layers): the per-edge pass
// writes, for every layer l, its input acts[l][e][:] and the gradient of its
// pre-activation output dz[l][e][:] (width W) to workspace planes, and the
// input gradient split per segment dseg[s][e][:width_s]; outer_sum_kernel
// then sums the products.
template <typename I, int W, int L>
__global__ __launch_bounds__(256) void edge_mlp_planes_kernel(
    const I* __restrict__ col, const int32_t* __restrict__ dst, int64_t n_edges, MlpView m,
    const float* __restrict__ dscore, float* __restrict__ acts, float* __restrict__ dz_out) {
  cfloat* wg = scalar_weights(m.w);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_edges) return;
  const int64_t plane = n_edges * W;
  float a[W];                       // input of the current layer
  float z[L > 1 ? L - 1 : 1][W];    // pre-activations of the hidden layers
  gather_inputs<I, W>(m, e, col, dst, a);
  static_for<L>([&](auto lc) TGX_INLINE_LAMBDA {
    constexpr int l = decltype(lc)::value;
    float* out = acts + l * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{a[i], a[i + 1], a[i + 2], a[i + 3]};
    if constexpr (l + 1 < L) {
      linear<W>(wg + l * (W * W + W), a, z[l], m.n_out[l], m.nb_in[l]);
      activate_all<W>(z[l], a, m.act[l], m.param[l], m.param2[l], m.nb_in[l + 1],
                    m.n_out[l]);
    }
  });
  // Last layer: one output, gradient ds: read, or formed here from the
  // replayed score (attention backward from the saved logsumexp).
  float g[W];
  float alpha = 0.f;   // attention backward: the edge's recomputed weight
  {
    cfloat* wl = wg + (L - 1) * (W * W + W);
    const float ds = m.att_lse != nullptr
                         ? attention_score_grad(m, e, dst[e], static_cast<int64_t>(col[e]),
                                                linear_out1<W>(wl, a, m.nb_in[L - 1]), alpha)
                         : dscore[e];
    float* out = dz_out + (L - 1) * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{i == 0 ? ds : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < W; ++i) g[i] = ds * wl[i];   // d a[L-1]
  }
  static_for<L - 1>([&](auto kc) TGX_INLINE_LAMBDA {
    constexpr int l = L - 2 - decltype(kc)::value;
    float dzl[W];
    activate_grad_all<W>(z[l], g, dzl, m.act[l], m.param[l], m.param2[l],
                         m.nb_in[l + 1], m.n_out[l]);
#pragma unroll
    for (int o = 0; o < W; ++o) pin(dzl[o]);
    float* out = dz_out + l * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{dzl[i], dzl[i + 1], dzl[i + 2], dzl[i + 3]};
    // d a[l] = W_l^T dz.
    linear_t<W>(wg + l * (W * W + W), dzl, g, m.n_out[l], m.nb_in[l]);
  });
  // g = d x: split per segment.
  scatter_segments<W>(m, e, g, alpha, dst[e]);
}

// v[0..B) = p[0..B) as 8- or 16-byte vector loads (p aligned to 4 B floats).
template <int B>
__device__ __forceinline__ void load_vec(const float* __restrict__ p, float (&v)[B]) {
  if constexpr (B % 4 == 0) {
#pragma unroll
    for (int j = 0; j < B; j += 4) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(p + j);
      v[j] = t[0], v[j + 1] = t[1], v[j + 2] = t[2], v[j + 3] = t[3];
    }
  } else {
    static_assert(B == 2, "2, 4 or 8 floats");
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x, v[1] = t.y;
  }
}

// Weight gradients of one layer: S[o][i] = sum_e G[e][o] A[e][i] and
// b[o] = sum_e G[e][o] over [n_edges, W] planes.  Each workgroup sums a chunk
// of edges (its four waves take every fourth edge), lane (ob, ib) of a wave
// owning the (W/8 x W/8) block of S at (ob, ib); the waves are added in LDS
// and every workgroup writes its partial (row stride `stride` floats); the
// column-sum kernels add the partials in workgroup order: deterministic.
template <int W>
__global__ __launch_bounds__(256) void outer_sum_kernel(const float* __restrict__ g,
                                                        const float* __restrict__ a,
                                                        int64_t n_edges, int64_t chunk,
                                                        int64_t stride,
                                                        float* __restrict__ partial) {
  constexpr int B = W / 8;
  constexpr int N = W * W + W;
  __shared__ float red[4][N];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ob = lane / 8, ib = lane % 8;
  float acc[B][B], bacc[B];
#pragma unroll
  for (int p = 0; p < B; ++p) {
    bacc[p] = 0.f;
#pragma unroll
    for (int q = 0; q < B; ++q) acc[p][q] = 0.f;
  }
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t e1 = e0 + chunk < n_edges ? e0 + chunk : n_edges;
  auto accumulate = [&](const float (&gv)[B], const float (&av)[B]) {
#pragma unroll
    for (int p = 0; p < B; ++p) {
      bacc[p] += gv[p];
#pragma unroll
      for (int q = 0; q < B; ++q) acc[p][q] = fmaf(gv[p], av[q], acc[p][q]);
    }
  };
  // Whole steps of U edges per wave (four row loads per lane in flight, as
  // vector loads), then the remainder one edge at a time.
  constexpr int U = 4;
  const int64_t full = e0 + (e1 - e0) / (4 * U) * (4 * U);
  for (int64_t base = e0 + wave; base < full; base += 4 * U) {
    float gv[U][B], av[U][B];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      load_vec<B>(g + (base + 4 * u) * W + ob * B, gv[u]);
      load_vec<B>(a + (base + 4 * u) * W + ib * B, av[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) accumulate(gv[u], av[u]);
  }
  for (int64_t e = full + wave; e < e1; e += 4) {
    float gv[B], av[B];
    load_vec<B>(g + e * W + ob * B, gv);
    load_vec<B>(a + e * W + ib * B, av);
    accumulate(gv, av);
  }
#pragma unroll
  for (int p = 0; p < B; ++p) {
#pragma unroll
    for (int q = 0; q < B; ++q) red[wave][(ob * B + p) * W + ib * B + q] = acc[p][q];
    if (ib == 0) red[wave][W * W + ob * B + p] = bacc[p];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < N; idx += 256)
    partial[static_cast<int64_t>(blockIdx.x) * stride + idx] =
        (red[0][idx] + red[1][idx]) + (red[2][idx] + red[3][idx]);
}

}  // namespace

int TGX_TIER(outer_blocks)(int64_t n_edges, int64_t* chunk) {
  // About four workgroups per CU; chunks of whole waves of edges.
  int64_t c = ceil_div(n_edges, 1024);
  c = c < 64 ? 64 : align_up(static_cast<size_t>(c), 64);
  *chunk = c;
  return static_cast<int>(ceil_div(n_edges, c));
}


namespace {
// 64 wide: per-edge planes, then one outer-sum launch per layer into the
// partial rows [block][l * NW ...].
template <typename I>
int planes_bwd_t(int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                const float* ds, float* acts, float* dz, int outer_nb, int64_t outer_chunk,
                float* partial, hipStream_t s) {
  constexpr int W = 64;
  constexpr int64_t NW = W * W + W;
  const int64_t blocks = ceil_div(E, 256);
  {
    TGX_PROFILE("edge_mlp_bwd_kernel", s);
    if constexpr (!TGX_NN_MATH)   // one layer: no function, never the second set
      if (L == 1) edge_mlp_planes_kernel<I, W, 1><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
    if (L == 2) edge_mlp_planes_kernel<I, W, 2><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
    if (L == 3) edge_mlp_planes_kernel<I, W, 3><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
    TGX_LAUNCHED("edge_mlp_planes_kernel");
  }
  TGX_PROFILE("outer_sum_kernel", s);
  for (int l = 0; l < L; ++l) {
    outer_sum_kernel<W><<<outer_nb, 256, 0, s>>>(dz + l * E * W, acts + l * E * W, E,
                                                 outer_chunk, L * NW, partial + l * NW);
    TGX_LAUNCHED("outer_sum_kernel");
  }
  return TGX_OK;
}
}  // namespace

int TGX_TIER(planes_backward)(int n_layers, int idx_bits, const void* col, const int32_t* dst,
                              int64_t n_edges, const MlpView& v, const float* dscore,
                              float* acts, float* dz, int outer_nb, int64_t outer_chunk,
                              float* partial, hipStream_t s) {
  return idx_bits == 32
             ? planes_bwd_t(n_layers, static_cast<const int32_t*>(col), dst, n_edges, v, dscore,
                            acts, dz, outer_nb, outer_chunk, partial, s)
             : planes_bwd_t(n_layers, static_cast<const int64_t*>(col), dst, n_edges, v, dscore,
                            acts, dz, outer_nb, outer_chunk, partial, s);
}

}  // namespace mlp
}  // namespace tgx
