// Device code shared by the edge-MLP kernels (tgx_nn.hip, tgx_nn_wide.hip):
// the network view, activations, per-edge input gathers and the row-by-row
// dense layers over LDS-staged weights.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "tgx_device.h"
#include "tgx_host.h"

namespace tgx {
namespace mlp {

constexpr int kMaxLayers = 3;
constexpr int kMaxSegments = 4;

struct MlpView {
  int n_layers;
  int in_width;
  int n_out[kMaxLayers];   // real output width of each layer (<= W)
  int nb_in[kMaxLayers];   // column blocks of 4 covering each layer's real input
  int act[kMaxLayers];
  float param[kMaxLayers];
  const float* w;   // n_layers x [W*W | W]
  int n_seg;
  int role[kMaxSegments];
  int width[kMaxSegments];
  int64_t stride[kMaxSegments];
  const float* ptr[kMaxSegments];
  int off[kMaxSegments];              // first input column of each segment
  float* grad[kMaxSegments];          // backward: per-segment input gradients
};

__device__ __forceinline__ float sigmoid(float z) { return 1.f / (1.f + __expf(-z)); }

// Component-wise activation (code uniform across the wave).
__device__ __forceinline__ float activate(float z, int act, float p) {
  switch (act) {
    case TGX_ACT_RELU: return fmaxf(z, 0.f);
    case TGX_ACT_LEAKY_RELU: return z > 0.f ? z : p * z;
    case TGX_ACT_TANH: return tanhf(z);
    case TGX_ACT_SIGMOID: return sigmoid(z);
    case TGX_ACT_SILU: return z * sigmoid(z);
    case TGX_ACT_GELU: return 0.5f * z * (1.f + erff(z * 0.70710678118654752f));
    case TGX_ACT_ELU: return z > 0.f ? z : p * (__expf(z) - 1.f);
    default: return z;
  }
}

// d activate / dz at z.
__device__ __forceinline__ float activate_grad(float z, int act, float p) {
  switch (act) {
    case TGX_ACT_RELU: return z > 0.f ? 1.f : 0.f;
    case TGX_ACT_LEAKY_RELU: return z > 0.f ? 1.f : p;
    case TGX_ACT_TANH: {
      const float t = tanhf(z);
      return 1.f - t * t;
    }
    case TGX_ACT_SIGMOID: {
      const float s = sigmoid(z);
      return s * (1.f - s);
    }
    case TGX_ACT_SILU: {
      const float s = sigmoid(z);
      return s * (1.f + z * (1.f - s));
    }
    case TGX_ACT_GELU:
      // Phi(z) + z phi(z)
      return 0.5f * (1.f + erff(z * 0.70710678118654752f)) +
             z * 0.39894228040143268f * __expf(-0.5f * z * z);
    case TGX_ACT_ELU: return z > 0.f ? 1.f : p * __expf(z);
    default: return 1.f;
  }
}

template <typename I>
__device__ __forceinline__ int64_t seg_row(int role, int64_t e, const I* col,
                                           const int32_t* dst) {
  return role == TGX_ROLE_SRC ? static_cast<int64_t>(col[e])
                              : (role == TGX_ROLE_DST ? static_cast<int64_t>(dst[e]) : e);
}

// x[k] for k < in_width from the concatenated segments (zero beyond).  The
// segment loop is compile-time, so each segment's row pointer is a plain
// per-lane value and every x index is a constant (no indexed register
// arrays); which columns a segment fills is a uniform range test.
template <typename I, int W>
__device__ __forceinline__ void gather_inputs(const MlpView& m, int64_t e, const I* col,
                                              const int32_t* dst, float (&x)[W]) {
#pragma unroll
  for (int k = 0; k < W; ++k) x[k] = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    if (s >= m.n_seg) break;
    const int off = m.off[s], wd = m.width[s];
    const float* p = m.ptr[s] + seg_row(m.role[s], e, col, dst) * m.stride[s] - off;
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (k >= off && k < off + wd) x[k] = p[k];
  }
}

// Keeps v's computation at this point of the program.  Without it the
// optimizer sinks each dot product to its first use, behind the uniform
// branches of the activation that follows, i.e. after every weight load of
// the layer, and all W*W weights of the layer end up live at once.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

// f(integral_constant<0>) ... f(integral_constant<N-1>): a loop whose index
// is a compile-time constant in the body (register arrays indexed by it stay
// in registers whatever the body's size).
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// One weight row of a layer held in LDS (16-byte reads) and its bias.
template <int W>
struct WRow {
  f32x4 w[W / 4];
  float b;
};
template <int W>
__device__ __forceinline__ void load_row(const float* wl, int o, WRow<W>& r) {
#pragma unroll
  for (int k = 0; k < W / 4; ++k) r.w[k] = *reinterpret_cast<const f32x4*>(wl + o * W + 4 * k);
  r.b = wl[W * W + o];
}

// z = W_l a + b_l, one weight row at a time (wl is uniform across the wave).
// Up to 32 wide and with kPrefetchRows, row o+1 is read from LDS while row
// o's dot product runs, so the read latency overlaps the FMAs (at the cost
// of one row of registers).  Otherwise only the layer's real shape is
// computed: rows o < n_out and the first nb column blocks of 4 (nb =
// ceil(n_in / 4)), padded rows getting z = 0; the skipped terms are products
// with zero padding weights (forward scores 0.205 -> 0.166 ms on the 19-16-1
// bench network).
template <int W, bool kPrefetchRows = true>
__device__ __forceinline__ void linear(const float* wl, const float (&a)[W], float (&z)[W],
                                       int n_out, int nb) {
  if constexpr (W <= 32 && kPrefetchRows) {
    // Every padded row and column is multiplied here: the kernel using this
    // path runs one wave per SIMD, where branches cost more than the FMAs
    // they skip.  Each dot product is four interleaved partial sums, so
    // consecutive FMAs are independent.
    WRow<W> cur, nxt;
    load_row<W>(wl, 0, cur);
    static_for<W>([&](auto oc) {
      constexpr int o = decltype(oc)::value;
      if constexpr (o + 1 < W) load_row<W>(wl, o + 1, nxt);
      float p[4] = {cur.b, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < W / 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = fmaf(cur.w[k][j], a[4 * k + j], p[j]);
      float acc = (p[0] + p[1]) + (p[2] + p[3]);
      pin(acc);
      z[o] = acc;
      if constexpr (o + 1 < W) cur = nxt;
      __builtin_amdgcn_sched_barrier(0);
    });
  } else {
#pragma unroll
    for (int o = 0; o < W; ++o) {
      if (o < n_out) {
        float acc = wl[W * W + o];
#pragma unroll
        for (int k = 0; k < W / 4; ++k)
          if (k < nb)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = fmaf(wl[o * W + 4 * k + j], a[4 * k + j], acc);
        pin(acc);
        z[o] = acc;
      } else {
        z[o] = 0.f;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// g = W_l^T dz (n_out and nb are unused: padded rows have dz = 0 and
// padded columns zero weights, and the one-wave-per-SIMD kernel that uses
// this runs faster without branches), W_l read row by row in order, row o+1
// fetched while row o is applied.
template <int W>
__device__ __forceinline__ void linear_t(const float* wl, const float (&dz)[W], float (&g)[W],
                                         int n_out, int nb) {
#pragma unroll
  for (int i = 0; i < W; ++i) g[i] = 0.f;
  WRow<W> cur, nxt;
  load_row<W>(wl, 0, cur);
  static_for<W>([&](auto oc) {
    constexpr int o = decltype(oc)::value;
    if constexpr (o + 1 < W) load_row<W>(wl, o + 1, nxt);
#pragma unroll
    for (int i = 0; i < W; ++i) {
      g[i] = fmaf(cur.w[i / 4][i % 4], dz[o], g[i]);
      pin(g[i]);
    }
    if constexpr (o + 1 < W) cur = nxt;
    __builtin_amdgcn_sched_barrier(0);
  });
}

// The weights of all layers, staged once per workgroup in LDS (every lane
// then reads the same address: a broadcast).
template <int W, int L>
__device__ __forceinline__ void stage_weights(const float* __restrict__ w, float* wsh) {
  for (int i = threadIdx.x; i < L * (W * W + W); i += 256) wsh[i] = w[i];
  __syncthreads();
}

// 64-wide chains: backward in two passes (tgx_nn_wide.hip).  Blocks and
// chunk of the outer-sum pass for n_edges edges.
int outer_blocks(int64_t n_edges, int64_t* chunk);

// Per-edge planes (acts, dz: n_layers x [n_edges, 64] each) and the
// per-segment input gradients, then the per-layer weight-gradient partial
// sums of outer_nb blocks into partial[block * n_layers * NW + l * NW + ...]
// (NW = 64 * 64 + 64).  Launches on `s`; TGX_* status.
int planes_backward(int n_layers, int idx_bits, const void* col, const int32_t* dst,
                    int64_t n_edges, const MlpView& v, const float* dscore, float* acts,
                    float* dz, int outer_nb, int64_t outer_chunk, float* partial,
                    hipStream_t s);

}  // namespace mlp
}  // namespace tgx
