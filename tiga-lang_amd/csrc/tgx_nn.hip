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
// weights are uniform across the wave, so they are read once per wave
// through scalar loads and used as SGPR operands of v_fma_f32.  Every layer
// is zero-padded to a common width W (16, 32 or 64) on the host, which keeps
// every register index compile-time.  The softmax and the value gather are
// separate row passes (segment softmax here, the weighted CSR sum of
// tgx_sum.hip for the values), which adds 8 bytes per edge (score, weight)
// to a gather of 4 F bytes per edge.
//
// Backward: segment softmax backward per row (ds = a (da - <a, da>)), then
// the per-edge MLP backward replays the chain, back-propagates ds, writes the
// per-layer inputs and pre-activation gradients (the weight gradients are
// their products over the edges, plain GEMMs) and the per-edge gradients of
// every input segment (reduced per source row over the transposed CSR and
// per destination row over the CSR by the caller).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "tgx_device.h"
#include "tgx_host.h"
#include "tgx_profile.h"

namespace tgx {
namespace {

constexpr int kMaxLayers = 3;
constexpr int kMaxSegments = 4;

struct MlpView {
  int n_layers;
  int in_width;
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

// z = W_l a + b_l over the padded width, one weight row at a time (wl is
// uniform across the wave).
template <int W>
__device__ __forceinline__ void linear(const float* wl, const float (&a)[W], float (&z)[W]) {
#pragma unroll
  for (int o = 0; o < W; ++o) {
    float acc = wl[W * W + o];
#pragma unroll
    for (int i = 0; i < W; ++i) acc = fmaf(wl[o * W + i], a[i], acc);
    pin(acc);
    z[o] = acc;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The weights of all layers, staged once per workgroup in LDS (every lane
// then reads the same address: a broadcast).
template <int W, int L>
__device__ __forceinline__ void stage_weights(const float* __restrict__ w, float* wsh) {
  for (int i = threadIdx.x; i < L * (W * W + W); i += 256) wsh[i] = w[i];
  __syncthreads();
}

template <typename I, int W, int L>
__global__ __launch_bounds__(256) void edge_mlp_fwd_kernel(const I* __restrict__ col,
                                                           const int32_t* __restrict__ dst,
                                                           int64_t n_edges, MlpView m,
                                                           float* __restrict__ scores) {
  __shared__ float wsh[L * (W * W + W)];
  stage_weights<W, L>(m.w, wsh);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_edges) return;
  float a[W], z[W];
  gather_inputs<I, W>(m, e, col, dst, a);
#pragma unroll
  for (int l = 0; l + 1 < L; ++l) {
    linear<W>(wsh + l * (W * W + W), a, z);
    const int act = m.act[l];
    const float p = m.param[l];
#pragma unroll
    for (int o = 0; o < W; ++o) a[o] = activate(z[o], act, p);
  }
  const float* wl = wsh + (L - 1) * (W * W + W);
  float s = wl[W * W];
#pragma unroll
  for (int i = 0; i < W; ++i) s = fmaf(wl[i], a[i], s);
  scores[e] = s;
}

// Per-edge backward of the score chain.  ds_e arrives from the softmax
// backward.  Writes, for every layer l: its input acts[l][e][:] and the
// gradient of its pre-activation output dz[l][e][:] (padded width W), and the
// input gradient split per segment dseg[s][e][:width_s].
template <typename I, int W, int L>
__global__ __launch_bounds__(256) void edge_mlp_bwd_kernel(
    const I* __restrict__ col, const int32_t* __restrict__ dst, int64_t n_edges, MlpView m,
    const float* __restrict__ dscore, float* __restrict__ acts, float* __restrict__ dz_out) {
  __shared__ float wsh[L * (W * W + W)];
  stage_weights<W, L>(m.w, wsh);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_edges) return;
  const int64_t plane = n_edges * W;
  float a[W];                       // input of the current layer
  float z[L > 1 ? L - 1 : 1][W];    // pre-activations of the hidden layers
  gather_inputs<I, W>(m, e, col, dst, a);
  static_for<L>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    float* out = acts + l * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{a[i], a[i + 1], a[i + 2], a[i + 3]};
    if constexpr (l + 1 < L) {
      linear<W>(wsh + l * (W * W + W), a, z[l]);
#pragma unroll
      for (int o = 0; o < W; ++o) a[o] = activate(z[l][o], m.act[l], m.param[l]);
    }
  });
  // Last layer: one output, gradient ds.
  const float ds = dscore[e];
  float g[W];
  {
    const float* wl = wsh + (L - 1) * (W * W + W);
    float* out = dz_out + (L - 1) * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{i == 0 ? ds : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < W; ++i) g[i] = ds * wl[i];   // d a[L-1]
  }
  static_for<L - 1>([&](auto kc) {
    constexpr int l = L - 2 - decltype(kc)::value;
    float dzl[W];
#pragma unroll
    for (int o = 0; o < W; ++o) {
      dzl[o] = g[o] * activate_grad(z[l][o], m.act[l], m.param[l]);
      pin(dzl[o]);
    }
    float* out = dz_out + l * plane + e * W;
#pragma unroll
    for (int i = 0; i < W; i += 4)
      *reinterpret_cast<f32x4*>(out + i) = f32x4{dzl[i], dzl[i + 1], dzl[i + 2], dzl[i + 3]};
    // d a[l] = W_l^T dz, accumulated row by row so W_l is read in order.
    const float* wl = wsh + l * (W * W + W);
#pragma unroll
    for (int i = 0; i < W; ++i) g[i] = 0.f;
    static_for<W>([&](auto oc) {
      constexpr int o = decltype(oc)::value;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        g[i] = fmaf(wl[o * W + i], dzl[o], g[i]);
        pin(g[i]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  });
  // g = d x: split per segment.
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    if (s >= m.n_seg) break;
    const int off = m.off[s], wd = m.width[s];
    float* q = m.grad[s] + e * wd - off;
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (k >= off && k < off + wd) q[k] = g[k];
  }
}

// One wave per row: alpha_e = exp(s_e - lse_i), lse_i = log sum exp s over
// the row (-inf and no weights for an empty row).
template <typename I>
__global__ __launch_bounds__(256) void segment_softmax_fwd_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, const float* __restrict__ scores,
    float* __restrict__ alpha, float* __restrict__ lse) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = lane_id();
  const int64_t e0 = row_ptr[row], e1 = row_ptr[row + 1];
  float m = kNegInf;
  for (int64_t e = e0 + lane; e < e1; e += kWave) m = fmaxf(m, scores[e]);
  m = group_max<kWave>(m);
  float l = 0.f;
  for (int64_t e = e0 + lane; e < e1; e += kWave) l += __expf(scores[e] - m);
  l = group_sum<kWave>(l);
  const float ls = e1 > e0 ? m + __logf(l) : kNegInf;
  for (int64_t e = e0 + lane; e < e1; e += kWave) alpha[e] = __expf(scores[e] - ls);
  if (lane == 0) lse[row] = ls;
}

// One wave per row: ds_e = alpha_e (dalpha_e - sum_row alpha dalpha).
template <typename I>
__global__ __launch_bounds__(256) void segment_softmax_bwd_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, const float* __restrict__ alpha,
    const float* __restrict__ dalpha, float* __restrict__ dscore) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = lane_id();
  const int64_t e0 = row_ptr[row], e1 = row_ptr[row + 1];
  float d = 0.f;
  for (int64_t e = e0 + lane; e < e1; e += kWave) d += alpha[e] * dalpha[e];
  d = group_sum<kWave>(d);
  for (int64_t e = e0 + lane; e < e1; e += kWave) dscore[e] = alpha[e] * (dalpha[e] - d);
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
// and every workgroup writes its partial.  A second kernel adds the partials
// in workgroup order: deterministic.
template <int W>
__global__ __launch_bounds__(256) void outer_sum_kernel(const float* __restrict__ g,
                                                        const float* __restrict__ a,
                                                        int64_t n_edges, int64_t chunk,
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
    partial[static_cast<int64_t>(blockIdx.x) * N + idx] =
        (red[0][idx] + red[1][idx]) + (red[2][idx] + red[3][idx]);
}

__global__ __launch_bounds__(256) void outer_sum_final_kernel(
    const float* __restrict__ partial, int n_blocks, int n, int w, float* __restrict__ dw,
    float* __restrict__ db) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= n) return;
  float s = 0.f;
  for (int b = 0; b < n_blocks; ++b) s += partial[static_cast<int64_t>(b) * n + idx];
  if (idx < w * w)
    dw[idx] = s;
  else if (db)
    db[idx - w * w] = s;
}

int outer_blocks(int64_t n_edges, int64_t* chunk) {
  // About four workgroups per CU; chunks of whole waves of edges.
  int64_t c = ceil_div(n_edges, 1024);
  c = c < 64 ? 64 : align_up(static_cast<size_t>(c), 64);
  *chunk = c;
  return static_cast<int>(ceil_div(n_edges, c));
}

int check_mlp(const tgx_edge_mlp* mlp, MlpView* view) {
  TGX_REQUIRE(mlp, "null mlp");
  TGX_REQUIRE(mlp->n_layers >= 1 && mlp->n_layers <= kMaxLayers, "1 to %d linear layers",
              kMaxLayers);
  TGX_REQUIRE(mlp->width == 16 || mlp->width == 32 || mlp->width == 64,
              "padded width must be 16, 32 or 64");
  TGX_REQUIRE(mlp->n_segments >= 1 && mlp->n_segments <= kMaxSegments,
              "1 to %d input segments", kMaxSegments);
  TGX_REQUIRE(mlp->weights_dev, "null weights");
  int in_width = 0;
  for (int s = 0; s < mlp->n_segments; ++s) {
    TGX_REQUIRE(mlp->seg_role[s] >= TGX_ROLE_SRC && mlp->seg_role[s] <= TGX_ROLE_EDGE,
                "bad segment role");
    TGX_REQUIRE(mlp->seg_width[s] > 0 && mlp->seg_stride[s] >= mlp->seg_width[s] &&
                    mlp->seg_dev[s],
                "bad segment %d", s);
    in_width += mlp->seg_width[s];
  }
  TGX_REQUIRE(in_width <= mlp->width, "inputs (%d) exceed the padded width", in_width);
  for (int l = 0; l + 1 < mlp->n_layers; ++l)
    TGX_REQUIRE(mlp->act[l] >= TGX_ACT_IDENTITY && mlp->act[l] <= TGX_ACT_ELU,
                "bad activation code");
  MlpView v{};
  v.n_layers = mlp->n_layers;
  v.in_width = in_width;
  for (int l = 0; l < kMaxLayers; ++l) {
    v.act[l] = l + 1 < mlp->n_layers ? mlp->act[l] : TGX_ACT_IDENTITY;
    v.param[l] = mlp->act_param[l];
  }
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
  if (L == 1) edge_mlp_fwd_kernel<I, W, 1><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
  if (L == 2) edge_mlp_fwd_kernel<I, W, 2><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
  if (L == 3) edge_mlp_fwd_kernel<I, W, 3><<<blocks, 256, 0, s>>>(col, dst, E, v, scores);
}

template <typename I, int W>
void launch_bwd(int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                const float* ds, float* acts, float* dz, hipStream_t s) {
  const int64_t blocks = ceil_div(E, 256);
  if (L == 1) edge_mlp_bwd_kernel<I, W, 1><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
  if (L == 2) edge_mlp_bwd_kernel<I, W, 2><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
  if (L == 3) edge_mlp_bwd_kernel<I, W, 3><<<blocks, 256, 0, s>>>(col, dst, E, v, ds, acts, dz);
}

template <typename I>
void dispatch_fwd(int W, int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                  float* scores, hipStream_t s) {
  if (W == 16) launch_fwd<I, 16>(L, col, dst, E, v, scores, s);
  if (W == 32) launch_fwd<I, 32>(L, col, dst, E, v, scores, s);
  if (W == 64) launch_fwd<I, 64>(L, col, dst, E, v, scores, s);
}

template <typename I>
void dispatch_bwd(int W, int L, const I* col, const int32_t* dst, int64_t E, const MlpView& v,
                  const float* ds, float* acts, float* dz, hipStream_t s) {
  if (W == 16) launch_bwd<I, 16>(L, col, dst, E, v, ds, acts, dz, s);
  if (W == 32) launch_bwd<I, 32>(L, col, dst, E, v, ds, acts, dz, s);
  if (W == 64) launch_bwd<I, 64>(L, col, dst, E, v, ds, acts, dz, s);
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_edge_mlp_scores(const void* col, const int32_t* dst_index, int idx_bits,
                                   int64_t n_edges, const tgx_edge_mlp* mlp, float* scores,
                                   void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v);
  if (st != TGX_OK) return st;
  if (n_edges == 0) return TGX_OK;
  TGX_REQUIRE(col && dst_index && scores, "null pointer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("edge_mlp_fwd_kernel", s);
  if (idx_bits == 32)
    dispatch_fwd(mlp->width, mlp->n_layers, static_cast<const int32_t*>(col), dst_index,
                 n_edges, v, scores, s);
  else
    dispatch_fwd(mlp->width, mlp->n_layers, static_cast<const int64_t*>(col), dst_index,
                 n_edges, v, scores, s);
  TGX_LAUNCHED("edge_mlp_fwd_kernel");
  return TGX_OK;
}

extern "C" int tgx_edge_mlp_backward(const void* col, const int32_t* dst_index, int idx_bits,
                                     int64_t n_edges, const tgx_edge_mlp* mlp,
                                     const float* dscore, float* acts, float* dz,
                                     float* const* dseg, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_edges >= 0, "negative size");
  MlpView v;
  int st = check_mlp(mlp, &v);
  if (st != TGX_OK) return st;
  if (n_edges == 0) return TGX_OK;
  TGX_REQUIRE(col && dst_index && dscore && acts && dz && dseg, "null pointer");
  for (int s = 0; s < mlp->n_segments; ++s) {
    TGX_REQUIRE(dseg[s], "null gradient for segment %d", s);
    v.grad[s] = dseg[s];
  }
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("edge_mlp_bwd_kernel", s);
  if (idx_bits == 32)
    dispatch_bwd(mlp->width, mlp->n_layers, static_cast<const int32_t*>(col), dst_index,
                 n_edges, v, dscore, acts, dz, s);
  else
    dispatch_bwd(mlp->width, mlp->n_layers, static_cast<const int64_t*>(col), dst_index,
                 n_edges, v, dscore, acts, dz, s);
  TGX_LAUNCHED("edge_mlp_bwd_kernel");
  return TGX_OK;
}

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
    segment_softmax_fwd_kernel<<<ceil_div(n_rows, 4), 256, 0, s>>>(
        static_cast<const int32_t*>(row_ptr), n_rows, scores, alpha, lse);
  else
    segment_softmax_fwd_kernel<<<ceil_div(n_rows, 4), 256, 0, s>>>(
        static_cast<const int64_t*>(row_ptr), n_rows, scores, alpha, lse);
  TGX_LAUNCHED("segment_softmax_fwd_kernel");
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
    segment_softmax_bwd_kernel<<<ceil_div(n_rows, 4), 256, 0, s>>>(
        static_cast<const int32_t*>(row_ptr), n_rows, alpha, dalpha, dscore);
  else
    segment_softmax_bwd_kernel<<<ceil_div(n_rows, 4), 256, 0, s>>>(
        static_cast<const int64_t*>(row_ptr), n_rows, alpha, dalpha, dscore);
  TGX_LAUNCHED("segment_softmax_bwd_kernel");
  return TGX_OK;
}

extern "C" int tgx_edge_outer_sum_workspace(int64_t n_edges, int width, size_t* bytes) {
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_edges >= 0 && (width == 16 || width == 32 || width == 64), "bad sizes");
  int64_t chunk = 0;
  const int nb = n_edges ? outer_blocks(n_edges, &chunk) : 0;
  *bytes = align_up(static_cast<size_t>(nb) * (width * width + width) * sizeof(float));
  return TGX_OK;
}

extern "C" int tgx_edge_outer_sum(const float* g, const float* a, int64_t n_edges, int width,
                                  float* dw, float* db, void* ws, size_t ws_bytes,
                                  void* stream) {
  TGX_REQUIRE(n_edges >= 0 && (width == 16 || width == 32 || width == 64), "bad sizes");
  TGX_REQUIRE(dw, "null dw");
  hipStream_t s = as_stream(stream);
  const int n = width * width + width;
  if (n_edges == 0) {
    // Zero sums, written by a kernel rather than a memset.
    outer_sum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(nullptr, 0, n, width, dw, db);
    TGX_LAUNCHED("outer_sum_final_kernel");
    return TGX_OK;
  }
  TGX_REQUIRE(g && a && ws, "null pointer");
  int64_t chunk = 0;
  const int nb = outer_blocks(n_edges, &chunk);
  TGX_REQUIRE(ws_bytes >= static_cast<size_t>(nb) * n * sizeof(float), "workspace too small");
  float* partial = static_cast<float*>(ws);
  TGX_PROFILE("outer_sum_kernel", s);
  if (width == 16) outer_sum_kernel<16><<<nb, 256, 0, s>>>(g, a, n_edges, chunk, partial);
  if (width == 32) outer_sum_kernel<32><<<nb, 256, 0, s>>>(g, a, n_edges, chunk, partial);
  if (width == 64) outer_sum_kernel<64><<<nb, 256, 0, s>>>(g, a, n_edges, chunk, partial);
  TGX_LAUNCHED("outer_sum_kernel");
  outer_sum_final_kernel<<<ceil_div(n, 256), 256, 0, s>>>(partial, nb, n, width, dw, db);
  TGX_LAUNCHED("outer_sum_final_kernel");
  return TGX_OK;
}
