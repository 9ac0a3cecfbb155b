// Device code shared by the edge-MLP kernels (tgx_nn.hip, tgx_nn_wide.hip):
// the network view, activations, per-edge input gathers and the dense
// layers over weights held in scalar registers.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "tgx_device.h"
#include "tgx_host.h"

// The component-wise functions a translation unit's kernels evaluate: the
// activations relu ... hardswish (TGX_NN_MATH 0), or those and exp, log,
// abs, sin, cos, the powers and LayerNorm (1).  The second set goes into kernels of
// their own (tgx_nn_math.hip and tgx_nn_wide_math.hip compile the same
// sources with TGX_NN_MATH 1), which the entry points call for a chain that
// uses one of them: the larger switch costs the backward kernels registers
// (spills at widths 16 and 24, one wave per SIMD less at width 32) that
// chains without them do not pay.
#ifndef TGX_NN_MATH
#define TGX_NN_MATH 0
#endif
#if TGX_NN_MATH
#define TGX_TIER(name) name##_math
#else
#define TGX_TIER(name) name
#endif

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
  float param2[kMaxLayers];
  const float* w;   // n_layers x [W*W | W]
  int n_seg;
  int role[kMaxSegments];
  int width[kMaxSegments];
  int64_t stride[kMaxSegments];
  const float* ptr[kMaxSegments];
  int off[kMaxSegments];              // first input column of each segment
  float* grad[kMaxSegments];          // backward: per-segment input gradients
  // LayerNorm over a hidden layer's real outputs before its activation
  // (kernels with the second set of functions only), and the floats per
  // layer of the weight blocks: W*W + W, or W*W + 3W (gamma, beta) when
  // some layer is normalized.
  int norm[kMaxLayers];
  float eps[kMaxLayers];
  int nw;
  // Backward of online-softmax attention over the chain's one-output score
  // when the forward kept only each row's logsumexp (att_lse non-null): the
  // kernels form each edge's score gradient themselves (attention_score_grad)
  // instead of reading it.  Rows of att_out / att_dout (destinations) and
  // att_value (sources) hold att_width floats.
  const float* att_lse;
  const float* att_out;
  const float* att_dout;
  const float* att_value;
  float* att_alpha;       // [n_edges]: the recomputed weights (null: not written)
  int att_width;
  // Segment whose per-edge gradient rows also receive alpha_e att_dout[dst_e]
  // (the value gradient's edge term, when the value is that source field),
  // or -1.
  int att_fold;
};

// Floats per layer of a chain's weight (and weight-gradient) blocks.
inline int block_floats(const tgx_edge_mlp* mlp) {
  int w = mlp->width * mlp->width + mlp->width;
  for (int l = 0; l + 1 < mlp->n_layers && l < kMaxLayers; ++l)
    if (mlp->norm[l]) return w + 2 * mlp->width;
  return w;
}

__device__ __forceinline__ float sigmoid(float z) { return 1.f / (1.f + __expf(-z)); }

// softplus with Torch's convention: z where beta z > threshold, else
// log(1 + exp(beta z)) / beta.
__device__ __forceinline__ float softplus(float z, float beta, float threshold) {
  const float bz = beta * z;
  return bz > threshold ? z : log1pf(__expf(bz)) / beta;
}

constexpr float kSeluAlpha = 1.6732632423543772848f;
constexpr float kSeluScale = 1.0507009873554804934f;

// Component-wise activation (code uniform across the wave).  Derivatives
// follow Torch's at the kinks (hardtanh's bounds excluded, hardswish's
// boundaries as its backward).
__device__ __forceinline__ float activate(float z, int act, float p, float p2) {
  switch (act) {
    case TGX_ACT_RELU: return fmaxf(z, 0.f);
    case TGX_ACT_LEAKY_RELU: return z > 0.f ? z : p * z;
    case TGX_ACT_TANH: return tanhf(z);
    case TGX_ACT_SIGMOID: return sigmoid(z);
    case TGX_ACT_SILU: return z * sigmoid(z);
    case TGX_ACT_GELU: return 0.5f * z * (1.f + erff(z * 0.70710678118654752f));
    case TGX_ACT_ELU: return z > 0.f ? z : p * (__expf(z) - 1.f);
    case TGX_ACT_HARDTANH: return fminf(fmaxf(z, p), p2);
    case TGX_ACT_SOFTPLUS: return softplus(z, p, p2);
    case TGX_ACT_SELU: return kSeluScale * (z > 0.f ? z : kSeluAlpha * (__expf(z) - 1.f));
    case TGX_ACT_MISH: return z * tanhf(softplus(z, 1.f, 20.f));
    case TGX_ACT_HARDSIGMOID: return fminf(fmaxf(z * (1.f / 6.f) + 0.5f, 0.f), 1.f);
    case TGX_ACT_HARDSWISH:
      return z <= -3.f ? 0.f : (z >= 3.f ? z : z * (z + 3.f) * (1.f / 6.f));
    default: return z;
  }
}

// d activate / dz at z.
__device__ __forceinline__ float activate_grad(float z, int act, float p, float p2) {
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
    case TGX_ACT_HARDTANH: return (z > p && z < p2) ? 1.f : 0.f;
    case TGX_ACT_SOFTPLUS: return p * z > p2 ? 1.f : sigmoid(p * z);
    case TGX_ACT_SELU: return kSeluScale * (z > 0.f ? 1.f : kSeluAlpha * __expf(z));
    case TGX_ACT_MISH: {
      const float t = tanhf(softplus(z, 1.f, 20.f));
      return t + z * sigmoid(z) * (1.f - t * t);
    }
    case TGX_ACT_HARDSIGMOID: return (z > -3.f && z < 3.f) ? (1.f / 6.f) : 0.f;
    case TGX_ACT_HARDSWISH: return z < -3.f ? 0.f : (z <= 3.f ? z * (1.f / 3.f) + 0.5f : 1.f);
    default: return 1.f;
  }
}

// x[k] for k < in_width from the concatenated segments (zero beyond), the
// edge's source and destination row ids given.  The segment loop is
// compile-time, so each segment's row pointer is a plain per-lane value and
// every x index is a constant (no indexed register arrays); which columns a
// segment fills is a uniform range test, made per block of 4 columns first.
template <int W>
__device__ __forceinline__ void gather_rows(const MlpView& m, int64_t e, int64_t src_row,
                                            int64_t dst_row, float (&x)[W]) {
#pragma unroll
  for (int k = 0; k < W; ++k) x[k] = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    if (s >= m.n_seg) break;
    const int off = m.off[s], end = m.off[s] + m.width[s];
    const int64_t row =
        m.role[s] == TGX_ROLE_SRC ? src_row : (m.role[s] == TGX_ROLE_DST ? dst_row : e);
    const float* p = m.ptr[s] + row * m.stride[s] - off;
#pragma unroll
    for (int b = 0; b < W; b += 4) {
      if (b + 4 > off && b < end) {
        if (b >= off && b + 4 <= end) {
#pragma unroll
          for (int k = b; k < b + 4; ++k) x[k] = p[k];
        } else {
#pragma unroll
          for (int k = b; k < b + 4; ++k)
            if (k >= off && k < end) x[k] = p[k];
        }
      }
    }
  }
}

// gather_rows, reading the row ids that the segments use.
template <typename I, int W>
__device__ __forceinline__ void gather_inputs(const MlpView& m, int64_t e, const I* col,
                                              const int32_t* dst, float (&x)[W]) {
  bool need_src = false, need_dst = false;
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    need_src |= s < m.n_seg && m.role[s] == TGX_ROLE_SRC;
    need_dst |= s < m.n_seg && m.role[s] == TGX_ROLE_DST;
  }
  gather_rows<W>(m, e, need_src ? static_cast<int64_t>(col[e]) : 0,
                 need_dst ? static_cast<int64_t>(dst[e]) : 0, x);
}

// Score gradient of edge e (destination row i, source row j) of an
// online-softmax attention out[i] = sum_e alpha_e value[j], from the
// replayed score s:
//   alpha = exp(s - lse[i]),  ds = alpha (<dout[i], value[j]> - <dout[i], out[i]>),
// the softmax Jacobian with the row term <dout, out> = sum_e alpha dalpha
// (the reference's edge-attention VJP, compiler/edge_nn_attention.py:
// 569-575).  alpha is stored for the value gradient's transposed sum.
__device__ __forceinline__ float attention_score_grad(const MlpView& m, int64_t e, int64_t i,
                                                      int64_t j, float s, float& alpha_out) {
  const float alpha = __expf(s - m.att_lse[i]);
  alpha_out = alpha;
  const int F = m.att_width;
  const float* d = m.att_dout + i * F;
  const float* o = m.att_out + i * F;
  const float* v = m.att_value + j * F;
  float dv = 0.f, dd = 0.f;
  if ((F & 3) == 0) {
    for (int f = 0; f < F; f += 4) {
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(d + f);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(v + f);
      const f32x4 o4 = *reinterpret_cast<const f32x4*>(o + f);
      dv += d4[0] * v4[0] + d4[1] * v4[1] + d4[2] * v4[2] + d4[3] * v4[3];
      dd += d4[0] * o4[0] + d4[1] * o4[1] + d4[2] * o4[2] + d4[3] * o4[3];
    }
  } else {
    for (int f = 0; f < F; ++f) {
      dv += d[f] * v[f];
      dd += d[f] * o[f];
    }
  }
  if (m.att_alpha) m.att_alpha[e] = alpha;
  return alpha * (dv - dd);
}

// q_s[e][k - off_s] = g[k] for every segment s (the per-edge input gradient
// split per segment), with the same block-then-column range tests.  Segment
// m.att_fold (when >= 0) also receives alpha * att_dout[i][k - off_s], the
// edge's term of the value gradient (i = the edge's destination row).
template <int W>
__device__ __forceinline__ void scatter_segments(const MlpView& m, int64_t e, const float (&g)[W],
                                                 float alpha = 0.f, int64_t i = 0) {
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    if (s >= m.n_seg) break;
    const int off = m.off[s], wd = m.width[s], end = off + wd;
    float* q = m.grad[s] + e * wd - off;
    const bool fold = s == m.att_fold;
    const float* d = fold ? m.att_dout + i * m.att_width - off : nullptr;   // d[k] pairs with g[k]
#pragma unroll
    for (int b = 0; b < W; b += 4) {
      if (b + 4 > off && b < end) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = g[b + k];
        if (b >= off && b + 4 <= end) {
          if (fold) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = fmaf(alpha, d[b + k], v[k]);
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) q[b + k] = v[k];
        } else {
#pragma unroll
          for (int k = b; k < b + 4; ++k)
            if (k >= off && k < end) q[k] = fold ? fmaf(alpha, d[k], v[k - b]) : v[k - b];
        }
      }
    }
  }
}

// Keeps v's computation at this point of the program.  Without it the
// optimizer sinks each value to its first use, past the uniform branches and
// weight loads in between, and the operands it needs stay live that long.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

// Lambdas in the kernels are inlined whatever the kernel's size: one left
// as a call takes the arrays it captures by reference out of registers (into
// private memory, spilled per lane).
#define TGX_INLINE_LAMBDA __attribute__((always_inline))

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

// Layer weights are read through the scalar data cache: every lane of a
// wave needs the same weight at the same time, so a uniform load from the
// constant address space puts it in a scalar register that feeds the FMA
// directly (one scalar operand per VALU instruction).  No LDS staging, no
// LDS read latency and no vector registers are spent on weights.
typedef __attribute__((address_space(4))) const float cfloat;

__device__ __forceinline__ cfloat* scalar_weights(const float* p) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wold-style-cast"
  return (cfloat*)p;   // generic -> constant address space (same address)
#pragma clang diagnostic pop
}

// p, with the compiler kept from knowing it is p (loads through it are not
// hoisted out of the enclosing loop).
__device__ __forceinline__ cfloat* opaque(cfloat* p) {
  asm volatile("" : "+s"(p));
  return p;
}

// The network's shape fields, hidden from the optimizer at this point (what
// is derived from them is recomputed after it rather than hoisted).
__device__ __forceinline__ void launder(MlpView& v) {
  asm volatile("" : "+s"(v.n_seg), "+s"(v.in_width));
#pragma unroll
  for (int l = 0; l < kMaxLayers; ++l)
    asm volatile("" : "+s"(v.n_out[l]), "+s"(v.nb_in[l]), "+s"(v.act[l]), "+s"(v.param[l]),
                 "+s"(v.param2[l]));
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s)
    asm volatile("" : "+s"(v.role[s]), "+s"(v.width[s]), "+s"(v.off[s]));
#if TGX_NN_MATH
  asm volatile("" : "+s"(v.nw));
#pragma unroll
  for (int l = 0; l < kMaxLayers; ++l) asm volatile("" : "+s"(v.norm[l]), "+s"(v.eps[l]));
#endif
}

// Floats per layer of the weight blocks (compile-time without LayerNorm).
template <int W>
__device__ __forceinline__ int layer_stride(const MlpView& m) {
#if TGX_NN_MATH
  return m.nw;
#else
  (void)m;
  return W * W + W;
#endif
}

#if TGX_NN_MATH
// LayerNorm over the n real outputs of a layer (Torch's nn.LayerNorm over
// the last axis: biased variance, eps inside the square root): z becomes
// x_hat = (z - mean) / sqrt(var + eps), 0 past n.  Returns 1 / sqrt(var + eps).
template <int W>
__device__ __forceinline__ float norm_rows(float (&z)[W], int n, float eps) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k) s += k < n ? z[k] : 0.f;
  const float inv_n = 1.f / static_cast<float>(n);
  const float mean = s * inv_n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const float d = z[k] - mean;
    q = k < n ? fmaf(d, d, q) : q;
  }
  const float rstd = 1.f / sqrtf(q * inv_n + eps);
#pragma unroll
  for (int k = 0; k < W; ++k) z[k] = k < n ? (z[k] - mean) * rstd : 0.f;
  return rstd;
}

// y = gamma x_hat + beta (gb: the layer's gamma, then beta; zero padding).
template <int W>
__device__ __forceinline__ void norm_affine(cfloat* gb, const float (&xh)[W], float (&y)[W]) {
#pragma unroll
  for (int k = 0; k < W; ++k) y[k] = fmaf(gb[k], xh[k], gb[W + k]);
}

// d (in: the gradient at y) becomes the gradient at the layer's z:
// d x_hat = gamma d, dz = rstd (d x_hat - mean(d x_hat) - x_hat mean(d x_hat
// x_hat)) over the n real outputs, 0 past n.
template <int W>
__device__ __forceinline__ void norm_rows_grad(cfloat* gb, const float (&xh)[W], float (&d)[W],
                                               int n, float rstd) {
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k) {
    d[k] *= gb[k];
    s1 += k < n ? d[k] : 0.f;
    s2 = k < n ? fmaf(d[k], xh[k], s2) : s2;
  }
  const float inv_n = 1.f / static_cast<float>(n);
  const float m1 = s1 * inv_n, m2 = s2 * inv_n;
#pragma unroll
  for (int k = 0; k < W; ++k) d[k] = k < n ? rstd * (d[k] - m1 - xh[k] * m2) : 0.f;
}
#endif

// A hidden layer's LayerNorm, when it has one, on its pre-activation z in
// place (wl: the layer's weight block).
template <int W>
__device__ __forceinline__ void norm_layer(const MlpView& m, int l, cfloat* wl, float (&z)[W]) {
#if TGX_NN_MATH
  if constexpr (W <= 32) {
    if (m.norm[l]) {
      norm_rows<W>(z, m.n_out[l], m.eps[l]);
      norm_affine<W>(wl + W * W + W, z, z);
    }
  }
#else
  (void)m, (void)l, (void)wl, (void)z;
#endif
}

// z = W_l a + b_l over the layer's real shape, in tiles of 8 rows x 8
// columns: a row tile runs when it holds a real output (o < n_out) and a
// column tile when it holds a real input (4 nb = n_in rounded up to 4), so
// one uniform branch skips 64 products with zero padding and the eight
// weights of a tile row are one scalar load.  Rows go in pairs, the next
// pair's weights loaded ahead of this pair's FMAs (the scheduling barriers
// keep the compiler from moving the loads back next to their use).  Each z[o] is the bias plus
// its products in ascending column order; padded rows get z = 0.  The
// padding of a column tile beyond n_in multiplies zero weights by the zero
// (or finite) padded inputs.
template <int W>
__device__ __forceinline__ void linear(cfloat* wl, const float (&a)[W], float (&z)[W], int n_out,
                                       int nb) {
  static_assert(W % 8 == 0, "tiles of 8");
  static_for<W / 8>([&](auto rc) TGX_INLINE_LAMBDA {
    constexpr int r0 = 8 * decltype(rc)::value;
    if (r0 < n_out) {
#pragma unroll
      for (int r = 0; r < 8; ++r) z[r0 + r] = wl[W * W + r0 + r];
#pragma unroll
      for (int c = 0; c < W / 8; ++c) {
        if (2 * c < nb) {
          // Rows in pairs; the next pair's weights are loaded before this
          // pair's FMAs so the scalar-cache latency overlaps them.
          float wp[2][2][8];
#pragma unroll
          for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) wp[0][r][j] = wl[(r0 + r) * W + 8 * c + j];
          static_for<4>([&](auto pc) TGX_INLINE_LAMBDA {
            constexpr int p = decltype(pc)::value;
            if constexpr (p + 1 < 4) {
#pragma unroll
              for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                  wp[(p + 1) & 1][r][j] = wl[(r0 + 2 * p + 2 + r) * W + 8 * c + j];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
              for (int j = 0; j < 8; ++j)
                z[r0 + 2 * p + r] = fmaf(wp[p & 1][r][j], a[8 * c + j], z[r0 + 2 * p + r]);
            __builtin_amdgcn_sched_barrier(0);
          });
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) z[r0 + r] = 0.f;
    }
  });
}

// g = W_l^T dz over the layer's real shape in the same 8 x 8 tiles (g is 0
// beyond the real column tiles); each g[i] adds its rows in ascending order.
template <int W>
__device__ __forceinline__ void linear_t(cfloat* wl, const float (&dz)[W], float (&g)[W],
                                         int n_out, int nb) {
  static_assert(W % 8 == 0, "tiles of 8");
#pragma unroll
  for (int i = 0; i < W; ++i) g[i] = 0.f;
  static_for<W / 8>([&](auto cc) TGX_INLINE_LAMBDA {
    constexpr int c0 = 8 * decltype(cc)::value;
    if (c0 < 4 * nb) {
#pragma unroll
      for (int t = 0; t < W / 8; ++t) {
        if (8 * t < n_out) {
          float wp[2][2][8];
#pragma unroll
          for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j) wp[0][r][j] = wl[(8 * t + r) * W + c0 + j];
          static_for<4>([&](auto pc) TGX_INLINE_LAMBDA {
            constexpr int p = decltype(pc)::value;
            if constexpr (p + 1 < 4) {
#pragma unroll
              for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                  wp[(p + 1) & 1][r][j] = wl[(8 * t + 2 * p + 2 + r) * W + c0 + j];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
              for (int j = 0; j < 8; ++j)
                g[c0 + j] = fmaf(wp[p & 1][r][j], dz[8 * t + 2 * p + r], g[c0 + j]);
            __builtin_amdgcn_sched_barrier(0);
          });
        }
      }
    }
  });
}

// The one output of a last layer: b + w . a over the real column tiles.
template <int W>
__device__ __forceinline__ float linear_out1(cfloat* wl, const float (&a)[W], int nb) {
  float z = wl[W * W];
#pragma unroll
  for (int c = 0; c < W / 8; ++c)
    if (2 * c < nb)
#pragma unroll
      for (int j = 0; j < 8; ++j) z = fmaf(wl[8 * c + j], a[8 * c + j], z);
  return z;
}

// g = ds w (the input gradient of a one-output last layer), 0 beyond the
// real column tiles.
template <int W>
__device__ __forceinline__ void linear_t_out1(cfloat* wl, float ds, float (&g)[W], int nb) {
#pragma unroll
  for (int c = 0; c < W / 8; ++c) {
    if (2 * c < nb) {
#pragma unroll
      for (int j = 0; j < 8; ++j) g[8 * c + j] = ds * wl[8 * c + j];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) g[8 * c + j] = 0.f;
    }
  }
}

// out[k] = f(z[k]) for the layer's real outputs (k < 4 nb, nb = its real
// width in blocks of 4), 0 beyond.  The switch on the activation code is
// taken once per layer; each case is a straight run over the elements.
template <int W, typename F>
__device__ __forceinline__ void map_real(const float (&z)[W], float (&out)[W], int nb, F f) {
#pragma unroll
  for (int k = 0; k < W / 4; ++k) {
    if (k < nb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * k + j] = f(z[4 * k + j], 4 * k + j);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * k + j] = 0.f;
    }
  }
}

#define TGX_ACT_CASES(X)                                                                 \
  X(TGX_ACT_RELU) X(TGX_ACT_LEAKY_RELU) X(TGX_ACT_TANH) X(TGX_ACT_SIGMOID) X(TGX_ACT_SILU) \
  X(TGX_ACT_GELU) X(TGX_ACT_ELU) X(TGX_ACT_HARDTANH) X(TGX_ACT_SOFTPLUS) X(TGX_ACT_SELU)   \
  X(TGX_ACT_MISH) X(TGX_ACT_HARDSIGMOID) X(TGX_ACT_HARDSWISH)

// The power functions as c z^e: sqrt (e = 1/2), rsqrt (-1/2), square (2),
// reciprocal p / z (e = -1, c = p), pow z^p.  One code path for the five
// keeps the kernels' size down (each case is a straight run over W values).
__device__ __forceinline__ void power_form(int act, float p, float& e, float& c) {
  c = 1.f;
  switch (act) {
    case TGX_ACT_SQRT: e = 0.5f; break;
    case TGX_ACT_RSQRT: e = -0.5f; break;
    case TGX_ACT_SQUARE: e = 2.f; break;
    case TGX_ACT_RECIPROCAL: e = -1.f; c = p; break;
    default: e = p; break;
  }
}

#define TGX_POWER_CASES \
  case TGX_ACT_SQRT: case TGX_ACT_RSQRT: case TGX_ACT_SQUARE: case TGX_ACT_RECIPROCAL: \
  case TGX_ACT_POW

// The per-layer activation sweeps differ between the two sets of functions:
// a namespace of their own per set keeps the two definitions apart.
namespace TGX_TIER(tier) {

// Activation of the n real outputs.  log and the power functions may not be
// finite at 0 (a padding column's 0 would become inf, and inf times a zero
// weight NaN downstream): their padding columns get 0.
template <int W>
__device__ __forceinline__ void activate_all(const float (&z)[W], float (&a)[W], int act,
                                             float p, float p2, int nb, int n) {
  switch (act) {
#define TGX_ACT_CASE(CODE)                                                             \
  case CODE:                                                                           \
    map_real<W>(z, a, nb, [p, p2](float v, int) TGX_INLINE_LAMBDA {                    \
      return activate(v, CODE, p, p2);                                                 \
    });                                                                                \
    break;
    TGX_ACT_CASES(TGX_ACT_CASE)
#undef TGX_ACT_CASE
#if TGX_NN_MATH
    case TGX_ACT_EXP:
      map_real<W>(z, a, nb, [](float v, int) TGX_INLINE_LAMBDA { return expf(v); });
      break;
    case TGX_ACT_LOG:
      map_real<W>(z, a, nb, [n](float v, int k) TGX_INLINE_LAMBDA {
        return k < n ? logf(v) : 0.f;
      });
      break;
    case TGX_ACT_ABS:
      map_real<W>(z, a, nb, [](float v, int) TGX_INLINE_LAMBDA { return fabsf(v); });
      break;
    case TGX_ACT_SIN:
    case TGX_ACT_COS: {
      const bool cosine = act == TGX_ACT_COS;
      map_real<W>(z, a, nb, [cosine](float v, int) TGX_INLINE_LAMBDA {
        float sv, cv;
        sincosf(v, &sv, &cv);
        return cosine ? cv : sv;
      });
      break;
    }
    TGX_POWER_CASES: {
      float e, c;
      power_form(act, p, e, c);
      map_real<W>(z, a, nb, [e, c, n](float v, int k) TGX_INLINE_LAMBDA {
        return k < n ? c * powf(v, e) : 0.f;
      });
      break;
    }
#endif
    default:
      map_real<W>(z, a, nb, [](float v, int) TGX_INLINE_LAMBDA { return v; });
      break;
  }
}

// dz[k] = g[k] * activate'(z[k]) for the n real outputs, 0 beyond for log
// and the power functions.  Torch's pow backward is 0 for a zero exponent.
template <int W>
__device__ __forceinline__ void activate_grad_all(const float (&z)[W], const float (&g)[W],
                                                  float (&dz)[W], int act, float p, float p2,
                                                  int nb, int n) {
  switch (act) {
#define TGX_ACT_CASE(CODE)                                                             \
  case CODE:                                                                           \
    map_real<W>(z, dz, nb, [&g, p, p2](float v, int k) TGX_INLINE_LAMBDA {             \
      return g[k] * activate_grad(v, CODE, p, p2);                                     \
    });                                                                                \
    break;
    TGX_ACT_CASES(TGX_ACT_CASE)
#undef TGX_ACT_CASE
#if TGX_NN_MATH
    case TGX_ACT_EXP:
      map_real<W>(z, dz, nb, [&g](float v, int k) TGX_INLINE_LAMBDA { return g[k] * expf(v); });
      break;
    case TGX_ACT_LOG:
      map_real<W>(z, dz, nb, [&g, n](float v, int k) TGX_INLINE_LAMBDA {
        return k < n ? g[k] / v : 0.f;
      });
      break;
    case TGX_ACT_ABS:
      map_real<W>(z, dz, nb, [&g](float v, int k) TGX_INLINE_LAMBDA {
        return v > 0.f ? g[k] : (v < 0.f ? -g[k] : 0.f);
      });
      break;
    case TGX_ACT_SIN:
    case TGX_ACT_COS: {
      const bool cosine = act == TGX_ACT_COS;
      map_real<W>(z, dz, nb, [&g, cosine](float v, int k) TGX_INLINE_LAMBDA {
        float sv, cv;
        sincosf(v, &sv, &cv);
        return cosine ? -g[k] * sv : g[k] * cv;
      });
      break;
    }
    TGX_POWER_CASES: {
      float e, c;
      power_form(act, p, e, c);
      const float ce = e == 0.f ? 0.f : c * e;
      map_real<W>(z, dz, nb, [&g, e, ce, n](float v, int k) TGX_INLINE_LAMBDA {
        return k < n ? g[k] * (ce * powf(v, e - 1.f)) : 0.f;
      });
      break;
    }
#endif
    default:
      map_real<W>(z, dz, nb, [&g](float, int k) TGX_INLINE_LAMBDA { return g[k]; });
      break;
  }
}

}  // namespace TGX_TIER(tier)
using namespace TGX_TIER(tier);

// Whether a chain uses a function of the second set (above) or LayerNorm.
inline bool uses_math_tier(const tgx_edge_mlp* mlp) {
  if (!mlp || mlp->n_layers < 1 || mlp->n_layers > kMaxLayers) return false;
  for (int l = 0; l < mlp->n_layers; ++l)
    if ((l + 1 < mlp->n_layers && mlp->act[l] >= TGX_ACT_EXP && mlp->act[l] <= TGX_ACT_POW) ||
        mlp->norm[l])
      return true;
  return false;
}

// The edge-MLP kernel launches per column index type: tgx_nn.hip builds the
// int32_t ones (with the entry points), tgx_nn_i64.hip the int64_t ones and
// the occupancy query (separately per tier, TGX_TIER).
void TGX_TIER(mlp_fwd)(int W, int L, const int32_t* col, const int32_t* dst, int64_t E,
                       const MlpView& v, float* scores, hipStream_t s);
void TGX_TIER(mlp_fwd)(int W, int L, const int64_t* col, const int32_t* dst, int64_t E,
                       const MlpView& v, float* scores, hipStream_t s);
void TGX_TIER(mlp_hidden)(int W, int L, const int32_t* col, const int32_t* dst, int64_t E,
                          const MlpView& v, float* hidden, int hw, hipStream_t s);
void TGX_TIER(mlp_hidden)(int W, int L, const int64_t* col, const int32_t* dst, int64_t E,
                          const MlpView& v, float* hidden, int hw, hipStream_t s);
// seeded: the edge-network sum's backward (seed per destination row, hw
// wide) in place of the score gradient ds.
void TGX_TIER(mlp_bwd)(bool seeded, int W, int L, const int32_t* col, const int32_t* dst,
                       int64_t E, int blocks, int64_t chunk, const MlpView& v, const float* ds,
                       float* partial, const float* seed, int hw, hipStream_t s);
void TGX_TIER(mlp_bwd)(bool seeded, int W, int L, const int64_t* col, const int32_t* dst,
                       int64_t E, int blocks, int64_t chunk, const MlpView& v, const float* ds,
                       float* partial, const float* seed, int hw, hipStream_t s);
// Blocks of the fused backward kernel (W <= 32) resident on the current
// device, from the int64_t instance's occupancy; it sizes the grid (and the
// workspace) of both index types.
int64_t TGX_TIER(mlp_bwd_resident)(int W, int L);

// 64-wide chains: backward in two passes (tgx_nn_wide.hip).  Blocks and
// chunk of the outer-sum pass for n_edges edges.
int TGX_TIER(outer_blocks)(int64_t n_edges, int64_t* chunk);

// Per-edge planes (acts, dz: n_layers x [n_edges, 64] each) and the
// per-segment input gradients, then the per-layer weight-gradient partial
// sums of outer_nb blocks into partial[block * n_layers * NW + l * NW + ...]
// (NW = 64 * 64 + 64).  Launches on `s`; TGX_* status.
int TGX_TIER(planes_backward)(int n_layers, int idx_bits, const void* col, const int32_t* dst,
                              int64_t n_edges, const MlpView& v, const float* dscore,
                              float* acts, float* dz, int outer_nb, int64_t outer_chunk,
                              float* partial, hipStream_t s);

}  // namespace mlp
}  // namespace tgx

// The edge-MLP entry points of tgx.h built with the second set of functions
// (tgx_nn_math.hip); the public entry points call them for chains that use
// one of those functions.  Same arguments and status codes.
#define TGX_NN_HIDDEN __attribute__((visibility("hidden")))
TGX_NN_HIDDEN int tgx_edge_mlp_scores_math(const void* col, const int32_t* dst_index,
                                           int idx_bits, int64_t n_edges,
                                           const tgx_edge_mlp* mlp, float* scores,
                                           void* stream);
TGX_NN_HIDDEN int tgx_edge_mlp_backward_workspace_math(int64_t n_edges, const tgx_edge_mlp* mlp,
                                                       size_t* bytes);
TGX_NN_HIDDEN int tgx_edge_mlp_backward_math(const void* col, const int32_t* dst_index,
                                             int idx_bits, int64_t n_edges,
                                             const tgx_edge_mlp* mlp, const float* dscore,
                                             float* dweights, float* const* dseg,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream);
TGX_NN_HIDDEN int tgx_edge_mlp_attention_backward_math(
    const void* col, const int32_t* dst_index, int idx_bits, int64_t n_edges,
    const tgx_edge_mlp* mlp, const float* lse, const float* out, const float* dout,
    const float* value, int32_t value_width, float* alpha, int fold_segment, float* dweights,
    float* const* dseg, void* workspace, size_t workspace_bytes, void* stream);
TGX_NN_HIDDEN int tgx_edge_mlp_hidden_math(const void* col, const int32_t* dst_index,
                                           int idx_bits, int64_t n_edges,
                                           const tgx_edge_mlp* mlp, float* hidden,
                                           int32_t hidden_width, void* stream);
TGX_NN_HIDDEN int tgx_edge_mlp_backward_seeded_math(const void* col, const int32_t* dst_index,
                                                    int idx_bits, int64_t n_edges,
                                                    const tgx_edge_mlp* mlp, const float* seed,
                                                    int32_t seed_width, float* dweights,
                                                    float* const* dseg, void* workspace,
                                                    size_t workspace_bytes, void* stream);
