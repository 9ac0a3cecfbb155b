// Dot-product edge attention over a destination-row CSR, bf16 in / fp32
// accumulate:
//
//   s_e = scale * (k[j, hd] . q[i, hd]) + bias[e, hd]     (j = col[e], i = row)
//   out[i, hd] = sum_e softmax_i(s)_e * v[j, hd]          (bf16 output)
//
// Reference semantics: edge() returning
//   reducer((src.k * dst.q).sum(-1) * scale + edge.bias, src.v)
// on the eager oracle (python/tiga/interop/torch/message_passing.py:2848-2894,
// reducer_oracle.py:60-137, fp32 accumulation for bf16 inputs, result cast
// back to bf16).
//
// Layout: q, k, v, dout are [N, H, D] bf16; one node row is 8*G values over G
// lanes (16 bytes = 8 bf16 per lane), head hd on HL = D/8 lanes.  bias/dbias
// are [E, H] fp32 in edge order.  ml [N, H, 2] fp32 = {logsumexp, delta}.
//
// Backward (no float atomics; alpha recomputed from the saved logsumexp):
//   B1 node pass     delta[i] = <dout[i], out[i]> per head
//   B2 destination pass over the CSR: ds_e = alpha_e (<dout[i], v[j]> - delta[i]),
//                    dbias[e] = ds_e, dq[i] = scale * sum ds_e k[j]
//   B3 source pass over the transposed CSR: dk[j] = scale * sum ds_e q[i],
//                    dv[j] = sum alpha_e dout[i]
//   Hub rows of either CSR are split into chunks whose fp32 partials are
//   summed in chunk order.
// Stored ds (the caller passes inv_perm): B3 runs first and also writes each
// edge's ds at its transposed position (coalesced, [E, H] fp32); B2 then
// reads ds through inv_perm instead of recomputing it, so it gathers only
// the k row per edge (the recomputation needs k and v rows, q, dout and
// the node state): one scattered 4H-byte read replaces a 2·D·H-byte row.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "tgx_device.h"
#include "tgx_host.h"
#include "tgx_profile.h"
#include "tgx_softmax.h"
#include "tgx_tasks.h"
#include "tgx_vals.h"

namespace tgx {
namespace {

template <class V>
__device__ __forceinline__ float dot8(const float (&a)[8], typename V::Raw b) {
  float f[8];
  V::unpack(b, f);
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) s += a[q] * f[q];
  return s;
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}

template <int EPW>
__device__ __forceinline__ int fetch_lane(int v, int src) {
  if constexpr (EPW == 1) return __builtin_amdgcn_readlane(v, src);
  return __shfl(v, src, 64);
}

template <int G>
__device__ __forceinline__ void fold_groups(float (&v)[8]) {
#pragma unroll
  for (int mask = G; mask < kWave; mask <<= 1)
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] += __shfl_xor(v[q], mask, 64);
}

// ---------------------------------------------------------------------------
// Forward

template <int DT, typename I>
struct DotFwdArgs {
  using T = typename Vals<DT, 8>::T;
  const I* row_ptr;
  const I* col;
  PlanView plan;
  const T* q;
  const T* k;
  const T* v;
  const float* bias;  // [E, H] or null
  float scale;
  T* out;
  float* ml;          // [N, H, 2]
  float* partial;     // per chunk: acc[8G] | m[H] | l[H]
  int64_t ld;         // values between consecutive nodes' rows of q, k, v, out
  int64_t mld;        // floats between consecutive nodes' rows of ml
  int64_t bld;        // floats between consecutive edges' rows of bias
};

template <int DT, typename I, int G, int HL, int U>
__global__ __launch_bounds__(kTaskBlock) void dot_fwd_kernel(DotFwdArgs<DT, I> a) {
  using V = Vals<DT, 8>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 8 * G;
  constexpr int H = G / HL;
  const Task t = decode_task(a.plan, a.row_ptr, global_wave());
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  const bool head_lead = (c % HL) == 0;
  if (t.kind == kTaskEmpty) {
    for (int r = 0; r < t.n_empty; ++r) {
      const int64_t i = uniform(a.plan.rows[t.empty0 + r]);
      if (g == 0) {
        V::store_zero(a.out + i * a.ld + 8 * c);
        if (head_lead) {
          a.ml[i * a.mld + hd * 2] = kNegInf;
          a.ml[i * a.mld + hd * 2 + 1] = 0.f;
        }
      }
    }
    return;
  }
  const int64_t row = t.row;
  float qf[8];
  V::unpack(V::load(a.q + row * a.ld + 8 * c), qf);
  SoftState<8> st;
  st.init();
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    const int my_col = lane < n ? static_cast<int>(a.col[base + lane]) : 0;
    for (int k = 0; k < n; k += EPW * U) {
      typename V::Raw kk[U], vv[U];
      float bb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const int j = fetch_lane<EPW>(my_col, slot < n ? slot : 0);
        kk[u] = V::load(a.k + static_cast<int64_t>(j) * a.ld + 8 * c);
        vv[u] = V::load(a.v + static_cast<int64_t>(j) * a.ld + 8 * c);
        bb[u] = (a.bias && slot < n) ? a.bias[(base + slot) * a.bld + hd] : 0.f;
      }
      float s[U];
      float mc = kNegInf;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const float sc = group_sum<HL>(dot8<V>(qf, kk[u])) * a.scale + bb[u];
        s[u] = slot < n ? sc : kNegInf;
        mc = fmaxf(mc, s[u]);
      }
      if (mc > st.m) st.rescale(mc);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = s[u] == kNegInf ? 0.f : fast_exp(s[u] - st.m);
        st.l += p;
        float vf[8];
        V::unpack(vv[u], vf);
#pragma unroll
        for (int q = 0; q < 8; ++q) st.acc[q] += p * vf[q];
      }
    }
  }
#pragma unroll
  for (int mask = G; mask < kWave; mask <<= 1) st.merge_xor(mask);
  if (g != 0) return;
  if (t.kind == kTaskChunk) {
    float* p = a.partial + static_cast<int64_t>(t.slot) * (HD + 2 * H);
    store8(p + 8 * c, st.acc);
    if (head_lead) {
      p[HD + hd] = st.m;
      p[HD + H + hd] = st.l;
    }
    return;
  }
  const float inv = 1.f / st.l;
  float o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = st.acc[q] * inv;
  V::store(a.out + row * a.ld + 8 * c, o);
  if (head_lead) {
    a.ml[row * a.mld + hd * 2] = st.m + __logf(st.l);
    a.ml[row * a.mld + hd * 2 + 1] = 0.f;
  }
}

template <int DT, int G, int HL>
__global__ __launch_bounds__(kTaskBlock) void dot_fwd_merge_kernel(
    PlanView plan, const float* __restrict__ partial, typename Vals<DT, 8>::T* __restrict__ out,
    float* __restrict__ ml, int64_t ld, int64_t mld) {
  using V = Vals<DT, 8>;
  constexpr int HD = 8 * G;
  constexpr int H = G / HL;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int c = lane_id();
  if (c >= G) return;
  const int hd = c / HL;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  SoftState<8> st;
  st.init();
  // Eight chunks' partials are requested before they are merged (a hub row
  // has up to hundreds of chunks; the merges depend on each other, the
  // loads do not): 0.115 -> 0.034 ms on the R-MAT scale-21 forward
  // (bench.py --config c3).
  int q = c0;
  for (; q + 8 <= c1; q += 8) {
    float acc[8][8], pm[8], pl[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float* p = partial + static_cast<int64_t>(q + u) * (HD + 2 * H);
      load8(p + 8 * c, acc[u]);
      pm[u] = p[HD + hd];
      pl[u] = p[HD + H + hd];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) st.merge(pm[u], pl[u], acc[u]);
  }
  for (; q < c1; ++q) {
    const float* p = partial + static_cast<int64_t>(q) * (HD + 2 * H);
    float acc[8];
    load8(p + 8 * c, acc);
    st.merge(p[HD + hd], p[HD + H + hd], acc);
  }
  const float inv = 1.f / st.l;
  float o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = st.acc[q] * inv;
  V::store(out + row * ld + 8 * c, o);
  if (c % HL == 0) {
    ml[row * mld + hd * 2] = st.m + __logf(st.l);
    ml[row * mld + hd * 2 + 1] = 0.f;
  }
}

// ---------------------------------------------------------------------------
// Backward

template <int DT, int G, int HL>
__global__ __launch_bounds__(kTaskBlock) void dot_delta_kernel(
    const typename Vals<DT, 8>::T* __restrict__ dout, const typename Vals<DT, 8>::T* __restrict__ out,
    float* __restrict__ ml, int64_t n_nodes, int64_t ld, int64_t mld) {
  using V = Vals<DT, 8>;
  constexpr int EPW = kWave / G;
  const int lane = lane_id();
  const int c = lane % G, hd = c / HL;
  const int64_t node = global_wave() * EPW + lane / G;
  if (node >= n_nodes) return;
  float d[8];
  V::unpack(V::load(dout + node * ld + 8 * c), d);
  const float delta = group_sum<HL>(dot8<V>(d, V::load(out + node * ld + 8 * c)));
  if (c % HL == 0) ml[node * mld + hd * 2 + 1] = delta;
}

template <int DT, typename I>
struct DotDstArgs {
  using T = typename Vals<DT, 8>::T;
  const I* row_ptr;
  const I* col;
  PlanView plan;
  const T* q;
  const T* k;
  const T* v;
  const float* bias;
  float scale;
  const float* ml;
  const T* dout;
  T* dq;
  float* dbias;     // [E, H] or null
  float* partial;   // per chunk: [8G] unscaled dq
  int64_t ld;       // values between consecutive nodes' rows of q, k, v, dout, dq
  int64_t mld;      // floats between consecutive nodes' rows of ml
  int64_t bld;      // floats between consecutive edges' rows of bias and dbias
  const int32_t* inv_perm;  // STORED: [E] transposed position of each edge
  const float* ds_t;        // STORED: [E, H] ds in transposed order (from B3)
  int64_t n_edges;          // STORED: E, the rows of ds_t (reads past it give 0)
};

// STORED: ds read through inv_perm (B3 ran first); otherwise recomputed.
// (The dbias stores stay in the loop: staging them in LDS like the source
// pass's ds measured slower here, 3.38 -> 3.60 ms on the R-MAT scale-21
// backward, bench.py --config c4.)
template <int DT, typename I, int G, int HL, int U, bool STORED>
__global__ __launch_bounds__(kTaskBlock) void dot_bwd_dst_kernel(DotDstArgs<DT, I> a) {
  using V = Vals<DT, 8>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 8 * G;
  const Task t = decode_task(a.plan, a.row_ptr, global_wave());
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  const bool head_lead = (c % HL) == 0;
  if (t.kind == kTaskEmpty) {
    for (int r = 0; r < t.n_empty; ++r) {
      const int64_t i = uniform(a.plan.rows[t.empty0 + r]);
      if (g == 0) V::store_zero(a.dq + i * a.ld + 8 * c);
    }
    return;
  }
  const int64_t row = t.row;
  float dq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (STORED) {
    constexpr int H = G / HL;
    for (int64_t base = t.e0; base < t.e1; base += kWave) {
      const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
      int my_col = 0, my_p = 0;
      if (lane < n) {
        my_col = static_cast<int>(a.col[base + lane]);
        my_p = a.inv_perm[base + lane];
      }
      for (int k = 0; k < n; k += EPW * U) {
        typename V::Raw kk[U];
        float dsv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int slot = k + u * EPW + g;
          const int src = slot < n ? slot : 0;
          const int j = fetch_lane<EPW>(my_col, src);
          const int64_t p = fetch_lane<EPW>(my_p, src);
          kk[u] = V::load(a.k + static_cast<int64_t>(j) * a.ld + 8 * c);
          dsv[u] = slot < n && p < a.n_edges ? a.ds_t[p * H + hd] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int slot = k + u * EPW + g;
          if (a.dbias && slot < n && head_lead) a.dbias[(base + slot) * a.bld + hd] = dsv[u];
          float kf[8];
          V::unpack(kk[u], kf);
#pragma unroll
          for (int q = 0; q < 8; ++q) dq[q] += dsv[u] * kf[q];
        }
      }
    }
  } else {
  float qf[8], df[8];
  V::unpack(V::load(a.q + row * a.ld + 8 * c), qf);
  V::unpack(V::load(a.dout + row * a.ld + 8 * c), df);
  const float lse = a.ml[row * a.mld + hd * 2];
  const float delta = a.ml[row * a.mld + hd * 2 + 1];
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    const int my_col = lane < n ? static_cast<int>(a.col[base + lane]) : 0;
    for (int k = 0; k < n; k += EPW * U) {
      typename V::Raw kk[U], vv[U];
      float bb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const int j = fetch_lane<EPW>(my_col, slot < n ? slot : 0);
        kk[u] = V::load(a.k + static_cast<int64_t>(j) * a.ld + 8 * c);
        vv[u] = V::load(a.v + static_cast<int64_t>(j) * a.ld + 8 * c);
        bb[u] = (a.bias && slot < n) ? a.bias[(base + slot) * a.bld + hd] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const bool valid = slot < n;
        const float s = group_sum<HL>(dot8<V>(qf, kk[u])) * a.scale + bb[u];
        const float alpha = valid ? fast_exp(s - lse) : 0.f;
        const float dalpha = group_sum<HL>(dot8<V>(df, vv[u]));
        const float ds = alpha * (dalpha - delta);
        if (a.dbias && valid && head_lead) a.dbias[(base + slot) * a.bld + hd] = ds;
        float kf[8];
        V::unpack(kk[u], kf);
#pragma unroll
        for (int q = 0; q < 8; ++q) dq[q] += ds * kf[q];
      }
    }
  }
  }
  fold_groups<G>(dq);
  if (g != 0) return;
  if (t.kind == kTaskChunk) {
    store8(a.partial + static_cast<int64_t>(t.slot) * HD + 8 * c, dq);
    return;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) dq[q] *= a.scale;
  V::store(a.dq + row * a.ld + 8 * c, dq);
}

template <int DT, int G>
__global__ __launch_bounds__(kTaskBlock) void dot_dq_merge_kernel(
    PlanView plan, const float* __restrict__ partial, float scale,
    typename Vals<DT, 8>::T* __restrict__ dq, int64_t ld) {
  using V = Vals<DT, 8>;
  constexpr int HD = 8 * G;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int c = lane_id();
  if (c >= G) return;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Eight chunks' partials in flight per step; summed in chunk order.
  int q = c0;
  for (; q + 8 <= c1; q += 8) {
    float p[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) load8(partial + static_cast<int64_t>(q + u) * HD + 8 * c, p[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int r = 0; r < 8; ++r) s[r] += p[u][r];
  }
  for (; q < c1; ++q) {
    float p[8];
    load8(partial + static_cast<int64_t>(q) * HD + 8 * c, p);
#pragma unroll
    for (int r = 0; r < 8; ++r) s[r] += p[r];
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) s[r] *= scale;
  V::store(dq + row * ld + 8 * c, s);
}

template <int DT>
struct DotSrcArgs {
  using T = typename Vals<DT, 8>::T;
  const int32_t* row_ptr_t;
  const int32_t* col_t;
  const int32_t* perm;
  PlanView plan;
  const T* q;
  const T* k;
  const T* v;
  const float* bias;
  float scale;
  const float* ml;
  const T* dout;
  T* dk;
  T* dv;
  float* partial;   // per chunk: [8G] unscaled dk | [8G] dv
  int64_t ld;       // values between consecutive nodes' rows of q, k, v, dout, dk, dv
  int64_t mld;      // floats between consecutive nodes' rows of ml
  int64_t bld;      // floats between consecutive edges' rows of bias
  float* ds_t;      // STORE_DS: [E, H] out, ds at each edge's transposed position
  int64_t n_edges;  // STORE_DS: E, the rows of ds_t (no write past it)
};

// STORE_DS: a window's ds (up to 64 edges x H) waits in LDS and leaves in
// one coalesced pass after the window (STAGE, H <= 16): a store per edge
// pair inside the loop would make every following gather wait for it, since
// loads and stores share one in-order completion counter.
template <int DT, int G, int HL, int U, bool STORE_DS>
__global__ __launch_bounds__(kTaskBlock) void dot_bwd_src_kernel(DotSrcArgs<DT> a) {
  using V = Vals<DT, 8>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 8 * G;
  constexpr int H = G / HL;
  constexpr bool STAGE = STORE_DS && H <= 16;
  __shared__ float stage[STAGE ? kWavesPerBlock : 1][STAGE ? kWave * H : 1];
  const int wave = threadIdx.x / kWave;
  const Task t = decode_task(a.plan, a.row_ptr_t, global_wave());
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  if (t.kind == kTaskEmpty) {
    for (int r = 0; r < t.n_empty; ++r) {
      const int64_t j = uniform(a.plan.rows[t.empty0 + r]);
      if (g == 0) {
        V::store_zero(a.dk + j * a.ld + 8 * c);
        V::store_zero(a.dv + j * a.ld + 8 * c);
      }
    }
    return;
  }
  const int64_t j = t.row;
  float kf[8], vf[8];
  V::unpack(V::load(a.k + j * a.ld + 8 * c), kf);
  V::unpack(V::load(a.v + j * a.ld + 8 * c), vf);
  float dk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float dv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    int my_i = 0, my_e = 0;
    if (lane < n) {
      my_i = a.col_t[base + lane];
      my_e = a.perm[base + lane];
    }
    for (int k = 0; k < n; k += EPW * U) {
      typename V::Raw qq[U], dd[U];
      float bb[U], lse[U], dl[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const int src = slot < n ? slot : 0;
        const int64_t i = fetch_lane<EPW>(my_i, src);
        const int64_t e = fetch_lane<EPW>(my_e, src);
        qq[u] = V::load(a.q + i * a.ld + 8 * c);
        dd[u] = V::load(a.dout + i * a.ld + 8 * c);
        lse[u] = a.ml[i * a.mld + hd * 2];
        dl[u] = a.ml[i * a.mld + hd * 2 + 1];
        bb[u] = a.bias ? a.bias[e * a.bld + hd] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const bool valid = slot < n;
        float qf[8], df[8];
        V::unpack(qq[u], qf);
        V::unpack(dd[u], df);
        float sp = 0.f, dp = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          sp += qf[q] * kf[q];
          dp += df[q] * vf[q];
        }
        const float s = group_sum<HL>(sp) * a.scale + bb[u];
        const float alpha = valid ? fast_exp(s - lse[u]) : 0.f;
        const float ds = alpha * (group_sum<HL>(dp) - dl[u]);
        if constexpr (STORE_DS) {
          if (valid && c % HL == 0) {
            if constexpr (STAGE)
              stage[wave][slot * H + hd] = ds;
            else if (base + slot < a.n_edges)
              a.ds_t[(base + slot) * H + hd] = ds;
          }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          dk[q] += ds * qf[q];
          dv[q] += alpha * df[q];
        }
      }
    }
    if constexpr (STAGE) {
      // One wave's LDS accesses complete in issue order, so every lane
      // reads the window's ds written above; the next window's writes come
      // after these reads.
      __builtin_amdgcn_wave_barrier();
      const int cnt = static_cast<int>(min(static_cast<int64_t>(n), a.n_edges - base)) * H;
      for (int x = lane; x < cnt; x += kWave) a.ds_t[base * H + x] = stage[wave][x];
      __builtin_amdgcn_wave_barrier();
    }
  }
  fold_groups<G>(dk);
  fold_groups<G>(dv);
  if (g != 0) return;
  if (t.kind == kTaskChunk) {
    float* p = a.partial + static_cast<int64_t>(t.slot) * (2 * HD);
    store8(p + 8 * c, dk);
    store8(p + HD + 8 * c, dv);
    return;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) dk[q] *= a.scale;
  V::store(a.dk + j * a.ld + 8 * c, dk);
  V::store(a.dv + j * a.ld + 8 * c, dv);
}

template <int DT, int G>
__global__ __launch_bounds__(kTaskBlock) void dot_kv_merge_kernel(
    PlanView plan, const float* __restrict__ partial, float scale,
    typename Vals<DT, 8>::T* __restrict__ dk, typename Vals<DT, 8>::T* __restrict__ dv,
    int64_t ld) {
  using V = Vals<DT, 8>;
  constexpr int HD = 8 * G;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int c = lane_id();
  if (c >= G) return;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  float sk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float sv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Four chunks' dk and dv partials in flight per step; summed in chunk
  // order.
  int q = c0;
  for (; q + 4 <= c1; q += 4) {
    float pk[4][8], pv[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      load8(partial + static_cast<int64_t>(q + u) * (2 * HD) + 8 * c, pk[u]);
      load8(partial + static_cast<int64_t>(q + u) * (2 * HD) + HD + 8 * c, pv[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        sk[r] += pk[u][r];
        sv[r] += pv[u][r];
      }
  }
  for (; q < c1; ++q) {
    float pk[8], pv[8];
    load8(partial + static_cast<int64_t>(q) * (2 * HD) + 8 * c, pk);
    load8(partial + static_cast<int64_t>(q) * (2 * HD) + HD + 8 * c, pv);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      sk[r] += pk[r];
      sv[r] += pv[r];
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) sk[r] *= scale;
  V::store(dk + row * ld + 8 * c, sk);
  V::store(dv + row * ld + 8 * c, sv);
}

// ---------------------------------------------------------------------------
// Host dispatch

struct DotShape {
  int G, HL;
};

// Heads run in groups (group_heads, kDotGroupValues): each group launches the
// kernels over its strided slice of q, k, v, out, dout, dq, dk, dv, ml, bias
// and dbias.
int dot_group_heads(int H, int D, int h0) { return group_heads(H, D, h0, kDotGroupValues); }

DotShape dot_shape(int Hg, int D) { return DotShape{Hg * D / 8, D / 8}; }

// Every (G, HL) a group can take: G = Hg * HL lanes, HL = D / 8 lanes per head.
#define TGX_DOT_SHAPES(X)                                                        \
  X(64, 64) X(64, 32) X(64, 16) X(64, 8) X(64, 4) X(64, 2) X(64, 1)            \
  X(32, 32) X(32, 16) X(32, 8) X(32, 4) X(32, 2) X(32, 1)                       \
  X(16, 16) X(16, 8) X(16, 4) X(16, 2) X(16, 1)                                 \
  X(8, 8) X(8, 4) X(8, 2) X(8, 1)                                               \
  X(4, 4) X(4, 2) X(4, 1)                                                       \
  X(2, 2) X(2, 1)                                                               \
  X(1, 1)

// Loads in flight per lane group (each covers a k and a v row, or a q and a
// dout row).  For H*D = 256 (32 lanes per row, two edges per wave-load) 1
// measured best on R-MAT scale 21, H=4, D=64 (2: +1.6% forward, +2.2%
// backward; 3: +4.6%), i.e. two edges' rows per wave in flight; other
// widths keep 2.
template <int G>
constexpr int dot_unroll() {
  return G == 32 ? 1 : 2;
}

template <int DT, typename I, int G, int HL>
int dot_fwd_launch(const DotFwdArgs<DT, I>& a, hipStream_t s) {
  constexpr int U = dot_unroll<G>();
  const int64_t waves = plan_waves(a.plan);
  if (waves > 0) {
    TGX_PROFILE("dot_fwd_kernel", s);
    dot_fwd_kernel<DT, I, G, HL, U><<<ceil_div(waves, kWavesPerBlock), kTaskBlock, 0, s>>>(a);
    TGX_LAUNCHED("dot_fwd_kernel");
  }
  if (a.plan.n_split > 0) {
    TGX_PROFILE("dot_fwd_merge_kernel", s);
    dot_fwd_merge_kernel<DT, G, HL>
        <<<ceil_div(a.plan.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(a.plan, a.partial, a.out,
                                                                          a.ml, a.ld, a.mld);
    TGX_LAUNCHED("dot_fwd_merge_kernel");
  }
  return TGX_OK;
}

struct DotBwdLayout {
  size_t dst_part_off, src_part_off, ds_off, bytes;
};

// stored: room for ds [E, H] of the widest head group.
DotBwdLayout dot_bwd_layout(const tgx_row_plan& plan, const tgx_row_plan& plan_t, int H, int D,
                            int64_t n_edges, bool stored) {
  DotBwdLayout L;
  const int64_t HD = static_cast<int64_t>(H) * D;
  Carve c{nullptr, 0};
  L.dst_part_off = reinterpret_cast<size_t>(c.take<float>(plan.n_chunks * HD));
  L.src_part_off = reinterpret_cast<size_t>(c.take<float>(plan_t.n_chunks * 2 * HD));
  L.ds_off = reinterpret_cast<size_t>(c.take<float>(stored ? n_edges * H : 0));
  L.bytes = align_up(c.used) + 256;
  return L;
}

template <int DT, typename I, int G, int HL>
int dot_bwd_launch(const DotDstArgs<DT, I>& da, const DotSrcArgs<DT>& sa,
                   const typename Vals<DT, 8>::T* out, float* ml, int64_t n_nodes,
                   hipStream_t s) {
  constexpr int U = dot_unroll<G>();
  constexpr int EPW = kWave / G;
  const bool stored = da.ds_t != nullptr;
  {
    TGX_PROFILE("dot_delta_kernel", s);
    dot_delta_kernel<DT, G, HL><<<ceil_div(ceil_div(n_nodes, EPW), kWavesPerBlock), kTaskBlock, 0,
                                  s>>>(da.dout, out, ml, n_nodes, da.ld, da.mld);
    TGX_LAUNCHED("dot_delta_kernel");
  }
  auto dst_pass = [&]() -> int {
    const int64_t dst_waves = plan_waves(da.plan);
    if (dst_waves > 0) {
      TGX_PROFILE("dot_bwd_dst_kernel", s);
      const auto k = stored ? dot_bwd_dst_kernel<DT, I, G, HL, U, true>
                            : dot_bwd_dst_kernel<DT, I, G, HL, U, false>;
      k<<<ceil_div(dst_waves, kWavesPerBlock), kTaskBlock, 0, s>>>(da);
      TGX_LAUNCHED("dot_bwd_dst_kernel");
    }
    if (da.plan.n_split > 0) {
      TGX_PROFILE("dot_dq_merge_kernel", s);
      dot_dq_merge_kernel<DT, G><<<ceil_div(da.plan.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
          da.plan, da.partial, da.scale, da.dq, da.ld);
      TGX_LAUNCHED("dot_dq_merge_kernel");
    }
    return TGX_OK;
  };
  // Stored ds: the source pass (which writes ds) runs before the
  // destination pass that reads it.
  if (!stored) {
    const int st = dst_pass();
    if (st != TGX_OK) return st;
  }
  const int64_t src_waves = plan_waves(sa.plan);
  if (src_waves > 0) {
    TGX_PROFILE("dot_bwd_src_kernel", s);
    const auto k = stored ? dot_bwd_src_kernel<DT, G, HL, U, true>
                          : dot_bwd_src_kernel<DT, G, HL, U, false>;
    k<<<ceil_div(src_waves, kWavesPerBlock), kTaskBlock, 0, s>>>(sa);
    TGX_LAUNCHED("dot_bwd_src_kernel");
  }
  if (sa.plan.n_split > 0) {
    TGX_PROFILE("dot_kv_merge_kernel", s);
    dot_kv_merge_kernel<DT, G><<<ceil_div(sa.plan.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
        sa.plan, sa.partial, sa.scale, sa.dk, sa.dv, sa.ld);
    TGX_LAUNCHED("dot_kv_merge_kernel");
  }
  if (stored) return dst_pass();
  return TGX_OK;
}

// One element format's forward over every head group.
template <int DT>
int dot_fwd_dtype(const void* row_ptr, const void* col, int idx_bits, const tgx_row_plan* plan,
                  const void* q, const void* k, const void* v, const float* bias, float scale,
                  void* out, float* ml, int H, int D, float* partial, hipStream_t s) {
  using T = typename Vals<DT, 8>::T;
  const int64_t ld = static_cast<int64_t>(H) * D, mld = 2 * static_cast<int64_t>(H), bld = H;
  for (int h0 = 0; h0 < H;) {
    const int hg = dot_group_heads(H, D, h0);
    const DotShape shp = dot_shape(hg, D);
    const int64_t off = static_cast<int64_t>(h0) * D;
    const T* qq = static_cast<const T*>(q) + off;
    const T* kk = k ? static_cast<const T*>(k) + off : nullptr;
    const T* vv = v ? static_cast<const T*>(v) + off : nullptr;
    T* oo = static_cast<T*>(out) + off;
    const float* bb = bias ? bias + h0 : nullptr;
    float* mm = ml + 2 * h0;
    int st = TGX_UNSUPPORTED;
#define TGX_DOT_FWD(GG, HH)                                                                  \
    if (shp.G == GG && shp.HL == HH) {                                                       \
      if (idx_bits == 32)                                                                    \
        st = dot_fwd_launch<DT, int32_t, GG, HH>(                                            \
            DotFwdArgs<DT, int32_t>{static_cast<const int32_t*>(row_ptr),                    \
                                    static_cast<const int32_t*>(col), plan_view(*plan), qq,  \
                                    kk, vv, bb, scale, oo, mm, partial, ld, mld, bld},       \
            s);                                                                              \
      else                                                                                   \
        st = dot_fwd_launch<DT, int64_t, GG, HH>(                                            \
            DotFwdArgs<DT, int64_t>{static_cast<const int64_t*>(row_ptr),                    \
                                    static_cast<const int64_t*>(col), plan_view(*plan), qq,  \
                                    kk, vv, bb, scale, oo, mm, partial, ld, mld, bld},       \
            s);                                                                              \
    } else
    TGX_DOT_SHAPES(TGX_DOT_FWD)
    set_error("unsupported dot attention head group G=%d HL=%d", shp.G, shp.HL);
#undef TGX_DOT_FWD
    if (st != TGX_OK) return st;
    h0 += hg;
  }
  return TGX_OK;
}

// One element format's backward over every head group.
template <int DT>
int dot_bwd_dtype(const void* row_ptr, const void* col, int idx_bits, const tgx_row_plan* plan,
                  const int32_t* row_ptr_t, const int32_t* col_t, const int32_t* perm,
                  const tgx_row_plan* plan_t, const void* q, const void* k, const void* v,
                  const float* bias, float scale, const void* out, float* ml, const void* dout,
                  void* dq, void* dk, void* dv, float* dbias, int64_t n_dst, int H, int D,
                  float* dst_part, float* src_part, const int32_t* inv_perm, float* ds_t,
                  int64_t n_edges, hipStream_t s) {
  using T = typename Vals<DT, 8>::T;
  const int64_t ld = static_cast<int64_t>(H) * D, mld = 2 * static_cast<int64_t>(H), bld = H;
  auto at = [](const void* p, int64_t off) {
    return p ? static_cast<const T*>(p) + off : nullptr;
  };
  auto at_mut = [](void* p, int64_t off) { return p ? static_cast<T*>(p) + off : nullptr; };
  for (int h0 = 0; h0 < H;) {
    const int hg = dot_group_heads(H, D, h0);
    const DotShape shp = dot_shape(hg, D);
    const int64_t off = static_cast<int64_t>(h0) * D;
    const T *qq = at(q, off), *kk = at(k, off), *vv = at(v, off), *oo = at(out, off),
            *gg = at(dout, off);
    T *dqq = at_mut(dq, off), *dkk = at_mut(dk, off), *dvv = at_mut(dv, off);
    const float* bb = bias ? bias + h0 : nullptr;
    float* dbb = dbias ? dbias + h0 : nullptr;
    float* mm = ml + 2 * h0;
    const DotSrcArgs<DT> sa{row_ptr_t, col_t, perm, plan_view(*plan_t), qq, kk, vv, bb, scale,
                            mm, gg, dkk, dvv, src_part, ld, mld, bld, ds_t, n_edges};
    int st = TGX_UNSUPPORTED;
#define TGX_DOT_BWD(GG, HH)                                                                   \
    if (shp.G == GG && shp.HL == HH) {                                                        \
      if (idx_bits == 32)                                                                     \
        st = dot_bwd_launch<DT, int32_t, GG, HH>(                                             \
            DotDstArgs<DT, int32_t>{static_cast<const int32_t*>(row_ptr),                     \
                                    static_cast<const int32_t*>(col), plan_view(*plan), qq,   \
                                    kk, vv, bb, scale, mm, gg, dqq, dbb, dst_part, ld, mld,   \
                                    bld, inv_perm, ds_t, n_edges},                            \
            sa, oo, mm, n_dst, s);                                                            \
      else                                                                                    \
        st = dot_bwd_launch<DT, int64_t, GG, HH>(                                             \
            DotDstArgs<DT, int64_t>{static_cast<const int64_t*>(row_ptr),                     \
                                    static_cast<const int64_t*>(col), plan_view(*plan), qq,   \
                                    kk, vv, bb, scale, mm, gg, dqq, dbb, dst_part, ld, mld,   \
                                    bld, inv_perm, ds_t, n_edges},                            \
            sa, oo, mm, n_dst, s);                                                            \
    } else
    TGX_DOT_SHAPES(TGX_DOT_BWD)
    set_error("unsupported dot attention head group G=%d HL=%d", shp.G, shp.HL);
#undef TGX_DOT_BWD
    if (st != TGX_OK) return st;
    h0 += hg;
  }
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_dot_attn_fwd(const void* row_ptr, const void* col, int idx_bits,
                                const tgx_row_plan* plan, const void* q, const void* k,
                                const void* v, const float* bias, float scale, void* out,
                                float* ml, int64_t n_dst, int64_t n_src, int H, int D,
                                int dtype, float* partial, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(dtype_bytes(dtype) != 0, "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)",
              dtype);
  if (!dot_heads_ok(H, D)) {
    set_error("dot attention supports H >= 1 and D in {8, 16, 32, 64, 128, 256, 512} "
              "(got H=%d D=%d)", H, D);
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && q && out && ml && ((k && v) || n_src == 0), "null pointer");
  TGX_REQUIRE(plan->n_chunks == 0 || partial, "split rows need a partial buffer");
  // Gathered row indices are held in 32 bits.
  TGX_REQUIRE(n_src < (int64_t{1} << 31), "source tables need fewer than 2^31 rows");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case TGX_DTYPE_BF16:
      return dot_fwd_dtype<TGX_DTYPE_BF16>(row_ptr, col, idx_bits, plan, q, k, v, bias, scale,
                                           out, ml, H, D, partial, s);
    case TGX_DTYPE_F16:
      return dot_fwd_dtype<TGX_DTYPE_F16>(row_ptr, col, idx_bits, plan, q, k, v, bias, scale,
                                          out, ml, H, D, partial, s);
    default:
      return dot_fwd_dtype<TGX_DTYPE_F32>(row_ptr, col, idx_bits, plan, q, k, v, bias, scale,
                                          out, ml, H, D, partial, s);
  }
}

extern "C" int tgx_dot_attn_bwd_workspace(const tgx_row_plan* plan, const tgx_row_plan* plan_t,
                                          int64_t n_edges, int H, int D, int stored_ds,
                                          size_t* bytes) {
  TGX_REQUIRE(plan && plan_t && bytes, "null pointer");
  if (!dot_heads_ok(H, D)) {
    set_error("unsupported dot attention shape H=%d D=%d", H, D);
    return TGX_UNSUPPORTED;
  }
  // Head groups run one after another on one stream and share the
  // workspace; the first group is the widest.
  TGX_REQUIRE(n_edges >= 0, "bad edge count");
  *bytes = dot_bwd_layout(*plan, *plan_t, dot_group_heads(H, D, 0), D, n_edges, stored_ds != 0)
               .bytes;
  return TGX_OK;
}

extern "C" int tgx_dot_attn_bwd(const void* row_ptr, const void* col, int idx_bits,
                                const tgx_row_plan* plan, const int32_t* row_ptr_t,
                                const int32_t* col_t, const int32_t* perm,
                                const int32_t* inv_perm, const tgx_row_plan* plan_t,
                                int64_t n_edges, const void* q, const void* k,
                                const void* v, const float* bias, float scale, const void* out,
                                float* ml, const void* dout, void* dq, void* dk, void* dv,
                                float* dbias, int64_t n_dst, int64_t n_src, int H, int D,
                                int dtype, void* ws, size_t ws_bytes, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(dtype_bytes(dtype) != 0, "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)",
              dtype);
  if (!dot_heads_ok(H, D)) {
    set_error("unsupported dot attention shape H=%d D=%d", H, D);
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  st = check_plan(plan_t, n_src);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(row_ptr && row_ptr_t && q && out && ml && dout && dq &&
                  ((k && v && dk && dv) || n_src == 0),
              "null pointer");
  TGX_REQUIRE(n_edges >= 0 && n_edges < (int64_t{1} << 31), "bad edge count");
  const bool stored = inv_perm != nullptr && n_edges > 0;
  const DotBwdLayout L =
      dot_bwd_layout(*plan, *plan_t, dot_group_heads(H, D, 0), D, n_edges, stored);
  TGX_REQUIRE(ws && ws_bytes >= L.bytes, "workspace too small: need %zu bytes", L.bytes);
  hipStream_t s = as_stream(stream);
  char* w = static_cast<char*>(ws);
  float* dst_part = reinterpret_cast<float*>(w + L.dst_part_off);
  float* src_part = reinterpret_cast<float*>(w + L.src_part_off);
  float* ds_t = stored ? reinterpret_cast<float*>(w + L.ds_off) : nullptr;
  switch (dtype) {
    case TGX_DTYPE_BF16:
      return dot_bwd_dtype<TGX_DTYPE_BF16>(row_ptr, col, idx_bits, plan, row_ptr_t, col_t, perm,
                                           plan_t, q, k, v, bias, scale, out, ml, dout, dq, dk,
                                           dv, dbias, n_dst, H, D, dst_part, src_part, inv_perm,
                                           ds_t, n_edges, s);
    case TGX_DTYPE_F16:
      return dot_bwd_dtype<TGX_DTYPE_F16>(row_ptr, col, idx_bits, plan, row_ptr_t, col_t, perm,
                                          plan_t, q, k, v, bias, scale, out, ml, dout, dq, dk,
                                          dv, dbias, n_dst, H, D, dst_part, src_part, inv_perm,
                                          ds_t, n_edges, s);
    default:
      return dot_bwd_dtype<TGX_DTYPE_F32>(row_ptr, col, idx_bits, plan, row_ptr_t, col_t, perm,
                                          plan_t, q, k, v, bias, scale, out, ml, dout, dq, dk,
                                          dv, dbias, n_dst, H, D, dst_part, src_part, inv_perm,
                                          ds_t, n_edges, s);
  }
}

// ---------------------------------------------------------------------------
// Forward without a caller buffer: the split-row partials live in a static
// device array.  For callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc).
namespace tgx {
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;   // 64 MiB per device
// Host code must never use this name as an address: it is a host-side
// stand-in.  The device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_init;
// Ordering of the calls that use a device's scratch: the event recorded
// after the last uncaptured call and the stream it ran on.  A call on
// another stream first waits for that event, so uncaptured calls on one
// device run one after another in the order the host made them, whatever
// their streams.  (Set up with the address; guarded by g_scratch_order.)
hipEvent_t g_scratch_done[kMaxDevices];
hipStream_t g_scratch_stream[kMaxDevices];
bool g_scratch_used[kMaxDevices];
std::mutex g_scratch_order;

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with that device current) and kept, with the
// device's ordering event.
int scratch_on_current_device(float** out, int* device) {
  int dev = -1;
  TGX_HIP(hipGetDevice(&dev));
  TGX_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal %d out of range", dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_init);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      TGX_HIP(hipEventCreateWithFlags(&g_scratch_done[dev], hipEventDisableTiming));
      TGX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
      TGX_REQUIRE(ptr != nullptr, "no device address for the static scratch");
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = static_cast<float*>(ptr);
  *device = dev;
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

extern "C" int tgx_dot_attn_fwd_noalloc(const void* row_ptr, const void* col, int idx_bits,
                                        const tgx_row_plan* plan, const void* q,
                                        const void* k, const void* v, const float* bias,
                                        float scale, void* out, float* ml, int64_t n_dst,
                                        int64_t n_src, int H, int D, int dtype, void* stream) {
  // Every size check comes before any HIP call.
  TGX_REQUIRE(plan != nullptr, "null plan");
  if (!dot_heads_ok(H, D)) {
    set_error("dot attention supports H >= 1 and D in {8, 16, 32, 64, 128, 256, 512} "
              "(got H=%d D=%d)", H, D);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(plan->n_chunks >= 0, "inconsistent plan");
  const size_t per_chunk = (static_cast<size_t>(H) * D + 2 * static_cast<size_t>(H)) *
                           sizeof(float);
  TGX_REQUIRE(static_cast<size_t>(plan->n_chunks) <= kScratchBytes / per_chunk,
              "%lld split-row chunks need %zu bytes of partials; the static scratch holds "
              "%zu bytes (64 MiB): use tgx_dot_attn_fwd with a caller buffer",
              static_cast<long long>(plan->n_chunks),
              static_cast<size_t>(plan->n_chunks) * per_chunk, kScratchBytes);
  float* partial = nullptr;
  int dev = -1;
  if (plan->n_chunks > 0 && n_dst > 0) {
    const int st = scratch_on_current_device(&partial, &dev);
    if (st != TGX_OK) return st;
  }
  if (!partial)   // no split rows: the scratch is not touched
    return tgx_dot_attn_fwd(row_ptr, col, idx_bits, plan, q, k, v, bias, scale, out, ml,
                            n_dst, n_src, H, D, dtype, nullptr, stream);
  hipStream_t s = as_stream(stream);
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  TGX_HIP(hipStreamIsCapturing(s, &capture));
  if (capture != hipStreamCaptureStatusNone)
    // Under capture the graph's own dependencies order its replays; an
    // event recorded outside the capture cannot be waited on inside it.
    return tgx_dot_attn_fwd(row_ptr, col, idx_bits, plan, q, k, v, bias, scale, out, ml,
                            n_dst, n_src, H, D, dtype, partial, stream);
  std::lock_guard<std::mutex> lock(g_scratch_order);
  if (g_scratch_used[dev] && g_scratch_stream[dev] != s)
    TGX_HIP(hipStreamWaitEvent(s, g_scratch_done[dev], 0));
  const int st = tgx_dot_attn_fwd(row_ptr, col, idx_bits, plan, q, k, v, bias, scale, out, ml,
                                  n_dst, n_src, H, D, dtype, partial, stream);
  if (st != TGX_OK) return st;
  TGX_HIP(hipEventRecord(g_scratch_done[dev], s));
  g_scratch_stream[dev] = s;
  g_scratch_used[dev] = true;
  return TGX_OK;
}
