// GAT additive edge attention over a destination-row CSR.
//
//   z_e = a_src[hd] . hs[j, hd] + a_dst[hd] . hd[i, hd]    (j = col[e], i = row)
//   s_e = LeakyReLU(z_e, slope)
//   out[i, hd] = sum_e softmax_i(s)_e * hs[j, hd]
//
// hs (source features) and hd (destination features) are one tensor for a
// homogeneous relation and two for a bipartite one.  Elements are fp32,
// bf16 or fp16; scores, softmax sums and products are fp32 and every output
// is rounded once (the reference accumulates 16-bit scores in fp32 and
// casts the result to the value's dtype, reducer_oracle.py:22-41, 137).
//
// Reference semantics: an edge() returning
//   reducer(leaky_relu((src.h*a_src).sum(-1) + (dst.h*a_dst).sum(-1)), src.h)
// evaluated by the eager oracle (python/tiga/interop/torch/message_passing.py:
// 2848-2894, reducer_oracle.py:60-137): per-(row, head) max shift, exp, sum,
// weighted sum, empty row -> 0.
//
// Layout: features are [N, H, D]; one node row is 4*G values spread over G
// lanes (4 values per lane: 16 bytes of fp32, 8 bytes of bf16/fp16), so head
// hd occupies HL = D/4 consecutive lanes and its dot products reduce with
// DPP inside the lane group.  node_state is [N_dst, H, 4] fp32 = {logsumexp,
// delta, a_dst.hd[i], a_src.hd[i]} so one 16-byte load per lane brings every
// per-(node, head) scalar the backward needs (slot 3, a_src.h of the same
// node, is not read by the backward).
//
// Backward (no float atomics, nothing per-edge saved by the forward):
//   B1 node pass   delta[i] = <dout[i], out[i]> per head
//   B2 source pass over the transposed CSR (row j = source): recompute
//      alpha_e = exp(s_e - lse[i]) and dz_e = alpha_e (<dout[i], hs[j]> - delta[i])
//      * LeakyReLU'(z_e); dhs[j] = sum alpha_e dout[i] + (sum dz_e) a_src;
//      dz_e stored at its transposed position (coalesced writes).
//   B3 destination pass over the CSR: dhd[i] = (sum_e dz_e) a_dst (added to
//      dhs[i] when hs and hd are one tensor) and da_dst += (sum_e dz_e) hd[i],
//      each edge's dz read through inv_perm; da_src += (sum dz_e) hs[j] over
//      the sources, fused here for a homogeneous relation, its own pass
//      otherwise.
//   da_* partials are fp64 per wave (static task striding), reduced in a
//   fixed order, so every output is deterministic.  With 16-bit elements and
//   one feature tensor, the source pass's dh contribution waits in an fp32
//   workspace until B3 adds the destination term and rounds once.
//
// Folded destination term (a forward that also writes `pos`): a row's sum
// of dz needs no per-edge pass.  With ds_e = alpha_e (<dout[i], hs[j]> -
// delta[i]), sum_e ds_e = <dout[i], out[i]> - delta[i] = 0 over a non-empty
// row, so
//   sum_e dz_e = sum_{z_e > 0} ds_e + slope sum_{z_e <= 0} ds_e
//              = (1 - slope) sum_{z_e > 0} ds_e
//              = (1 - slope) <dout[i], pos[i]>,
//   pos[i] = sum_{z_e > 0} alpha_e (hs[j] - out[i])      (fp32, [N_dst, H, D]),
// which the forward accumulates beside out (the z > 0 test is the same fp32
// z the source pass branches on).  B1 then also forms sdz_dst[i], B2 adds
// sdz_dst[j] a_dst to a homogeneous relation's dh[j] (or B1 writes a
// bipartite relation's dhd[i] = sdz_dst[i] a_dst), no dz is stored and B3
// becomes a node pass over h for da_src and da_dst.
#include <hip/hip_runtime.h>

#include "tgx_device.h"
#include "tgx_host.h"
#include "tgx_profile.h"
#include "tgx_softmax.h"
#include "tgx_tasks.h"
#include "tgx_vals.h"

namespace tgx {
namespace {

constexpr int kPersistBlocks = 2048;  // persistent backward grid (8 waves / CU)

__device__ __forceinline__ f32x4 ld4(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
typedef float f32x3 __attribute__((ext_vector_type(3)));
__device__ __forceinline__ f32x3 ld3(const float* p) {
  return *reinterpret_cast<const f32x3*>(p);
}
__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  return a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
}

template <int DT, typename I>
struct GatFwdArgs {
  using T = typename Vals<DT, 4>::T;
  const I* row_ptr;
  const I* col;
  PlanView plan;
  const T* hs;     // source features (gathered)
  const T* hd;     // destination features (== hs for a homogeneous relation)
  const float* a_src;
  const float* a_dst;
  float slope;
  T* out;
  float* ns;
  float* partial;  // per chunk: acc[4G] | m[H] | l[H] (POS: | pacc[4G] | pl[H])
  float* pos;      // POS: [N_dst, H, D] fp32, the folded destination term's rows
  int64_t ld;      // values between consecutive nodes' rows of hs, hd, out and pos
  int64_t nsld;    // floats between consecutive nodes' rows of ns
};

// Floats per chunk of the forward's partial buffer.
__host__ __device__ constexpr int64_t gat_partial_floats(int64_t HD, int64_t H, bool pos) {
  return pos ? 2 * HD + 3 * H : HD + 2 * H;
}

// Index of lane `src` in a wave, read by every lane (edge groups differ).
template <int EPW>
__device__ __forceinline__ int fetch_lane(int v, int src) {
  if constexpr (EPW == 1) return __builtin_amdgcn_readlane(v, src);
  return __shfl(v, src, 64);
}

// A finished row: out = acc / l and (POS) pos = (pacc - pl out) / l, both
// from the fp32 state.
template <class V, bool POS, int NA>
__device__ __forceinline__ void store_row(typename V::T* out, float* pos, int64_t off,
                                          const SoftState<NA>& st) {
  const float inv = 1.f / st.l;
  const f32x4 o = {st.acc[0] * inv, st.acc[1] * inv, st.acc[2] * inv, st.acc[3] * inv};
  V::store(out + off, o);
  if constexpr (POS) {
    const float w = st.acc[8] * inv;
    st4(pos + off, f32x4{st.acc[4] * inv - w * o[0], st.acc[5] * inv - w * o[1],
                         st.acc[6] * inv - w * o[2], st.acc[7] * inv - w * o[3]});
  }
}

// POS: the softmax state also carries pacc = sum over z > 0 of p hs[j]
// (acc[4..7]) and pl = sum over z > 0 of p (acc[8]), rescaled with acc and
// l, so pos[i] = (pacc - pl out[i]) / l.
// (POS adds 5 accumulators: held to 96 VGPRs, the plain kernel's 5 waves
// per SIMD, where that needs no spill: heads of up to 64 values.)
template <int DT, typename I, int G, int HL, int U, bool POS>
__global__ __launch_bounds__(kTaskBlock, POS && HL <= 16 ? 5 : 1) void gat_fwd_kernel(
    GatFwdArgs<DT, I> a) {
  using V = Vals<DT, 4>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  constexpr int NA = POS ? 9 : 4;
  const Task t = decode_task(a.plan, a.row_ptr, global_wave());
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  const bool head_lead = (c % HL) == 0;
  const f32x4 as4 = ld4(a.a_src + 4 * c);
  const f32x4 ad4 = ld4(a.a_dst + 4 * c);

  if (t.kind == kTaskEmpty) {
    for (int k = 0; k < t.n_empty; ++k) {
      const int64_t i = uniform(a.plan.rows[t.empty0 + k]);
      const f32x4 hi = V::widen(V::load(a.hd + i * a.ld + 4 * c));
      const float sdst = group_sum<HL>(dot4(ad4, hi));
      const float ssrc = group_sum<HL>(dot4(as4, hi));
      if (g == 0) {
        V::store(a.out + i * a.ld + 4 * c, f32x4{0.f, 0.f, 0.f, 0.f});
        if constexpr (POS) st4(a.pos + i * a.ld + 4 * c, f32x4{0.f, 0.f, 0.f, 0.f});
        if (head_lead) st4(a.ns + i * a.nsld + hd * 4, f32x4{kNegInf, 0.f, sdst, ssrc});
      }
    }
    return;
  }

  const int64_t row = t.row;
  const f32x4 hi = V::widen(V::load(a.hd + row * a.ld + 4 * c));
  const float sdst = group_sum<HL>(dot4(ad4, hi));

  SoftState<NA> st;
  st.init();
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    const int my_col = lane < n ? static_cast<int>(a.col[base + lane]) : 0;
    for (int k = 0; k < n; k += EPW * U) {
      typename V::Raw x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const int j = fetch_lane<EPW>(my_col, slot < n ? slot : 0);
        x[u] = V::load(a.hs + static_cast<int64_t>(j) * a.ld + 4 * c);
      }
      float s[U];
      bool up[U];
      float mc = kNegInf;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const float z = group_sum<HL>(dot4(as4, V::widen(x[u]))) + sdst;
        s[u] = slot < n ? leaky_relu(z, a.slope) : kNegInf;
        up[u] = z > 0.f;
        mc = fmaxf(mc, s[u]);
      }
      if (mc > st.m) st.rescale(mc);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = s[u] == kNegInf ? 0.f : fast_exp(s[u] - st.m);
        st.l += p;
        const f32x4 xv = V::widen(x[u]);
#pragma unroll
        for (int q = 0; q < 4; ++q) st.acc[q] += p * xv[q];
        if constexpr (POS) {
          const float pp = up[u] ? p : 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) st.acc[4 + q] += pp * xv[q];
          st.acc[8] += pp;
        }
      }
    }
  }
#pragma unroll
  for (int mask = G; mask < kWave; mask <<= 1) st.merge_xor(mask);
  if (g != 0) return;
  if (t.kind == kTaskChunk) {
    float* p = a.partial + t.slot * gat_partial_floats(HD, H, POS);
    st4(p + 4 * c, f32x4{st.acc[0], st.acc[1], st.acc[2], st.acc[3]});
    if (head_lead) {
      p[HD + hd] = st.m;
      p[HD + H + hd] = st.l;
    }
    if constexpr (POS) {
      st4(p + HD + 2 * H + 4 * c, f32x4{st.acc[4], st.acc[5], st.acc[6], st.acc[7]});
      if (head_lead) p[2 * HD + 2 * H + hd] = st.acc[8];
    }
    return;
  }
  store_row<V, POS>(a.out, a.pos, row * a.ld + 4 * c, st);
  const float ssrc_i = group_sum<HL>(dot4(as4, hi));
  if (head_lead) st4(a.ns + row * a.nsld + hd * 4, f32x4{st.m + __logf(st.l), 0.f, sdst, ssrc_i});
}

template <int DT, int G, int HL, bool POS>
__global__ __launch_bounds__(kTaskBlock) void gat_fwd_merge_kernel(
    PlanView plan, const float* __restrict__ partial,
    const typename Vals<DT, 4>::T* __restrict__ hd_rows, const float* __restrict__ a_src,
    const float* __restrict__ a_dst, typename Vals<DT, 4>::T* __restrict__ out,
    float* __restrict__ pos, float* __restrict__ ns, int64_t ld, int64_t nsld) {
  using V = Vals<DT, 4>;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  constexpr int NA = POS ? 9 : 4;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int lane = lane_id();
  if (lane >= G) return;
  const int c = lane, hd = c / HL;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  SoftState<NA> st;
  st.init();
  // The partials of up to eight chunks are requested before they are merged
  // in chunk order (the merges depend on each other, the loads do not).
  constexpr int B = 8;
  for (int q0 = c0; q0 < c1; q0 += B) {
    float accs[B][NA], pm[B], pl[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int q = q0 + u < c1 ? q0 + u : c1 - 1;
      const float* p = partial + static_cast<int64_t>(q) * gat_partial_floats(HD, H, POS);
      const f32x4 acc = ld4(p + 4 * c);
#pragma unroll
      for (int k = 0; k < 4; ++k) accs[u][k] = acc[k];
      if constexpr (POS) {
        const f32x4 pacc = ld4(p + HD + 2 * H + 4 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) accs[u][4 + k] = pacc[k];
        accs[u][8] = p[2 * HD + 2 * H + hd];
      }
      pm[u] = p[HD + hd];
      pl[u] = p[HD + H + hd];
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (q0 + u < c1) st.merge(pm[u], pl[u], accs[u]);
  }
  store_row<V, POS>(out, pos, row * ld + 4 * c, st);
  const f32x4 hi = V::widen(V::load(hd_rows + row * ld + 4 * c));
  const float sdst = group_sum<HL>(dot4(ld4(a_dst + 4 * c), hi));
  const float ssrc = group_sum<HL>(dot4(ld4(a_src + 4 * c), hi));
  if (c % HL == 0) st4(ns + row * nsld + hd * 4, f32x4{st.m + __logf(st.l), 0.f, sdst, ssrc});
}

// ---------------------------------------------------------------------------
// Backward.

// Destination term of a folded backward (B1 with `pos`).
template <int DT>
struct GatFold {
  const float* pos;   // [N_dst, H, D] fp32 from the forward
  float one_minus_slope;
  float* sdz_dst;     // [N_dst, H] out: sum of dz over each row's in-edges
  const float* a_dst;
  typename Vals<DT, 4>::T* dhd;  // FOLD == 2: the bipartite destination gradient
};

// FOLD 0: delta only; 1: and sdz_dst = (1 - slope) <dout, pos>; 2: and
// dhd[i] = sdz_dst[i] a_dst (a bipartite relation's destination gradient).
template <int DT, int G, int HL, int FOLD>
__global__ __launch_bounds__(kTaskBlock) void gat_delta_kernel(
    const typename Vals<DT, 4>::T* __restrict__ dout,
    const typename Vals<DT, 4>::T* __restrict__ out, float* __restrict__ ns, int64_t n_nodes,
    int64_t ld, int64_t nsld, GatFold<DT> f) {
  using V = Vals<DT, 4>;
  constexpr int EPW = kWave / G;
  constexpr int H = G / HL;
  const int lane = lane_id();
  const int c = lane % G, hd = c / HL;
  const int64_t node = global_wave() * EPW + lane / G;
  if (node >= n_nodes) return;
  const int64_t off = node * ld + 4 * c;
  const f32x4 dv = V::widen(V::load(dout + off));
  const float d = group_sum<HL>(dot4(dv, V::widen(V::load(out + off))));
  if (c % HL == 0) ns[node * nsld + hd * 4 + 1] = d;
  if constexpr (FOLD > 0) {
    const float sd = f.one_minus_slope * group_sum<HL>(dot4(dv, ld4(f.pos + off)));
    if (c % HL == 0) f.sdz_dst[node * H + hd] = sd;
    if constexpr (FOLD == 2) V::store(f.dhd + off, sd * ld4(f.a_dst + 4 * c));
  }
}

template <int DT>
struct GatSrcArgs {
  using T = typename Vals<DT, 4>::T;
  const int32_t* row_ptr_t;
  const int32_t* col_t;
  const int32_t* perm;
  PlanView plan;
  const T* hs;
  const float* a_src;
  float slope;
  const float* ns;
  const T* dout;
  float* dh_acc;    // fp32 [N, HD] (one feature tensor: B3 adds to it), or null
  T* dhs;           // the source gradient itself when dh_acc is null
  float* partial;   // per chunk: [4G] dh contribution | [H] sum of dz
  float* dz;        // [E, H] in transposed edge order (coalesced); MODE 0 only
  float* sdz_src;   // [N_src, H] sum of dz over each source's out-edges
  const float* a_dst;    // MODE 2
  const float* sdz_dst;  // MODE 2: [N, H] from B1
  int64_t ld;       // values between consecutive nodes' rows of hs, dout, dh
  int64_t nsld;     // floats between consecutive nodes' rows of ns
};

// One wave per task of the transposed-CSR plan (source rows).  MODE 0: dz
// stored for B3; 1 (folded, bipartite): no dz; 2 (folded, one feature
// tensor): no dz, and dh[j] also takes the destination term sdz_dst[j] a_dst.
// (The folded modes are held to the per-edge mode's 7 waves per SIMD.)
template <int DT, int G, int HL, int U, int MODE>
__global__ __launch_bounds__(kTaskBlock, MODE ? 7 : 1) void gat_bwd_src_kernel(
    GatSrcArgs<DT> a) {
  using V = Vals<DT, 4>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  const Task t = decode_task(a.plan, a.row_ptr_t, global_wave());
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  const bool head_lead = (c % HL) == 0;
  if (t.kind == kTaskEmpty) {
    for (int k = 0; k < t.n_empty; ++k) {
      const int64_t j = uniform(a.plan.rows[t.empty0 + k]);
      if (g == 0) {
        if constexpr (MODE == 2)
          V::store(a.dhs + j * a.ld + 4 * c, a.sdz_dst[j * H + hd] * ld4(a.a_dst + 4 * c));
        else if (a.dh_acc)
          st4(a.dh_acc + j * a.ld + 4 * c, f32x4{0.f, 0.f, 0.f, 0.f});
        else
          V::store(a.dhs + j * a.ld + 4 * c, f32x4{0.f, 0.f, 0.f, 0.f});
        if (head_lead) a.sdz_src[j * H + hd] = 0.f;
      }
    }
    return;
  }
  const f32x4 as4 = ld4(a.a_src + 4 * c);
  const int64_t j = t.row;
  const f32x4 hj = V::widen(V::load(a.hs + j * a.ld + 4 * c));
  // a_src . hs[j], the same fp32 arithmetic as the forward's.
  const float ssrc = group_sum<HL>(dot4(as4, hj));
  f32x4 dha = {0.f, 0.f, 0.f, 0.f};
  float sdz = 0.f;
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    const int my_i = lane < n ? a.col_t[base + lane] : 0;
    for (int k = 0; k < n; k += EPW * U) {
      typename V::Raw d[U];
      f32x3 nst[U];  // {lse, delta, a_dst.hd[i]} of the destination
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const int64_t i = fetch_lane<EPW>(my_i, slot < n ? slot : 0);
        d[u] = V::load(a.dout + i * a.ld + 4 * c);
        nst[u] = ld3(a.ns + i * a.nsld + hd * 4);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int slot = k + u * EPW + g;
        const bool valid = slot < n;
        const f32x4 du = V::widen(d[u]);
        const float z = ssrc + nst[u][2];
        const float s = leaky_relu(z, a.slope);
        const float alpha = valid ? fast_exp(s - nst[u][0]) : 0.f;
        const float dalpha = group_sum<HL>(dot4(du, hj));
        const float ds = alpha * (dalpha - nst[u][1]);
        const float dzv = z > 0.f ? ds : ds * a.slope;
        dha += alpha * du;
        sdz += dzv;
        if constexpr (MODE == 0) {
          if (valid && head_lead) a.dz[(base + slot) * H + hd] = dzv;
        }
      }
    }
  }
#pragma unroll
  for (int mask = G; mask < kWave; mask <<= 1) {
    dha[0] += __shfl_xor(dha[0], mask, 64);
    dha[1] += __shfl_xor(dha[1], mask, 64);
    dha[2] += __shfl_xor(dha[2], mask, 64);
    dha[3] += __shfl_xor(dha[3], mask, 64);
    sdz += __shfl_xor(sdz, mask, 64);
  }
  if (g != 0) return;
  f32x4 contrib = dha + sdz * as4;
  if (t.kind == kTaskChunk) {
    float* p = a.partial + static_cast<int64_t>(t.slot) * (HD + H);
    st4(p + 4 * c, contrib);
    if (head_lead) p[HD + hd] = sdz;
  } else {
    // (Folded modes run with dh_acc == null: dh is final here.)
    if constexpr (MODE == 2) contrib = contrib + a.sdz_dst[j * H + hd] * ld4(a.a_dst + 4 * c);
    if (a.dh_acc)
      st4(a.dh_acc + j * a.ld + 4 * c, contrib);
    else
      V::store(a.dhs + j * a.ld + 4 * c, contrib);
    if (head_lead) a.sdz_src[j * H + hd] = sdz;
  }
}

// FOLD: a homogeneous relation's dh also takes sdz_dst[row] a_dst.
template <int DT, int G, int HL, bool FOLD>
__global__ __launch_bounds__(kTaskBlock) void gat_bwd_src_merge_kernel(
    PlanView plan, const float* __restrict__ partial, float* __restrict__ dh_acc,
    typename Vals<DT, 4>::T* __restrict__ dhs, float* __restrict__ sdz_src,
    const float* __restrict__ a_dst, const float* __restrict__ sdz_dst, int64_t ld) {
  using V = Vals<DT, 4>;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int c = lane_id();
  if (c >= G) return;
  const int hd = c / HL;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  float z = 0.f;
  // Up to eight chunks' partials in flight, summed in chunk order.
  constexpr int B = 8;
  for (int q0 = c0; q0 < c1; q0 += B) {
    f32x4 ps[B];
    float pz[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int q = q0 + u < c1 ? q0 + u : c1 - 1;
      const float* p = partial + static_cast<int64_t>(q) * (HD + H);
      ps[u] = ld4(p + 4 * c);
      pz[u] = p[HD + hd];
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (q0 + u < c1) {
        s += ps[u];
        z += pz[u];
      }
  }
  if constexpr (FOLD) s = s + sdz_dst[row * H + hd] * ld4(a_dst + 4 * c);
  if (dh_acc)
    st4(dh_acc + row * ld + 4 * c, s);
  else
    V::store(dhs + row * ld + 4 * c, s);
  if (c % HL == 0) sdz_src[row * H + hd] = z;
}

template <int DT, typename I>
struct GatDstArgs {
  using T = typename Vals<DT, 4>::T;
  const I* row_ptr;
  PlanView plan;
  const T* hd;
  const float* a_dst;
  const float* dz;       // [E, H] in transposed edge order
  const int32_t* inv_perm;  // [E] transposed position of each edge
  const float* sdz_src;  // [N, H]; read only with `fused_src`
  const float* dh_acc;   // fp32 source-pass contribution to add, or null
  T* dhd;                // destination gradient (the one dh of a homogeneous relation)
  float* partial;        // per chunk: [H]
  double* dap_src;       // [waves, 4G]
  double* dap_dst;       // [waves, 4G]
  int64_t n_tasks;
  int64_t ld;            // values between consecutive nodes' rows of hd and dhd
};

__device__ __forceinline__ void acc_f64(f64x4& acc, float scale, f32x4 v) {
  const double sd = static_cast<double>(scale);
  acc[0] += sd * v[0];
  acc[1] += sd * v[1];
  acc[2] += sd * v[2];
  acc[3] += sd * v[3];
}

// dhd[i] = base + sdz * a_dst, base = the source pass's fp32 contribution
// (one feature tensor: FUSED) or 0, rounded once.
template <class V, bool FUSED>
__device__ __forceinline__ void finish_dh(typename V::T* dhd, const float* dh_acc, int64_t off,
                                          float sdz, f32x4 ad4) {
  f32x4 base = {0.f, 0.f, 0.f, 0.f};
  if constexpr (FUSED) base = ld4(dh_acc + off);
  V::store(dhd + off, base + sdz * ad4);
}

// Persistent over the CSR plan (static task striding keeps the fp64
// partials deterministic).  Every destination row of hd is read exactly
// once here: da_dst += (sum over its in-edges of dz) hd[i], and with one
// feature tensor (FUSED) da_src += sdz_src[i] h[i].
template <int DT, typename I, int G, int HL, bool FUSED>
__global__ __launch_bounds__(kTaskBlock) void gat_bwd_dst_kernel(GatDstArgs<DT, I> a) {
  using V = Vals<DT, 4>;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  const f32x4 ad4 = ld4(a.a_dst + 4 * c);
  f64x4 ds = {0.0, 0.0, 0.0, 0.0};
  f64x4 dd = {0.0, 0.0, 0.0, 0.0};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t w = global_wave(); w < a.n_tasks; w += stride) {
    const Task t = decode_task(a.plan, a.row_ptr, w);
    if (t.kind == kTaskNone) continue;
    if (t.kind == kTaskEmpty) {
      for (int k = 0; k < t.n_empty; ++k) {
        const int64_t i = uniform(a.plan.rows[t.empty0 + k]);
        if (g == 0) {
          if constexpr (FUSED)
            acc_f64(ds, a.sdz_src[i * H + hd], V::widen(V::load(a.hd + i * a.ld + 4 * c)));
          // An fp32 gradient of one feature tensor already holds its value.
          if constexpr (!(FUSED && DT == TGX_DTYPE_F32))
            finish_dh<V, FUSED>(a.dhd, a.dh_acc, i * a.ld + 4 * c, 0.f, ad4);
        }
      }
      continue;
    }
    const int64_t i = t.row;
    // Sum dz over the edge range, fetching each edge's H values from its
    // transposed position; lane l always handles head l % H.
    // Batches of 4 x 64 values: all index loads, then all gathers, so a
    // row of up to 32 edges costs two dependent memory round trips.
    float s = 0.f;
    const int64_t p0 = t.e0 * H, p1 = t.e1 * H;
    for (int64_t pb = p0; pb < p1; pb += 4 * kWave) {
      int32_t ip[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t p = pb + k * kWave + lane;
        ip[k] = p < p1 ? a.inv_perm[p / H] : -1;
      }
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t p = pb + k * kWave + lane;
        v[k] = ip[k] >= 0 ? a.dz[static_cast<int64_t>(ip[k]) * H + (p % H)] : 0.f;
      }
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
#pragma unroll
    for (int mask = H; mask < kWave; mask <<= 1) s += __shfl_xor(s, mask, 64);
    const float sdz = __shfl(s, hd, 64);
    if (t.kind == kTaskChunk && lane < H)
      a.partial[static_cast<int64_t>(t.slot) * H + lane] = s;
    if (g == 0) {
      const f32x4 hi = V::widen(V::load(a.hd + i * a.ld + 4 * c));
      acc_f64(dd, sdz, hi);
      const bool first = t.kind == kTaskRow || t.e0 == static_cast<int64_t>(a.row_ptr[i]);
      if constexpr (FUSED) {
        if (first) acc_f64(ds, a.sdz_src[i * H + hd], hi);
      }
      if (t.kind == kTaskRow) finish_dh<V, FUSED>(a.dhd, a.dh_acc, i * a.ld + 4 * c, sdz, ad4);
    }
  }
  if (g == 0) {
    double* q = a.dap_dst + global_wave() * HD + 4 * c;
    q[0] = dd[0]; q[1] = dd[1]; q[2] = dd[2]; q[3] = dd[3];
    if constexpr (FUSED) {
      double* p = a.dap_src + global_wave() * HD + 4 * c;
      p[0] = ds[0]; p[1] = ds[1]; p[2] = ds[2]; p[3] = ds[3];
    }
  }
}

template <int DT, int G, int HL, bool FUSED>
__global__ __launch_bounds__(kTaskBlock) void gat_bwd_dst_merge_kernel(
    PlanView plan, const float* __restrict__ partial, const float* __restrict__ a_dst,
    const float* dh_acc, typename Vals<DT, 4>::T* dhd, int64_t ld) {
  using V = Vals<DT, 4>;
  constexpr int H = G / HL;
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int c = lane_id();
  if (c >= G) return;
  const int hd = c / HL;
  const int64_t row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  float s = 0.f;
  for (int q = c0; q < c1; ++q) s += partial[static_cast<int64_t>(q) * H + hd];
  finish_dh<V, FUSED>(dhd, dh_acc, row * ld + 4 * c, s, ld4(a_dst + 4 * c));
}

// Per-wave partials of da over node rows: sum_j sdz_a[j] h[j] (and with
// BOTH, sum_j sdz_b[j] h[j] from the same row read), persistent with static
// striding (deterministic).  A bipartite relation's da_src (sdz_src over
// hs), and in a folded backward its da_dst (sdz_dst over hd), or both of a
// homogeneous relation's in one pass.
template <int G>
__device__ __forceinline__ void wave_sum_f64(f64x4& v) {
#pragma unroll
  for (int mask = G; mask < kWave; mask <<= 1) {
    v[0] += __shfl_xor(v[0], mask, 64);
    v[1] += __shfl_xor(v[1], mask, 64);
    v[2] += __shfl_xor(v[2], mask, 64);
    v[3] += __shfl_xor(v[3], mask, 64);
  }
}

template <int DT, int G, int HL, bool BOTH>
__global__ __launch_bounds__(kTaskBlock) void gat_da_nodes_kernel(
    const typename Vals<DT, 4>::T* __restrict__ h, const float* __restrict__ sdz_a,
    double* __restrict__ dap_a, const float* __restrict__ sdz_b, double* __restrict__ dap_b,
    int64_t n, int64_t ld) {
  using V = Vals<DT, 4>;
  constexpr int EPW = kWave / G;
  constexpr int HD = 4 * G;
  constexpr int H = G / HL;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int hd = c / HL;
  f64x4 da = {0.0, 0.0, 0.0, 0.0};
  f64x4 db = {0.0, 0.0, 0.0, 0.0};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWavesPerBlock * EPW;
  for (int64_t j = global_wave() * EPW + g; j < n; j += stride) {
    const f32x4 hv = V::widen(V::load(h + j * ld + 4 * c));
    acc_f64(da, sdz_a[j * H + hd], hv);
    if constexpr (BOTH) acc_f64(db, sdz_b[j * H + hd], hv);
  }
  wave_sum_f64<G>(da);
  if constexpr (BOTH) wave_sum_f64<G>(db);
  if (g == 0) {
    double* p = dap_a + global_wave() * HD + 4 * c;
    p[0] = da[0]; p[1] = da[1]; p[2] = da[2]; p[3] = da[3];
    if constexpr (BOTH) {
      double* q = dap_b + global_wave() * HD + 4 * c;
      q[0] = db[0]; q[1] = db[1]; q[2] = db[2]; q[3] = db[3];
    }
  }
}

// da[x] = sum over waves of dapart[w][x] in a fixed order, fp64, two levels:
// block (tensor, slice) sums a contiguous range of wave rows with coalesced
// 2 KB row reads, then one wave per element adds the kDaSlices slice sums.
constexpr int kDaSlices = 64;

__global__ __launch_bounds__(256) void da_slice_kernel(const double* __restrict__ part_src,
                                                       const double* __restrict__ part_dst,
                                                       int64_t src_waves, int64_t dst_waves,
                                                       int HD, double* __restrict__ slices) {
  const int tensor = blockIdx.y;
  const int slice = blockIdx.x;
  const int e = threadIdx.x;
  if (e >= HD) return;
  const double* p = tensor ? part_dst : part_src;
  const int64_t waves = tensor ? dst_waves : src_waves;
  const int64_t per = (waves + kDaSlices - 1) / kDaSlices;
  const int64_t w0 = slice * per;
  const int64_t w1 = w0 + per < waves ? w0 + per : waves;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  int64_t w = w0;
  for (; w + 4 <= w1; w += 4) {
    s0 += p[(w + 0) * HD + e];
    s1 += p[(w + 1) * HD + e];
    s2 += p[(w + 2) * HD + e];
    s3 += p[(w + 3) * HD + e];
  }
  for (; w < w1; ++w) s0 += p[w * HD + e];
  slices[(static_cast<int64_t>(tensor) * kDaSlices + slice) * HD + e] = (s0 + s1) + (s2 + s3);
}

__global__ __launch_bounds__(256) void da_final_kernel(const double* __restrict__ slices, int HD,
                                                       float* __restrict__ da_src,
                                                       float* __restrict__ da_dst) {
  const int x = blockIdx.x * 256 + threadIdx.x;
  if (x >= 2 * HD) return;
  const int tensor = x >= HD;
  const int e = tensor ? x - HD : x;
  double s = 0.0;
  for (int k = 0; k < kDaSlices; ++k) s += slices[(static_cast<int64_t>(tensor) * kDaSlices + k) * HD + e];
  (tensor ? da_dst : da_src)[e] = static_cast<float>(s);
}

// ---------------------------------------------------------------------------
// Host dispatch.

struct GatShape {
  int G, HL;
};

// Heads run in groups (group_heads, kGatGroupFloats): each group launches the
// kernels over its strided slice of h, out, dout, dh and the node state, and
// its own contiguous slice of a_src, a_dst, da_src and da_dst.
int gat_group_heads(int H, int D, int h0) { return group_heads(H, D, h0, kGatGroupFloats); }

GatShape gat_shape(int Hg, int D) { return GatShape{Hg * D / 4, D / 4}; }

// Persistent grid: enough workgroups for the tasks, at most what stays
// resident at once, at most kPersistBlocks (the partial buffers' capacity).
int64_t persist_blocks(int64_t tasks, int64_t resident) {
  int64_t b = ceil_div(tasks, kWavesPerBlock);
  if (b > resident) b = resident;
  if (b > kPersistBlocks) b = kPersistBlocks;
  return b > 0 ? b : 1;
}

// Every (G, HL) a group can take: G = Hg * HL lanes, HL = D / 4 lanes per head.
#define TGX_GAT_SHAPES(X)                                                        \
  X(64, 64) X(64, 32) X(64, 16) X(64, 8) X(64, 4) X(64, 2) X(64, 1)            \
  X(32, 32) X(32, 16) X(32, 8) X(32, 4) X(32, 2) X(32, 1)                       \
  X(16, 16) X(16, 8) X(16, 4) X(16, 2) X(16, 1)                                 \
  X(8, 8) X(8, 4) X(8, 2) X(8, 1)                                               \
  X(4, 4) X(4, 2) X(4, 1)                                                       \
  X(2, 2) X(2, 1)                                                               \
  X(1, 1)

template <int DT, typename I, int G, int HL>
int gat_fwd_launch(const GatFwdArgs<DT, I>& a, hipStream_t s) {
  constexpr int EPW = kWave / G;
  // Rows in flight per lane group: 10 x 1 KB per wave measured best for the
  // fp32 forward (8: +2%, 12: +1%, 16: +5% time on the 1M-node graph).
  constexpr int U = EPW >= 10 ? 1 : 10 / EPW;
  const int64_t waves = plan_waves(a.plan);
  const bool pos = a.pos != nullptr;
  if (waves > 0) {
    TGX_PROFILE("gat_fwd_kernel", s);
    const auto k = pos ? gat_fwd_kernel<DT, I, G, HL, U, true>
                       : gat_fwd_kernel<DT, I, G, HL, U, false>;
    k<<<ceil_div(waves, kWavesPerBlock), kTaskBlock, 0, s>>>(a);
    TGX_LAUNCHED("gat_fwd_kernel");
  }
  if (a.plan.n_split > 0) {
    TGX_PROFILE("gat_fwd_merge_kernel", s);
    const auto k = pos ? gat_fwd_merge_kernel<DT, G, HL, true>
                       : gat_fwd_merge_kernel<DT, G, HL, false>;
    k<<<ceil_div(a.plan.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
        a.plan, a.partial, a.hd, a.a_src, a.a_dst, a.out, a.pos, a.ns, a.ld, a.nsld);
    TGX_LAUNCHED("gat_fwd_merge_kernel");
  }
  return TGX_OK;
}

struct GatBwdLayout {
  size_t dz_off, sdz_off, sdz_dst_off, src_part_off, dst_part_off, dap_src_off, dap_dst_off,
      slices_off, dh_acc_off, bytes;
  int64_t src_waves, dst_waves;
};

// Workspace of one head group of H heads out of H_total.  dh_acc, only for
// 16-bit elements (where a homogeneous relation's dh waits there between
// passes), comes first and spans whole rows, [n_dst, H_total * D] fp32: the
// kernels index it with the row stride of dh itself, each head group at its
// own column offset.
// Folded (the forward wrote pos): no dz, no dh_acc and no B3 partials; an
// sdz_dst row per destination, and the dst da partials sized for a node pass.
GatBwdLayout gat_bwd_layout(const tgx_row_plan& plan, const tgx_row_plan& plan_t,
                            int64_t n_edges, int H, int D, int dtype, int H_total,
                            bool folded) {
  GatBwdLayout L;
  const int64_t HD = static_cast<int64_t>(H) * D;
  // Partial buffers are sized for the largest grid; launches may use fewer.
  // The node passes over da take at most one wave per node.
  const PlanView pv = plan_view(plan);
  L.dst_waves = persist_blocks(folded ? plan.n_rows : plan_waves(pv), kPersistBlocks) *
                kWavesPerBlock;
  L.src_waves = persist_blocks(plan_t.n_rows, kPersistBlocks) * kWavesPerBlock;
  if (L.src_waves < L.dst_waves) L.src_waves = L.dst_waves;
  const int64_t nodes = plan.n_rows > plan_t.n_rows ? plan.n_rows : plan_t.n_rows;
  Carve c{nullptr, 0};
  L.dh_acc_off = reinterpret_cast<size_t>(c.take<float>(
      dtype == TGX_DTYPE_F32 || folded ? 0 : plan.n_rows * static_cast<int64_t>(H_total) * D));
  L.dz_off = reinterpret_cast<size_t>(c.take<float>(folded ? 0 : n_edges * H));
  L.sdz_off = reinterpret_cast<size_t>(c.take<float>(nodes * H));
  L.sdz_dst_off = reinterpret_cast<size_t>(c.take<float>(folded ? plan.n_rows * H : 0));
  L.src_part_off = reinterpret_cast<size_t>(c.take<float>(plan_t.n_chunks * (HD + H)));
  L.dst_part_off = reinterpret_cast<size_t>(c.take<float>(folded ? 0 : plan.n_chunks * H));
  L.dap_src_off = reinterpret_cast<size_t>(c.take<double>(L.src_waves * HD));
  L.dap_dst_off = reinterpret_cast<size_t>(c.take<double>(L.dst_waves * HD));
  L.slices_off = reinterpret_cast<size_t>(c.take<double>(2 * kDaSlices * HD));
  L.bytes = align_up(c.used);
  return L;
}

struct GatBwdIo {
  const void *hs, *hd, *out, *dout;
  const float *a_src, *a_dst;
  void *dhs, *dhd;
  float *ns, *da_src, *da_dst;
  const float* pos;  // the forward's folded destination rows, or null
  int64_t n_dst, n_src, ld, nsld;
  float slope;
  int64_t col_off;   // the head group's first column (h0 * D) within a row
};

// Node-pass grid: one wave per EPW nodes, at most what stays resident.
template <class Kernel>
int64_t node_blocks(Kernel k, int64_t n, int epw) {
  return persist_blocks(ceil_div(n, epw), resident_blocks(k, kTaskBlock));
}

template <int DT, typename I, int G, int HL>
int gat_bwd_launch(const I* row_ptr, const tgx_row_plan& plan, const int32_t* row_ptr_t,
                   const int32_t* col_t, const int32_t* perm, const int32_t* inv_perm,
                   const tgx_row_plan& plan_t, const GatBwdIo& io, char* ws,
                   const GatBwdLayout& L, hipStream_t s) {
  using T = typename Vals<DT, 4>::T;
  constexpr int EPW = kWave / G;
  // The source pass holds dout rows plus node state per edge: 4 in flight
  // per wave measured best (2: +4%, 3: +2%, 6: +5%, 8: +6% time).
  constexpr int U = EPW >= 4 ? 1 : 4 / EPW;
  constexpr int HD = 4 * G;
  const bool homogeneous = io.dhs == io.dhd;
  const bool folded = io.pos != nullptr;
  float* dz = folded ? nullptr : reinterpret_cast<float*>(ws + L.dz_off);
  float* sdz_src = reinterpret_cast<float*>(ws + L.sdz_off);
  float* sdz_dst = folded ? reinterpret_cast<float*>(ws + L.sdz_dst_off) : nullptr;
  float* src_part = reinterpret_cast<float*>(ws + L.src_part_off);
  float* dst_part = reinterpret_cast<float*>(ws + L.dst_part_off);
  double* dap_src = reinterpret_cast<double*>(ws + L.dap_src_off);
  double* dap_dst = reinterpret_cast<double*>(ws + L.dap_dst_off);
  // One feature tensor, not folded: the source pass's contribution to dh is
  // completed by the destination pass, in place for fp32, in fp32 workspace
  // otherwise.  Folded, the source pass writes the final dh.
  float* dh_acc = nullptr;
  if (homogeneous && !folded)
    dh_acc = DT == TGX_DTYPE_F32
                 ? static_cast<float*>(io.dhd)
                 : reinterpret_cast<float*>(ws + L.dh_acc_off) + io.col_off;
  const T* hs = static_cast<const T*>(io.hs);
  const T* hd = static_cast<const T*>(io.hd);
  const PlanView pv = plan_view(plan), pt = plan_view(plan_t);
  const int src_mode = !folded ? 0 : homogeneous ? 2 : 1;

  if (io.n_dst > 0) {
    TGX_PROFILE("gat_delta_kernel", s);
    const GatFold<DT> f{io.pos, 1.f - io.slope, sdz_dst, io.a_dst, static_cast<T*>(io.dhd)};
    const auto k = !folded ? gat_delta_kernel<DT, G, HL, 0>
                   : homogeneous ? gat_delta_kernel<DT, G, HL, 1>
                                 : gat_delta_kernel<DT, G, HL, 2>;
    k<<<ceil_div(ceil_div(io.n_dst, EPW), kWavesPerBlock), kTaskBlock, 0, s>>>(
        static_cast<const T*>(io.dout), static_cast<const T*>(io.out), io.ns, io.n_dst, io.ld,
        io.nsld, f);
    TGX_LAUNCHED("gat_delta_kernel");
  }

  const GatSrcArgs<DT> sa{row_ptr_t, col_t, perm, pt, hs, io.a_src, io.slope, io.ns,
                          static_cast<const T*>(io.dout), dh_acc, static_cast<T*>(io.dhs),
                          src_part, dz, sdz_src, io.a_dst, sdz_dst, io.ld, io.nsld};
  if (plan_waves(pt) > 0) {
    TGX_PROFILE("gat_bwd_src_kernel", s);
    const auto k = src_mode == 0 ? gat_bwd_src_kernel<DT, G, HL, U, 0>
                   : src_mode == 1 ? gat_bwd_src_kernel<DT, G, HL, U, 1>
                                   : gat_bwd_src_kernel<DT, G, HL, U, 2>;
    k<<<ceil_div(plan_waves(pt), kWavesPerBlock), kTaskBlock, 0, s>>>(sa);
    TGX_LAUNCHED("gat_bwd_src_kernel");
  }
  if (pt.n_split > 0) {
    TGX_PROFILE("gat_bwd_src_merge_kernel", s);
    const auto k = src_mode == 2 ? gat_bwd_src_merge_kernel<DT, G, HL, true>
                                 : gat_bwd_src_merge_kernel<DT, G, HL, false>;
    k<<<ceil_div(pt.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
        pt, src_part, dh_acc, static_cast<T*>(io.dhs), sdz_src, io.a_dst, sdz_dst, io.ld);
    TGX_LAUNCHED("gat_bwd_src_merge_kernel");
  }

  int64_t src_blocks = 0, dst_blocks = 0;
  if (folded) {
    // da from node passes: both sums in one read of h for one feature
    // tensor, hs and hd each read once for two.
    if (homogeneous) {
      const auto k = gat_da_nodes_kernel<DT, G, HL, true>;
      src_blocks = dst_blocks = node_blocks(k, io.n_src, EPW);
      TGX_PROFILE("gat_da_nodes_kernel", s);
      k<<<src_blocks, kTaskBlock, 0, s>>>(hs, sdz_src, dap_src, sdz_dst, dap_dst, io.n_src,
                                          io.ld);
      TGX_LAUNCHED("gat_da_nodes_kernel");
    } else {
      const auto k = gat_da_nodes_kernel<DT, G, HL, false>;
      src_blocks = node_blocks(k, io.n_src, EPW);
      dst_blocks = node_blocks(k, io.n_dst, EPW);
      TGX_PROFILE("gat_da_nodes_kernel", s);
      k<<<src_blocks, kTaskBlock, 0, s>>>(hs, sdz_src, dap_src, nullptr, nullptr, io.n_src,
                                          io.ld);
      TGX_LAUNCHED("gat_da_nodes_kernel");
      TGX_PROFILE("gat_da_nodes_kernel", s);
      k<<<dst_blocks, kTaskBlock, 0, s>>>(hd, sdz_dst, dap_dst, nullptr, nullptr, io.n_dst,
                                          io.ld);
      TGX_LAUNCHED("gat_da_nodes_kernel");
    }
  } else {
    const GatDstArgs<DT, I> da{row_ptr, pv, hd, io.a_dst, dz, inv_perm, sdz_src, dh_acc,
                               static_cast<T*>(io.dhd), dst_part, dap_src, dap_dst,
                               plan_waves(pv), io.ld};
    const auto dst_kernel = homogeneous ? gat_bwd_dst_kernel<DT, I, G, HL, true>
                                        : gat_bwd_dst_kernel<DT, I, G, HL, false>;
    dst_blocks = persist_blocks(plan_waves(pv), resident_blocks(dst_kernel, kTaskBlock));
    {
      TGX_PROFILE("gat_bwd_dst_kernel", s);
      dst_kernel<<<dst_blocks, kTaskBlock, 0, s>>>(da);
      TGX_LAUNCHED("gat_bwd_dst_kernel");
    }
    if (pv.n_split > 0) {
      TGX_PROFILE("gat_bwd_dst_merge_kernel", s);
      const auto merge = homogeneous ? gat_bwd_dst_merge_kernel<DT, G, HL, true>
                                     : gat_bwd_dst_merge_kernel<DT, G, HL, false>;
      merge<<<ceil_div(pv.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
          pv, dst_part, io.a_dst, dh_acc, static_cast<T*>(io.dhd), io.ld);
      TGX_LAUNCHED("gat_bwd_dst_merge_kernel");
    }
    src_blocks = dst_blocks;
    if (!homogeneous) {
      const auto k = gat_da_nodes_kernel<DT, G, HL, false>;
      src_blocks = node_blocks(k, io.n_src, EPW);
      TGX_PROFILE("gat_da_nodes_kernel", s);
      k<<<src_blocks, kTaskBlock, 0, s>>>(hs, sdz_src, dap_src, nullptr, nullptr, io.n_src,
                                          io.ld);
      TGX_LAUNCHED("gat_da_nodes_kernel");
    }
  }
  {
    TGX_PROFILE("da_reduce_kernel", s);
    double* slices = reinterpret_cast<double*>(ws + L.slices_off);
    da_slice_kernel<<<dim3(kDaSlices, 2), 256, 0, s>>>(dap_src, dap_dst,
                                                        src_blocks * kWavesPerBlock,
                                                        dst_blocks * kWavesPerBlock, HD, slices);
    TGX_LAUNCHED("da_slice_kernel");
    da_final_kernel<<<ceil_div(2 * HD, 256), 256, 0, s>>>(slices, HD, io.da_src, io.da_dst);
    TGX_LAUNCHED("da_final_kernel");
  }
  return TGX_OK;
}

template <int DT>
int gat_fwd_dtype(const void* row_ptr, const void* col, int idx_bits, const tgx_row_plan* plan,
                  const void* hs, const void* hd, const float* a_src, const float* a_dst,
                  float slope, void* out, float* ns, int H, int D, float* partial,
                  float* pos, hipStream_t s) {
  using T = typename Vals<DT, 4>::T;
  const int64_t ld = static_cast<int64_t>(H) * D, nsld = 4 * static_cast<int64_t>(H);
  for (int h0 = 0; h0 < H;) {
    const int hg = gat_group_heads(H, D, h0);
    const GatShape shp = gat_shape(hg, D);
    const int64_t off = static_cast<int64_t>(h0) * D;
    const T* hs_g = hs ? static_cast<const T*>(hs) + off : nullptr;
    const T* hd_g = static_cast<const T*>(hd) + off;
    T* out_g = static_cast<T*>(out) + off;
    float* pos_g = pos ? pos + off : nullptr;
    int st = TGX_UNSUPPORTED;
#define TGX_GAT_FWD(GG, HH)                                                                  \
    if (shp.G == GG && shp.HL == HH) {                                                       \
      if (idx_bits == 32)                                                                    \
        st = gat_fwd_launch<DT, int32_t, GG, HH>(                                            \
            GatFwdArgs<DT, int32_t>{static_cast<const int32_t*>(row_ptr),                    \
                                    static_cast<const int32_t*>(col), plan_view(*plan),      \
                                    hs_g, hd_g, a_src + off, a_dst + off, slope, out_g,      \
                                    ns + 4 * h0, partial, pos_g, ld, nsld},                  \
            s);                                                                              \
      else                                                                                   \
        st = gat_fwd_launch<DT, int64_t, GG, HH>(                                            \
            GatFwdArgs<DT, int64_t>{static_cast<const int64_t*>(row_ptr),                    \
                                    static_cast<const int64_t*>(col), plan_view(*plan),      \
                                    hs_g, hd_g, a_src + off, a_dst + off, slope, out_g,      \
                                    ns + 4 * h0, partial, pos_g, ld, nsld},                  \
            s);                                                                              \
    } else
    TGX_GAT_SHAPES(TGX_GAT_FWD)
    set_error("unsupported GAT head group G=%d HL=%d", shp.G, shp.HL);
#undef TGX_GAT_FWD
    if (st != TGX_OK) return st;
    h0 += hg;
  }
  return TGX_OK;
}

template <int DT>
int gat_bwd_dtype(const void* row_ptr, int idx_bits, const tgx_row_plan* plan,
                  const int32_t* row_ptr_t, const int32_t* col_t, const int32_t* perm,
                  const int32_t* inv_perm, const tgx_row_plan* plan_t, const GatBwdIo& all,
                  int64_t n_edges, int H, int D, char* w, hipStream_t s) {
  using T = typename Vals<DT, 4>::T;
  auto at = [](const void* p, int64_t off) -> const void* {
    return p ? static_cast<const T*>(p) + off : nullptr;
  };
  auto at_mut = [](void* p, int64_t off) -> void* {
    return p ? static_cast<T*>(p) + off : nullptr;
  };
  for (int h0 = 0; h0 < H;) {
    const int hg = gat_group_heads(H, D, h0);
    const GatShape shp = gat_shape(hg, D);
    const GatBwdLayout L =
        gat_bwd_layout(*plan, *plan_t, n_edges, hg, D, DT, H, all.pos != nullptr);
    const int64_t off = static_cast<int64_t>(h0) * D;
    GatBwdIo io = all;
    io.col_off = off;
    io.hs = at(all.hs, off);
    io.hd = at(all.hd, off);
    io.out = at(all.out, off);
    io.dout = at(all.dout, off);
    io.dhs = at_mut(all.dhs, off);
    io.dhd = at_mut(all.dhd, off);
    io.a_src = all.a_src + off;
    io.a_dst = all.a_dst + off;
    io.da_src = all.da_src + off;
    io.da_dst = all.da_dst + off;
    io.ns = all.ns + 4 * h0;
    io.pos = all.pos ? all.pos + off : nullptr;
    int st = TGX_UNSUPPORTED;
#define TGX_GAT_BWD(GG, HH)                                                                 \
    if (shp.G == GG && shp.HL == HH) {                                                      \
      if (idx_bits == 32)                                                                   \
        st = gat_bwd_launch<DT, int32_t, GG, HH>(static_cast<const int32_t*>(row_ptr),      \
                                                 *plan, row_ptr_t, col_t, perm, inv_perm,   \
                                                 *plan_t, io, w, L, s);                     \
      else                                                                                  \
        st = gat_bwd_launch<DT, int64_t, GG, HH>(static_cast<const int64_t*>(row_ptr),      \
                                                 *plan, row_ptr_t, col_t, perm, inv_perm,   \
                                                 *plan_t, io, w, L, s);                     \
    } else
    TGX_GAT_SHAPES(TGX_GAT_BWD)
    set_error("unsupported GAT head group G=%d HL=%d", shp.G, shp.HL);
#undef TGX_GAT_BWD
    if (st != TGX_OK) return st;
    h0 += hg;
  }
  return TGX_OK;
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_gat_fwd(const void* row_ptr, const void* col, int idx_bits,
                           const tgx_row_plan* plan, const void* h_src, const void* h_dst,
                           const float* a_src, const float* a_dst, float slope, void* out,
                           float* ns, int64_t n_dst, int64_t n_src, int H, int D, int dtype,
                           float* partial, float* pos, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(dtype_bytes(dtype) != 0, "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)",
              dtype);
  if (!gat_heads_ok(H, D)) {
    set_error("GAT kernel supports H >= 1 and D in {4, 8, 16, 32, 64, 128, 256} "
              "(got H=%d D=%d)", H, D);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(h_src != h_dst || n_src == n_dst,
              "one feature tensor for both roles needs n_src == n_dst");
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && h_dst && a_src && a_dst && out && ns && (h_src || n_src == 0),
              "null pointer");
  TGX_REQUIRE(plan->n_chunks == 0 || partial, "split rows need a partial buffer");
  TGX_REQUIRE(reinterpret_cast<uintptr_t>(pos) % 16 == 0, "pos must be 16-byte aligned");
  TGX_REQUIRE(n_src < (int64_t{1} << 31), "source tables need fewer than 2^31 rows");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case TGX_DTYPE_F32:
      return gat_fwd_dtype<TGX_DTYPE_F32>(row_ptr, col, idx_bits, plan, h_src, h_dst, a_src,
                                          a_dst, slope, out, ns, H, D, partial, pos, s);
    case TGX_DTYPE_BF16:
      return gat_fwd_dtype<TGX_DTYPE_BF16>(row_ptr, col, idx_bits, plan, h_src, h_dst, a_src,
                                           a_dst, slope, out, ns, H, D, partial, pos, s);
    default:
      return gat_fwd_dtype<TGX_DTYPE_F16>(row_ptr, col, idx_bits, plan, h_src, h_dst, a_src,
                                          a_dst, slope, out, ns, H, D, partial, pos, s);
  }
}

extern "C" int tgx_gat_bwd_workspace(const tgx_row_plan* plan, const tgx_row_plan* plan_t,
                                     int64_t n_edges, int H, int D, int dtype, int folded,
                                     size_t* bytes) {
  TGX_REQUIRE(plan && plan_t && bytes, "null pointer");
  TGX_REQUIRE(dtype_bytes(dtype) != 0, "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)",
              dtype);
  if (!gat_heads_ok(H, D)) {
    set_error("unsupported GAT shape H=%d D=%d", H, D);
    return TGX_UNSUPPORTED;
  }
  // Head groups run one after another on one stream and share the
  // workspace; the first group is the widest.
  *bytes = gat_bwd_layout(*plan, *plan_t, n_edges, gat_group_heads(H, D, 0), D, dtype, H,
                          folded != 0)
               .bytes;
  return TGX_OK;
}

extern "C" int tgx_gat_bwd(const void* row_ptr, const void* col, int idx_bits,
                           const tgx_row_plan* plan, const int32_t* row_ptr_t,
                           const int32_t* col_t, const int32_t* perm, const int32_t* inv_perm,
                           const tgx_row_plan* plan_t, const void* h_src, const void* h_dst,
                           const float* a_src, const float* a_dst, float slope, const void* out,
                           float* ns, const float* pos, const void* dout, void* dh_src,
                           void* dh_dst,
                           float* da_src, float* da_dst, int64_t n_dst, int64_t n_src,
                           int64_t n_edges, int H, int D, int dtype, void* ws, size_t ws_bytes,
                           void* stream) {
  (void)col;
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(dtype_bytes(dtype) != 0, "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)",
              dtype);
  if (!gat_heads_ok(H, D)) {
    set_error("unsupported GAT shape H=%d D=%d", H, D);
    return TGX_UNSUPPORTED;
  }
  // One gradient buffer for both roles declares one feature tensor.
  const bool homogeneous = dh_src == dh_dst;
  TGX_REQUIRE(!homogeneous || (h_src == h_dst && n_src == n_dst),
              "one gradient for both roles (dh_src == dh_dst) needs one feature tensor "
              "(h_src == h_dst) and n_src == n_dst");
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  st = check_plan(plan_t, n_src);
  if (st != TGX_OK) return st;
  if (n_dst == 0 && n_src == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && h_src && h_dst && a_src && a_dst && out && ns && dout && dh_src &&
                  dh_dst && da_src && da_dst,
              "null pointer");
  TGX_REQUIRE(n_edges == 0 || (row_ptr_t && col_t && (pos || inv_perm)),
              "null transposed CSR");
  TGX_REQUIRE(reinterpret_cast<uintptr_t>(pos) % 16 == 0, "pos must be 16-byte aligned");
  TGX_REQUIRE(n_src < (int64_t{1} << 31) && n_dst < (int64_t{1} << 31),
              "node tables need fewer than 2^31 rows");
  const size_t need = gat_bwd_layout(*plan, *plan_t, n_edges, gat_group_heads(H, D, 0), D,
                                     dtype, H, pos != nullptr)
                          .bytes;
  TGX_REQUIRE(ws && ws_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const GatBwdIo io{h_src, h_dst, out, dout, a_src, a_dst, dh_src, dh_dst, ns, da_src, da_dst,
                    pos, n_dst, n_src, static_cast<int64_t>(H) * D, 4 * static_cast<int64_t>(H),
                    slope, 0};
  char* w = static_cast<char*>(ws);
  switch (dtype) {
    case TGX_DTYPE_F32:
      return gat_bwd_dtype<TGX_DTYPE_F32>(row_ptr, idx_bits, plan, row_ptr_t, col_t, perm,
                                          inv_perm, plan_t, io, n_edges, H, D, w, s);
    case TGX_DTYPE_BF16:
      return gat_bwd_dtype<TGX_DTYPE_BF16>(row_ptr, idx_bits, plan, row_ptr_t, col_t, perm,
                                           inv_perm, plan_t, io, n_edges, H, D, w, s);
    default:
      return gat_bwd_dtype<TGX_DTYPE_F16>(row_ptr, idx_bits, plan, row_ptr_t, col_t, perm,
                                          inv_perm, plan_t, io, n_edges, H, D, w, s);
  }
}
