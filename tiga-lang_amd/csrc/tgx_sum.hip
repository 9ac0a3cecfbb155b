// Sum reducer over a destination-row CSR:  out[i, :] = sum_e w[e] * x[col[e], :]
//
// Layout: a gathered row of F fp32 features is split into feature tiles of
// G*VEC floats; G lanes hold one tile of one edge, VEC floats per lane
// (16-byte loads when VEC == 4), so one wave keeps 64/G edges in flight per
// vector load and U such loads per lane before consuming them.  The edge
// groups are folded at the end of the row with cross-lane adds.
//
// The same kernel is the backward's dx pass: run over the transposed CSR with
// x := dout and the weight fetched through the transpose permutation, it
// computes dx[j] = sum_{e'} w[perm[e']] * dout[col_t[e']] with no atomics.  With
// `self_x` set it also produces dw[perm[e']] = <dout[col_t[e']], x[j]> from the
// row it already holds.
#include <hip/hip_runtime.h>

#include "tgx_device.h"
#include "tgx_host.h"
#include "tgx_profile.h"
#include "tgx_tasks.h"

namespace tgx {
namespace {

// Element storage of the feature tables (x, out, dout, dx); weights and the
// split-row partials are always fp32, and so is every sum.
template <int DT>
struct Elem;
template <>
struct Elem<TGX_DTYPE_F32> {
  typedef float S;
  static __device__ __forceinline__ f32x4 load4(const S* p) {
    return *reinterpret_cast<const f32x4*>(p);
  }
  static __device__ __forceinline__ void store4(S* p, f32x4 v) {
    *reinterpret_cast<f32x4*>(p) = v;
  }
  static __device__ __forceinline__ float load1(const S* p) { return *p; }
  static __device__ __forceinline__ void store1(S* p, float v) { *p = v; }
};
template <>
struct Elem<TGX_DTYPE_BF16> {
  typedef uint16_t S;
  static __device__ __forceinline__ f32x4 load4(const S* p) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    return f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
  }
  static __device__ __forceinline__ void store4(S* p, f32x4 v) {
    *reinterpret_cast<uint2*>(p) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
  static __device__ __forceinline__ float load1(const S* p) { return bf16_lo(*p); }
  static __device__ __forceinline__ void store1(S* p, float v) {
    *p = static_cast<uint16_t>(f32_to_bf16_bits(v));
  }
};
template <>
struct Elem<TGX_DTYPE_F16> {
  typedef _Float16 S;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 load4(const S* p) {
    const h4 h = *reinterpret_cast<const h4*>(p);
    return f32x4{static_cast<float>(h[0]), static_cast<float>(h[1]), static_cast<float>(h[2]),
                 static_cast<float>(h[3])};
  }
  static __device__ __forceinline__ void store4(S* p, f32x4 v) {
    *reinterpret_cast<h4*>(p) = h4{static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]),
                                   static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
  }
  static __device__ __forceinline__ float load1(const S* p) { return static_cast<float>(*p); }
  static __device__ __forceinline__ void store1(S* p, float v) { *p = static_cast<_Float16>(v); }
};

template <typename I, int DT>
struct SumArgs {
  typedef typename Elem<DT>::S S;
  const I* row_ptr;
  const I* col;
  PlanView plan;
  const S* x;              // gathered table [*, F]
  const float* w;          // per-edge weight or null (=1)
  const int32_t* wperm;    // weight index = wperm[e] when non-null
  S* out;                  // [rows, F]
  float* partial;          // [n_chunks, F]
  const S* self_x;         // dw: row's own features [rows, F] (null = no dw)
  float* dw;               // dw output, written at wperm ? wperm[e] : e
  int64_t F;
};

// VEC consecutive features per lane, held in fp32.
template <int VEC, int DT>
struct Vec;
template <int DT>
struct Vec<4, DT> {
  typedef f32x4 T;
  typedef typename Elem<DT>::S S;
  static __device__ __forceinline__ T load(const S* p) { return Elem<DT>::load4(p); }
  static __device__ __forceinline__ void store(S* p, T v) { Elem<DT>::store4(p, v); }
  static __device__ __forceinline__ T zero() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  static __device__ __forceinline__ float dot(T a, T b) {
    return a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
  }
  static __device__ __forceinline__ T shfl_xor(T v, int m) {
    return f32x4{__shfl_xor(v[0], m, 64), __shfl_xor(v[1], m, 64),
                 __shfl_xor(v[2], m, 64), __shfl_xor(v[3], m, 64)};
  }
};
template <int DT>
struct Vec<1, DT> {
  typedef float T;
  typedef typename Elem<DT>::S S;
  static __device__ __forceinline__ T load(const S* p) { return Elem<DT>::load1(p); }
  static __device__ __forceinline__ void store(S* p, T v) { Elem<DT>::store1(p, v); }
  static __device__ __forceinline__ T zero() { return 0.f; }
  static __device__ __forceinline__ float dot(T a, T b) { return a * b; }
  static __device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, 64); }
};

template <int G>
__device__ __forceinline__ float group_reduce_sum(float v) {
  // Sum over the G lanes of one edge group (aligned, contiguous).
  return group_sum<G>(v);
}

// One whole-wave task (a row, a split-row chunk or a group of empty rows).
template <typename I, int DT, int VEC, int G, int U>
__device__ __forceinline__ void sum_task(const SumArgs<I, DT>& a, const Task& t) {
  typedef Vec<VEC, DT> V;
  typedef typename V::T T;
  constexpr int EPW = kWave / G;  // edges per wave-wide load
  if (t.kind == kTaskNone) return;
  const int lane = lane_id();
  const int g = lane / G;
  const int c = lane % G;
  const int64_t F = a.F;
  const int64_t fo = static_cast<int64_t>(blockIdx.y) * (G * VEC) + c * VEC;
  const bool active = fo < F;

  if (t.kind == kTaskEmpty) {
    for (int k = 0; k < t.n_empty; ++k) {
      const int row = uniform(a.plan.rows[t.empty0 + k]);
      if (g == 0 && active && a.out)
        V::store(a.out + static_cast<int64_t>(row) * F + fo, V::zero());
    }
    return;
  }

  T self = V::zero();
  const bool want_dw = a.self_x != nullptr;
  if (want_dw && active) self = V::load(a.self_x + static_cast<int64_t>(t.row) * F + fo);
  // A window's dw values wait in LDS and leave with one store per lane
  // after the window, not one store per edge group inside the gather loop
  // (whose following gathers would share its in-order completion count).
  // Measured on bench.py --config c1: the backward unchanged (0.109 ms), the forward, which
  // writes no dw, 0.061 -> 0.059 ms with this kernel shape.
  __shared__ float dw_stage[kWavesPerBlock][kWave];
  const int wv = threadIdx.x / kWave;

  T acc = V::zero();
  for (int64_t base = t.e0; base < t.e1; base += kWave) {
    const int n = static_cast<int>(t.e1 - base < kWave ? t.e1 - base : kWave);
    int my_col = 0;
    float my_w = 0.f;
    int my_wp = 0;   // wperm[e] (int32: a permuted relation has < 2^31 edges)
    if (lane < n) {
      // No column array: the columns are the edge ids (a per-edge field
      // summed per row, read contiguously).
      const int64_t e = base + lane;
      my_col = a.col ? static_cast<int>(a.col[e]) : static_cast<int>(e);
      if (a.wperm) my_wp = a.wperm[e];
      my_w = a.w ? a.w[a.wperm ? static_cast<int64_t>(my_wp) : e] : 1.f;
    }
    for (int k = 0; k < n; k += EPW * U) {
      T v[U];
      float wt[U];
      int slot[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        slot[u] = k + u * EPW + g;
        const int src = slot[u] < n ? slot[u] : 0;
        const int j = __shfl(my_col, src, 64);
        wt[u] = __shfl(my_w, src, 64);
        v[u] = (slot[u] < n && active) ? V::load(a.x + static_cast<int64_t>(j) * F + fo)
                                       : V::zero();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (slot[u] < n) acc += wt[u] * v[u];
      }
      if (want_dw) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float d = group_reduce_sum<G>(V::dot(v[u], self));
          if (c == 0 && slot[u] < n) dw_stage[wv][slot[u]] = d;
        }
      }
    }
    if (want_dw) {
      // One wave's LDS accesses complete in issue order: lane e reads the
      // value another lane wrote for edge base + e.
      __builtin_amdgcn_wave_barrier();
      if (lane < n) a.dw[a.wperm ? static_cast<int64_t>(my_wp) : base + lane] = dw_stage[wv][lane];
      __builtin_amdgcn_wave_barrier();
    }
  }
  // Fold the EPW edge groups (lanes with equal c).
#pragma unroll
  for (int m = G; m < kWave; m <<= 1) acc += V::shfl_xor(acc, m);
  // A null out: only the per-edge dot products (dw) are wanted.
  if (g != 0 || !active || !a.out) return;
  if (t.kind == kTaskChunk)
    Vec<VEC, TGX_DTYPE_F32>::store(a.partial + static_cast<int64_t>(t.slot) * F + fo, acc);
  else
    V::store(a.out + static_cast<int64_t>(t.row) * F + fo, acc);
}

template <typename I, int DT, int VEC, int G, int U>
__global__ __launch_bounds__(kTaskBlock) void sum_rows_kernel(SumArgs<I, DT> a) {
  sum_task<I, DT, VEC, G, U>(a, decode_task(a.plan, a.row_ptr, global_wave()));
}

// Narrow rows (G <= 8 lanes per edge): the wave splits into 64 / SLOT lane
// slots of SLOT lanes, each taking P rows of the wave bin, so a wave's fixed
// cost (task decode, the dependent row_ptr -> col -> gather chain) covers
// (64 / SLOT) P rows, and the loads of a slot's P rows are in flight
// together.  A slot keeps SLOT edges per row in flight (U = G loads of
// SLOT / G edges).  The task list is
//   [split-row chunks | row groups | empty-row groups];
// chunks and empty groups run as whole-wave tasks.  Slot s of group w takes
// the wave-bin rows S P w + S q + s, q < P, S = 64 / SLOT.
template <typename I, int DT, int VEC, int G, int UC, int SLOT, int P>
__global__ __launch_bounds__(kTaskBlock) void sum_pairs_kernel(SumArgs<I, DT> a) {
  typedef Vec<VEC, DT> V;
  typedef typename V::T T;
  constexpr int NS = kWave / SLOT;   // slots per wave
  constexpr int EPH = SLOT / G;      // edges per slot load
  constexpr int U = G;               // loads in flight per row: SLOT edges
  const PlanView& p = a.plan;
  const int64_t w = global_wave();
  const int64_t n_groups = (p.n_wave + NS * P - 1) / (NS * P);
  if (w < p.n_chunks) {
    sum_task<I, DT, VEC, G, UC>(a, decode_task(p, a.row_ptr, w));
    return;
  }
  const int64_t pw = w - p.n_chunks;
  if (pw >= n_groups) {
    sum_task<I, DT, VEC, G, UC>(a, decode_task(p, a.row_ptr, p.n_chunks + p.n_wave + (pw - n_groups)));
    return;
  }
  const int lane = lane_id();
  const int slot_id = lane / SLOT, hl = lane % SLOT;
  const int g = hl / G, c = hl % G;
  const int64_t F = a.F;
  const int64_t fo = c * VEC;   // G * VEC <= F's tile: one feature tile
  const bool active = fo < F;
  const bool want_dw = a.self_x != nullptr;
  int row[P], len[P];
  int64_t e0[P];
  bool has[P];
  int len_max = 0;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int64_t k = NS * P * pw + NS * q + slot_id;   // position in the wave bin
    has[q] = k < p.n_wave;
    row[q] = has[q] ? p.rows[p.n_empty + k] : 0;
    e0[q] = has[q] ? static_cast<int64_t>(a.row_ptr[row[q]]) : 0;
    len[q] = has[q] ? static_cast<int>(static_cast<int64_t>(a.row_ptr[row[q] + 1]) - e0[q]) : 0;
    len_max = max(len_max, len[q]);
  }
  // Every slot loops to the longest row (wave-uniform bounds keep every
  // shuffle's source lanes active); each row masks its own tail.
#pragma unroll
  for (int m = SLOT; m < kWave; m <<= 1) len_max = max(len_max, __shfl_xor(len_max, m, 64));
  T self[P], acc[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    self[q] = V::zero();
    acc[q] = V::zero();
    if (want_dw && active && has[q])
      self[q] = V::load(a.self_x + static_cast<int64_t>(row[q]) * F + fo);
  }
  for (int base = 0; base < len_max; base += SLOT) {
    int n[P], my_col[P], my_wp[P];
    float my_w[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
      n[q] = min(max(len[q] - base, 0), SLOT);   // this row's edges
      my_col[q] = 0;
      my_wp[q] = 0;
      my_w[q] = 0.f;
      if (hl < n[q]) {
        const int64_t e = e0[q] + base + hl;
        my_col[q] = a.col ? static_cast<int>(a.col[e]) : static_cast<int>(e);
        if (a.wperm) my_wp[q] = a.wperm[e];
        my_w[q] = a.w ? a.w[a.wperm ? static_cast<int64_t>(my_wp[q]) : e] : 1.f;
      }
    }
    const int n_max = min(len_max - base, SLOT);   // wave-uniform
    for (int kk = 0; kk < n_max; kk += EPH * U) {
      T v[P][U];
      float wt[P][U];
      int slot[U];
#pragma unroll
      for (int u = 0; u < U; ++u) slot[u] = kk + u * EPH + g;
#pragma unroll
      for (int q = 0; q < P; ++q)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int src = SLOT * slot_id + (slot[u] < n[q] ? slot[u] : 0);
          const int j = __shfl(my_col[q], src, 64);
          wt[q][u] = __shfl(my_w[q], src, 64);
          v[q][u] = (slot[u] < n[q] && active) ? V::load(a.x + static_cast<int64_t>(j) * F + fo)
                                               : V::zero();
        }
#pragma unroll
      for (int q = 0; q < P; ++q)
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (slot[u] < n[q]) acc[q] += wt[q][u] * v[q][u];
      if (want_dw) {
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const float d = group_reduce_sum<G>(V::dot(v[q][u], self[q]));
            const int k = slot[u] < n[q] ? slot[u] : 0;
            const int wp = __shfl(my_wp[q], SLOT * slot_id + k, 64);
            const int64_t widx = a.wperm ? static_cast<int64_t>(wp) : e0[q] + base + k;
            if (c == 0 && slot[u] < n[q]) a.dw[widx] = d;
          }
      }
    }
  }
  // Fold each row's edge groups (lanes with equal c; masks below SLOT stay
  // inside the slot).
#pragma unroll
  for (int q = 0; q < P; ++q) {
#pragma unroll
    for (int m = G; m < SLOT; m <<= 1) acc[q] += V::shfl_xor(acc[q], m);
    if (g == 0 && active && has[q] && a.out)
      V::store(a.out + static_cast<int64_t>(row[q]) * F + fo, acc[q]);
  }
}

// Combine split-row chunk partials in chunk order (deterministic).
template <int DT>
__global__ __launch_bounds__(kTaskBlock) void sum_merge_kernel(
    PlanView plan, const float* __restrict__ partial, typename Elem<DT>::S* __restrict__ out,
    int64_t F) {
  const int64_t k = global_wave();
  if (k >= plan.n_split) return;
  const int row = uniform(plan.rows[plan.n_empty + plan.n_wave + k]);
  const int c0 = plan.chunk_off[k], c1 = plan.chunk_off[k + 1];
  for (int64_t f = lane_id(); f < F; f += kWave) {
    float s = 0.f;
    for (int c = c0; c < c1; ++c) s += partial[static_cast<int64_t>(c) * F + f];
    Elem<DT>::store1(out + static_cast<int64_t>(row) * F + f, s);
  }
}

template <typename I, int DT, int VEC, int G>
void launch_sum(const SumArgs<I, DT>& a, int64_t ftiles, hipStream_t s) {
  constexpr int U = (kWave / G) >= 16 ? 1 : (16 / (kWave / G) < 8 ? 16 / (kWave / G) : 8);
  if constexpr (G <= 8) {
    // ftiles == 1 here: G * VEC <= 32 covers F.
    // One lane per edge (F = 1, or F = 4 as one 4-wide vector): 16-lane
    // slots of 2 rows each, 8 rows per wave (the reference's F = 1 case,
    // 131072 rows of 16 edges: 0.0254 ms with 32-lane slots of 2 rows,
    // 0.0182 ms with these).  Wider rows: 32-lane slots of one row (two rows
    // per wave measured 5% faster than four on 8-wide rows).
    constexpr int SLOT = G == 1 ? 16 : 32;
    constexpr int P = G == 1 ? 2 : 1;
    constexpr int NS = kWave / SLOT;
    const PlanView& p = a.plan;
    const int64_t waves = p.n_chunks + (p.n_wave + NS * P - 1) / (NS * P) +
                          (p.n_empty + kEmptyPerWave - 1) / kEmptyPerWave;
    sum_pairs_kernel<I, DT, VEC, G, U, SLOT, P>
        <<<static_cast<unsigned>(ceil_div(waves, kWavesPerBlock)), kTaskBlock, 0, s>>>(a);
  } else {
    const int64_t waves = plan_waves(a.plan);
    dim3 grid(static_cast<unsigned>(ceil_div(waves, kWavesPerBlock)),
              static_cast<unsigned>(ftiles));
    sum_rows_kernel<I, DT, VEC, G, U><<<grid, kTaskBlock, 0, s>>>(a);
  }
}

template <typename I, int DT>
int sum_dispatch(const SumArgs<I, DT>& a, hipStream_t s) {
  const int64_t F = a.F;
  if (F % 4 == 0) {
    const int64_t lanes = F / 4;
    if (lanes <= 1) launch_sum<I, DT, 4, 1>(a, 1, s);
    else if (lanes <= 2) launch_sum<I, DT, 4, 2>(a, 1, s);
    else if (lanes <= 4) launch_sum<I, DT, 4, 4>(a, 1, s);
    else if (lanes <= 8) launch_sum<I, DT, 4, 8>(a, 1, s);
    else if (lanes <= 16) launch_sum<I, DT, 4, 16>(a, 1, s);
    else if (lanes <= 32) launch_sum<I, DT, 4, 32>(a, 1, s);
    else launch_sum<I, DT, 4, 64>(a, ceil_div(lanes, 64), s);
  } else {
    if (F <= 1) launch_sum<I, DT, 1, 1>(a, 1, s);
    else if (F <= 2) launch_sum<I, DT, 1, 2>(a, 1, s);
    else if (F <= 4) launch_sum<I, DT, 1, 4>(a, 1, s);
    else if (F <= 8) launch_sum<I, DT, 1, 8>(a, 1, s);
    else if (F <= 16) launch_sum<I, DT, 1, 16>(a, 1, s);
    else if (F <= 32) launch_sum<I, DT, 1, 32>(a, 1, s);
    else launch_sum<I, DT, 1, 64>(a, ceil_div(F, 64), s);
  }
  TGX_LAUNCHED("sum_rows_kernel");
  if (a.plan.n_split > 0 && a.out) {
    sum_merge_kernel<DT><<<ceil_div(a.plan.n_split, kWavesPerBlock), kTaskBlock, 0, s>>>(
        a.plan, a.partial, a.out, F);
    TGX_LAUNCHED("sum_merge_kernel");
  }
  return TGX_OK;
}

// dw for feature widths that span several tiles: one wave per edge group of
// the transposed CSR row, full-width dot product.
template <int DT>
__global__ __launch_bounds__(kTaskBlock) void sum_dw_wide_kernel(
    const int32_t* __restrict__ row_ptr_t, const int32_t* __restrict__ col_t,
    const int32_t* __restrict__ perm, const typename Elem<DT>::S* __restrict__ x,
    const typename Elem<DT>::S* __restrict__ dout, float* __restrict__ dw, int64_t n_src,
    int64_t F) {
  const int64_t j = global_wave();
  if (j >= n_src) return;
  const int64_t b = row_ptr_t[j], e = row_ptr_t[j + 1];
  for (int64_t k = b; k < e; ++k) {
    const int64_t i = col_t[k];
    float s = 0.f;
    for (int64_t f = lane_id(); f < F; f += kWave)
      s += Elem<DT>::load1(dout + i * F + f) * Elem<DT>::load1(x + j * F + f);
    s = group_sum<64>(s);
    if (lane_id() == 0) dw[perm[k]] = s;
  }
}

template <int V>
struct DtConst {
  static constexpr int value = V;
};
template <typename T>
struct IdxType {
  typedef T type;
};

// Calls f(DtConst<dtype>, IdxType<index type>) for a checked dtype code and
// index width.
template <typename F>
int with_types(int dtype, int idx_bits, F f) {
  if (dtype == TGX_DTYPE_BF16)
    return idx_bits == 32 ? f(DtConst<TGX_DTYPE_BF16>{}, IdxType<int32_t>{})
                          : f(DtConst<TGX_DTYPE_BF16>{}, IdxType<int64_t>{});
  if (dtype == TGX_DTYPE_F16)
    return idx_bits == 32 ? f(DtConst<TGX_DTYPE_F16>{}, IdxType<int32_t>{})
                          : f(DtConst<TGX_DTYPE_F16>{}, IdxType<int64_t>{});
  return idx_bits == 32 ? f(DtConst<TGX_DTYPE_F32>{}, IdxType<int32_t>{})
                        : f(DtConst<TGX_DTYPE_F32>{}, IdxType<int64_t>{});
}

}  // namespace

}  // namespace tgx

using namespace tgx;

extern "C" int tgx_partial_bytes(const tgx_row_plan* plan, int64_t state_floats,
                                 size_t* bytes) {
  TGX_REQUIRE(plan && bytes, "null pointer");
  TGX_REQUIRE(state_floats >= 0, "negative state size");
  *bytes = static_cast<size_t>(plan->n_chunks) * state_floats * sizeof(float);
  return TGX_OK;
}

extern "C" int tgx_csr_sum_fwd(const void* row_ptr, const void* col, int idx_bits,
                               const tgx_row_plan* plan, const void* x, const float* w,
                               void* out, int64_t n_dst, int64_t n_src, int64_t F, int dtype,
                               float* partial, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  if (dtype != TGX_DTYPE_F32 && dtype != TGX_DTYPE_BF16 && dtype != TGX_DTYPE_F16) {
    set_error("sum supports fp32, bf16 and fp16 features (dtype code %d)", dtype);
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && out && (x || n_src == 0), "null pointer");
  // A null col means the columns are the edge ids (x holds one row per edge).
  TGX_REQUIRE(col || n_src < (int64_t{1} << 31), "edge-id columns need fewer than 2^31 edges");
  // Gathered row indices are held in 32 bits.
  TGX_REQUIRE(n_src < (int64_t{1} << 31), "source tables need fewer than 2^31 rows");
  TGX_REQUIRE(plan->n_chunks == 0 || partial, "split rows need a partial buffer");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("csr_sum_fwd", s);
  auto run = [&](auto dt, auto idx) -> int {
    constexpr int DT = decltype(dt)::value;
    typedef typename decltype(idx)::type I;
    typedef typename Elem<DT>::S S;
    SumArgs<I, DT> a{static_cast<const I*>(row_ptr), static_cast<const I*>(col),
                     plan_view(*plan), static_cast<const S*>(x), w, nullptr,
                     static_cast<S*>(out), partial, nullptr, nullptr, F};
    return sum_dispatch(a, s);
  };
  return with_types(dtype, idx_bits, run);
}

extern "C" int tgx_csr_sum_bwd(const int32_t* row_ptr_t, const int32_t* col_t,
                               const int32_t* perm, const tgx_row_plan* plan_t,
                               const void* x, const float* w, const void* dout, void* dx,
                               float* dw, int64_t n_dst, int64_t n_src, int64_t F, int dtype,
                               float* partial, void* stream) {
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  if (dtype != TGX_DTYPE_F32 && dtype != TGX_DTYPE_BF16 && dtype != TGX_DTYPE_F16) {
    set_error("sum supports fp32, bf16 and fp16 features (dtype code %d)", dtype);
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan_t, n_src);
  if (st != TGX_OK) return st;
  if (n_src == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr_t && dout, "null pointer");
  // col_t / perm may be null for a graph without edges.
  TGX_REQUIRE(!dw || x, "dw needs x");
  TGX_REQUIRE(plan_t->n_chunks == 0 || partial || !dx, "split rows need a partial buffer");
  hipStream_t s = as_stream(stream);
  const bool single_tile = (F % 4 == 0) ? (F / 4 <= 64) : (F <= 64);
  TGX_PROFILE("csr_sum_bwd", s);
  auto run = [&](auto dt, auto) -> int {
    constexpr int DT = decltype(dt)::value;
    typedef typename Elem<DT>::S S;
    const S* xs = static_cast<const S*>(x);
    const S* gs = static_cast<const S*>(dout);
    if (dx) {
      SumArgs<int32_t, DT> a{row_ptr_t, col_t, plan_view(*plan_t), gs, w, perm,
                             static_cast<S*>(dx), partial,
                             (dw && single_tile) ? xs : nullptr,
                             (dw && single_tile) ? dw : nullptr, F};
      const int r = sum_dispatch(a, s);
      if (r != TGX_OK) return r;
    }
    if (dw && (!dx || !single_tile)) {
      sum_dw_wide_kernel<DT><<<ceil_div(n_src, kWavesPerBlock), kTaskBlock, 0, s>>>(
          row_ptr_t, col_t, perm, xs, gs, dw, n_src, F);
      TGX_LAUNCHED("sum_dw_wide_kernel");
    }
    return TGX_OK;
  };
  return with_types(dtype, 32, run);
}

extern "C" int tgx_csr_edge_dot(const void* row_ptr, const void* col, int idx_bits,
                                const tgx_row_plan* plan, const void* x, const void* dout,
                                float* dw, int64_t n_dst, int64_t n_src, int64_t F, int dtype,
                                void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  if (dtype != TGX_DTYPE_F32 && dtype != TGX_DTYPE_BF16 && dtype != TGX_DTYPE_F16) {
    set_error("sum supports fp32, bf16 and fp16 features (dtype code %d)", dtype);
    return TGX_UNSUPPORTED;
  }
  if (F > 32) {
    set_error("tgx_csr_edge_dot covers F <= 32 (got %lld); wider rows take the dw output "
              "of tgx_csr_sum_bwd", static_cast<long long>(F));
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && col && x && dout && dw, "null pointer");
  TGX_REQUIRE(n_src < (int64_t{1} << 31), "source tables need fewer than 2^31 rows");
  hipStream_t s = as_stream(stream);
  TGX_PROFILE("csr_edge_dot", s);
  auto run = [&](auto dt, auto idx) -> int {
    constexpr int DT = decltype(dt)::value;
    typedef typename decltype(idx)::type I;
    typedef typename Elem<DT>::S S;
    // The sum kernel over the CSR with the row's own dout as `self`: it
    // writes dw[e] = <dout[i], x[col[e]]> in edge order and no sums.
    SumArgs<I, DT> a{static_cast<const I*>(row_ptr), static_cast<const I*>(col),
                     plan_view(*plan), static_cast<const S*>(x), nullptr, nullptr, nullptr,
                     nullptr, static_cast<const S*>(dout), dw, F};
    return sum_dispatch(a, s);
  };
  return with_types(dtype, idx_bits, run);
}
