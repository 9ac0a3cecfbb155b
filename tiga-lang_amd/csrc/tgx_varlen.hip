// Varlen causal attention on MFMA (gfx950, bf16 in, fp32 accumulate).
//
// The relation is Graph.cu_seqlens(causal=True) (reference
// python/tiga/interop/torch/graph.py:260-294): token i of sequence k attends
// to keys [s_k, i].  The edge function is the dot-product score
// scale * q[i].k[j] with value v[j]; the reference evaluates it on its eager
// oracle (examples/varlen_causal_attention.py:46-48) and its only compiled
// streaming tile is dense/triangular fp16 forward (lib/Target/Triton/
// Translate.cpp:1603-1912).  Here it stays implicit (no materialized CSR).
//
// Layout: q, k, v, out, dout are [T, H, 128] bf16 (token-major); lse and
// delta are [T, H] fp32.
//
// MFMA: v_mfma_f32_16x16x32_bf16 with lane l, g = l / 16:
//   A[i = l % 16][k = 8g + j], B[k = 8g + j][n = l % 16], C[4g + r][n = l % 16].
// The forward computes S^T = K Q^T, so each lane's accumulators hold 4 keys of
// one query; two 16-key tiles together are exactly the B operand of
// O^T = V^T P^T under the key order {4g..4g+3, 16+4g..16+4g+3}, so P never
// leaves registers.  Operands needed "down a column" (V^T here, Q^T/dO^T/K^T
// in the backward) are read from row-major LDS tiles with ds_read_b64_tr_b16:
// inside each 16-lane group it returns lane i, element j = F[4j + i/4][i % 4]
// of the 4 x 16-bit values F[lane][0..3] the group's lanes address, so lane i'
// addressing X[r0 + i'/4][c0 + 4 (i' % 4)] receives X[r0 + j][c0 + i]; two such
// reads build the permuted 8-key A fragment.  Tiles are staged row-major with
// 16-byte writes, double-buffered, with the next tile's global loads in
// flight during the current tile's MFMAs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "tgx_device.h"
#include "tgx_host.h"
#include "tgx_profile.h"

namespace tgx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int VD = 128;    // head dim
constexpr int VBM = 128;   // queries per workgroup (4 waves x 32)
constexpr int VBN = 64;    // keys per iteration
// LDS row stride (bf16) of every staged tile: 288 B rows keep both the 16 B
// row-fragment reads and the transposing 8 B reads free of bank conflicts
// (measured: SQ_LDS_BANK_CONFLICT = 0).
constexpr int TPAD = 144;
constexpr int KPAD = TPAD;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// gfx950 (MI355X) has 8 XCDs, each with its own L2; workgroup i of a launch
// runs on XCD i % 8.
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4v mfma(bf16x8 a, bf16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const __bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

struct VarlenFwdArgs {
  const int32_t* cu;      // [n_seq + 1]
  const int32_t* tasks;   // [n_tasks, 4] = (sequence, first query, head, 0)
  int H;
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  __bf16* out;
  float* lse;             // [T, H]
  float scale_log2;       // softmax scale * log2(e)
};

// Stage one 64-key tile: thread t holds 4 rows x 16 B of K and of V.  Rows
// past the sequence end are clamped to its last row (finite values whose
// scores the causal mask removes), so the loads need no branches; every tile
// handed to a workgroup has at least one key (s1 > s0).
struct KvStage {
  bf16x8 k[4], v[4];
};

__device__ __forceinline__ void load_kv(KvStage& st, const __bf16* kb, const __bf16* vb,
                                        int64_t row_stride, int kbase, int s1) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int key = min(kbase + (idx >> 4), s1 - 1);
    const int64_t off = static_cast<int64_t>(key) * row_stride + (idx & 15) * 8;
    st.k[it] = ld_bf16x8(kb + off);
    st.v[it] = ld_bf16x8(vb + off);
  }
}

// Max / sum of a value over the four 16-lane groups (lanes l, l^16, l^32,
// l^48) with gfx950's row-swap permutes: with both operands equal, each swap
// hands every lane its partner's value in one of the two results.
__device__ __forceinline__ float group4_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 2^x on the hardware unit (v_exp_f32): exact 0 for -inf; results below the
// fp32 normal range flush to zero, which softmax weights tolerate.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// The running max is only moved when a tile's max exceeds it by more than
// this many (log2 units): weights then stay below 2^8, exact in the final
// normalisation, and the O rescale is skipped for nearly every tile.
constexpr float kRescaleLog2 = 8.f;

__device__ __forceinline__ void store_kv(const KvStage& st, __bf16 (*ks)[KPAD],
                                         __bf16 (*vs)[TPAD]) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int key = idx >> 4;
    const int dc = idx & 15;
    *reinterpret_cast<bf16x8*>(&ks[key][dc * 8]) = st.k[it];
    *reinterpret_cast<bf16x8*>(&vs[key][dc * 8]) = st.v[it];
  }
}

// A fragment of X^T (rows of X are the contraction index) from a row-major
// LDS tile X[row][col] with row stride TPAD: lane (lr, g) receives
// X[r0 + 4g + j][c0 + lr] for j < 4 and X[r0 + 16 + 4g + j - 4][c0 + lr] for
// j >= 4, i.e. 8 rows of one column in the permuted order of the B operand.
__device__ __forceinline__ bf16x8 tr_frag(__bf16 (*x)[TPAD], int r0, int c0, int lr, int g) {
  const __bf16* p = &x[r0 + 4 * g + (lr >> 2)][c0 + 4 * (lr & 3)];
  const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 16 * TPAD));
  // Assemble at dword granularity (elements 0-3 from a, 4-7 from b).
  const u32x2 aw = __builtin_bit_cast(u32x2, a);
  const u32x2 bw = __builtin_bit_cast(u32x2, b);
  const u32x4 w = {aw[0], aw[1], bw[0], bw[1]};
  return __builtin_bit_cast(bf16x8, w);
}

__global__ __launch_bounds__(256, 2) void varlen_fwd_kernel(VarlenFwdArgs a) {
  __shared__ __bf16 ks[2][VBN][KPAD];
  __shared__ __bf16 vs[2][VBN][TPAD];
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int seq = task[0];
  if (seq < 0) return;   // padding slot of a shorter XCD queue
  const int q0 = task[1];
  const int h = task[2];
  const int s0 = a.cu[seq], s1 = a.cu[seq + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t row_stride = static_cast<int64_t>(a.H) * VD;
  const __bf16* qh = a.q + h * VD;
  const __bf16* kh = a.k + h * VD;
  const __bf16* vh = a.v + h * VD;
  const int qb = q0 + wave * 32;

  // Q^T fragments (B operand): lane holds Q[q = qb + 16 qt + lr][32 ks + 8g .. +8].
  bf16x8 qf[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
      qf[qt][kc] = qq < s1 ? ld_bf16x8(qh + qq * row_stride + 32 * kc + 8 * g) : bf16x8{};
  }

  const int kv_end = (q0 + VBM < s1) ? q0 + VBM : s1;
  const int n_kv = (kv_end - s0 + VBN - 1) / VBN;
  const float sl2 = a.scale_log2;
  // Running max in scaled log2 units (-inf until a score is seen); lp is this
  // lane's share of the softmax denominator.
  float m[2] = {kNegInf, kNegInf};
  float lp[2] = {0.f, 0.f};
  // Last unmasked key of each query row (padded rows past s1 use s1 - 1).
  int qlim[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) qlim[qt] = min(qb + 16 * qt + lr, s1 - 1);
  f32x4v o[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[dt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};

  KvStage stage;
  load_kv(stage, kh, vh, row_stride, s0, s1);
  store_kv(stage, ks[0], vs[0]);
  for (int it = 0; it < n_kv; ++it) {
    __syncthreads();
    const int buf = it & 1;
    const int kbase = s0 + it * VBN;
    const bool more = it + 1 < n_kv;
    if (more) load_kv(stage, kh, vh, row_stride, kbase + VBN, s1);

    // A wave whose 32 queries all precede this key tile has nothing to add.
    if (kbase <= qb + 31) {
    // S^T = K Q^T over D = 128 (4 k-steps of 32).
    f32x4v c[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) c[kt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 kf = ld_bf16x8(&ks[buf][16 * kt + lr][32 * kc + 8 * g]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) c[kt][qt] = mfma(kf, qf[qt][kc], c[kt][qt]);
      }
    }

    // Causal/sequence mask (diagonal and last tiles only), then the tile max
    // of the raw scores (scale > 0, so scaling commutes with max).
    if (kbase + VBN > qb || kbase + VBN > s1) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kbase + 16 * kt + 4 * g + r > qlim[qt]) c[kt][qt][r] = kNegInf;
    }
    float mt[2];
    bool grow = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float x = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) x = fmaxf(x, c[kt][qt][r]);
      mt[qt] = group4_max(x) * sl2;
      grow |= mt[qt] > m[qt] + kRescaleLog2;
    }
    if (__any(grow)) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const float mn = fmaxf(m[qt], mt[qt]);
        const float alpha = mn == kNegInf ? 1.f : exp2_hw(m[qt] - mn);
        lp[qt] *= alpha;
        m[qt] = mn;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt][qt] *= alpha;
      }
    }
    bf16x8 pf[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float mo = m[qt] == kNegInf ? 0.f : m[qt];
      float p[4][4];
      float rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kt][r] = exp2_hw(c[kt][qt][r] * sl2 - mo);
          rs += p[kt][r];
        }
      lp[qt] += rs;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pf[qt][k2][j] = static_cast<__bf16>(p[2 * k2][j]);
          pf[qt][k2][4 + j] = static_cast<__bf16>(p[2 * k2 + 1][j]);
        }
    }

    // O^T += V^T P^T over the 64 keys (2 k-steps of 32).
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const bf16x8 vf = tr_frag(vs[buf], 32 * k2, 16 * dt, lr, g);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[dt][qt] = mfma(vf, pf[qt][k2], o[dt][qt]);
      }
    }
    }
    if (more) store_kv(stage, ks[buf ^ 1], vs[buf ^ 1]);
  }

  // Finalize: l summed over the 4 lane groups, O = O^T / l, natural-log lse.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l = group4_sum(lp[qt]);
    const int qq = qb + 16 * qt + lr;
    if (qq >= s1) continue;
    const float inv = 1.f / l;
    __bf16* orow = a.out + qq * row_stride + h * VD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      bf16x4 w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = static_cast<__bf16>(o[dt][qt][r] * inv);
      *reinterpret_cast<bf16x4*>(orow + 16 * dt + 4 * g) = w;
    }
    if (g == 0) a.lse[static_cast<int64_t>(qq) * a.H + h] = (m[qt] + __log2f(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Backward.  Three launches, no atomics:
//   delta[t, h] = <dout, out>;
//   dK/dV: one workgroup per 64-key tile (4 waves x 16 keys), looping over
//          64-query blocks q >= key; S = Q K^T and dP = dO V^T give P and dS
//          in C layout [q][key], which (two q-tiles, permuted) is directly the
//          B operand of dV^T = dO^T P and dK^T = Q^T dS;
//   dQ:    one workgroup per 128-query tile like the forward; S^T = K Q^T and
//          dP^T = V dO^T give dS^T, the B operand of dQ^T = K^T dS^T.
// dO^T, Q^T and K^T operands are staged transposed in LDS in the same
// permuted order as V^T in the forward.

struct VarlenBwdArgs {
  const int32_t* cu;
  const int32_t* tasks;   // [n_tasks, 4] = (sequence, first key or query, head, 0)
  int H;
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  const __bf16* dout;
  const float* lse;       // [T, H]
  const float* delta;     // [T, H]
  __bf16* dq;
  __bf16* dk;
  __bf16* dv;
  float scale;            // softmax scale
  float scale_log2;       // scale * log2(e)
};

__global__ __launch_bounds__(256) void varlen_delta_kernel(const __bf16* __restrict__ dout,
                                                           const __bf16* __restrict__ out,
                                                           float* __restrict__ delta,
                                                           int64_t T, int H) {
  // One wave per (token, group of 4 heads): lane l covers 8 elements of head
  // 4 * blockpart + l / 16.
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int groups = (H + 3) / 4;
  const int64_t t = wid / groups;
  const int hg = static_cast<int>(wid - t * groups);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  const int h = 4 * hg + (lane >> 4);
  float s = 0.f;
  if (h < H) {
    const int64_t off = (t * H + h) * VD + (lane & 15) * 8;
    const bf16x8 a = ld_bf16x8(dout + off);
    const bf16x8 b = ld_bf16x8(out + off);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += static_cast<float>(a[j]) * static_cast<float>(b[j]);
  }
  s = group_sum<16>(s);
  if (h < H && (lane & 15) == 0) delta[t * H + h] = s;
}

// Staging of one 64-row block of two [T, H, 128] tensors: thread t holds 4
// rows x 16 B of each (rows beyond `end` are zero).
struct Stage2 {
  bf16x8 a[4], b[4];
};

__device__ __forceinline__ void load2(Stage2& st, const __bf16* xa, const __bf16* xb,
                                      int64_t row_stride, int base, int end) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int row = idx >> 4;
    const int dc = idx & 15;
    if (base + row < end) {
      const int64_t off = static_cast<int64_t>(base + row) * row_stride + dc * 8;
      st.a[it] = ld_bf16x8(xa + off);
      st.b[it] = ld_bf16x8(xb + off);
    } else {
      st.a[it] = bf16x8{};
      st.b[it] = bf16x8{};
    }
  }
}

// Row-major copies of the two staged tensors (either may be skipped).
template <int SA, int SB>
__device__ __forceinline__ void store2(const Stage2& st, __bf16 (*ra)[SA], __bf16 (*rb)[SB]) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int row = idx >> 4;
    const int dc = idx & 15;
    *reinterpret_cast<bf16x8*>(&ra[row][dc * 8]) = st.a[it];
    *reinterpret_cast<bf16x8*>(&rb[row][dc * 8]) = st.b[it];
  }
}

// dK/dV: workgroup = (64-key tile, head); wave w owns keys k0 + 16w .. +16.
__global__ __launch_bounds__(256, 2) void varlen_dkdv_kernel(VarlenBwdArgs a) {
  __shared__ __bf16 qs[VBN][TPAD];    // Q rows of the query block
  __shared__ __bf16 dos[VBN][TPAD];   // dO rows
  __shared__ float lse_s[VBN], del_s[VBN];
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int seq = task[0];
  if (seq < 0) return;   // padding slot of a shorter XCD queue
  const int k0 = task[1];
  const int h = task[2];
  const int s1 = a.cu[seq + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t row_stride = static_cast<int64_t>(a.H) * VD;
  const int key = k0 + 16 * wave + lr;   // this lane's key (B operand column)

  // K^T and V^T fragments (B operands): K[key][32 kc + 8g .. +8].
  bf16x8 kf[4], vf[4];
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    if (key < s1) {
      kf[kc] = ld_bf16x8(a.k + key * row_stride + h * VD + 32 * kc + 8 * g);
      vf[kc] = ld_bf16x8(a.v + key * row_stride + h * VD + 32 * kc + 8 * g);
    } else {
      kf[kc] = bf16x8{};
      vf[kc] = bf16x8{};
    }
  }
  f32x4v dkt[8], dvt[8];   // dK^T / dV^T tiles [d = 16 dt + 4g + r][key]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    dkt[dt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    dvt[dt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  }
  const __bf16* qh = a.q + h * VD;
  const __bf16* doh = a.dout + h * VD;
  // Query blocks run last to first: every key tile of a (sequence, head)
  // starts on the sequence's last block, so tiles that run together (they
  // are queued together on one XCD) read each block at about the same time
  // and share it through L2.
  const int n_qb = (s1 - k0 + VBN - 1) / VBN;
  Stage2 st;
  load2(st, qh, doh, row_stride, k0 + (n_qb - 1) * VBN, s1);
  for (int step = 0; step < n_qb; ++step) {
    const int ib = n_qb - 1 - step;
    const int qbase = k0 + ib * VBN;
    __syncthreads();   // previous block's LDS reads are done
    store2<TPAD, TPAD>(st, qs, dos);
    if (threadIdx.x < VBN) {
      const int qq = qbase + threadIdx.x;
      lse_s[threadIdx.x] = qq < s1 ? a.lse[static_cast<int64_t>(qq) * a.H + h] * kLog2e
                                   : __builtin_huge_valf();
      del_s[threadIdx.x] = qq < s1 ? a.delta[static_cast<int64_t>(qq) * a.H + h] : 0.f;
    }
    __syncthreads();
    if (ib > 0) load2(st, qh, doh, row_stride, qbase - VBN, s1);
    // Keys of this wave that precede every query of the block all count;
    // a wave whose keys all exceed the block's last query skips it.
    if (k0 + 16 * wave > qbase + VBN - 1) continue;

    // S = Q K^T, dP = dO V^T: C tiles [q = 16 qt + 4g + r][key].
    f32x4v sc[4], dp[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      sc[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
      dp[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const bf16x8 qa = ld_bf16x8(&qs[16 * qt + lr][32 * kc + 8 * g]);
        const bf16x8 da = ld_bf16x8(&dos[16 * qt + lr][32 * kc + 8 * g]);
        sc[qt] = mfma(qa, kf[kc], sc[qt]);
        dp[qt] = mfma(da, vf[kc], dp[qt]);
      }
    }
    // P = exp(S*scale - lse), dS = P (dP - delta); packed per 32-query step.
    // Only the first block holds queries that precede keys of the tile, so
    // only it is masked (padded queries have lse = +inf, so P = 0).
    bf16x8 pb[2], sb[2];
    auto weights = [&](auto masked) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = 16 * qt + 4 * g + r;
          float p = exp2_hw(sc[qt][r] * a.scale_log2 - lse_s[qi]);
          if (decltype(masked)::value && qbase + qi < key) p = 0.f;
          const float ds = p * (dp[qt][r] - del_s[qi]);
          pb[qt >> 1][4 * (qt & 1) + r] = static_cast<__bf16>(p);
          sb[qt >> 1][4 * (qt & 1) + r] = static_cast<__bf16>(ds);
        }
      }
    };
    if (ib == 0)
      weights(std::true_type{});
    else
      weights(std::false_type{});
    // dV^T += dO^T P, dK^T += Q^T dS over the block's 64 queries.
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const bf16x8 ot = tr_frag(dos, 32 * k2, 16 * dt, lr, g);
        const bf16x8 qtv = tr_frag(qs, 32 * k2, 16 * dt, lr, g);
        dvt[dt] = mfma(ot, pb[k2], dvt[dt]);
        dkt[dt] = mfma(qtv, sb[k2], dkt[dt]);
      }
    }
  }
  if (key >= s1) return;
  __bf16* dkrow = a.dk + key * row_stride + h * VD;
  __bf16* dvrow = a.dv + key * row_stride + h * VD;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    bf16x4 wk, wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wk[r] = static_cast<__bf16>(dkt[dt][r] * a.scale);
      wv[r] = static_cast<__bf16>(dvt[dt][r]);
    }
    *reinterpret_cast<bf16x4*>(dkrow + 16 * dt + 4 * g) = wk;
    *reinterpret_cast<bf16x4*>(dvrow + 16 * dt + 4 * g) = wv;
  }
}

// dQ: workgroup = (128-query tile, head), wave w owns queries q0 + 32w .. +32.
__global__ __launch_bounds__(256, 2) void varlen_dq_kernel(VarlenBwdArgs a) {
  __shared__ __bf16 ks[VBN][TPAD];     // K rows of the key tile
  __shared__ __bf16 vs[VBN][KPAD];     // V rows
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int seq = task[0];
  if (seq < 0) return;   // padding slot of a shorter XCD queue
  const int q0 = task[1];
  const int h = task[2];
  const int s0 = a.cu[seq], s1 = a.cu[seq + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t row_stride = static_cast<int64_t>(a.H) * VD;
  const int qb = q0 + wave * 32;
  bf16x8 qf[2][4], df[2][4];
  float lse2[2], del[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
    const bool ok = qq < s1;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      qf[qt][kc] = ok ? ld_bf16x8(a.q + qq * row_stride + h * VD + 32 * kc + 8 * g) : bf16x8{};
      df[qt][kc] = ok ? ld_bf16x8(a.dout + qq * row_stride + h * VD + 32 * kc + 8 * g)
                      : bf16x8{};
    }
    lse2[qt] = ok ? a.lse[static_cast<int64_t>(qq) * a.H + h] * kLog2e : __builtin_huge_valf();
    del[qt] = ok ? a.delta[static_cast<int64_t>(qq) * a.H + h] : 0.f;
  }
  int qlim[2];         // last key each query row may see
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) qlim[qt] = min(qb + 16 * qt + lr, s1 - 1);
  f32x4v dqt[8][2];   // dQ^T [d = 16 dt + 4g + r][q]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const __bf16* kh = a.k + h * VD;
  const __bf16* vh = a.v + h * VD;
  const int kv_end = (q0 + VBM < s1) ? q0 + VBM : s1;
  const int n_kv = (kv_end - s0 + VBN - 1) / VBN;
  Stage2 st;
  load2(st, kh, vh, row_stride, s0, s1);
  for (int it = 0; it < n_kv; ++it) {
    const int kbase = s0 + it * VBN;
    __syncthreads();
    store2<TPAD, KPAD>(st, ks, vs);
    __syncthreads();
    if (it + 1 < n_kv) load2(st, kh, vh, row_stride, kbase + VBN, s1);
    if (kbase > qb + 31) continue;
    const bool edge_tile = kbase + VBN > qb || kbase + VBN > s1;
    // S^T = K Q^T and dP^T = V dO^T one 16-key subtile at a time (C tiles
    // [key = 16 kt + 4g + r][q]), turned straight into dS^T fragments.
    bf16x8 sb[2][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4v sc[2], dp[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        sc[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
        dp[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const bf16x8 ka = ld_bf16x8(&ks[16 * kt + lr][32 * kc + 8 * g]);
        const bf16x8 va = ld_bf16x8(&vs[16 * kt + lr][32 * kc + 8 * g]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          sc[qt] = mfma(ka, qf[qt][kc], sc[qt]);
          dp[qt] = mfma(va, df[qt][kc], dp[qt]);
        }
      }
      // Keys past a query (diagonal and last tiles only) get no weight;
      // padded queries have lse = +inf, so their P is 0.
      auto weights = [&](auto masked) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float p = exp2_hw(sc[qt][r] * a.scale_log2 - lse2[qt]);
            if (decltype(masked)::value && kbase + 16 * kt + 4 * g + r > qlim[qt]) p = 0.f;
            const float ds = p * (dp[qt][r] - del[qt]);
            sb[qt][kt >> 1][4 * (kt & 1) + r] = static_cast<__bf16>(ds);
          }
        }
      };
      if (edge_tile)
        weights(std::true_type{});
      else
        weights(std::false_type{});
    }
    // dQ^T += K^T dS^T.
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const bf16x8 kta = tr_frag(ks, 32 * k2, 16 * dt, lr, g);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = mfma(kta, sb[qt][k2], dqt[dt][qt]);
      }
    }
  }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
    if (qq >= s1) continue;
    __bf16* row = a.dq + qq * row_stride + h * VD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      bf16x4 w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = static_cast<__bf16>(dqt[dt][qt][r] * a.scale);
      *reinterpret_cast<bf16x4*>(row + 16 * dt + 4 * g) = w;
    }
  }
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_varlen_causal_tasks(const int32_t* cu_seqlens_host, int n_seq, int H,
                                       int block, int kind, int32_t* tasks_host,
                                       int64_t* n_tasks) {
  TGX_REQUIRE(cu_seqlens_host && n_tasks && n_seq >= 0 && H > 0 && block > 0,
              "bad arguments");
  TGX_REQUIRE(kind == 0 || kind == 1, "kind must be 0 (query tiles) or 1 (key tiles)");
  // Work of a tile: the causal keys a query tile sees, or the queries that
  // see a key tile.  A group is every tile of one (sequence, head).
  struct Group {
    int seq, head;
    int64_t work;
  };
  std::vector<Group> groups;
  for (int b = 0; b < n_seq; ++b) {
    const int s0 = cu_seqlens_host[b], s1 = cu_seqlens_host[b + 1];
    TGX_REQUIRE(s1 >= s0 && s0 >= 0, "cu_seqlens must be non-decreasing from 0");
    if (s1 == s0) continue;
    int64_t w = 0;
    for (int r0 = s0; r0 < s1; r0 += block)
      w += kind == 0 ? std::min(r0 + block, s1) - s0 : s1 - r0;
    for (int h = 0; h < H; ++h) groups.push_back(Group{b, h, w});
  }
  // Longest-processing-time assignment of groups to the XCDs (stable, so
  // ties keep sequence then head order).
  std::stable_sort(groups.begin(), groups.end(),
                   [](const Group& x, const Group& y) { return x.work > y.work; });
  std::vector<std::vector<int32_t>> queue(kXcds);
  int64_t load[kXcds] = {};
  for (const Group& gr : groups) {
    int x = 0;
    for (int i = 1; i < kXcds; ++i)
      if (load[i] < load[x]) x = i;
    load[x] += gr.work;
    const int s0 = cu_seqlens_host[gr.seq], s1 = cu_seqlens_host[gr.seq + 1];
    // Heaviest tile first: the last query tile, or the first key tile.
    const int n_t = (s1 - s0 + block - 1) / block;
    for (int t = 0; t < n_t; ++t) {
      const int r0 = kind == 0 ? s0 + (n_t - 1 - t) * block : s0 + t * block;
      queue[x].insert(queue[x].end(), {gr.seq, r0, gr.head, 0});
    }
  }
  size_t longest = 0;
  for (const auto& qx : queue) longest = std::max(longest, qx.size() / 4);
  const int64_t n = static_cast<int64_t>(longest) * kXcds;
  TGX_REQUIRE(n < (int64_t{1} << 31), "too many tasks");
  *n_tasks = n;
  if (tasks_host) {
    // Dispatch hands workgroup i to XCD i % 8: slot 8 i + x is XCD x's i-th
    // task, or padding (sequence -1) once its queue is exhausted.
    for (size_t i = 0; i < longest; ++i)
      for (int x = 0; x < kXcds; ++x) {
        int32_t* dst = tasks_host + 4 * (static_cast<int64_t>(i) * kXcds + x);
        if (4 * i < queue[x].size()) {
          for (int c = 0; c < 4; ++c) dst[c] = queue[x][4 * i + c];
        } else {
          dst[0] = -1;
          dst[1] = dst[2] = dst[3] = 0;
        }
      }
  }
  return TGX_OK;
}

extern "C" int tgx_varlen_causal_fwd(const int32_t* cu_seqlens_dev, const int32_t* tasks_dev,
                                     int64_t n_tasks, const void* q, const void* k,
                                     const void* v, float scale, void* out, float* lse,
                                     int64_t total_tokens, int H, int D, void* stream) {
  if (D != VD) {
    set_error("varlen causal attention supports head_dim 128 (got %d)", D);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(H > 0 && n_tasks >= 0 && total_tokens >= 0, "bad sizes");
  TGX_REQUIRE(total_tokens * H * VD < (int64_t{1} << 31), "tensor too large for 32-bit offsets");
  if (n_tasks == 0) return TGX_OK;
  TGX_REQUIRE(cu_seqlens_dev && tasks_dev && q && k && v && out && lse, "null pointer");
  TGX_REQUIRE(n_tasks < (int64_t{1} << 31), "too many tasks");
  hipStream_t s = as_stream(stream);
  VarlenFwdArgs a{cu_seqlens_dev, tasks_dev, H,
                  static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                  static_cast<const __bf16*>(v), static_cast<__bf16*>(out), lse,
                  scale * kLog2e};
  TGX_PROFILE("varlen_fwd_kernel", s);
  varlen_fwd_kernel<<<static_cast<unsigned>(n_tasks), 256, 0, s>>>(a);
  TGX_LAUNCHED("varlen_fwd_kernel");
  return TGX_OK;
}

extern "C" int tgx_varlen_causal_bwd(const int32_t* cu_seqlens_dev, const int32_t* q_tasks_dev,
                                     int64_t n_q_tasks, const int32_t* k_tasks_dev,
                                     int64_t n_k_tasks, const void* q, const void* k,
                                     const void* v, const void* out, const float* lse,
                                     const void* dout, float scale, void* dq, void* dk, void* dv,
                                     float* delta, int64_t total_tokens, int H, int D,
                                     void* stream) {
  if (D != VD) {
    set_error("varlen causal attention supports head_dim 128 (got %d)", D);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(H > 0 && n_q_tasks >= 0 && n_k_tasks >= 0 && total_tokens >= 0, "bad sizes");
  TGX_REQUIRE(n_q_tasks < (int64_t{1} << 31) && n_k_tasks < (int64_t{1} << 31),
              "too many tasks");
  TGX_REQUIRE(total_tokens * H * VD < (int64_t{1} << 31), "tensor too large for 32-bit offsets");
  if (total_tokens == 0) return TGX_OK;
  TGX_REQUIRE(cu_seqlens_dev && q_tasks_dev && k_tasks_dev && q && k && v && out && lse &&
                  dout && dq && dk && dv && delta,
              "null pointer");
  hipStream_t s = as_stream(stream);
  {
    TGX_PROFILE("varlen_delta_kernel", s);
    const int64_t waves = total_tokens * ((H + 3) / 4);
    varlen_delta_kernel<<<ceil_div(waves, 4), 256, 0, s>>>(
        static_cast<const __bf16*>(dout), static_cast<const __bf16*>(out), delta, total_tokens,
        H);
    TGX_LAUNCHED("varlen_delta_kernel");
  }
  VarlenBwdArgs a{cu_seqlens_dev, k_tasks_dev, H,
                  static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                  static_cast<const __bf16*>(v), static_cast<const __bf16*>(dout), lse, delta,
                  static_cast<__bf16*>(dq), static_cast<__bf16*>(dk), static_cast<__bf16*>(dv),
                  scale, scale * kLog2e};
  if (n_k_tasks > 0) {
    TGX_PROFILE("varlen_dkdv_kernel", s);
    varlen_dkdv_kernel<<<static_cast<unsigned>(n_k_tasks), 256, 0, s>>>(a);
    TGX_LAUNCHED("varlen_dkdv_kernel");
  }
  a.tasks = q_tasks_dev;
  if (n_q_tasks > 0) {
    TGX_PROFILE("varlen_dq_kernel", s);
    varlen_dq_kernel<<<static_cast<unsigned>(n_q_tasks), 256, 0, s>>>(a);
    TGX_LAUNCHED("varlen_dq_kernel");
  }
  return TGX_OK;
}
