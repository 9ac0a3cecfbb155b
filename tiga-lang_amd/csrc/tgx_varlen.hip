// Dense attention tiles on MFMA (gfx950, bf16 or fp16 in, fp32 accumulate)
// over block-diagonal relations: block k relates queries
// [cu_q[k], cu_q[k+1]) to keys [cu_k[k], cu_k[k+1]), either every pair
// (causal = false) or key <= query (causal = true, cu_q == cu_k).
//
// Relations covered (reference python/tiga/interop/torch/graph.py):
//   Graph.cu_seqlens(causal=True/False)  (:260-294)  varlen, cu_q = cu_k
//   Graph.dense(num_src, num_dst)        (:535-574)  one block, all pairs
//   Graph.triangular(n)                  (:576-592)  one block, key <= query
// The edge function is the dot-product score scale * q[i].k[j] with value
// v[j] under online softmax; the reference evaluates varlen on its eager
// oracle (examples/varlen_causal_attention.py) and dense/triangular with one
// compiled fp16 streaming forward tile (lib/Target/Triton/Translate.cpp:
// 1603-1912), whose optional block pruning (:1760-1860) this file restates.
// The relation stays implicit (no materialized CSR).
//
// Layout: q, k, v are [N, H, D] with element strides (sn, sh, 1), one pair
// for q and one shared by k and v (contiguous [N, H, D], or [H, N, D] storage
// viewed as [N, H, D]);
// out, dout, dq, dk, dv are contiguous [N, H, D]; lse and delta are [N, H]
// fp32.  D is 64 or 128.
//
// MFMA: v_mfma_f32_16x16x32_{bf16,f16} with lane l, g = l / 16:
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
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <typename T>
struct Vec;
template <>
struct Vec<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
};
template <>
struct Vec<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
};
template <typename T>
using vec8 = typename Vec<T>::v8;
template <typename T>
using vec4 = typename Vec<T>::v4;

constexpr int VBM = 128;   // queries per workgroup (4 waves x 32)
constexpr int VBN = 64;    // keys per iteration
// LDS row stride (elements) of every staged tile: 288 B rows keep both the
// 16 B row-fragment reads and the transposing 8 B reads free of bank
// conflicts (measured: SQ_LDS_BANK_CONFLICT = 0).  D = 64 uses the first half
// of each row.
constexpr int TPAD = 144;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// gfx950 (MI355X) has 8 XCDs, each with its own L2; workgroup i of a launch
// runs on XCD i % 8.
constexpr int kXcds = 8;

// Stored dS (the dK/dV kernel writes it, the dQ kernel reads it back instead
// of recomputing S and dP): 64 x 64 tiles per (block, head), query blocks qi
// and key blocks kj of 64 rows from the block's start; a causal (square)
// block keeps the tiles qi >= kj.  A tile is dS^T, row = key, 64 queries
// per row: the dK/dV lanes hold runs of four queries of one key, and the dQ
// kernel stages the rows in LDS and reads them down the key columns
// (ds_read_b64_tr_b16), as it reads K^T.
constexpr int kDsTile = 64 * 64;
__host__ __device__ inline int64_t ds_tiles(int64_t lq, int64_t lk, bool causal) {
  const int64_t nq = (lq + 63) / 64, nk = (lk + 63) / 64;
  return causal ? nq * (nq + 1) / 2 : nq * nk;
}
__host__ __device__ inline int64_t ds_tile(int qi, int kj, int nk, bool causal) {
  return causal ? static_cast<int64_t>(qi) * (qi + 1) / 2 + kj
                : static_cast<int64_t>(qi) * nk + kj;
}

__device__ __forceinline__ f32x4v mfma(bf16x8 a, bf16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4v mfma(f16x8 a, f16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ vec8<T> ld8(const T* p) {
  return *reinterpret_cast<const vec8<T>*>(p);
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

// MFMA clusters run at wave priority 1 (s_setprio) and the softmax work
// between them at 0: of the two waves sharing a SIMD, the one with MFMAs
// ready issues them back to back while the other fills the VALU (dK/dV
// 2.32 -> 2.26 ms on bench.py --config c5; forward and dQ unchanged).

// Staging of one 64-row block of two [N, H, D] tensors by 256 threads:
// thread t holds D / 32 chunks of 16 B of each.  Rows at or past `end` are
// clamped to row end - 1 (finite values the caller masks; every staged
// block has end > base) when CLAMP, else zero-filled.
template <typename T, int D>
struct Stage {
  static constexpr int N = D / 32;
  vec8<T> a[N], b[N];
};

// Row strides (elements) of the staged tensors stay below this, so a row's
// byte offset inside a 64-row block is one 24-bit multiply (checked by the
// entry points).
constexpr int64_t kMaxRowStride = (int64_t{1} << 24) / 8;

// The block's first row is a uniform address; each chunk is a 32-bit byte
// offset from it (local row x row bytes + column bytes, one v_mad_u32_u24),
// so the loads take the scalar-base form and no 64-bit address arithmetic
// runs per block.
template <typename T, int D, bool CLAMP>
__device__ __forceinline__ void stage_load(Stage<T, D>& st, const T* xa, int64_t sa,
                                           const T* xb, int64_t sb, int base, int end) {
  constexpr int CPR = D / 8;   // 16-byte chunks per row
  const char* ta = reinterpret_cast<const char*>(xa + static_cast<int64_t>(base) * sa);
  const char* tb = reinterpret_cast<const char*>(xb + static_cast<int64_t>(base) * sb);
  const uint32_t rba = static_cast<uint32_t>(sa) * sizeof(T);
  const uint32_t rbb = static_cast<uint32_t>(sb) * sizeof(T);
  const int last = end - 1 - base;   // last local row inside the tensor
#pragma unroll
  for (int it = 0; it < Stage<T, D>::N; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int r = idx / CPR;
    const uint32_t cb = static_cast<uint32_t>(idx % CPR) * 16;
    if (CLAMP || r <= last) {
      const uint32_t rr = static_cast<uint32_t>(CLAMP ? min(r, last) : r);
      st.a[it] = *reinterpret_cast<const vec8<T>*>(ta + (__umul24(rr, rba) + cb));
      st.b[it] = *reinterpret_cast<const vec8<T>*>(tb + (__umul24(rr, rbb) + cb));
    } else {
      st.a[it] = vec8<T>{};
      st.b[it] = vec8<T>{};
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ void stage_store(const Stage<T, D>& st, T (*ra)[TPAD],
                                            T (*rb)[TPAD]) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int it = 0; it < Stage<T, D>::N; ++it) {
    const int idx = threadIdx.x + 256 * it;
    *reinterpret_cast<vec8<T>*>(&ra[idx / CPR][(idx % CPR) * 8]) = st.a[it];
    *reinterpret_cast<vec8<T>*>(&rb[idx / CPR][(idx % CPR) * 8]) = st.b[it];
  }
}

// A fragment of X^T (rows of X are the contraction index) from a row-major
// LDS tile X[row][col] with row stride TPAD: lane (lr, g) receives
// X[r0 + 4g + j][c0 + lr] for j < 4 and X[r0 + 16 + 4g + j - 4][c0 + lr] for
// j >= 4, i.e. 8 rows of one column in the permuted order of the B operand.
template <typename T>
__device__ __forceinline__ vec8<T> tr_frag(T (*x)[TPAD], int r0, int c0, int lr, int g) {
  const T* p = &x[r0 + 4 * g + (lr >> 2)][c0 + 4 * (lr & 3)];
  const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 16 * TPAD));
  // Assemble at dword granularity (elements 0-3 from a, 4-7 from b).
  const u32x2 aw = __builtin_bit_cast(u32x2, a);
  const u32x2 bw = __builtin_bit_cast(u32x2, b);
  const u32x4 w = {aw[0], aw[1], bw[0], bw[1]};
  return __builtin_bit_cast(vec8<T>, w);
}

// ---------------------------------------------------------------------------
// Forward

template <typename T>
struct FwdArgs {
  const int32_t* cu_q;    // [n_blocks + 1] query ranges
  const int32_t* cu_k;    // [n_blocks + 1] key ranges
  const int32_t* tasks;   // [n_tasks, 4] = (block, first query, head, 0)
  int H;
  const T* q;
  const T* k;
  const T* v;
  int64_t qsn, qsh;       // element strides of q (token, head)
  int64_t ksn, ksh;       // element strides of k and v
  T* out;                 // [n_q, H, D]
  float* lse;             // [n_q, H]
  float scale_log2;       // softmax scale * log2(e)
  float prune_log2;       // log2(block_prune_threshold) (PRUNE only)
  // Split key ranges (chunk_tiles > 0): task[3] >= 0 is the partial slot of
  // a key chunk, which covers the tile's 64-key tiles [c, c + 1) *
  // chunk_tiles, c = slot % max_chunks, and writes its unnormalized O, its
  // running max and its sum to partial (kPartialFloats<D> per slot) for
  // varlen_fwd_merge_kernel; task[3] = -1 is a whole tile.
  int chunk_tiles;
  int max_chunks;
  float* partial;
};

// Floats of one key chunk's partial: O [128 queries][D], then the running
// max (scaled log2 units) and the sum per query.
template <int D>
constexpr int64_t kPartialFloats = static_cast<int64_t>(VBM) * (D + 2);

template <typename T, int D, bool CAUSAL, bool PRUNE>
__global__ __launch_bounds__(256, 2) void varlen_fwd_kernel(FwdArgs<T> a) {
  constexpr int KC = D / 32;   // contraction steps of S over D
  constexpr int DT = D / 16;   // 16-row tiles of O^T
  __shared__ T ks[2][VBN][TPAD];
  __shared__ T vs[2][VBN][TPAD];
  __shared__ float wave_max[PRUNE ? 4 : 1];
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int blk = task[0];
  if (blk < 0) return;   // padding slot of a shorter XCD queue
  const int q0 = task[1];
  const int h = task[2];
  const int qs1 = a.cu_q[blk + 1];
  const int ks0 = a.cu_k[blk], ks1 = a.cu_k[blk + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const T* qh = a.q + h * a.qsh;
  const T* kh = a.k + h * a.ksh;
  const T* vh = a.v + h * a.ksh;
  const int qb = q0 + wave * 32;

  // Q^T fragments (B operand): lane holds Q[q = qb + 16 qt + lr][32 kc + 8g .. +8].
  vec8<T> qf[2][KC];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      qf[qt][kc] = qq < qs1 ? ld8(qh + qq * a.qsn + 32 * kc + 8 * g) : vec8<T>{};
  }

  const int kv_end = CAUSAL ? min(q0 + VBM, ks1) : ks1;
  const int n_kv_all = (kv_end - ks0 + VBN - 1) / VBN;
  // The key tiles this task covers: all, or one chunk of them.
  const int slot = a.chunk_tiles > 0 ? task[3] : -1;
  const int it0 = slot >= 0 ? (slot % a.max_chunks) * a.chunk_tiles : 0;
  const int n_kv = slot >= 0 ? min(n_kv_all, it0 + a.chunk_tiles) : n_kv_all;
  const float sl2 = a.scale_log2;
  // Running max in scaled log2 units (-inf until a score is seen).
  float m[2] = {kNegInf, kNegInf};
  // Last key each query row may see (padded rows past the block use the
  // last key, their output is discarded).
  int qlim[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
    qlim[qt] = CAUSAL ? min(qb + 16 * qt + lr, ks1 - 1) : ks1 - 1;
  f32x4v o[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[dt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  // The softmax denominators: a row of ones times P^T on the MFMA (four
  // products per key tile in place of 32 adds per lane), every element of
  // lsum[qt] the sum over the tile's keys for query lr.  The sum is of the
  // same rounded weights that multiply V.
  f32x4v lsum[2] = {f32x4v{0.f, 0.f, 0.f, 0.f}, f32x4v{0.f, 0.f, 0.f, 0.f}};
  vec8<T> ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = static_cast<T>(1.f);
  // Running max over the whole workgroup tile (PRUNE), scaled log2 units.
  float block_m = kNegInf;

  Stage<T, D> stage;
  if (it0 < n_kv) {
    stage_load<T, D, true>(stage, kh, a.ksn, vh, a.ksn, ks0 + it0 * VBN, ks1);
    stage_store<T, D>(stage, ks[it0 & 1], vs[it0 & 1]);
  }
  for (int it = it0; it < n_kv; ++it) {
    __syncthreads();
    const int buf = it & 1;
    const int kbase = ks0 + it * VBN;
    const bool more = it + 1 < n_kv;
    if (more) stage_load<T, D, true>(stage, kh, a.ksn, vh, a.ksn, kbase + VBN, ks1);

    // A wave whose 32 queries all precede this key tile has nothing to add.
    const bool active = !CAUSAL || kbase <= qb + 31;
    f32x4v c[4][2];
    float mt[2] = {kNegInf, kNegInf};
    if (active) {
      // S^T = K Q^T over D (k-steps of 32).
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) c[kt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const vec8<T> kf = ld8(&ks[buf][16 * kt + lr][32 * kc + 8 * g]);
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) c[kt][qt] = mfma(kf, qf[qt][kc], c[kt][qt]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      // Causal/sequence mask (diagonal and last tiles only), then the tile
      // max of the raw scores (scale > 0, so scaling commutes with max).
      const bool edge = CAUSAL ? (kbase + VBN > qb || kbase + VBN > ks1) : kbase + VBN > ks1;
      if (edge) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (kbase + 16 * kt + 4 * g + r > qlim[qt]) c[kt][qt][r] = kNegInf;
      }
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        float x = kNegInf;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) x = fmaxf(x, c[kt][qt][r]);
        mt[qt] = group4_max(x) * sl2;
      }
    }
    bool admit = active;
    if constexpr (PRUNE) {
      // Tile admission (Translate.cpp:1793-1815): the tile's max over the
      // whole query block against the block's running max; a tile whose
      // best weight is below threshold x the best weight so far is skipped.
      const float wm = group_max<16>(fmaxf(mt[0], mt[1]));
      if (lane == 0) wave_max[wave] = wm;
      __syncthreads();
      const float tile_m =
          fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
      const bool skip = tile_m - block_m < a.prune_log2;
      if (!skip) block_m = fmaxf(block_m, tile_m);
      admit = admit && !skip;
    }
    if (admit) {
      bool grow = false;
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) grow |= mt[qt] > m[qt] + kRescaleLog2;
      if (__any(grow)) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          const float mn = fmaxf(m[qt], mt[qt]);
          const float alpha = mn == kNegInf ? 1.f : exp2_hw(m[qt] - mn);
          lsum[qt] *= alpha;
          m[qt] = mn;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[dt][qt] *= alpha;
        }
      }
      vec8<T> pf[2][2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const float mo = m[qt] == kNegInf ? 0.f : m[qt];
        float p[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) p[kt][r] = exp2_hw(c[kt][qt][r] * sl2 - mo);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            pf[qt][k2][j] = static_cast<T>(p[2 * k2][j]);
            pf[qt][k2][4 + j] = static_cast<T>(p[2 * k2 + 1][j]);
          }
      }
      // O^T += V^T P^T over the 64 keys (2 k-steps of 32).
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const vec8<T> vf = tr_frag(vs[buf], 32 * k2, 16 * dt, lr, g);
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) o[dt][qt] = mfma(vf, pf[qt][k2], o[dt][qt]);
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) lsum[qt] = mfma(ones, pf[qt][k2], lsum[qt]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    if (more) stage_store<T, D>(stage, ks[buf ^ 1], vs[buf ^ 1]);
  }

  if (slot >= 0) {
    // A key chunk: O^T (not normalized), the running max and the sum of
    // each of the tile's queries, for the merge.
    float* part = a.partial + static_cast<int64_t>(slot) * kPartialFloats<D>;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int qr = qb - q0 + 16 * qt + lr;   // query row in the tile
      if (qb + 16 * qt + lr >= qs1) continue;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4v*>(part + qr * D + 16 * dt + 4 * g) = o[dt][qt];
      if (g == 0) {
        part[VBM * D + qr] = m[qt];
        part[VBM * D + VBM + qr] = lsum[qt][0];
      }
    }
    return;
  }
  // Finalize: O = O^T / l, natural-log lse (a row that sees no key gets 0
  // and -inf).
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l = lsum[qt][0];
    const int qq = qb + 16 * qt + lr;
    if (qq >= qs1) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T* orow = a.out + (static_cast<int64_t>(qq) * a.H + h) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vec4<T> w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = static_cast<T>(o[dt][qt][r] * inv);
      *reinterpret_cast<vec4<T>*>(orow + 16 * dt + 4 * g) = w;
    }
    if (g == 0)
      a.lse[static_cast<int64_t>(qq) * a.H + h] = l > 0.f ? (m[qt] + __log2f(l)) * kLn2
                                                           : kNegInf;
  }
}

// Combine the key chunks of each split query tile (merge[m] = (block, first
// query, head, chunks), slots m * max_chunks + c) in chunk order: the
// largest running max M, l = sum_c l_c 2^(m_c - M), O = sum_c O_c 2^(m_c -
// M) / l; then out and lse as the whole-tile epilogue writes them.  A
// thread per (query, 4 features): kMergeBlocks<D> workgroups per split tile.
template <int D>
constexpr int kMergeBlocks = VBM * (D / 4) / 256;

template <typename T, int D>
__global__ __launch_bounds__(256) void varlen_fwd_merge_kernel(
    const int32_t* __restrict__ merge, const int32_t* __restrict__ cu_q, int H,
    int max_chunks, const float* __restrict__ partial, T* __restrict__ out,
    float* __restrict__ lse) {
  const int64_t mi = blockIdx.x / kMergeBlocks<D>;
  const int32_t* mt = merge + 4 * mi;
  const int blk = mt[0], q0 = mt[1], h = mt[2], nc = mt[3];
  const int qs1 = cu_q[blk + 1];
  const float* base = partial + mi * max_chunks * kPartialFloats<D>;
  constexpr int CPR = D / 4;   // 4-feature chunks per query row
  {
    const int w = (blockIdx.x % kMergeBlocks<D>) * 256 + threadIdx.x;
    const int qr = w / CPR, d4 = 4 * (w % CPR);
    const int qq = q0 + qr;
    if (qq >= qs1) return;
    float mx = kNegInf;
    for (int c = 0; c < nc; ++c) mx = fmaxf(mx, base[c * kPartialFloats<D> + VBM * D + qr]);
    float l = 0.f;
    f32x4v acc = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nc; ++c) {
      const float* pc = base + c * kPartialFloats<D>;
      const float mc = pc[VBM * D + qr];
      const float f = mc == kNegInf ? 0.f : exp2_hw(mc - mx);
      l += pc[VBM * D + VBM + qr] * f;
      acc += *reinterpret_cast<const f32x4v*>(pc + qr * D + d4) * f;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    vec4<T> wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[r] = static_cast<T>(acc[r] * inv);
    *reinterpret_cast<vec4<T>*>(out + (static_cast<int64_t>(qq) * H + h) * D + d4) = wv;
    if (d4 == 0)
      lse[static_cast<int64_t>(qq) * H + h] = l > 0.f ? (mx + __log2f(l)) * kLn2 : kNegInf;
  }
}

// ---------------------------------------------------------------------------
// Backward.  Three launches, no atomics:
//   delta[t, h] = <dout, out>;
//   dK/dV: one workgroup per 64-key tile (4 waves x 16 keys), looping over
//          64-query blocks (q >= key when causal); S = Q K^T and dP = dO V^T
//          give P and dS in C layout [q][key], which (two q-tiles, permuted)
//          is directly the B operand of dV^T = dO^T P and dK^T = Q^T dS;
//   dQ:    one workgroup per 128-query tile like the forward; S^T = K Q^T and
//          dP^T = V dO^T give dS^T, the B operand of dQ^T = K^T dS^T.
// dO^T, Q^T and K^T operands are staged transposed in LDS in the same
// permuted order as V^T in the forward.

template <typename T>
struct BwdArgs {
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* tasks;   // [n_tasks, 4] = (block, first key or query, head, 0)
  int H;
  const T* q;
  const T* k;
  const T* v;
  int64_t qsn, qsh;       // element strides of q
  int64_t ksn, ksh;       // element strides of k and v
  const T* dout;          // contiguous [n_q, H, D]
  const float* lse;       // [n_q, H]
  const float* delta;     // [n_q, H]
  T* dq;
  T* dk;
  T* dv;
  float scale;            // softmax scale
  float scale_log2;       // scale * log2(e)
  T* ds;                  // stored dS tiles (null: the dQ kernel recomputes)
};

template <typename T, int D>
__global__ __launch_bounds__(256) void varlen_delta_kernel(const T* __restrict__ dout,
                                                           const T* __restrict__ out,
                                                           float* __restrict__ delta,
                                                           int64_t n, int H) {
  // One wave per (token, group of heads): a head spans D / 8 lanes of 8
  // elements each.
  constexpr int LPH = D / 8;
  constexpr int HPW = kWave / LPH;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int groups = (H + HPW - 1) / HPW;
  const int64_t t = wid / groups;
  const int hg = static_cast<int>(wid - t * groups);
  if (t >= n) return;
  const int lane = threadIdx.x & 63;
  const int h = HPW * hg + lane / LPH;
  float s = 0.f;
  if (h < H) {
    const int64_t off = (t * H + h) * D + (lane % LPH) * 8;
    const vec8<T> x = ld8(dout + off);
    const vec8<T> y = ld8(out + off);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += static_cast<float>(x[j]) * static_cast<float>(y[j]);
  }
  s = group_sum<LPH>(s);
  if (h < H && lane % LPH == 0) delta[t * H + h] = s;
}

// dK/dV: workgroup = (64-key tile, head); wave w owns keys k0 + 16w .. +16.
// STORE: dS of every (query block, key tile) also goes to a.ds, the tiles of
// (block, head) from task[3].
template <typename T, int D, bool CAUSAL, bool STORE>
__global__ __launch_bounds__(256, 2) void varlen_dkdv_kernel(BwdArgs<T> a) {
  constexpr int KC = D / 32;
  constexpr int DT = D / 16;
  __shared__ T qs[VBN][TPAD];    // Q rows of the query block
  __shared__ T dos[VBN][TPAD];   // dO rows
  __shared__ float lse_s[VBN], del_s[VBN];
  // STORE: the block's dS^T tile, written to a.ds in the next step (or after
  // the loop) with full-row 16-byte stores.  Row stride 34 dwords: the 16
  // lanes an 8-byte LDS access serves together (16 rows, or two rows of 8
  // chunks) fall on 32 distinct banks.  (A 36-dword stride or a 16-byte
  // chunk swizzle gives 2-way conflicts on the writes.)
  constexpr int DSP = VBN + 4;
  __shared__ T dsw[STORE ? VBN : 1][STORE ? DSP : 1];
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int blk = task[0];
  if (blk < 0) return;   // padding slot of a shorter XCD queue
  const int k0 = task[1];
  const int h = task[2];
  const int qs0 = a.cu_q[blk], qs1 = a.cu_q[blk + 1];
  const int ks1 = a.cu_k[blk + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t cs = static_cast<int64_t>(a.H) * D;   // contiguous token stride
  const int key = k0 + 16 * wave + lr;   // this lane's key (B operand column)

  // K^T and V^T fragments (B operands): K[key][32 kc + 8g .. +8].
  vec8<T> kf[KC], vf[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    if (key < ks1) {
      kf[kc] = ld8(a.k + key * a.ksn + h * a.ksh + 32 * kc + 8 * g);
      vf[kc] = ld8(a.v + key * a.ksn + h * a.ksh + 32 * kc + 8 * g);
    } else {
      kf[kc] = vec8<T>{};
      vf[kc] = vec8<T>{};
    }
  }
  f32x4v dkt[DT], dvt[DT];   // dK^T / dV^T tiles [d = 16 dt + 4g + r][key]
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkt[dt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    dvt[dt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  }
  const T* qh = a.q + h * a.qsh;
  const T* doh = a.dout + h * D;
  // Queries that see the tile: from the tile's first key (causal) or the
  // block's first query.  Blocks run last to first: every key tile of a
  // (block, head) starts on the same last query block, so tiles that run
  // together (queued together on one XCD) read each block at about the same
  // time and share it through L2.
  const int qstart = CAUSAL ? k0 : qs0;
  const int n_qb = (qs1 - qstart + VBN - 1) / VBN;
  // Stored dS: this key tile's column of tiles, (qi, kj) for the blocks qi.
  const int ks0 = a.cu_k[blk];
  const int kj = (k0 - ks0) / VBN, nk = (ks1 - ks0 + VBN - 1) / VBN;
  T* const ds_blk = STORE ? a.ds + static_cast<int64_t>(task[3]) * kDsTile : nullptr;
  // The staged dS^T tile of query block qi (its 64 x 64 elements, thread t
  // the 16-byte chunks t and t + 256, each read as two 8-byte halves) to its
  // place in a.ds.
  auto flush_ds = [&](int qi) {
    T* tile = ds_blk + ds_tile(qi, kj, nk, CAUSAL) * kDsTile;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c >> 3, col = 8 * (c & 7);
      const vec4<T> lo = *reinterpret_cast<const vec4<T>*>(&dsw[row][col]);
      const vec4<T> hi = *reinterpret_cast<const vec4<T>*>(&dsw[row][col + 4]);
      *reinterpret_cast<vec8<T>*>(tile + row * VBN + col) =
          vec8<T>{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  // The block's Q/dO rows and its lse/delta are loaded one block ahead, all
  // before this block's dS stores: a wait for them then never waits for
  // the stores (vector memory counts complete in order).
  Stage<T, D> st;
  // Raw lse/delta of the next block's rows (rows past the block read the
  // last row; replaced when stored to LDS, so no use of the loaded values
  // comes before the stores).
  float lse_n = 0.f, del_n = 0.f;
  auto load_rows = [&](int qbase) {
    stage_load<T, D, false>(st, qh, a.qsn, doh, cs, qbase, qs1);
    if (threadIdx.x < VBN) {
      const int64_t qq = min(qbase + static_cast<int>(threadIdx.x), qs1 - 1);
      lse_n = a.lse[qq * a.H + h];
      del_n = a.delta[qq * a.H + h];
    }
  };
  if (n_qb > 0) load_rows(qstart + (n_qb - 1) * VBN);
  for (int step = 0; step < n_qb; ++step) {
    const int ib = n_qb - 1 - step;
    const int qbase = qstart + ib * VBN;
    __syncthreads();   // previous block's LDS reads are done
    if constexpr (STORE) {
      if (step > 0) flush_ds((qbase + VBN - qs0) / VBN);
    }
    stage_store<T, D>(st, qs, dos);
    if (threadIdx.x < VBN) {
      const bool ok = qbase + static_cast<int>(threadIdx.x) < qs1;
      lse_s[threadIdx.x] = ok ? lse_n * kLog2e : __builtin_huge_valf();
      del_s[threadIdx.x] = ok ? del_n : 0.f;
    }
    __syncthreads();
    if (ib > 0) load_rows(qbase - VBN);
    // (Causal blocks start at the tile's first key, so every wave has a key
    // at or before the block's last query: no wave skips a block.)

    // S = Q K^T, dP = dO V^T: C tiles [q = 16 qt + 4g + r][key].
    f32x4v sc[4], dp[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      sc[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
      dp[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const vec8<T> qa = ld8(&qs[16 * qt + lr][32 * kc + 8 * g]);
        const vec8<T> da = ld8(&dos[16 * qt + lr][32 * kc + 8 * g]);
        sc[qt] = mfma(qa, kf[kc], sc[qt]);
        dp[qt] = mfma(da, vf[kc], dp[qt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // P = exp(S*scale - lse), dS = P (dP - delta); packed per 32-query step.
    // Causal: only the first block holds queries that precede keys of the
    // tile, so only it is masked (padded queries have lse = +inf, so P = 0).
    vec8<T> pb[2], sb[2];
    auto weights = [&](auto masked) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = 16 * qt + 4 * g + r;
          float p = exp2_hw(sc[qt][r] * a.scale_log2 - lse_s[qi]);
          if (decltype(masked)::value && qbase + qi < key) p = 0.f;
          const float ds = p * (dp[qt][r] - del_s[qi]);
          pb[qt >> 1][4 * (qt & 1) + r] = static_cast<T>(p);
          sb[qt >> 1][4 * (qt & 1) + r] = static_cast<T>(ds);
        }
      }
    };
    if (CAUSAL && ib == 0)
      weights(std::true_type{});
    else
      weights(std::false_type{});
    if constexpr (STORE) {
      // dS^T row of this lane's key over the block's 64 queries, four
      // consecutive queries per 8-byte LDS write.  (Rows of keys past the
      // block hold P (0 - delta) of a zero K row; the dQ pass skips them.)
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        vec4<T> w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = sb[qt >> 1][4 * (qt & 1) + r];
        *reinterpret_cast<vec4<T>*>(&dsw[16 * wave + lr][16 * qt + 4 * g]) = w;
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS over the block's 64 queries.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const vec8<T> ot = tr_frag(dos, 32 * k2, 16 * dt, lr, g);
        const vec8<T> qtv = tr_frag(qs, 32 * k2, 16 * dt, lr, g);
        dvt[dt] = mfma(ot, pb[k2], dvt[dt]);
        dkt[dt] = mfma(qtv, sb[k2], dkt[dt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }
  if constexpr (STORE) {
    if (n_qb > 0) {
      __syncthreads();
      flush_ds((qstart - qs0) / VBN);
    }
  }
  if (key >= ks1) return;
  T* dkrow = a.dk + key * cs + h * D;
  T* dvrow = a.dv + key * cs + h * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    vec4<T> wk, wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wk[r] = static_cast<T>(dkt[dt][r] * a.scale);
      wv[r] = static_cast<T>(dvt[dt][r]);
    }
    *reinterpret_cast<vec4<T>*>(dkrow + 16 * dt + 4 * g) = wk;
    *reinterpret_cast<vec4<T>*>(dvrow + 16 * dt + 4 * g) = wv;
  }
}

// dQ: workgroup = (128-query tile, head), wave w owns queries q0 + 32w .. +32.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void varlen_dq_kernel(BwdArgs<T> a) {
  constexpr int KC = D / 32;
  constexpr int DT = D / 16;
  __shared__ T ks[VBN][TPAD];   // K rows of the key tile
  __shared__ T vs[VBN][TPAD];   // V rows
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int blk = task[0];
  if (blk < 0) return;   // padding slot of a shorter XCD queue
  const int q0 = task[1];
  const int h = task[2];
  const int qs1 = a.cu_q[blk + 1];
  const int ks0 = a.cu_k[blk], ks1 = a.cu_k[blk + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t cs = static_cast<int64_t>(a.H) * D;
  const int qb = q0 + wave * 32;
  vec8<T> qf[2][KC], df[2][KC];
  float lse2[2], del[2];
  int qlim[2];         // last key each query row may see
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
    const bool ok = qq < qs1;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      qf[qt][kc] = ok ? ld8(a.q + qq * a.qsn + h * a.qsh + 32 * kc + 8 * g) : vec8<T>{};
      df[qt][kc] = ok ? ld8(a.dout + qq * cs + h * D + 32 * kc + 8 * g) : vec8<T>{};
    }
    lse2[qt] = ok ? a.lse[static_cast<int64_t>(qq) * a.H + h] * kLog2e : __builtin_huge_valf();
    del[qt] = ok ? a.delta[static_cast<int64_t>(qq) * a.H + h] : 0.f;
    qlim[qt] = CAUSAL ? min(qq, ks1 - 1) : ks1 - 1;
  }
  f32x4v dqt[DT][2];   // dQ^T [d = 16 dt + 4g + r][q]
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const T* kh = a.k + h * a.ksh;
  const T* vh = a.v + h * a.ksh;
  const int kv_end = CAUSAL ? min(q0 + VBM, ks1) : ks1;
  const int n_kv = (kv_end - ks0 + VBN - 1) / VBN;
  Stage<T, D> st;
  // Key rows past the block are zero: their dS^T meets a zero K row, so
  // non-causal tiles need no mask.
  if (n_kv > 0) stage_load<T, D, false>(st, kh, a.ksn, vh, a.ksn, ks0, ks1);
  for (int it = 0; it < n_kv; ++it) {
    const int kbase = ks0 + it * VBN;
    __syncthreads();
    stage_store<T, D>(st, ks, vs);
    __syncthreads();
    if (it + 1 < n_kv) stage_load<T, D, false>(st, kh, a.ksn, vh, a.ksn, kbase + VBN, ks1);
    if (CAUSAL && kbase > qb + 31) continue;
    const bool edge_tile = CAUSAL && (kbase + VBN > qb || kbase + VBN > ks1);
    // S^T = K Q^T and dP^T = V dO^T one 16-key subtile at a time (C tiles
    // [key = 16 kt + 4g + r][q]), turned straight into dS^T fragments.
    vec8<T> sb[2][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4v sc[2], dp[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        sc[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
        dp[qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const vec8<T> ka = ld8(&ks[16 * kt + lr][32 * kc + 8 * g]);
        const vec8<T> va = ld8(&vs[16 * kt + lr][32 * kc + 8 * g]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          sc[qt] = mfma(ka, qf[qt][kc], sc[qt]);
          dp[qt] = mfma(va, df[qt][kc], dp[qt]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
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
            sb[qt][kt >> 1][4 * (kt & 1) + r] = static_cast<T>(ds);
          }
        }
      };
      if (edge_tile)
        weights(std::true_type{});
      else
        weights(std::false_type{});
    }
    // dQ^T += K^T dS^T.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const vec8<T> kta = tr_frag(ks, 32 * k2, 16 * dt, lr, g);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = mfma(kta, sb[qt][k2], dqt[dt][qt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
    if (qq >= qs1) continue;
    T* row = a.dq + qq * cs + h * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vec4<T> w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = static_cast<T>(dqt[dt][qt][r] * a.scale);
      *reinterpret_cast<vec4<T>*>(row + 16 * dt + 4 * g) = w;
    }
  }
}

// Staging of one 64-row block of one [N, H, D] tensor (K for the stored-dS
// dQ kernel); rows past `end` zero-filled.
template <typename T, int D>
struct Stage1 {
  static constexpr int N = D / 32;
  vec8<T> a[N];
};

template <typename T, int D>
__device__ __forceinline__ void stage1_load(Stage1<T, D>& st, const T* x, int64_t sx, int base,
                                            int end) {
  constexpr int CPR = D / 8;
  const char* t = reinterpret_cast<const char*>(x + static_cast<int64_t>(base) * sx);
  const uint32_t rb = static_cast<uint32_t>(sx) * sizeof(T);
  const int last = end - 1 - base;
#pragma unroll
  for (int it = 0; it < Stage1<T, D>::N; ++it) {
    const int idx = threadIdx.x + 256 * it;
    const int r = idx / CPR;
    const uint32_t cb = static_cast<uint32_t>(idx % CPR) * 16;
    st.a[it] = r <= last ? *reinterpret_cast<const vec8<T>*>(
                               t + (__umul24(static_cast<uint32_t>(r), rb) + cb))
                         : vec8<T>{};
  }
}

template <typename T, int D>
__device__ __forceinline__ void stage1_store(const Stage1<T, D>& st, T (*x)[TPAD]) {
  constexpr int CPR = D / 8;
#pragma unroll
  for (int it = 0; it < Stage1<T, D>::N; ++it) {
    const int idx = threadIdx.x + 256 * it;
    *reinterpret_cast<vec8<T>*>(&x[idx / CPR][(idx % CPR) * 8]) = st.a[it];
  }
}

// dQ from stored dS: workgroup = (128-query tile, head), wave w owns queries
// q0 + 32w .. +32, i.e. rows 32 (w % 2) .. +32 of query block qi0 + w / 2.
// Per 64-key tile: K and the two stored dS^T tiles (qi0, kj), (qi0 + 1, kj)
// staged in LDS (loaded one tile ahead), then dQ^T += K^T dS^T with both
// operands read down their key columns: one product per tile instead of
// three.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void varlen_dq_stored_kernel(BwdArgs<T> a) {
  constexpr int DT = D / 16;
  __shared__ T ks[VBN][TPAD];    // K rows of the key tile
  __shared__ T dss[VBN][TPAD];   // dS^T rows: keys x the workgroup's 128 queries
  const int32_t* task = a.tasks + 4 * static_cast<int64_t>(blockIdx.x);
  const int blk = task[0];
  if (blk < 0) return;   // padding slot of a shorter XCD queue
  const int q0 = task[1];
  const int h = task[2];
  const int qs0 = a.cu_q[blk], qs1 = a.cu_q[blk + 1];
  const int ks0 = a.cu_k[blk], ks1 = a.cu_k[blk + 1];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int64_t cs = static_cast<int64_t>(a.H) * D;
  const int qb = q0 + wave * 32;
  const int qi0 = (q0 - qs0) / VBN;
  const int nq = (qs1 - qs0 + VBN - 1) / VBN;
  const int nk = (ks1 - ks0 + VBN - 1) / VBN;
  const T* tiles = a.ds + static_cast<int64_t>(task[3]) * kDsTile;
  f32x4v dqt[DT][2];   // dQ^T [d = 16 dt + 4g + r][q]
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const T* kh = a.k + h * a.ksh;
  const int kv_end = CAUSAL ? min(q0 + VBM, ks1) : ks1;
  const int n_kv = (kv_end - ks0 + VBN - 1) / VBN;
  // Key tiles this wave has stored dS for (causal: those at or before its
  // query block; none when its queries all lie past the block).
  const int qi = qi0 + (wave >> 1);
  const int n_own = qb >= qs1 ? 0 : CAUSAL ? min(n_kv, qi + 1) : n_kv;
  // Staging of the two dS^T tiles: 2 x 64 rows x 128 B, four 16-byte
  // chunks per thread (chunk c: tile c / 512, row (c % 512) / 8, column
  // 8 (c % 8)); a tile that does not exist, and the rows of keys past the
  // block (written by the dK/dV pass but not zero), are zero-filled.
  vec8<T> dstage[4];
  auto ds_load = [&](int kj) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int t = c >> 9, row = (c & 511) >> 3, col = 8 * (c & 7);
      const int tq = qi0 + t;
      const bool ok = tq < nq && (!CAUSAL || kj <= tq) && ks0 + VBN * kj + row < ks1;
      dstage[i] = ok ? ld8(tiles + ds_tile(tq, kj, nk, CAUSAL) * kDsTile + row * VBN + col)
                     : vec8<T>{};
    }
  };
  auto ds_store = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int t = c >> 9, row = (c & 511) >> 3, col = 8 * (c & 7);
      *reinterpret_cast<vec8<T>*>(&dss[row][VBN * t + col]) = dstage[i];
    }
  };
  Stage1<T, D> st;
  if (n_kv > 0) {
    stage1_load<T, D>(st, kh, a.ksn, ks0, ks1);
    ds_load(0);
  }
  const int c0 = 32 * wave;   // this wave's first query column in dss
  for (int it = 0; it < n_kv; ++it) {
    const int kbase = ks0 + it * VBN;
    __syncthreads();
    stage1_store<T, D>(st, ks);
    ds_store();
    __syncthreads();
    if (it + 1 < n_kv) {
      stage1_load<T, D>(st, kh, a.ksn, kbase + VBN, ks1);
      ds_load(it + 1);
    }
    if (it >= n_own) continue;
    // dQ^T += K^T dS^T (key rows past the block are zero in ks and dss).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      vec8<T> sb[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) sb[qt] = tr_frag(dss, 32 * k2, c0 + 16 * qt, lr, g);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const vec8<T> kta = tr_frag(ks, 32 * k2, 16 * dt, lr, g);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) dqt[dt][qt] = mfma(kta, sb[qt], dqt[dt][qt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qq = qb + 16 * qt + lr;
    if (qq >= qs1) continue;
    T* row = a.dq + qq * cs + h * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vec4<T> w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = static_cast<T>(dqt[dt][qt][r] * a.scale);
      *reinterpret_cast<vec4<T>*>(row + 16 * dt + 4 * g) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// Launch helpers (dtype x head dim x causal x prune dispatch).

struct AttnShape {
  int64_t n_q, n_k;
  int H, D, dtype, causal;
  int64_t qsn, qsh, ksn, ksh;
};

int check_shape(const AttnShape& s) {
  if (s.D != 32 && s.D != 64 && s.D != 128) {
    set_error("dense attention tiles support head_dim 32, 64 and 128 (got %d)", s.D);
    return TGX_UNSUPPORTED;
  }
  if (s.dtype != TGX_DTYPE_BF16 && s.dtype != TGX_DTYPE_F16) {
    set_error("dense attention tiles support bf16 and fp16 (dtype code %d)", s.dtype);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(s.H > 0 && s.n_q >= 0 && s.n_k >= 0, "bad sizes");
  TGX_REQUIRE(s.qsn > 0 && s.qsh > 0 && s.ksn > 0 && s.ksh > 0, "strides must be positive");
  if (s.qsn >= kMaxRowStride || s.ksn >= kMaxRowStride ||
      static_cast<int64_t>(s.H) * s.D >= kMaxRowStride) {
    set_error("dense attention tiles need token strides below %lld elements",
              static_cast<long long>(kMaxRowStride));
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(s.n_q < (int64_t{1} << 31) && s.n_k < (int64_t{1} << 31),
              "token counts must fit int32");
  return TGX_OK;
}

template <typename T, int D>
int launch_fwd(const AttnShape& s, FwdArgs<T> a, int64_t n_tasks, bool prune,
               hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(n_tasks);
  TGX_PROFILE("varlen_fwd_kernel", stream);
  if (s.causal) {
    if (prune)
      varlen_fwd_kernel<T, D, true, true><<<grid, 256, 0, stream>>>(a);
    else
      varlen_fwd_kernel<T, D, true, false><<<grid, 256, 0, stream>>>(a);
  } else {
    if (prune)
      varlen_fwd_kernel<T, D, false, true><<<grid, 256, 0, stream>>>(a);
    else
      varlen_fwd_kernel<T, D, false, false><<<grid, 256, 0, stream>>>(a);
  }
  TGX_LAUNCHED("varlen_fwd_kernel");
  return TGX_OK;
}

template <typename T, int D>
int launch_bwd(const AttnShape& s, BwdArgs<T> a, const T* out, const int32_t* q_tasks,
               int64_t n_q_tasks, const int32_t* k_tasks, int64_t n_k_tasks, float* delta,
               hipStream_t stream) {
  {
    TGX_PROFILE("varlen_delta_kernel", stream);
    const int hpw = kWave / (D / 8);
    const int64_t waves = s.n_q * ((s.H + hpw - 1) / hpw);
    if (waves > 0) {
      varlen_delta_kernel<T, D><<<ceil_div(waves, 4), 256, 0, stream>>>(a.dout, out, delta,
                                                                         s.n_q, s.H);
      TGX_LAUNCHED("varlen_delta_kernel");
    }
  }
  a.delta = delta;
  const unsigned gk = static_cast<unsigned>(n_k_tasks), gq = static_cast<unsigned>(n_q_tasks);
  if (n_k_tasks > 0) {
    TGX_PROFILE("varlen_dkdv_kernel", stream);
    a.tasks = k_tasks;
    if (a.ds) {
      if (s.causal)
        varlen_dkdv_kernel<T, D, true, true><<<gk, 256, 0, stream>>>(a);
      else
        varlen_dkdv_kernel<T, D, false, true><<<gk, 256, 0, stream>>>(a);
    } else {
      if (s.causal)
        varlen_dkdv_kernel<T, D, true, false><<<gk, 256, 0, stream>>>(a);
      else
        varlen_dkdv_kernel<T, D, false, false><<<gk, 256, 0, stream>>>(a);
    }
    TGX_LAUNCHED("varlen_dkdv_kernel");
  }
  if (n_q_tasks > 0) {
    const char* dq_name = a.ds ? "varlen_dq_stored_kernel" : "varlen_dq_kernel";
    TGX_PROFILE(dq_name, stream);
    a.tasks = q_tasks;
    if (a.ds) {
      if (s.causal)
        varlen_dq_stored_kernel<T, D, true><<<gq, 256, 0, stream>>>(a);
      else
        varlen_dq_stored_kernel<T, D, false><<<gq, 256, 0, stream>>>(a);
    } else {
      if (s.causal)
        varlen_dq_kernel<T, D, true><<<gq, 256, 0, stream>>>(a);
      else
        varlen_dq_kernel<T, D, false><<<gq, 256, 0, stream>>>(a);
    }
    TGX_LAUNCHED(dq_name);
  }
  return TGX_OK;
}

// f(std::integral_constant<int, D>) for the head dims the tiles are built for
// (check_shape has admitted D).
template <typename F>
int with_head_dim(int D, F&& f) {
  if (D == 32) return f(std::integral_constant<int, 32>{});
  if (D == 64) return f(std::integral_constant<int, 64>{});
  return f(std::integral_constant<int, 128>{});
}

template <typename T>
int fwd_dtype(const AttnShape& s, const int32_t* cu_q, const int32_t* cu_k,
              const int32_t* tasks, int64_t n_tasks, const void* q, const void* k,
              const void* v, float scale, float prune, void* out, float* lse,
              hipStream_t stream) {
  FwdArgs<T> a{cu_q, cu_k, tasks, s.H,
               static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
               s.qsn, s.qsh, s.ksn, s.ksh, static_cast<T*>(out), lse, scale * kLog2e,
               prune > 0.f ? __builtin_log2f(prune) : 0.f};
  return with_head_dim(s.D, [&](auto dc) -> int {
    return launch_fwd<T, decltype(dc)::value>(s, a, n_tasks, prune > 0.f, stream);
  });
}

template <typename T>
int bwd_dtype(const AttnShape& s, const int32_t* cu_q, const int32_t* cu_k,
              const int32_t* q_tasks, int64_t n_q_tasks, const int32_t* k_tasks,
              int64_t n_k_tasks, const void* q, const void* k, const void* v, const void* out,
              const float* lse, const void* dout, float scale, void* dq, void* dk, void* dv,
              float* delta, void* ds, hipStream_t stream) {
  BwdArgs<T> a{cu_q, cu_k, nullptr, s.H,
               static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
               s.qsn, s.qsh, s.ksn, s.ksh, static_cast<const T*>(dout), lse, delta,
               static_cast<T*>(dq), static_cast<T*>(dk), static_cast<T*>(dv),
               scale, scale * kLog2e, static_cast<T*>(ds)};
  return with_head_dim(s.D, [&](auto dc) -> int {
    return launch_bwd<T, decltype(dc)::value>(s, a, static_cast<const T*>(out), q_tasks,
                                              n_q_tasks, k_tasks, n_k_tasks, delta, stream);
  });
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_attn_tasks(const int32_t* cu_q_host, const int32_t* cu_k_host, int n_blocks,
                              int H, int block, int kind, int causal, int32_t* tasks_host,
                              int64_t* n_tasks) {
  TGX_REQUIRE(cu_q_host && cu_k_host && n_tasks && n_blocks >= 0 && H > 0 && block > 0,
              "bad arguments");
  TGX_REQUIRE(kind == 0 || kind == 1, "kind must be 0 (query tiles) or 1 (key tiles)");
  // Work of a tile: the keys a query tile sees, or the queries that see a
  // key tile.  A group is every tile of one (block, head).
  struct Group {
    int blk, head;
    int64_t work;
    int64_t tile0;   // first stored dS tile of (block, head)
  };
  std::vector<Group> groups;
  int64_t tiles = 0;   // stored dS tiles of the blocks before b, all heads
  for (int b = 0; b < n_blocks; ++b) {
    const int q0 = cu_q_host[b], q1 = cu_q_host[b + 1];
    const int k0 = cu_k_host[b], k1 = cu_k_host[b + 1];
    TGX_REQUIRE(q1 >= q0 && q0 >= 0 && k1 >= k0 && k0 >= 0,
                "cu_seqlens must be non-decreasing from 0");
    TGX_REQUIRE(!causal || (q0 == k0 && q1 == k1), "causal blocks must be square");
    const int64_t nt = ds_tiles(q1 - q0, k1 - k0, causal != 0);
    const int64_t tile_b = tiles;
    tiles += nt * H;
    const int r0 = kind == 0 ? q0 : k0, r1 = kind == 0 ? q1 : k1;
    if (r1 == r0) continue;
    int64_t w = 0;
    for (int r = r0; r < r1; r += block) {
      const int end = std::min(r + block, r1);
      if (kind == 0)
        w += causal ? end - k0 : k1 - k0;
      else
        w += causal ? q1 - r : q1 - q0;
    }
    for (int h = 0; h < H; ++h)
      groups.push_back(Group{b, h, std::max<int64_t>(w, 1), tile_b + h * nt});
  }
  // Longest-processing-time assignment of groups to the XCDs (stable, so
  // ties keep block then head order).
  std::stable_sort(groups.begin(), groups.end(),
                   [](const Group& x, const Group& y) { return x.work > y.work; });
  std::vector<std::vector<int32_t>> queue(kXcds);
  int64_t load[kXcds] = {};
  for (const Group& gr : groups) {
    int x = 0;
    for (int i = 1; i < kXcds; ++i)
      if (load[i] < load[x]) x = i;
    load[x] += gr.work;
    const int r0 = kind == 0 ? cu_q_host[gr.blk] : cu_k_host[gr.blk];
    const int r1 = kind == 0 ? cu_q_host[gr.blk + 1] : cu_k_host[gr.blk + 1];
    // Heaviest tile first: causal query tiles from the last, key tiles from
    // the first (equal work otherwise: in order).
    const int n_t = (r1 - r0 + block - 1) / block;
    for (int t = 0; t < n_t; ++t) {
      const int tt = (kind == 0 && causal) ? n_t - 1 - t : t;
      // The dS tile offset fits int32 when the stored path can hold it
      // (tgx_attn_ds_tiles refuses more); past that it is unused.
      const int32_t t0 = gr.tile0 < (int64_t{1} << 31) ? static_cast<int32_t>(gr.tile0) : 0;
      queue[x].insert(queue[x].end(), {gr.blk, r0 + tt * block, gr.head, t0});
    }
  }
  size_t longest = 0;
  for (const auto& qx : queue) longest = std::max(longest, qx.size() / 4);
  const int64_t n = static_cast<int64_t>(longest) * kXcds;
  TGX_REQUIRE(n < (int64_t{1} << 31), "too many tasks");
  *n_tasks = n;
  if (tasks_host) {
    // Dispatch hands workgroup i to XCD i % 8: slot 8 i + x is XCD x's i-th
    // task, or padding (block -1) once its queue is exhausted.
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

extern "C" int tgx_attn_fwd_split_tasks(const int32_t* cu_q_host, const int32_t* cu_k_host,
                                        int n_blocks, int H, int causal, int slots,
                                        int32_t* tasks_host, int64_t* n_tasks,
                                        int32_t* merge_host, int64_t* n_merge,
                                        int32_t* chunk_tiles, int32_t* max_chunks) {
  TGX_REQUIRE(cu_q_host && cu_k_host && n_tasks && n_merge && chunk_tiles && max_chunks &&
                  n_blocks >= 0 && H > 0 && slots > 0,
              "bad arguments");
  // Key tiles (64 keys) each 128-query tile sees; their total over the
  // relation and heads spread over the resident workgroup slots is the
  // balanced load.  Tiles seeing more than that are split into chunks of
  // that many key tiles (when the longest tile is at least 5/4 of it).
  int64_t total = 0, longest = 0;
  for (int b = 0; b < n_blocks; ++b) {
    const int q0 = cu_q_host[b], q1 = cu_q_host[b + 1];
    const int k0 = cu_k_host[b], k1 = cu_k_host[b + 1];
    TGX_REQUIRE(q1 >= q0 && q0 >= 0 && k1 >= k0 && k0 >= 0,
                "cu_seqlens must be non-decreasing from 0");
    TGX_REQUIRE(!causal || (q0 == k0 && q1 == k1), "causal blocks must be square");
    for (int r = q0; r < q1; r += VBM) {
      const int kv_end = causal ? std::min(r + VBM, k1) : k1;
      const int64_t nk = (kv_end - k0 + VBN - 1) / VBN;
      total += nk * H;
      longest = std::max(longest, nk);
    }
  }
  const int64_t balanced = std::max<int64_t>((total + slots - 1) / slots, 8);
  const bool split = 4 * longest >= 5 * balanced;
  const int64_t chunk = split ? balanced : std::max<int64_t>(longest, 1);
  TGX_REQUIRE(chunk < (int64_t{1} << 31), "too many key tiles");
  const int64_t mc = (longest + chunk - 1) / chunk;
  *chunk_tiles = static_cast<int32_t>(chunk);
  *max_chunks = static_cast<int32_t>(std::max<int64_t>(mc, 1));
  // Tasks per (block, head) group, groups over the XCDs as in
  // tgx_attn_tasks; within a group the heaviest task first.
  struct Task4 {
    int64_t work;
    int32_t v[4];
  };
  struct Group {
    int blk, head;
    int64_t work;
  };
  std::vector<Group> groups;
  for (int b = 0; b < n_blocks; ++b) {
    const int q0 = cu_q_host[b], q1 = cu_q_host[b + 1], k0 = cu_k_host[b], k1 = cu_k_host[b + 1];
    if (q1 == q0) continue;
    int64_t w = 0;
    for (int r = q0; r < q1; r += VBM) w += causal ? std::min(r + VBM, k1) - k0 : k1 - k0;
    for (int h = 0; h < H; ++h) groups.push_back(Group{b, h, std::max<int64_t>(w, 1)});
  }
  std::stable_sort(groups.begin(), groups.end(),
                   [](const Group& x, const Group& y) { return x.work > y.work; });
  std::vector<std::vector<int32_t>> queue(kXcds);
  std::vector<int32_t> merges;
  int64_t load[kXcds] = {};
  for (const Group& gr : groups) {
    int x = 0;
    for (int i = 1; i < kXcds; ++i)
      if (load[i] < load[x]) x = i;
    load[x] += gr.work;
    const int q0 = cu_q_host[gr.blk], q1 = cu_q_host[gr.blk + 1];
    const int k0 = cu_k_host[gr.blk], k1 = cu_k_host[gr.blk + 1];
    std::vector<Task4> tasks;
    for (int r = q0; r < q1; r += VBM) {
      const int kv_end = causal ? std::min(r + VBM, k1) : k1;
      const int64_t nk = (kv_end - k0 + VBN - 1) / VBN;
      if (nk <= chunk) {
        tasks.push_back(Task4{std::max<int64_t>(nk, 1), {gr.blk, r, gr.head, -1}});
        continue;
      }
      const int64_t m = static_cast<int64_t>(merges.size()) / 4;
      const int64_t nc = (nk + chunk - 1) / chunk;
      TGX_REQUIRE((m + 1) * *max_chunks < (int64_t{1} << 31), "too many split tiles");
      merges.insert(merges.end(), {gr.blk, r, gr.head, static_cast<int32_t>(nc)});
      for (int64_t c = 0; c < nc; ++c)
        tasks.push_back(Task4{std::min(chunk, nk - c * chunk),
                              {gr.blk, r, gr.head, static_cast<int32_t>(m * *max_chunks + c)}});
    }
    std::stable_sort(tasks.begin(), tasks.end(),
                     [](const Task4& a, const Task4& b) { return a.work > b.work; });
    for (const Task4& t : tasks) queue[x].insert(queue[x].end(), t.v, t.v + 4);
  }
  size_t deepest = 0;
  for (const auto& qx : queue) deepest = std::max(deepest, qx.size() / 4);
  const int64_t n = static_cast<int64_t>(deepest) * kXcds;
  TGX_REQUIRE(n < (int64_t{1} << 31), "too many tasks");
  *n_tasks = n;
  *n_merge = static_cast<int64_t>(merges.size()) / 4;
  if (tasks_host) {
    for (size_t i = 0; i < deepest; ++i)
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
  if (merge_host) std::copy(merges.begin(), merges.end(), merge_host);
  return TGX_OK;
}

extern "C" int tgx_attn_fwd(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                            const int32_t* tasks_dev, int64_t n_tasks, int causal, int dtype,
                            const void* q, const void* k, const void* v, const int64_t* strides,
                            float scale, float prune_threshold, void* out, float* lse,
                            int64_t n_q, int64_t n_k, int H, int D, void* stream) {
  TGX_REQUIRE(strides, "null strides");
  const AttnShape s{n_q, n_k, H, D, dtype, causal != 0,
                    strides[0], strides[1], strides[2], strides[3]};
  int st = check_shape(s);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(!(prune_threshold < 0.f) && prune_threshold <= 1.f,
              "block_prune_threshold must be in (0, 1] (0 = exact)");
  TGX_REQUIRE(n_tasks >= 0 && n_tasks < (int64_t{1} << 31), "bad task count");
  if (n_tasks == 0) return TGX_OK;
  TGX_REQUIRE(cu_q_dev && cu_k_dev && tasks_dev && q && k && v && out && lse, "null pointer");
  hipStream_t hs = as_stream(stream);
  if (dtype == TGX_DTYPE_BF16)
    return fwd_dtype<__bf16>(s, cu_q_dev, cu_k_dev, tasks_dev, n_tasks, q, k, v, scale,
                             prune_threshold, out, lse, hs);
  return fwd_dtype<_Float16>(s, cu_q_dev, cu_k_dev, tasks_dev, n_tasks, q, k, v, scale,
                             prune_threshold, out, lse, hs);
}

extern "C" int tgx_attn_fwd_split(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                                  const int32_t* tasks_dev, int64_t n_tasks,
                                  const int32_t* merge_dev, int64_t n_merge,
                                  int32_t chunk_tiles, int32_t max_chunks, int causal, int dtype,
                                  const void* q, const void* k, const void* v,
                                  const int64_t* strides, float scale, void* out, float* lse,
                                  float* partial_dev, int64_t n_q, int64_t n_k, int H, int D,
                                  void* stream) {
  TGX_REQUIRE(strides, "null strides");
  const AttnShape s{n_q, n_k, H, D, dtype, causal != 0,
                    strides[0], strides[1], strides[2], strides[3]};
  int st = check_shape(s);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(n_tasks >= 0 && n_tasks < (int64_t{1} << 31), "bad task count");
  TGX_REQUIRE(n_merge >= 0 && chunk_tiles > 0 && max_chunks > 0 &&
                  n_merge * max_chunks < (int64_t{1} << 31) && n_merge < (int64_t{1} << 26),
              "bad split plan");
  if (n_tasks == 0) return TGX_OK;
  TGX_REQUIRE(cu_q_dev && cu_k_dev && tasks_dev && q && k && v && out && lse, "null pointer");
  TGX_REQUIRE(n_merge == 0 || (merge_dev && partial_dev), "split tiles need merge and partial");
  hipStream_t hs = as_stream(stream);
  auto run = [&](auto tag) -> int {
    typedef decltype(tag) T;
    FwdArgs<T> a{cu_q_dev, cu_k_dev, tasks_dev, s.H,
                 static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                 s.qsn, s.qsh, s.ksn, s.ksh, static_cast<T*>(out), lse, scale * kLog2e, 0.f,
                 chunk_tiles, max_chunks, partial_dev};
    return with_head_dim(D, [&](auto dc) -> int {
      constexpr int DD = decltype(dc)::value;
      const int r = launch_fwd<T, DD>(s, a, n_tasks, false, hs);
      if (r != TGX_OK || n_merge == 0) return r;
      TGX_PROFILE("varlen_fwd_merge_kernel", hs);
      const unsigned grid = static_cast<unsigned>(n_merge * kMergeBlocks<DD>);
      varlen_fwd_merge_kernel<T, DD><<<grid, 256, 0, hs>>>(
          merge_dev, cu_q_dev, s.H, max_chunks, partial_dev, static_cast<T*>(out), lse);
      TGX_LAUNCHED("varlen_fwd_merge_kernel");
      return TGX_OK;
    });
  };
  if (dtype == TGX_DTYPE_BF16) return run(__bf16{});
  return run(_Float16{});
}

extern "C" int tgx_attn_bwd(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                            const int32_t* q_tasks_dev, int64_t n_q_tasks,
                            const int32_t* k_tasks_dev, int64_t n_k_tasks, int causal,
                            int dtype, const void* q, const void* k, const void* v,
                            const int64_t* strides, const void* out, const float* lse,
                            const void* dout, float scale, void* dq, void* dk, void* dv,
                            float* delta, int64_t n_q, int64_t n_k, int H, int D,
                            void* stream) {
  TGX_REQUIRE(strides, "null strides");
  const AttnShape s{n_q, n_k, H, D, dtype, causal != 0,
                    strides[0], strides[1], strides[2], strides[3]};
  int st = check_shape(s);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(n_q_tasks >= 0 && n_k_tasks >= 0 && n_q_tasks < (int64_t{1} << 31) &&
                  n_k_tasks < (int64_t{1} << 31),
              "bad task count");
  if (n_q == 0 && n_k == 0) return TGX_OK;
  TGX_REQUIRE(cu_q_dev && cu_k_dev && q_tasks_dev && k_tasks_dev && q && k && v && out &&
                  lse && dout && dq && dk && dv && delta,
              "null pointer");
  hipStream_t hs = as_stream(stream);
  if (dtype == TGX_DTYPE_BF16)
    return bwd_dtype<__bf16>(s, cu_q_dev, cu_k_dev, q_tasks_dev, n_q_tasks, k_tasks_dev,
                             n_k_tasks, q, k, v, out, lse, dout, scale, dq, dk, dv, delta,
                             nullptr, hs);
  return bwd_dtype<_Float16>(s, cu_q_dev, cu_k_dev, q_tasks_dev, n_q_tasks, k_tasks_dev,
                             n_k_tasks, q, k, v, out, lse, dout, scale, dq, dk, dv, delta,
                             nullptr, hs);
}

extern "C" int tgx_attn_ds_tiles(const int32_t* cu_q_host, const int32_t* cu_k_host,
                                 int n_blocks, int H, int causal, int64_t* n_tiles) {
  TGX_REQUIRE(cu_q_host && cu_k_host && n_tiles && n_blocks >= 0 && H > 0, "bad arguments");
  int64_t tiles = 0;
  for (int b = 0; b < n_blocks; ++b) {
    const int64_t lq = int64_t{cu_q_host[b + 1]} - cu_q_host[b];
    const int64_t lk = int64_t{cu_k_host[b + 1]} - cu_k_host[b];
    TGX_REQUIRE(lq >= 0 && lk >= 0, "cu_seqlens must be non-decreasing");
    TGX_REQUIRE(!causal || lq == lk, "causal blocks must be square");
    tiles += ds_tiles(lq, lk, causal != 0) * H;
  }
  if (tiles >= (int64_t{1} << 31)) {
    set_error("%lld stored dS tiles exceed the task list's int32 offsets",
              static_cast<long long>(tiles));
    return TGX_UNSUPPORTED;
  }
  *n_tiles = tiles;
  return TGX_OK;
}

extern "C" int tgx_attn_bwd_stored(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                                   const int32_t* q_tasks_dev, int64_t n_q_tasks,
                                   const int32_t* k_tasks_dev, int64_t n_k_tasks, int causal,
                                   int dtype, const void* q, const void* k, const void* v,
                                   const int64_t* strides, const void* out, const float* lse,
                                   const void* dout, float scale, void* dq, void* dk, void* dv,
                                   float* delta, void* ds, int64_t n_q, int64_t n_k, int H,
                                   int D, void* stream) {
  TGX_REQUIRE(strides, "null strides");
  const AttnShape s{n_q, n_k, H, D, dtype, causal != 0,
                    strides[0], strides[1], strides[2], strides[3]};
  int st = check_shape(s);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(n_q_tasks >= 0 && n_k_tasks >= 0 && n_q_tasks < (int64_t{1} << 31) &&
                  n_k_tasks < (int64_t{1} << 31),
              "bad task count");
  if (n_q == 0 && n_k == 0) return TGX_OK;
  TGX_REQUIRE(cu_q_dev && cu_k_dev && q_tasks_dev && k_tasks_dev && q && k && v && out &&
                  lse && dout && dq && dk && dv && delta && ds,
              "null pointer");
  hipStream_t hs = as_stream(stream);
  if (dtype == TGX_DTYPE_BF16)
    return bwd_dtype<__bf16>(s, cu_q_dev, cu_k_dev, q_tasks_dev, n_q_tasks, k_tasks_dev,
                             n_k_tasks, q, k, v, out, lse, dout, scale, dq, dk, dv, delta, ds,
                             hs);
  return bwd_dtype<_Float16>(s, cu_q_dev, cu_k_dev, q_tasks_dev, n_q_tasks, k_tasks_dev,
                             n_k_tasks, q, k, v, out, lse, dout, scale, dq, dk, dv, delta, ds,
                             hs);
}
