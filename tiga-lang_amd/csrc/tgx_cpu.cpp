// CPU twins of the device entry points (declared in include/tgx_cpu.h).
//
// Plain C++17 over host memory: the same argument checks and status codes as
// the device entry points, the same row-plan walk (whole rows, split rows
// chunk by chunk with the chunk states merged in chunk order, empty rows),
// plus full checks of the CSR, the plan and the transposed CSR that a device
// launch cannot afford.  Threads take fixed contiguous ranges of plan
// positions, and the one cross-row reduction (GAT's da_src / da_dst) is
// summed in fp64 over a fixed number of row blocks, so results do not depend
// on the thread count.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <limits>
#include <new>
#include <system_error>
#include <thread>
#include <vector>

#include "tgx.h"
#include "tgx_check.h"
#include "tgx_cpu.h"

namespace tgx {
namespace {

constexpr float kInf = std::numeric_limits<float>::infinity();

std::atomic<int> g_threads{0};

int thread_count() {
  int t = g_threads.load(std::memory_order_relaxed);
  if (t <= 0) t = static_cast<int>(std::thread::hardware_concurrency());
  return t > 0 ? t : 1;
}

// f(lo, hi) over [0, n) in at most thread_count() contiguous ranges of at
// least `grain` items.
template <typename F>
void parallel_ranges(int64_t n, F f, int64_t grain = 64) {
  if (n <= 0) return;
  const int64_t t = std::min<int64_t>(thread_count(), std::max<int64_t>(1, n / grain));
  if (t <= 1) {
    f(int64_t{0}, n);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(static_cast<size_t>(t - 1));
  const int64_t per = (n + t - 1) / t;
  for (int64_t k = 1; k < t; ++k) {
    const int64_t lo = k * per, hi = std::min(n, lo + per);
    if (lo < hi) pool.emplace_back([=] { f(lo, hi); });
  }
  f(int64_t{0}, std::min(n, per));
  for (auto& th : pool) th.join();
}

// Runs an entry point body; C++ exceptions never cross the C ABI.
template <typename Body>
int guarded(Body body) {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    set_error("host allocation failed");
    return TGX_OUT_OF_MEMORY;
  } catch (const std::system_error& e) {
    set_error("thread start failed: %s", e.what());
    return TGX_INTERNAL;
  } catch (...) {
    set_error("unexpected exception");
    return TGX_INTERNAL;
  }
}

// Index arrays are int32 or int64 (idx_bits).
struct Idx {
  const void* p;
  int bits;
  int64_t operator[](int64_t i) const {
    return bits == 32 ? static_cast<const int32_t*>(p)[i] : static_cast<const int64_t*>(p)[i];
  }
};

// ---- 16-bit floating point storage ------------------------------------------

float bf16_to_float(uint16_t b) {
  const uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t float_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest, ties to even
  return static_cast<uint16_t>(u >> 16);
}

// IEEE binary16: 1 sign, 5 exponent (bias 15), 10 mantissa bits.
float f16_to_float(uint16_t h) {
  const int sign = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0)
    v = ldexpf(static_cast<float>(m), -24);
  else if (e == 31)
    v = m ? std::numeric_limits<float>::quiet_NaN() : kInf;
  else
    v = ldexpf(static_cast<float>(m | 0x400), e - 25);
  return sign ? -v : v;
}

uint16_t float_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (ax < 0x38800000u) {                                                // below 2^-14: subnormal
    float a;
    memcpy(&a, &ax, 4);
    return static_cast<uint16_t>(sign | static_cast<uint32_t>(nearbyintf(a * 16777216.0f)));
  }
  uint32_t r = ax - 0x38000000u;  // exponent bias 127 -> 15
  r += 0xfffu + ((r >> 13) & 1u);
  return static_cast<uint16_t>(sign | (r >> 13));
}

struct Half16 {
  int dtype;  // TGX_DTYPE_BF16 or TGX_DTYPE_F16
  float load(const uint16_t* p, int64_t i) const {
    return dtype == TGX_DTYPE_BF16 ? bf16_to_float(p[i]) : f16_to_float(p[i]);
  }
  uint16_t store(float v) const {
    return dtype == TGX_DTYPE_BF16 ? float_to_bf16(v) : float_to_f16(v);
  }
};

// ---- CSR and plan checks ------------------------------------------------------

// row_ptr [n_rows+1] starts at 0 and never decreases; *n_edges = row_ptr[n_rows];
// every column (when col is given) lies in [0, n_cols).
int check_csr(Idx rp, const Idx* col, int64_t n_rows, int64_t n_cols, int64_t* n_edges) {
  TGX_REQUIRE(rp.p, "null row_ptr");
  TGX_REQUIRE(rp[0] == 0, "row_ptr[0] must be 0 (got %lld)", static_cast<long long>(rp[0]));
  for (int64_t i = 0; i < n_rows; ++i)
    TGX_REQUIRE(rp[i + 1] >= rp[i], "row_ptr decreases at row %lld", static_cast<long long>(i));
  const int64_t E = rp[n_rows];
  if (col) {
    TGX_REQUIRE(E == 0 || col->p, "null col");
    for (int64_t e = 0; e < E; ++e) {
      const int64_t c = (*col)[e];
      TGX_REQUIRE(c >= 0 && c < n_cols, "col[%lld] = %lld outside [0, %lld)",
                  static_cast<long long>(e), static_cast<long long>(c),
                  static_cast<long long>(n_cols));
    }
  }
  if (n_edges) *n_edges = E;
  return TGX_OK;
}

// The plan's rows are a permutation of [0, n_rows) in three bins that match
// the degrees (0 | 1..wave_max | > wave_max) and the split rows' chunk
// offsets count ceil(degree / chunk_edges) chunks each.
int check_plan_rows(const tgx_row_plan* p, Idx rp, int64_t n_rows) {
  int st = check_plan(p, n_rows);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(p->wave_max > 0, "plan wave_max must be positive");
  std::vector<unsigned char> seen(static_cast<size_t>(n_rows), 0);
  const int32_t* rows = p->rows_dev;
  for (int64_t k = 0; k < n_rows; ++k) {
    const int64_t r = rows[k];
    TGX_REQUIRE(r >= 0 && r < n_rows, "plan row %lld out of range", static_cast<long long>(r));
    TGX_REQUIRE(!seen[r], "plan lists row %lld twice", static_cast<long long>(r));
    seen[r] = 1;
    const int64_t deg = rp[r + 1] - rp[r];
    const bool ok = k < p->n_empty ? deg == 0
                    : k < p->n_empty + p->n_wave ? deg >= 1 && deg <= p->wave_max
                                                 : deg > p->wave_max;
    TGX_REQUIRE(ok, "plan puts row %lld (degree %lld) in the wrong bin",
                static_cast<long long>(r), static_cast<long long>(deg));
  }
  if (p->n_split > 0) {
    const int32_t* off = p->chunk_offsets_dev;
    TGX_REQUIRE(off[0] == 0, "chunk_offsets[0] must be 0");
    for (int64_t k = 0; k < p->n_split; ++k) {
      const int64_t r = rows[p->n_empty + p->n_wave + k];
      const int64_t want = ceil_div(rp[r + 1] - rp[r], p->chunk_edges);
      TGX_REQUIRE(off[k + 1] - off[k] == want, "split row %lld needs %lld chunks",
                  static_cast<long long>(r), static_cast<long long>(want));
    }
    TGX_REQUIRE(off[p->n_split] == p->n_chunks, "n_chunks does not match chunk_offsets");
  } else {
    TGX_REQUIRE(p->n_chunks == 0, "chunks without split rows");
  }
  return TGX_OK;
}

// The transposed CSR of an E-edge relation with n_dst destinations: a CSR
// over n_src sources with columns in [0, n_dst), perm a permutation of the
// edge ids and inv_perm (when given) its inverse.
int check_transposed(const int32_t* rpt, const int32_t* colt, const int32_t* perm,
                     const int32_t* inv_perm, int64_t n_src, int64_t n_dst, int64_t* n_edges) {
  Idx r{rpt, 32}, c{colt, 32};
  int64_t E = 0;
  int st = check_csr(r, &c, n_src, n_dst, &E);
  if (st != TGX_OK) return st;
  if (E == 0) {
    *n_edges = 0;
    return TGX_OK;
  }
  TGX_REQUIRE(perm, "null perm");
  std::vector<unsigned char> seen(static_cast<size_t>(E), 0);
  for (int64_t k = 0; k < E; ++k) {
    const int64_t e = perm[k];
    TGX_REQUIRE(e >= 0 && e < E && !seen[e], "perm is not a permutation at %lld",
                static_cast<long long>(k));
    seen[e] = 1;
    if (inv_perm)
      TGX_REQUIRE(inv_perm[e] == k, "inv_perm[perm[%lld]] != %lld", static_cast<long long>(k),
                  static_cast<long long>(k));
  }
  *n_edges = E;
  return TGX_OK;
}

// ---- Plan walk ----------------------------------------------------------------

// Calls whole(row, e0, e1) for every non-empty row done in one piece,
// chunks(row, offsets of its chunks) for every split row, empty(row) for
// every empty row; plan positions are spread over the threads.
template <typename Whole, typename Split, typename Empty>
void walk_plan(const tgx_row_plan& p, Idx rp, Whole whole, Split split, Empty empty) {
  parallel_ranges(p.n_rows, [&](int64_t lo, int64_t hi) {
    for (int64_t k = lo; k < hi; ++k) {
      const int64_t row = p.rows_dev[k];
      if (k < p.n_empty) {
        empty(row);
      } else if (k < p.n_empty + p.n_wave) {
        whole(row, rp[row], rp[row + 1]);
      } else {
        const int64_t s = k - p.n_empty - p.n_wave;
        const int64_t rb = rp[row], re = rp[row + 1];
        std::vector<std::pair<int64_t, int64_t>> ranges;
        for (int64_t c = p.chunk_offsets_dev[s]; c < p.chunk_offsets_dev[s + 1]; ++c) {
          const int64_t e0 = rb + (c - p.chunk_offsets_dev[s]) * p.chunk_edges;
          ranges.emplace_back(e0, std::min(e0 + p.chunk_edges, re));
        }
        split(row, ranges);
      }
    }
  });
}

// Online softmax state of one (row, head): running max, sum and weighted sum.
struct Soft {
  float m = -kInf, l = 0.f;
  std::vector<float> acc;
  explicit Soft(int D) : acc(static_cast<size_t>(D), 0.f) {}
  void add(float s, const float* v) {
    if (s == -kInf) return;  // weight exp(-inf) = 0
    if (s > m) {
      const float c = m == -kInf ? 0.f : expf(m - s);
      l *= c;
      for (float& a : acc) a *= c;
      m = s;
    }
    const float p = expf(s - m);
    l += p;
    for (size_t d = 0; d < acc.size(); ++d) acc[d] += p * v[d];
  }
  void merge(const Soft& o) {
    if (o.m == -kInf) return;
    const float mm = std::max(m, o.m);
    const float a = m == -kInf ? 0.f : expf(m - mm), b = expf(o.m - mm);
    l = l * a + o.l * b;
    for (size_t d = 0; d < acc.size(); ++d) acc[d] = acc[d] * a + o.acc[d] * b;
    m = mm;
  }
};

float leaky(float z, float slope) { return z > 0.f ? z : z * slope; }

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_cpu_set_threads(int threads) {
  return g_threads.exchange(threads < 0 ? 0 : threads);
}

// ---- Graph construction and planning --------------------------------------------

extern "C" int tgx_cpu_destination_index(const void* row_ptr, int idx_bits, int64_t n_rows,
                                         int64_t n_edges, void* out, int out_bits) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(out_bits == 32 || out_bits == 64, "out_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0 && n_edges >= 0, "bad sizes");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits};
    int64_t E = 0;
    int st = check_csr(rp, nullptr, n_rows, 0, &E);
    if (st != TGX_OK) return st;
    TGX_REQUIRE(E == n_edges, "row_ptr[n_rows] = %lld, expected %lld edges",
                static_cast<long long>(E), static_cast<long long>(n_edges));
    TGX_REQUIRE(out_bits == 64 || n_rows <= INT32_MAX, "row ids need 64-bit output");
    TGX_REQUIRE(n_edges == 0 || out, "null out");
    parallel_ranges(n_rows, [&](int64_t lo, int64_t hi) {
      for (int64_t i = lo; i < hi; ++i)
        for (int64_t e = rp[i]; e < rp[i + 1]; ++e) {
          if (out_bits == 32)
            static_cast<int32_t*>(out)[e] = static_cast<int32_t>(i);
          else
            static_cast<int64_t*>(out)[e] = i;
        }
    });
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_csr_transpose(const void* row_ptr, const void* col, int idx_bits,
                                     int64_t n_dst, int64_t n_src, int64_t n_edges,
                                     int32_t* row_ptr_t, int32_t* col_t, int32_t* perm,
                                     int32_t* inv_perm) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_dst >= 0 && n_src >= 0 && n_edges >= 0, "bad sizes");
  TGX_REQUIRE(n_edges < (int64_t{1} << 31) && n_dst < (int64_t{1} << 31) &&
                  n_src < (int64_t{1} << 31),
              "the transposed CSR is int32: sizes must be below 2^31");
  TGX_REQUIRE(row_ptr_t, "null row_ptr_t");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    int64_t E = 0;
    int st = check_csr(rp, &c, n_dst, n_src, &E);
    if (st != TGX_OK) return st;
    TGX_REQUIRE(E == n_edges, "row_ptr[n_dst] = %lld, expected %lld edges",
                static_cast<long long>(E), static_cast<long long>(n_edges));
    TGX_REQUIRE(n_edges == 0 || (col_t && perm), "null output");
    // Counting sort by source, stable in edge order.
    std::vector<int64_t> count(static_cast<size_t>(n_src) + 1, 0);
    for (int64_t e = 0; e < E; ++e) ++count[c[e] + 1];
    for (int64_t j = 0; j < n_src; ++j) count[j + 1] += count[j];
    for (int64_t j = 0; j <= n_src; ++j) row_ptr_t[j] = static_cast<int32_t>(count[j]);
    for (int64_t i = 0; i < n_dst; ++i)
      for (int64_t e = rp[i]; e < rp[i + 1]; ++e) {
        const int64_t k = count[c[e]]++;
        col_t[k] = static_cast<int32_t>(i);
        perm[k] = static_cast<int32_t>(e);
        if (inv_perm) inv_perm[e] = static_cast<int32_t>(k);
      }
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_plan_degree_bins(const void* row_ptr, int idx_bits, int64_t n_rows,
                                        const int64_t* upper_bounds, int n_bins,
                                        int32_t* rows_out, int64_t* bin_offsets) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_bins >= 1 && n_bins <= 8, "n_bins must be in [1, 8]");
  TGX_REQUIRE(upper_bounds && bin_offsets, "null host pointer");
  TGX_REQUIRE(n_rows >= 0 && n_rows <= INT32_MAX, "n_rows must fit int32");
  for (int b = 1; b < n_bins; ++b)
    TGX_REQUIRE(upper_bounds[b] > upper_bounds[b - 1], "upper_bounds must ascend");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits};
    int st = check_csr(rp, nullptr, n_rows, 0, nullptr);
    if (st != TGX_OK) return st;
    TGX_REQUIRE(n_rows == 0 || rows_out, "null rows_out");
    std::vector<int> bin(static_cast<size_t>(n_rows));
    std::vector<int64_t> count(static_cast<size_t>(n_bins) + 1, 0);
    for (int64_t i = 0; i < n_rows; ++i) {
      const int64_t deg = rp[i + 1] - rp[i];
      const int b = static_cast<int>(
          std::lower_bound(upper_bounds, upper_bounds + n_bins, deg) - upper_bounds);
      TGX_REQUIRE(b < n_bins, "row %lld has degree %lld above the last bound %lld",
                  static_cast<long long>(i), static_cast<long long>(deg),
                  static_cast<long long>(upper_bounds[n_bins - 1]));
      bin[i] = b;
      ++count[b + 1];
    }
    for (int b = 0; b < n_bins; ++b) count[b + 1] += count[b];
    for (int b = 0; b <= n_bins; ++b) bin_offsets[b] = count[b];
    for (int64_t i = 0; i < n_rows; ++i) rows_out[count[bin[i]]++] = static_cast<int32_t>(i);
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_plan_split_chunks(const void* row_ptr, int idx_bits,
                                         const int32_t* split_rows, int64_t n_split,
                                         int32_t chunk_edges, int32_t* chunk_offsets,
                                         int64_t* n_chunks) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_split >= 0 && chunk_edges > 0, "bad sizes");
  TGX_REQUIRE(row_ptr && chunk_offsets && n_chunks && (split_rows || n_split == 0),
              "null pointer");
  const Idx rp{row_ptr, idx_bits};
  int64_t total = 0;
  chunk_offsets[0] = 0;
  for (int64_t k = 0; k < n_split; ++k) {
    const int64_t r = split_rows[k];
    TGX_REQUIRE(r >= 0, "negative split row");
    total += ceil_div(rp[r + 1] - rp[r], chunk_edges);
    TGX_REQUIRE(total <= INT32_MAX, "more than 2^31 chunks");
    chunk_offsets[k + 1] = static_cast<int32_t>(total);
  }
  *n_chunks = total;
  return TGX_OK;
}

// ---- Weighted sum -----------------------------------------------------------------

namespace {

// Feature storage of the sum (x, out, dout, dx) by dtype code.
struct Feat {
  int dtype;
  float load(const void* p, int64_t i) const {
    if (dtype == TGX_DTYPE_F32) return static_cast<const float*>(p)[i];
    return Half16{dtype}.load(static_cast<const uint16_t*>(p), i);
  }
  void store(void* p, int64_t i, float v) const {
    if (dtype == TGX_DTYPE_F32)
      static_cast<float*>(p)[i] = v;
    else
      static_cast<uint16_t*>(p)[i] = Half16{dtype}.store(v);
  }
};

int check_sum_dtype(int dtype) {
  if (dtype != TGX_DTYPE_F32 && dtype != TGX_DTYPE_BF16 && dtype != TGX_DTYPE_F16) {
    set_error("sum supports fp32, bf16 and fp16 features (dtype code %d)", dtype);
    return TGX_UNSUPPORTED;
  }
  return TGX_OK;
}

}  // namespace

extern "C" int tgx_cpu_csr_sum_fwd(const void* row_ptr, const void* col, int idx_bits,
                                   const tgx_row_plan* plan, const void* x, const float* w,
                                   void* out, int64_t n_dst, int64_t n_src, int64_t F,
                                   int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  int st = check_sum_dtype(dtype);
  if (st != TGX_OK) return st;
  st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && out && (x || n_src == 0), "null pointer");
  TGX_REQUIRE(col || n_src < (int64_t{1} << 31), "edge-id columns need fewer than 2^31 edges");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    const Feat ft{dtype};
    int64_t E = 0;
    int s = check_csr(rp, col ? &c : nullptr, n_dst, n_src, &E);
    if (s != TGX_OK) return s;
    TGX_REQUIRE(col || E == n_src, "edge-id columns need x with one row per edge");
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    auto range = [&](int64_t e0, int64_t e1, float* acc) {
      for (int64_t e = e0; e < e1; ++e) {
        const float we = w ? w[e] : 1.f;
        const int64_t base = (col ? c[e] : e) * F;
        for (int64_t f = 0; f < F; ++f) acc[f] += we * ft.load(x, base + f);
      }
    };
    auto store = [&](int64_t row, const float* acc) {
      for (int64_t f = 0; f < F; ++f) ft.store(out, row * F + f, acc[f]);
    };
    walk_plan(
        *plan, rp,
        [&](int64_t row, int64_t e0, int64_t e1) {
          std::vector<float> acc(static_cast<size_t>(F), 0.f);
          range(e0, e1, acc.data());
          store(row, acc.data());
        },
        [&](int64_t row, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> acc(static_cast<size_t>(F), 0.f), part(acc.size());
          for (const auto& ch : chunks) {
            std::fill(part.begin(), part.end(), 0.f);
            range(ch.first, ch.second, part.data());
            for (int64_t f = 0; f < F; ++f) acc[f] += part[f];
          }
          store(row, acc.data());
        },
        [&](int64_t row) {
          for (int64_t f = 0; f < F; ++f) ft.store(out, row * F + f, 0.f);
        });
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_csr_sum_bwd(const int32_t* row_ptr_t, const int32_t* col_t,
                                   const int32_t* perm, const tgx_row_plan* plan_t,
                                   const void* x, const float* w, const void* dout, void* dx,
                                   float* dw, int64_t n_dst, int64_t n_src, int64_t F,
                                   int dtype) {
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  int st = check_sum_dtype(dtype);
  if (st != TGX_OK) return st;
  st = check_plan(plan_t, n_src);
  if (st != TGX_OK) return st;
  if (n_src == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr_t && dout, "null pointer");
  TGX_REQUIRE(!dw || x, "dw needs x");
  return guarded([&]() -> int {
    int64_t E = 0;
    int s = check_transposed(row_ptr_t, col_t, perm, nullptr, n_src, n_dst, &E);
    if (s != TGX_OK) return s;
    const Idx rpt{row_ptr_t, 32};
    const Feat ft{dtype};
    s = check_plan_rows(plan_t, rpt, n_src);
    if (s != TGX_OK) return s;
    auto range = [&](int64_t j, int64_t e0, int64_t e1, float* acc) {
      for (int64_t k = e0; k < e1; ++k) {
        const int64_t e = perm[k];
        const int64_t gb = static_cast<int64_t>(col_t[k]) * F;
        if (acc) {
          const float we = w ? w[e] : 1.f;
          for (int64_t f = 0; f < F; ++f) acc[f] += we * ft.load(dout, gb + f);
        }
        if (dw) {
          float d = 0.f;
          for (int64_t f = 0; f < F; ++f) d += ft.load(dout, gb + f) * ft.load(x, j * F + f);
          dw[e] = d;
        }
      }
    };
    auto store = [&](int64_t j, const float* acc) {
      if (dx)
        for (int64_t f = 0; f < F; ++f) ft.store(dx, j * F + f, acc[f]);
    };
    walk_plan(
        *plan_t, rpt,
        [&](int64_t j, int64_t e0, int64_t e1) {
          std::vector<float> acc(static_cast<size_t>(F), 0.f);
          range(j, e0, e1, dx ? acc.data() : nullptr);
          store(j, acc.data());
        },
        [&](int64_t j, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> acc(static_cast<size_t>(F), 0.f), part(acc.size());
          for (const auto& ch : chunks) {
            std::fill(part.begin(), part.end(), 0.f);
            range(j, ch.first, ch.second, dx ? part.data() : nullptr);
            for (int64_t f = 0; f < F; ++f) acc[f] += part[f];
          }
          store(j, acc.data());
        },
        [&](int64_t j) {
          const std::vector<float> zero(static_cast<size_t>(F), 0.f);
          store(j, zero.data());
        });
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_csr_edge_dot(const void* row_ptr, const void* col, int idx_bits,
                                    const tgx_row_plan* plan, const void* x, const void* dout,
                                    float* dw, int64_t n_dst, int64_t n_src, int64_t F,
                                    int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(F > 0 && n_dst >= 0 && n_src >= 0, "bad sizes");
  int st = check_sum_dtype(dtype);
  if (st != TGX_OK) return st;
  if (F > 32) {
    set_error("tgx_csr_edge_dot covers F <= 32 (got %lld); wider rows take the dw output "
              "of tgx_csr_sum_bwd", static_cast<long long>(F));
    return TGX_UNSUPPORTED;
  }
  st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && col && x && dout && dw, "null pointer");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    const Feat ft{dtype};
    int s = check_csr(rp, &c, n_dst, n_src, nullptr);
    if (s != TGX_OK) return s;
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    auto range = [&](int64_t i, int64_t e0, int64_t e1) {
      for (int64_t e = e0; e < e1; ++e) {
        float d = 0.f;
        for (int64_t f = 0; f < F; ++f) d += ft.load(dout, i * F + f) * ft.load(x, c[e] * F + f);
        dw[e] = d;
      }
    };
    walk_plan(
        *plan, rp, [&](int64_t i, int64_t e0, int64_t e1) { range(i, e0, e1); },
        [&](int64_t i, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          for (const auto& ch : chunks) range(i, ch.first, ch.second);
        },
        [](int64_t) {});
    return TGX_OK;
  });
}

// ---- Element types ------------------------------------------------------------------

namespace {

// One element type of the q/k/v/out/dout/dq/dk/dv tensors, read as fp32 and
// written with one round-to-nearest-even.
struct Elem {
  int dtype;  // TGX_DTYPE_*
  float get(const void* base, int64_t i) const {
    if (dtype == TGX_DTYPE_F32) return static_cast<const float*>(base)[i];
    return Half16{dtype}.load(static_cast<const uint16_t*>(base), i);
  }
  void put(void* base, int64_t i, float v) const {
    if (dtype == TGX_DTYPE_F32)
      static_cast<float*>(base)[i] = v;
    else
      static_cast<uint16_t*>(base)[i] = Half16{dtype}.store(v);
  }
};

bool elem_ok(int dtype) {
  return dtype == TGX_DTYPE_BF16 || dtype == TGX_DTYPE_F16 || dtype == TGX_DTYPE_F32;
}

// n values of `base` widened to fp32.
std::vector<float> widen_all(const Elem& el, const void* base, int64_t n) {
  std::vector<float> v(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) v[i] = el.get(base, i);
  return v;
}

void round_all(const Elem& el, const std::vector<float>& v, void* base) {
  for (size_t i = 0; i < v.size(); ++i) el.put(base, static_cast<int64_t>(i), v[i]);
}

}  // namespace

// ---- GAT additive attention -------------------------------------------------------

extern "C" int tgx_cpu_gat_fwd(const void* row_ptr, const void* col, int idx_bits,
                               const tgx_row_plan* plan, const void* h_src, const void* h_dst,
                               const float* a_src, const float* a_dst, float slope, void* out,
                               float* ns, int64_t n_dst, int64_t n_src, int H, int D,
                               int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(elem_ok(dtype), "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)", dtype);
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
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    int s = check_csr(rp, &c, n_dst, n_src, nullptr);
    if (s != TGX_OK) return s;
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    const int64_t HD = static_cast<int64_t>(H) * D;
    const Elem el{dtype};
    const std::vector<float> hs = widen_all(el, h_src, n_src * HD);
    const std::vector<float> hd_own = h_src == h_dst ? std::vector<float>()
                                                     : widen_all(el, h_dst, n_dst * HD);
    const float* HS = hs.data();
    const float* HDv = h_src == h_dst ? hs.data() : hd_own.data();
    // a . h per (node, head): a_src over the sources, a_dst and a_src over the
    // destinations (node state slots 2 and 3).
    auto half = [&](const float* rows, const float* a, int64_t n) {
      std::vector<float> z(static_cast<size_t>(n * H));
      parallel_ranges(n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i)
          for (int hd = 0; hd < H; ++hd) {
            float acc = 0.f;
            for (int d = 0; d < D; ++d) acc += a[hd * D + d] * rows[i * HD + hd * D + d];
            z[i * H + hd] = acc;
          }
      });
      return z;
    };
    const std::vector<float> zs = half(HS, a_src, n_src), zd = half(HDv, a_dst, n_dst),
                             zsd = half(HDv, a_src, n_dst);
    std::vector<float> o32(static_cast<size_t>(n_dst * HD));
    auto state = [&](int64_t i, int hd, int64_t e0, int64_t e1) {
      Soft st(D);
      for (int64_t e = e0; e < e1; ++e) {
        const int64_t j = c[e];
        st.add(leaky(zs[j * H + hd] + zd[i * H + hd], slope), HS + j * HD + hd * D);
      }
      return st;
    };
    auto finish = [&](int64_t i, int hd, const Soft& st) {
      float* o = o32.data() + i * HD + hd * D;
      float* n = ns + (i * H + hd) * 4;
      n[1] = 0.f;
      n[2] = zd[i * H + hd];
      n[3] = zsd[i * H + hd];
      if (st.l > 0.f) {
        const float inv = 1.f / st.l;
        for (int d = 0; d < D; ++d) o[d] = st.acc[d] * inv;
        n[0] = st.m + logf(st.l);
      } else {
        std::fill(o, o + D, 0.f);
        n[0] = -kInf;
      }
    };
    walk_plan(
        *plan, rp,
        [&](int64_t i, int64_t e0, int64_t e1) {
          for (int hd = 0; hd < H; ++hd) finish(i, hd, state(i, hd, e0, e1));
        },
        [&](int64_t i, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          for (int hd = 0; hd < H; ++hd) {
            Soft total(D);
            for (const auto& ch : chunks) total.merge(state(i, hd, ch.first, ch.second));
            finish(i, hd, total);
          }
        },
        [&](int64_t i) {
          for (int hd = 0; hd < H; ++hd) finish(i, hd, Soft(D));
        });
    round_all(el, o32, out);
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_gat_bwd(const void* row_ptr, const void* col, int idx_bits,
                               const tgx_row_plan* plan, const int32_t* row_ptr_t,
                               const int32_t* col_t, const int32_t* perm,
                               const int32_t* inv_perm, const tgx_row_plan* plan_t,
                               const void* h_src, const void* h_dst, const float* a_src,
                               const float* a_dst, float slope, const void* out, float* ns,
                               const void* dout, void* dh_src, void* dh_dst, float* da_src,
                               float* da_dst, int64_t n_dst, int64_t n_src, int64_t n_edges,
                               int H, int D, int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(elem_ok(dtype), "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)", dtype);
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
  TGX_REQUIRE(n_edges == 0 || (row_ptr_t && col_t && inv_perm), "null transposed CSR");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    int64_t E = 0, Et = 0;
    int s = check_csr(rp, &c, n_dst, n_src, &E);
    if (s != TGX_OK) return s;
    TGX_REQUIRE(E == n_edges, "row_ptr[n_dst] = %lld, expected %lld edges",
                static_cast<long long>(E), static_cast<long long>(n_edges));
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    s = check_transposed(row_ptr_t, col_t, perm, inv_perm, n_src, n_dst, &Et);
    if (s != TGX_OK) return s;
    TGX_REQUIRE(Et == E, "transposed CSR has %lld edges, expected %lld",
                static_cast<long long>(Et), static_cast<long long>(E));
    const Idx rpt{row_ptr_t, 32};
    s = check_plan_rows(plan_t, rpt, n_src);
    if (s != TGX_OK) return s;
    const int64_t HD = static_cast<int64_t>(H) * D;
    const Elem el{dtype};
    const std::vector<float> hs = widen_all(el, h_src, n_src * HD);
    const std::vector<float> hd_own = homogeneous ? std::vector<float>()
                                                  : widen_all(el, h_dst, n_dst * HD);
    const float* HS = hs.data();
    const float* HDv = homogeneous ? hs.data() : hd_own.data();
    const std::vector<float> o32 = widen_all(el, out, n_dst * HD);
    const std::vector<float> g32 = widen_all(el, dout, n_dst * HD);
    // B1: delta = <dout, out> per (node, head).
    parallel_ranges(n_dst, [&](int64_t lo, int64_t hi) {
      for (int64_t i = lo; i < hi; ++i)
        for (int hd = 0; hd < H; ++hd) {
          float d = 0.f;
          for (int q = 0; q < D; ++q) d += g32[i * HD + hd * D + q] * o32[i * HD + hd * D + q];
          ns[(i * H + hd) * 4 + 1] = d;
        }
    });
    // B2: source pass over the transposed CSR; dz per edge at its transposed
    // position, the source-side sums per (node, head).
    std::vector<float> dz(static_cast<size_t>(E * H)), sdz_src(static_cast<size_t>(n_src * H));
    std::vector<float> dhs(static_cast<size_t>(n_src * HD)), dhd(static_cast<size_t>(n_dst * HD));
    auto src_range = [&](int64_t j, int hd, int64_t k0, int64_t k1, float* dh_acc,
                         float& sdz) {
      const float* hj = HS + j * HD + hd * D;
      float zs = 0.f;
      for (int q = 0; q < D; ++q) zs += a_src[hd * D + q] * hj[q];
      for (int64_t k = k0; k < k1; ++k) {
        const int64_t i = col_t[k];
        const float* n = ns + (i * H + hd) * 4;
        const float z = zs + n[2];
        const float alpha = expf(leaky(z, slope) - n[0]);
        const float* g = g32.data() + i * HD + hd * D;
        float dalpha = 0.f;
        for (int q = 0; q < D; ++q) dalpha += g[q] * hj[q];
        const float ds = alpha * (dalpha - n[1]);
        const float dzv = z > 0.f ? ds : ds * slope;
        for (int q = 0; q < D; ++q) dh_acc[q] += alpha * g[q];
        sdz += dzv;
        dz[k * H + hd] = dzv;
      }
    };
    auto src_finish = [&](int64_t j, int hd, const float* acc, float sdz) {
      float* o = dhs.data() + j * HD + hd * D;
      for (int q = 0; q < D; ++q) o[q] = acc[q] + sdz * a_src[hd * D + q];
      sdz_src[j * H + hd] = sdz;
    };
    walk_plan(
        *plan_t, rpt,
        [&](int64_t j, int64_t k0, int64_t k1) {
          std::vector<float> acc(static_cast<size_t>(D));
          for (int hd = 0; hd < H; ++hd) {
            std::fill(acc.begin(), acc.end(), 0.f);
            float sdz = 0.f;
            src_range(j, hd, k0, k1, acc.data(), sdz);
            src_finish(j, hd, acc.data(), sdz);
          }
        },
        [&](int64_t j, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> acc(static_cast<size_t>(D)), part(static_cast<size_t>(D));
          for (int hd = 0; hd < H; ++hd) {
            std::fill(acc.begin(), acc.end(), 0.f);
            float sdz = 0.f;
            for (const auto& ch : chunks) {
              std::fill(part.begin(), part.end(), 0.f);
              float ps = 0.f;
              src_range(j, hd, ch.first, ch.second, part.data(), ps);
              for (int q = 0; q < D; ++q) acc[q] += part[q];
              sdz += ps;
            }
            src_finish(j, hd, acc.data(), sdz);
          }
        },
        [&](int64_t j) {
          std::fill(dhs.begin() + j * HD, dhs.begin() + (j + 1) * HD, 0.f);
          for (int hd = 0; hd < H; ++hd) sdz_src[j * H + hd] = 0.f;
        });
    // B3: destination pass over the CSR: dhd[i] = (sum of the row's dz) a_dst,
    // and fp64 parameter-gradient partials over fixed node blocks.
    constexpr int64_t kBlocks = 64;
    std::vector<double> pds(static_cast<size_t>(kBlocks * HD), 0.0), pdd(pds.size(), 0.0);
    const int64_t per_dst = ceil_div(n_dst, kBlocks), per_src = ceil_div(n_src, kBlocks);
    parallel_ranges(kBlocks, [&](int64_t b0, int64_t b1) {
      for (int64_t b = b0; b < b1; ++b) {
        double* ps = pds.data() + b * HD;
        double* pd = pdd.data() + b * HD;
        for (int64_t i = b * per_dst; i < std::min(n_dst, (b + 1) * per_dst); ++i)
          for (int hd = 0; hd < H; ++hd) {
            float sdz = 0.f;
            for (int64_t e = rp[i]; e < rp[i + 1]; ++e) sdz += dz[inv_perm[e] * H + hd];
            const float* hi = HDv + i * HD + hd * D;
            float* o = dhd.data() + i * HD + hd * D;
            for (int q = 0; q < D; ++q) {
              o[q] = sdz * a_dst[hd * D + q];
              pd[hd * D + q] += static_cast<double>(sdz) * hi[q];
            }
          }
        for (int64_t j = b * per_src; j < std::min(n_src, (b + 1) * per_src); ++j)
          for (int hd = 0; hd < H; ++hd) {
            const double ss = sdz_src[j * H + hd];
            const float* hj = HS + j * HD + hd * D;
            for (int q = 0; q < D; ++q) ps[hd * D + q] += ss * hj[q];
          }
      }
    }, 1);
    for (int64_t x = 0; x < HD; ++x) {
      double a = 0.0, b = 0.0;
      for (int64_t k = 0; k < kBlocks; ++k) {
        a += pds[k * HD + x];
        b += pdd[k * HD + x];
      }
      da_src[x] = static_cast<float>(a);
      da_dst[x] = static_cast<float>(b);
    }
    if (homogeneous) {
      // One tensor: both roles' terms, rounded once.
      for (size_t x = 0; x < dhs.size(); ++x) dhs[x] += dhd[x];
      round_all(el, dhs, dh_src);
    } else {
      round_all(el, dhs, dh_src);
      round_all(el, dhd, dh_dst);
    }
    return TGX_OK;
  });
}

// ---- Dot-product attention (bf16, fp16 or fp32 elements) --------------------------

namespace {

// Head hd of a [N, H, D] row, in fp32.
void load_head(const Elem& el, const void* base, int64_t node, int H, int D, int hd,
               float* dst) {
  const int64_t o = (node * H + hd) * D;
  for (int d = 0; d < D; ++d) dst[d] = el.get(base, o + d);
}


}  // namespace

extern "C" int tgx_cpu_dot_attn_fwd(const void* row_ptr, const void* col, int idx_bits,
                                    const tgx_row_plan* plan, const void* q, const void* k,
                                    const void* v, const float* bias, float scale, void* out,
                                    float* ml, int64_t n_dst, int64_t n_src, int H, int D,
                                    int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(elem_ok(dtype), "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)", dtype);
  if (!dot_heads_ok(H, D)) {
    set_error("dot attention supports H >= 1 and D in {8, 16, 32, 64, 128, 256, 512} "
              "(got H=%d D=%d)", H, D);
    return TGX_UNSUPPORTED;
  }
  int st = check_plan(plan, n_dst);
  if (st != TGX_OK) return st;
  if (n_dst == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && q && out && ml && ((k && v) || n_src == 0), "null pointer");
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    int s = check_csr(rp, &c, n_dst, n_src, nullptr);
    if (s != TGX_OK) return s;
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    const Elem el{dtype};
    const void *Q = q, *K = k, *V = v;
    auto state = [&](int64_t i, int hd, const float* qf, int64_t e0, int64_t e1) {
      Soft st(D);
      std::vector<float> kf(static_cast<size_t>(D)), vf(static_cast<size_t>(D));
      for (int64_t e = e0; e < e1; ++e) {
        const int64_t j = c[e];
        load_head(el, K, j, H, D, hd, kf.data());
        load_head(el, V, j, H, D, hd, vf.data());
        float dotp = 0.f;
        for (int d = 0; d < D; ++d) dotp += qf[d] * kf[d];
        st.add(dotp * scale + (bias ? bias[e * H + hd] : 0.f), vf.data());
      }
      (void)i;
      return st;
    };
    auto finish = [&](int64_t i, int hd, const Soft& st) {
      const int64_t o = (i * H + hd) * D;
      if (st.l > 0.f) {
        const float inv = 1.f / st.l;
        for (int d = 0; d < D; ++d) el.put(out, o + d, st.acc[d] * inv);
        ml[(i * H + hd) * 2] = st.m + logf(st.l);
      } else {
        for (int d = 0; d < D; ++d) el.put(out, o + d, 0.f);
        ml[(i * H + hd) * 2] = -kInf;
      }
      ml[(i * H + hd) * 2 + 1] = 0.f;
    };
    walk_plan(
        *plan, rp,
        [&](int64_t i, int64_t e0, int64_t e1) {
          std::vector<float> qf(static_cast<size_t>(D));
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, Q, i, H, D, hd, qf.data());
            finish(i, hd, state(i, hd, qf.data(), e0, e1));
          }
        },
        [&](int64_t i, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> qf(static_cast<size_t>(D));
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, Q, i, H, D, hd, qf.data());
            Soft total(D);
            for (const auto& ch : chunks) total.merge(state(i, hd, qf.data(), ch.first, ch.second));
            finish(i, hd, total);
          }
        },
        [&](int64_t i) {
          for (int hd = 0; hd < H; ++hd) finish(i, hd, Soft(D));
        });
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_dot_attn_bwd(const void* row_ptr, const void* col, int idx_bits,
                                    const tgx_row_plan* plan, const int32_t* row_ptr_t,
                                    const int32_t* col_t, const int32_t* perm,
                                    const tgx_row_plan* plan_t, const void* q, const void* k,
                                    const void* v, const float* bias, float scale,
                                    const void* out, float* ml, const void* dout, void* dq,
                                    void* dk, void* dv, float* dbias, int64_t n_dst,
                                    int64_t n_src, int H, int D, int dtype) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(elem_ok(dtype), "dtype must be TGX_DTYPE_BF16, _F16 or _F32 (got %d)", dtype);
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
  return guarded([&]() -> int {
    const Idx rp{row_ptr, idx_bits}, c{col, idx_bits};
    int64_t E = 0, Et = 0;
    int s = check_csr(rp, &c, n_dst, n_src, &E);
    if (s != TGX_OK) return s;
    s = check_plan_rows(plan, rp, n_dst);
    if (s != TGX_OK) return s;
    s = check_transposed(row_ptr_t, col_t, perm, nullptr, n_src, n_dst, &Et);
    if (s != TGX_OK) return s;
    TGX_REQUIRE(Et == E, "transposed CSR has %lld edges, expected %lld",
                static_cast<long long>(Et), static_cast<long long>(E));
    const Idx rpt{row_ptr_t, 32};
    s = check_plan_rows(plan_t, rpt, n_src);
    if (s != TGX_OK) return s;
    const Elem el{dtype};
    const void *Q = q, *K = k, *V = v, *Oo = out, *G = dout;
    // B1: delta = <dout, out>.
    parallel_ranges(n_dst, [&](int64_t lo, int64_t hi) {
      std::vector<float> a(static_cast<size_t>(D)), b(static_cast<size_t>(D));
      for (int64_t i = lo; i < hi; ++i)
        for (int hd = 0; hd < H; ++hd) {
          load_head(el, G, i, H, D, hd, a.data());
          load_head(el, Oo, i, H, D, hd, b.data());
          float d = 0.f;
          for (int x = 0; x < D; ++x) d += a[x] * b[x];
          ml[(i * H + hd) * 2 + 1] = d;
        }
    });
    // B2: destination pass: ds per edge (dbias), dq = scale * sum ds k.
    auto dst_range = [&](int64_t i, int hd, const float* qf, const float* gf, int64_t e0,
                         int64_t e1, float* acc) {
      const float lse = ml[(i * H + hd) * 2], delta = ml[(i * H + hd) * 2 + 1];
      std::vector<float> kf(static_cast<size_t>(D)), vf(static_cast<size_t>(D));
      for (int64_t e = e0; e < e1; ++e) {
        const int64_t j = c[e];
        load_head(el, K, j, H, D, hd, kf.data());
        load_head(el, V, j, H, D, hd, vf.data());
        float sp = 0.f, dp = 0.f;
        for (int x = 0; x < D; ++x) {
          sp += qf[x] * kf[x];
          dp += gf[x] * vf[x];
        }
        const float alpha = expf(sp * scale + (bias ? bias[e * H + hd] : 0.f) - lse);
        const float ds = alpha * (dp - delta);
        if (dbias) dbias[e * H + hd] = ds;
        for (int x = 0; x < D; ++x) acc[x] += ds * kf[x];
      }
    };
    auto dq_store = [&](int64_t i, int hd, const float* acc) {
      const int64_t o = (i * H + hd) * D;
      for (int x = 0; x < D; ++x) el.put(dq, o + x, acc[x] * scale);
    };
    walk_plan(
        *plan, rp,
        [&](int64_t i, int64_t e0, int64_t e1) {
          std::vector<float> qf(D), gf(D), acc(D);
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, Q, i, H, D, hd, qf.data());
            load_head(el, G, i, H, D, hd, gf.data());
            std::fill(acc.begin(), acc.end(), 0.f);
            dst_range(i, hd, qf.data(), gf.data(), e0, e1, acc.data());
            dq_store(i, hd, acc.data());
          }
        },
        [&](int64_t i, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> qf(D), gf(D), acc(D), part(D);
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, Q, i, H, D, hd, qf.data());
            load_head(el, G, i, H, D, hd, gf.data());
            std::fill(acc.begin(), acc.end(), 0.f);
            for (const auto& ch : chunks) {
              std::fill(part.begin(), part.end(), 0.f);
              dst_range(i, hd, qf.data(), gf.data(), ch.first, ch.second, part.data());
              for (int x = 0; x < D; ++x) acc[x] += part[x];
            }
            dq_store(i, hd, acc.data());
          }
        },
        [&](int64_t i) {
          for (int64_t x = i * H * D; x < (i + 1) * H * D; ++x) el.put(dq, x, 0.f);
        });
    if (n_src == 0) return TGX_OK;
    // B3: source pass over the transposed CSR: dk = scale * sum ds q, dv = sum alpha dout.
    auto src_range = [&](int hd, const float* kf, const float* vf, int64_t k0, int64_t k1,
                         float* ak, float* av) {
      std::vector<float> qf(static_cast<size_t>(D)), gf(static_cast<size_t>(D));
      for (int64_t t = k0; t < k1; ++t) {
        const int64_t i = col_t[t], e = perm[t];
        load_head(el, Q, i, H, D, hd, qf.data());
        load_head(el, G, i, H, D, hd, gf.data());
        float sp = 0.f, dp = 0.f;
        for (int x = 0; x < D; ++x) {
          sp += qf[x] * kf[x];
          dp += gf[x] * vf[x];
        }
        const float alpha =
            expf(sp * scale + (bias ? bias[e * H + hd] : 0.f) - ml[(i * H + hd) * 2]);
        const float ds = alpha * (dp - ml[(i * H + hd) * 2 + 1]);
        for (int x = 0; x < D; ++x) {
          ak[x] += ds * qf[x];
          av[x] += alpha * gf[x];
        }
      }
    };
    auto kv_store = [&](int64_t j, int hd, const float* ak, const float* av) {
      const int64_t o = (j * H + hd) * D;
      for (int x = 0; x < D; ++x) {
        el.put(dk, o + x, ak[x] * scale);
        el.put(dv, o + x, av[x]);
      }
    };
    walk_plan(
        *plan_t, rpt,
        [&](int64_t j, int64_t k0, int64_t k1) {
          std::vector<float> kf(D), vf(D), ak(D), av(D);
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, K, j, H, D, hd, kf.data());
            load_head(el, V, j, H, D, hd, vf.data());
            std::fill(ak.begin(), ak.end(), 0.f);
            std::fill(av.begin(), av.end(), 0.f);
            src_range(hd, kf.data(), vf.data(), k0, k1, ak.data(), av.data());
            kv_store(j, hd, ak.data(), av.data());
          }
        },
        [&](int64_t j, const std::vector<std::pair<int64_t, int64_t>>& chunks) {
          std::vector<float> kf(D), vf(D), ak(D), av(D), pk(D), pv(D);
          for (int hd = 0; hd < H; ++hd) {
            load_head(el, K, j, H, D, hd, kf.data());
            load_head(el, V, j, H, D, hd, vf.data());
            std::fill(ak.begin(), ak.end(), 0.f);
            std::fill(av.begin(), av.end(), 0.f);
            for (const auto& ch : chunks) {
              std::fill(pk.begin(), pk.end(), 0.f);
              std::fill(pv.begin(), pv.end(), 0.f);
              src_range(hd, kf.data(), vf.data(), ch.first, ch.second, pk.data(), pv.data());
              for (int x = 0; x < D; ++x) {
                ak[x] += pk[x];
                av[x] += pv[x];
              }
            }
            kv_store(j, hd, ak.data(), av.data());
          }
        },
        [&](int64_t j) {
          for (int64_t x = j * H * D; x < (j + 1) * H * D; ++x) {
            el.put(dk, x, 0.f);
            el.put(dv, x, 0.f);
          }
        });
    return TGX_OK;
  });
}

// ---- Dense attention over block-diagonal relations ---------------------------------

namespace {

struct AttnView {
  int64_t n_q, n_k;
  int H, D;
  Half16 t;
  int64_t qsn, qsh, ksn, ksh;
};

int check_attn(const int32_t* cu_q, const int32_t* cu_k, int n_blocks, int causal, int dtype,
               const int64_t* strides, int64_t n_q, int64_t n_k, int H, int D) {
  if (D != 32 && D != 64 && D != 128) {
    set_error("dense attention tiles support head_dim 32, 64 and 128 (got %d)", D);
    return TGX_UNSUPPORTED;
  }
  if (dtype != TGX_DTYPE_BF16 && dtype != TGX_DTYPE_F16) {
    set_error("dense attention tiles support bf16 and fp16 (dtype code %d)", dtype);
    return TGX_UNSUPPORTED;
  }
  TGX_REQUIRE(strides, "null strides");
  TGX_REQUIRE(H > 0 && n_q >= 0 && n_k >= 0 && n_blocks >= 0, "bad sizes");
  TGX_REQUIRE(strides[0] > 0 && strides[1] > 0 && strides[2] > 0 && strides[3] > 0,
              "strides must be positive");
  TGX_REQUIRE(n_q < (int64_t{1} << 31) && n_k < (int64_t{1} << 31),
              "token counts must fit int32");
  TGX_REQUIRE(n_blocks == 0 || (cu_q && cu_k), "null cu_seqlens");
  for (int b = 0; b < n_blocks; ++b) {
    const int64_t q0 = cu_q[b], q1 = cu_q[b + 1], k0 = cu_k[b], k1 = cu_k[b + 1];
    TGX_REQUIRE(q1 >= q0 && q0 >= 0 && q1 <= n_q && k1 >= k0 && k0 >= 0 && k1 <= n_k,
                "block %d out of range", b);
    TGX_REQUIRE(!causal || (q0 == k0 && q1 == k1), "causal blocks must be square");
  }
  return TGX_OK;
}

// Keys [k0, k1) of block b that query row r sees.
void block_keys(const int32_t* cu_q, const int32_t* cu_k, int b, int causal, int64_t r,
                int64_t* k0, int64_t* k1) {
  *k0 = cu_k[b];
  *k1 = causal ? cu_k[b] + (r - cu_q[b]) + 1 : cu_k[b + 1];
}

}  // namespace

extern "C" int tgx_cpu_attn_fwd(const int32_t* cu_q, const int32_t* cu_k, int n_blocks,
                                int causal, int dtype, const void* q, const void* k,
                                const void* v, const int64_t* strides, float scale,
                                float prune_threshold, void* out, float* lse, int64_t n_q,
                                int64_t n_k, int H, int D) {
  int st = check_attn(cu_q, cu_k, n_blocks, causal, dtype, strides, n_q, n_k, H, D);
  if (st != TGX_OK) return st;
  TGX_REQUIRE(!(prune_threshold < 0.f) && prune_threshold <= 1.f,
              "block_prune_threshold must be in (0, 1] (0 = exact)");
  if (prune_threshold > 0.f) {
    set_error("the CPU twin computes exact softmax only (block pruning depends on the "
              "device tile schedule)");
    return TGX_UNSUPPORTED;
  }
  if (n_blocks == 0) return TGX_OK;
  TGX_REQUIRE(q && k && v && out && lse, "null pointer");
  return guarded([&]() -> int {
    const AttnView a{n_q, n_k, H, D, Half16{dtype}, strides[0], strides[1], strides[2],
                     strides[3]};
    const auto* Q = static_cast<const uint16_t*>(q);
    const auto* K = static_cast<const uint16_t*>(k);
    const auto* V = static_cast<const uint16_t*>(v);
    auto* O = static_cast<uint16_t*>(out);
    // Work items: (block, head) pairs; each writes its own rows of one head.
    parallel_ranges(static_cast<int64_t>(n_blocks) * H, [&](int64_t lo, int64_t hi) {
      std::vector<float> qf(D), vf(D);
      for (int64_t w = lo; w < hi; ++w) {
        const int b = static_cast<int>(w / H), hd = static_cast<int>(w % H);
        for (int64_t r = cu_q[b]; r < cu_q[b + 1]; ++r) {
          for (int d = 0; d < D; ++d) qf[d] = a.t.load(Q, r * a.qsn + hd * a.qsh + d);
          int64_t k0, k1;
          block_keys(cu_q, cu_k, b, causal, r, &k0, &k1);
          Soft s(D);
          for (int64_t kk = k0; kk < k1; ++kk) {
            float sp = 0.f;
            for (int d = 0; d < D; ++d) sp += qf[d] * a.t.load(K, kk * a.ksn + hd * a.ksh + d);
            for (int d = 0; d < D; ++d) vf[d] = a.t.load(V, kk * a.ksn + hd * a.ksh + d);
            s.add(sp * scale, vf.data());
          }
          uint16_t* o = O + (r * H + hd) * D;
          if (s.l > 0.f) {
            const float inv = 1.f / s.l;
            for (int d = 0; d < D; ++d) o[d] = a.t.store(s.acc[d] * inv);
            lse[r * H + hd] = s.m + logf(s.l);
          } else {
            for (int d = 0; d < D; ++d) o[d] = a.t.store(0.f);
            lse[r * H + hd] = -kInf;
          }
        }
      }
    });
    return TGX_OK;
  });
}

extern "C" int tgx_cpu_attn_bwd(const int32_t* cu_q, const int32_t* cu_k, int n_blocks,
                                int causal, int dtype, const void* q, const void* k,
                                const void* v, const int64_t* strides, const void* out,
                                const float* lse, const void* dout, float scale, void* dq,
                                void* dk, void* dv, float* delta, int64_t n_q, int64_t n_k,
                                int H, int D) {
  int st = check_attn(cu_q, cu_k, n_blocks, causal, dtype, strides, n_q, n_k, H, D);
  if (st != TGX_OK) return st;
  if (n_blocks == 0) return TGX_OK;
  TGX_REQUIRE(q && k && v && out && lse && dout && dq && dk && dv && delta, "null pointer");
  return guarded([&]() -> int {
    const AttnView a{n_q, n_k, H, D, Half16{dtype}, strides[0], strides[1], strides[2],
                     strides[3]};
    const auto* Q = static_cast<const uint16_t*>(q);
    const auto* K = static_cast<const uint16_t*>(k);
    const auto* V = static_cast<const uint16_t*>(v);
    const auto* O = static_cast<const uint16_t*>(out);
    const auto* G = static_cast<const uint16_t*>(dout);
    auto* DQ = static_cast<uint16_t*>(dq);
    auto* DK = static_cast<uint16_t*>(dk);
    auto* DV = static_cast<uint16_t*>(dv);
    parallel_ranges(static_cast<int64_t>(n_blocks) * H, [&](int64_t lo, int64_t hi) {
      std::vector<float> qf(D), gf(D), kf(D), vf(D), aq(D);
      for (int64_t w = lo; w < hi; ++w) {
        const int b = static_cast<int>(w / H), hd = static_cast<int>(w % H);
        const int64_t kb = cu_k[b], nk = cu_k[b + 1] - kb;
        std::vector<float> ak(static_cast<size_t>(nk * D), 0.f), av(ak.size(), 0.f);
        for (int64_t r = cu_q[b]; r < cu_q[b + 1]; ++r) {
          float d0 = 0.f;
          for (int d = 0; d < D; ++d) {
            qf[d] = a.t.load(Q, r * a.qsn + hd * a.qsh + d);
            gf[d] = a.t.load(G, (r * H + hd) * D + d);
            d0 += gf[d] * a.t.load(O, (r * H + hd) * D + d);
          }
          delta[r * H + hd] = d0;
          std::fill(aq.begin(), aq.end(), 0.f);
          int64_t k0, k1;
          block_keys(cu_q, cu_k, b, causal, r, &k0, &k1);
          const float l = lse[r * H + hd];
          for (int64_t kk = k0; kk < k1; ++kk) {
            float sp = 0.f, dp = 0.f;
            for (int d = 0; d < D; ++d) {
              kf[d] = a.t.load(K, kk * a.ksn + hd * a.ksh + d);
              vf[d] = a.t.load(V, kk * a.ksn + hd * a.ksh + d);
              sp += qf[d] * kf[d];
              dp += gf[d] * vf[d];
            }
            const float p = l == -kInf ? 0.f : expf(sp * scale - l);
            const float ds = p * (dp - d0);
            float* rk = ak.data() + (kk - kb) * D;
            float* rv = av.data() + (kk - kb) * D;
            for (int d = 0; d < D; ++d) {
              aq[d] += ds * kf[d];
              rk[d] += ds * qf[d];
              rv[d] += p * gf[d];
            }
          }
          for (int d = 0; d < D; ++d) DQ[(r * H + hd) * D + d] = a.t.store(aq[d] * scale);
        }
        for (int64_t kk = 0; kk < nk; ++kk)
          for (int d = 0; d < D; ++d) {
            DK[((kb + kk) * H + hd) * D + d] = a.t.store(ak[kk * D + d] * scale);
            DV[((kb + kk) * H + hd) * D + d] = a.t.store(av[kk * D + d]);
          }
      }
    });
    return TGX_OK;
  });
}
