// Argument checks and small helpers shared by the device entry points and the
// CPU twins: plain C++, no HIP headers.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "tgx.h"

namespace tgx {

// Last error message for the calling thread; read by tgx_last_error().
void set_error(const char* fmt, ...);

#define TGX_REQUIRE(cond, ...)                  \
  do {                                          \
    if (!(cond)) {                              \
      ::tgx::set_error(__VA_ARGS__);            \
      return TGX_INVALID_ARGUMENT;              \
    }                                           \
  } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t v, size_t a = 256) { return (v + a - 1) / a * a; }

// Validate a row plan's counts against the number of rows it must cover.
inline int check_plan(const tgx_row_plan* p, int64_t rows) {
  TGX_REQUIRE(p != nullptr, "null plan");
  TGX_REQUIRE(p->n_rows == rows, "plan covers %lld rows, expected %lld",
              static_cast<long long>(p->n_rows), static_cast<long long>(rows));
  TGX_REQUIRE(p->n_empty >= 0 && p->n_wave >= 0 && p->n_split >= 0 &&
                  p->n_chunks >= 0 && p->n_empty + p->n_wave + p->n_split == p->n_rows,
              "inconsistent plan");
  TGX_REQUIRE(p->n_rows == 0 || p->rows_dev, "plan without rows");
  TGX_REQUIRE(p->n_rows < (int64_t{1} << 31), "plan rows are 32-bit: fewer than 2^31 rows");
  TGX_REQUIRE(p->n_split == 0 || (p->chunk_offsets_dev && p->chunk_edges > 0 &&
                                  p->n_chunks >= p->n_split),
              "plan without chunk offsets");
  return TGX_OK;
}

// Head grouping of the attention kernels.  A GAT group of Hg heads holds
// Hg * D <= 256 floats per node (a float4 per lane over at most 64 lanes), a
// dot-product group Hg * D <= 512 bf16 values (8 per lane); Hg is a power of
// two and the head width D / 4 (GAT) or D / 8 (dot) is a power of two.  Any
// H splits greedily into such groups.
constexpr int kGatGroupFloats = 256;
constexpr int kDotGroupValues = 512;

inline bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

inline bool gat_heads_ok(int H, int D) {
  return H >= 1 && D > 0 && D % 4 == 0 && D <= kGatGroupFloats && pow2(D / 4);
}

inline bool dot_heads_ok(int H, int D) {
  return H >= 1 && D > 0 && D % 8 == 0 && D <= kDotGroupValues && pow2(D / 8);
}

// Heads in the group starting at head h0 (groups of at most `cap` values).
inline int group_heads(int H, int D, int h0, int cap) {
  int hg = cap / D;
  while (hg > H - h0) hg >>= 1;
  return hg;
}

}  // namespace tgx
