// Host-side helpers for the C ABI: status mapping, argument checks and
// launch error capture.  Every exported entry point returns a TGX status and
// never throws across the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

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

#define TGX_HIP(call)                                                  \
  do {                                                                 \
    hipError_t tgx_err_ = (call);                                      \
    if (tgx_err_ != hipSuccess) {                                      \
      ::tgx::set_error("%s failed: %s", #call,                        \
                       hipGetErrorString(tgx_err_));                   \
      return TGX_INTERNAL;                                             \
    }                                                                  \
  } while (0)

// Check the launch that was just enqueued.
#define TGX_LAUNCHED(name)                                             \
  do {                                                                 \
    hipError_t tgx_err_ = hipGetLastError();                           \
    if (tgx_err_ != hipSuccess) {                                      \
      ::tgx::set_error("launch of %s failed: %s", name,               \
                       hipGetErrorString(tgx_err_));                   \
      return TGX_INTERNAL;                                             \
    }                                                                  \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t v, size_t a = 256) { return (v + a - 1) / a * a; }

// Bump allocator over a caller-provided workspace.
struct Carve {
  char* base;
  size_t cap;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    size_t off = align_up(used);
    used = off + count * sizeof(T);
    return reinterpret_cast<T*>(base + off);
  }
  bool ok() const { return used <= cap; }
};

// Device scan over int32 (exclusive).  out may alias in.  Writes the total to
// *total_dev when non-null.  scratch must hold scan_scratch_ints(n) ints.
size_t scan_scratch_ints(int64_t n);
int scan_exclusive_i32(const int32_t* in, int32_t* out, int64_t n,
                       int32_t* total_dev, int32_t* scratch, hipStream_t stream);

// Workgroups of `block` threads that a kernel can keep resident on the whole
// device at once (occupancy x compute units); persistent grids use this so no
// workgroup waits for a second round.
template <typename Kernel>
inline int64_t resident_blocks(Kernel kernel, int block) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess)
    return 1;
  const int64_t n = static_cast<int64_t>(cus) * (per_cu > 0 ? per_cu : 1);
  return n > 0 ? n : 1;
}

// Validate a row plan against the number of rows it must cover.
inline int check_plan(const tgx_row_plan* p, int64_t rows) {
  TGX_REQUIRE(p != nullptr, "null plan");
  TGX_REQUIRE(p->n_rows == rows, "plan covers %lld rows, expected %lld",
              static_cast<long long>(p->n_rows), static_cast<long long>(rows));
  TGX_REQUIRE(p->n_empty >= 0 && p->n_wave >= 0 && p->n_split >= 0 &&
                  p->n_chunks >= 0 && p->n_empty + p->n_wave + p->n_split == p->n_rows,
              "inconsistent plan");
  TGX_REQUIRE(p->n_rows == 0 || p->rows_dev, "plan without rows");
  TGX_REQUIRE(p->n_split == 0 || (p->chunk_offsets_dev && p->chunk_edges > 0 &&
                                  p->n_chunks >= p->n_split),
              "plan without chunk offsets");
  return TGX_OK;
}

}  // namespace tgx
