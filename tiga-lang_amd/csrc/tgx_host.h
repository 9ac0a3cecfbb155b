// Host-side helpers for the C ABI: status mapping, argument checks and
// launch error capture.  Every exported entry point returns a TGX status and
// never throws across the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "tgx.h"
#include "tgx_check.h"

namespace tgx {

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

}  // namespace tgx
