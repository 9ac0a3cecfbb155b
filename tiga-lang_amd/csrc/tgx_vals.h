// Element formats of gathered node rows: a lane loads N consecutive values of
// one row (N = 8 for the dot-product kernels, 4 for the GAT kernels), keeps
// them in their storage form while the load is in flight, and widens them to
// fp32 for arithmetic.  Results are rounded back with round-to-nearest-even.
//
//   TGX_DTYPE_BF16  16-bit storage, 8 values = one 16-byte vector
//   TGX_DTYPE_F16   16-bit storage, 8 values = one 16-byte vector
//   TGX_DTYPE_F32   8 values = two 16-byte vectors, 4 values = one
//
// The 16-bit formats hold element 2k in the low half of 32-bit word k.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tgx.h"
#include "tgx_device.h"

namespace tgx {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void f16_pair(uint32_t w, float& lo, float& hi) {
  const f16x2 h = __builtin_bit_cast(f16x2, w);
  lo = static_cast<float>(h[0]);
  hi = static_cast<float>(h[1]);
}
// fp32 -> fp16 with the hardware's round-to-nearest-even conversion.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const f16x2 h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
  return __builtin_bit_cast(uint32_t, h);
}

template <int DT, int N>
struct Vals;

// ---- 8 values per lane -------------------------------------------------------
template <>
struct Vals<TGX_DTYPE_BF16, 8> {
  using T = uint16_t;
  using Raw = u32x4;
  static __device__ __forceinline__ Raw load(const T* p) {
    return *reinterpret_cast<const u32x4*>(p);
  }
  static __device__ __forceinline__ void unpack(Raw r, float (&f)[8]) { unpack8(r, f); }
  static __device__ __forceinline__ void store(T* p, const float (&f)[8]) {
    *reinterpret_cast<u32x4*>(p) = pack8(f);
  }
  static __device__ __forceinline__ void store_zero(T* p) {
    *reinterpret_cast<u32x4*>(p) = u32x4{0u, 0u, 0u, 0u};
  }
};

template <>
struct Vals<TGX_DTYPE_F16, 8> {
  using T = uint16_t;
  using Raw = u32x4;
  static __device__ __forceinline__ Raw load(const T* p) {
    return *reinterpret_cast<const u32x4*>(p);
  }
  static __device__ __forceinline__ void unpack(Raw r, float (&f)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) f16_pair(r[k], f[2 * k], f[2 * k + 1]);
  }
  static __device__ __forceinline__ void store(T* p, const float (&f)[8]) {
    u32x4 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = pack_f16x2(f[2 * k], f[2 * k + 1]);
    *reinterpret_cast<u32x4*>(p) = r;
  }
  static __device__ __forceinline__ void store_zero(T* p) {
    *reinterpret_cast<u32x4*>(p) = u32x4{0u, 0u, 0u, 0u};
  }
};

template <>
struct Vals<TGX_DTYPE_F32, 8> {
  using T = float;
  struct Raw {
    f32x4 lo, hi;
  };
  static __device__ __forceinline__ Raw load(const T* p) {
    return Raw{*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4)};
  }
  static __device__ __forceinline__ void unpack(Raw r, float (&f)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[k] = r.lo[k];
      f[4 + k] = r.hi[k];
    }
  }
  static __device__ __forceinline__ void store(T* p, const float (&f)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{f[4], f[5], f[6], f[7]};
  }
  static __device__ __forceinline__ void store_zero(T* p) {
    *reinterpret_cast<f32x4*>(p) = f32x4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
  }
};

// ---- 4 values per lane (held as f32x4 after the load) -------------------------
template <>
struct Vals<TGX_DTYPE_F32, 4> {
  using T = float;
  using Raw = f32x4;
  static __device__ __forceinline__ Raw load(const T* p) {
    return *reinterpret_cast<const f32x4*>(p);
  }
  static __device__ __forceinline__ f32x4 widen(Raw r) { return r; }
  static __device__ __forceinline__ void store(T* p, f32x4 v) {
    *reinterpret_cast<f32x4*>(p) = v;
  }
};

template <>
struct Vals<TGX_DTYPE_BF16, 4> {
  using T = uint16_t;
  using Raw = u32x2;
  static __device__ __forceinline__ Raw load(const T* p) {
    return *reinterpret_cast<const u32x2*>(p);
  }
  static __device__ __forceinline__ f32x4 widen(Raw r) {
    return f32x4{bf16_lo(r[0]), bf16_hi(r[0]), bf16_lo(r[1]), bf16_hi(r[1])};
  }
  static __device__ __forceinline__ void store(T* p, f32x4 v) {
    *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
};

template <>
struct Vals<TGX_DTYPE_F16, 4> {
  using T = uint16_t;
  using Raw = u32x2;
  static __device__ __forceinline__ Raw load(const T* p) {
    return *reinterpret_cast<const u32x2*>(p);
  }
  static __device__ __forceinline__ f32x4 widen(Raw r) {
    f32x4 v;
    float a, b, c, d;
    f16_pair(r[0], a, b);
    f16_pair(r[1], c, d);
    v[0] = a; v[1] = b; v[2] = c; v[3] = d;
    return v;
  }
  static __device__ __forceinline__ void store(T* p, f32x4 v) {
    *reinterpret_cast<u32x2*>(p) = u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
  }
};

// Host: element size of a TGX_DTYPE_* code, 0 for an unknown code.
inline int dtype_bytes(int dtype) {
  return dtype == TGX_DTYPE_F32 ? 4 : (dtype == TGX_DTYPE_BF16 || dtype == TGX_DTYPE_F16) ? 2 : 0;
}

}  // namespace tgx
