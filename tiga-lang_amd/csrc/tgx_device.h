// Device-side helpers shared by the CSR message-passing kernels (gfx950 only).
//
// Lane layout used by every sparse kernel: one gathered node row is spread
// over a group of G consecutive lanes, each lane owning one 16-byte vector
// (4 x fp32 or 8 x bf16).  A 64-wide wave therefore covers 64/G rows per
// vector load.  Per-head dot products reduce over the lanes that hold one
// head with DPP butterflies (quad_perm, row_half_mirror, row_mirror), which
// stay inside a 16-lane DPP row and never touch LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tgx {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// ---- DPP lane exchange ------------------------------------------------------
// dpp_ctrl encodings (GCN/CDNA DPP): quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in 1,2,4,8,16,32,64); every lane of
// the group receives the group total.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<0xB1>(v);
  if constexpr (N >= 4) v += dpp<0x4E>(v);
  if constexpr (N >= 8) v += dpp<0x141>(v);
  if constexpr (N >= 16) v += dpp<0x140>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<0xB1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<0x4E>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<0x140>(v));
  if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if constexpr (N >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// ---- wave-uniform helpers ---------------------------------------------------
__device__ __forceinline__ int uniform(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int read_lane(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

// ---- bf16 <-> fp32 ----------------------------------------------------------
// A 16-byte lane vector holds eight bf16 values; element 2k sits in the low
// half of word k.
__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __uint_as_float(w & 0xFFFF0000u);
}
// Round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu))
    return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}
__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = bf16_lo(v[k]);
    f[2 * k + 1] = bf16_hi(v[k]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = pack_bf16x2(f[2 * k], f[2 * k + 1]);
  return v;
}

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }

}  // namespace tgx
