// Online-softmax state (running max m, denominator l, weighted sum acc) held
// per lane, plus the merges used when several edge groups of one wave, or
// several chunks of one hub row, each hold a partial state of the same row.
#pragma once

#include "tgx_device.h"

namespace tgx {

template <int N>
struct SoftState {
  float m;
  float l;
  float acc[N];

  __device__ __forceinline__ void init() {
    m = kNegInf;
    l = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) acc[k] = 0.f;
  }

  // Rescale to a new running max (m_new >= m, finite).
  __device__ __forceinline__ void rescale(float m_new) {
    const float sc = (m == kNegInf) ? 0.f : fast_exp(m - m_new);
    l *= sc;
#pragma unroll
    for (int k = 0; k < N; ++k) acc[k] *= sc;
    m = m_new;
  }

  // Merge another partial state of the same row.
  __device__ __forceinline__ void merge(float m2, float l2, const float (&acc2)[N]) {
    const float mn = fmaxf(m, m2);
    if (mn == kNegInf) return;
    const float a = (m == kNegInf) ? 0.f : fast_exp(m - mn);
    const float b = (m2 == kNegInf) ? 0.f : fast_exp(m2 - mn);
    l = l * a + l2 * b;
#pragma unroll
    for (int k = 0; k < N; ++k) acc[k] = acc[k] * a + acc2[k] * b;
    m = mn;
  }

  // Merge with the lane at lane ^ mask.
  __device__ __forceinline__ void merge_xor(int mask) {
    const float m2 = __shfl_xor(m, mask, 64);
    const float l2 = __shfl_xor(l, mask, 64);
    float acc2[N];
#pragma unroll
    for (int k = 0; k < N; ++k) acc2[k] = __shfl_xor(acc[k], mask, 64);
    merge(m2, l2, acc2);
  }
};

__device__ __forceinline__ float leaky_relu(float z, float slope) {
  return z > 0.f ? z : z * slope;
}

}  // namespace tgx
