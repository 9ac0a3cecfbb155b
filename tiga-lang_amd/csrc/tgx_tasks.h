// Row-task decoding shared by the sparse kernels.
//
// A launch over a tgx_row_plan is a flat list of wave tasks laid out as
//   [ split-row chunks | whole rows (1..wave_max edges) | empty-row groups ]
// so the heavy hub chunks start first.  Each wave decodes its own task from
// its global wave index; every decoded value is wave-uniform.
#pragma once

#include "tgx.h"
#include "tgx_device.h"

namespace tgx {

constexpr int kTaskBlock = 256;                      // 4 waves per workgroup
constexpr int kWavesPerBlock = kTaskBlock / kWave;
constexpr int kEmptyPerWave = 8;                     // empty rows per wave

struct PlanView {
  const int32_t* rows;
  const int32_t* chunk_off;
  int64_t n_empty, n_wave, n_split, n_chunks;
  int32_t chunk_edges;
};

inline PlanView plan_view(const tgx_row_plan& p) {
  return PlanView{p.rows_dev, p.chunk_offsets_dev, p.n_empty, p.n_wave,
                  p.n_split, p.n_chunks, p.chunk_edges};
}

inline int64_t plan_waves(const PlanView& p) {
  return p.n_chunks + p.n_wave + (p.n_empty + kEmptyPerWave - 1) / kEmptyPerWave;
}

enum TaskKind { kTaskNone = 0, kTaskChunk = 1, kTaskRow = 2, kTaskEmpty = 3 };

struct Task {
  int kind;
  int row;        // destination row (row/chunk tasks)
  int64_t e0, e1; // edge range
  int slot;       // chunk index for chunk tasks
  int64_t empty0; // first index into rows[] for an empty group
  int n_empty;    // rows in the empty group
};

template <typename I>
__device__ __forceinline__ Task decode_task(const PlanView& p, const I* row_ptr,
                                            int64_t wave_id) {
  Task t;
  t.kind = kTaskNone;
  if (wave_id < p.n_chunks) {
    const int c = static_cast<int>(wave_id);
    // Split row owning chunk c: last k with chunk_off[k] <= c.
    int lo = 0, hi = static_cast<int>(p.n_split) - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (p.chunk_off[mid] <= c) lo = mid; else hi = mid - 1;
    }
    lo = uniform(lo);
    const int row = uniform(p.rows[p.n_empty + p.n_wave + lo]);
    const int64_t rb = static_cast<int64_t>(row_ptr[row]);
    const int64_t re = static_cast<int64_t>(row_ptr[row + 1]);
    const int64_t e0 = rb + static_cast<int64_t>(c - p.chunk_off[lo]) * p.chunk_edges;
    t.kind = kTaskChunk;
    t.row = row;
    t.e0 = e0;
    t.e1 = e0 + p.chunk_edges < re ? e0 + p.chunk_edges : re;
    t.slot = c;
    return t;
  }
  wave_id -= p.n_chunks;
  if (wave_id < p.n_wave) {
    const int row = uniform(p.rows[p.n_empty + wave_id]);
    t.kind = kTaskRow;
    t.row = row;
    t.e0 = static_cast<int64_t>(row_ptr[row]);
    t.e1 = static_cast<int64_t>(row_ptr[row + 1]);
    t.slot = -1;
    return t;
  }
  wave_id -= p.n_wave;
  const int64_t first = wave_id * kEmptyPerWave;
  if (first < p.n_empty) {
    t.kind = kTaskEmpty;
    t.empty0 = first;
    const int64_t left = p.n_empty - first;
    t.n_empty = static_cast<int>(left < kEmptyPerWave ? left : kEmptyPerWave);
  }
  return t;
}

__device__ __forceinline__ int64_t global_wave() {
  return static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
}

}  // namespace tgx
