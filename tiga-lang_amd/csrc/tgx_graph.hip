// Graph indexing on the device: exclusive scan, per-edge destination index,
// stable CSR transpose (LSD radix sort of col_idx) and the deterministic
// degree-binned row partition.
//
// All of these are integer kernels; every output is a pure function of the
// input (no atomics decide positions), so results are bit-identical across
// runs.  LDS integer atomics are used only to count, never to place.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstring>
#include <vector>

#include "tgx_device.h"
#include "tgx_host.h"

namespace tgx {
namespace {

constexpr int kBlock = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kBlock * kScanItems;  // 4096 ints per block

template <typename I>
__device__ __forceinline__ int64_t ld_idx(const I* p, int64_t i) {
  return static_cast<int64_t>(p[i]);
}

// Inclusive scan across one 64-lane wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    int t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

// Exclusive scan over the block; returns the thread's exclusive prefix and
// writes the block total to *total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds4, int* total) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) lds4[wave] = inc;
  __syncthreads();
  int base = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; ++w) {
    int t = lds4[w];
    if (w < wave) base += t;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return base + inc - v;
}

__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(
    const int32_t* __restrict__ in, int64_t n, int32_t* __restrict__ partial) {
  __shared__ int lds4[kBlock / kWave];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t idx = base + static_cast<int64_t>(k) * kBlock + threadIdx.x;
    if (idx < n) s += in[idx];
  }
  int total;
  block_exclusive_scan(s, lds4, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// Scan of one tile with a per-block carry-in.
__global__ __launch_bounds__(kBlock) void scan_tile_kernel(
    const int32_t* __restrict__ in, int32_t* __restrict__ out, int64_t n,
    const int32_t* __restrict__ carry, int32_t* __restrict__ total_dev) {
  __shared__ int lds4[kBlock / kWave];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  int v[kScanItems];
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t idx = base + k;
    v[k] = idx < n ? in[idx] : 0;
    s += v[k];
  }
  int total;
  int prefix = block_exclusive_scan(s, lds4, &total);
  prefix += carry ? carry[blockIdx.x] : 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t idx = base + k;
    if (idx < n) out[idx] = prefix;
    prefix += v[k];
  }
  if (total_dev && blockIdx.x == gridDim.x - 1 && threadIdx.x == kBlock - 1)
    *total_dev = prefix;
}

}  // namespace

size_t scan_scratch_ints(int64_t n) {
  size_t total = 0;
  while (n > kScanTile) {
    n = ceil_div(n, kScanTile);
    total += static_cast<size_t>(n) + 64;
  }
  return total + 64;
}

int scan_exclusive_i32(const int32_t* in, int32_t* out, int64_t n,
                       int32_t* total_dev, int32_t* scratch, hipStream_t stream) {
  if (n <= 0) {
    if (total_dev) TGX_HIP(hipMemsetAsync(total_dev, 0, sizeof(int32_t), stream));
    return TGX_OK;
  }
  const int64_t blocks = ceil_div(n, kScanTile);
  if (blocks == 1) {
    scan_tile_kernel<<<1, kBlock, 0, stream>>>(in, out, n, nullptr, total_dev);
    TGX_LAUNCHED("scan_tile_kernel");
    return TGX_OK;
  }
  int32_t* partial = scratch;
  int32_t* rest = scratch + align_up(static_cast<size_t>(blocks), 64);
  scan_reduce_kernel<<<blocks, kBlock, 0, stream>>>(in, n, partial);
  TGX_LAUNCHED("scan_reduce_kernel");
  int st = scan_exclusive_i32(partial, partial, blocks, nullptr, rest, stream);
  if (st != TGX_OK) return st;
  scan_tile_kernel<<<blocks, kBlock, 0, stream>>>(in, out, n, partial, total_dev);
  TGX_LAUNCHED("scan_tile_kernel");
  return TGX_OK;
}

namespace {

// ---------------------------------------------------------------------------
// destination index: one wave per row writes the row id over its edge range.
template <typename I, typename O>
__global__ __launch_bounds__(kBlock) void destination_index_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, O* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) +
                      threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t b = ld_idx(row_ptr, row), e = ld_idx(row_ptr, row + 1);
  for (int64_t k = b + lane_id(); k < e; k += kWave) out[k] = static_cast<O>(row);
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort of 32-bit keys with 32-bit payload (8-bit digits).
constexpr int kSortItems = 8;
constexpr int kSortTile = kBlock * kSortItems;  // 2048 keys per block

template <typename K>
__device__ __forceinline__ uint32_t key_at(const K* keys, int64_t i) {
  return static_cast<uint32_t>(keys[i]);
}

template <typename K>
__global__ __launch_bounds__(kBlock) void radix_hist_kernel(
    const K* __restrict__ keys, int64_t n, int shift, int nblocks,
    int32_t* __restrict__ hist) {
  __shared__ int counts[256];
  counts[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    int64_t idx = base + r * kBlock + threadIdx.x;
    if (idx < n) atomicAdd(&counts[(key_at(keys, idx) >> shift) & 255u], 1);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = counts[threadIdx.x];
}

// Scatter one tile.  Keys are visited in round-major, then lane order, which
// is exactly the tile's index order, so equal digits keep their order.
// vals_in == nullptr means the payload is the key's own index.
template <typename K>
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(
    const K* __restrict__ keys_in, const int32_t* __restrict__ vals_in,
    int64_t n, int shift, int nblocks, const int32_t* __restrict__ offsets,
    uint32_t* __restrict__ keys_out, int32_t* __restrict__ vals_out) {
  __shared__ int running[256];
  __shared__ int wave_count[kBlock / kWave][256];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  running[threadIdx.x] =
      offsets[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x];
  for (int w = 0; w < kBlock / kWave; ++w) wave_count[w][threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t idx = base + r * kBlock + threadIdx.x;
    const bool valid = idx < n;
    uint32_t key = valid ? key_at(keys_in, idx) : 0u;
    int32_t val = valid ? (vals_in ? vals_in[idx] : static_cast<int32_t>(idx)) : 0;
    uint32_t digit = (key >> shift) & 255u;
    // Lanes of this wave holding the same digit.
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      uint64_t bal = __ballot((digit >> b) & 1u);
      peers &= ((digit >> b) & 1u) ? bal : ~bal;
    }
    const int lane_rank = __popcll(peers & lt_mask);
    if (valid && lane_rank == 0) wave_count[wave][digit] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = running[digit] + lane_rank;
      for (int w = 0; w < wave; ++w) pos += wave_count[w][digit];
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
    int add = 0;
#pragma unroll
    for (int w = 0; w < kBlock / kWave; ++w) {
      add += wave_count[w][threadIdx.x];
      wave_count[w][threadIdx.x] = 0;
    }
    running[threadIdx.x] += add;
    __syncthreads();
  }
}

// out[k] for k in [0, n_keys] = number of sorted keys < k (lower bound), i.e.
// the CSR row pointer of the rows the keys name.
template <typename O>
__global__ __launch_bounds__(kBlock) void run_end_fill_kernel(
    const uint32_t* __restrict__ sorted_keys, int64_t n, int64_t n_keys,
    O* __restrict__ row_ptr) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (k > n_keys) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(sorted_keys[mid]) < k) lo = mid + 1; else hi = mid;
  }
  row_ptr[k] = static_cast<O>(lo);
}

// col[i] = src[perm[i]]: the source id of each edge in destination order.
template <typename S>
__global__ __launch_bounds__(kBlock) void gather_src_kernel(
    const int32_t* __restrict__ perm, const S* __restrict__ src, int64_t n,
    S* __restrict__ col) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  col[i] = src[perm[i]];
}

// Varlen block-diagonal relation: sequence k owns positions [cu[k], cu[k+1]).
template <typename I>
__global__ __launch_bounds__(kBlock) void varlen_seq_edges_kernel(
    const I* __restrict__ cu, int64_t n_seq, int causal, int32_t* __restrict__ out) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (k >= n_seq) return;
  const int64_t len = ld_idx(cu, k + 1) - ld_idx(cu, k);
  out[k] = static_cast<int32_t>(causal ? len * (len + 1) / 2 : len * len);
}

// One wave per position: row i of sequence k (start s, length L) relates to
// sources s..i (causal) or s..s+L-1; its edges start at the sequence's first
// edge plus the edges of the earlier rows of the same sequence.
template <typename I>
__global__ __launch_bounds__(kBlock) void varlen_rows_kernel(
    const I* __restrict__ cu, int64_t n_seq, const int32_t* __restrict__ seq_edge0,
    int causal, int64_t total, I* __restrict__ row_ptr, I* __restrict__ col) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) +
                      threadIdx.x / kWave;
  if (row >= total) return;
  // Largest k < n_seq with cu[k] <= row (empty sequences share a start).
  int64_t lo = 0, hi = n_seq - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (ld_idx(cu, mid) <= row) lo = mid; else hi = mid - 1;
  }
  const int64_t s = ld_idx(cu, lo);
  const int64_t len = ld_idx(cu, lo + 1) - s;
  const int64_t p = row - s;
  if (p < 0 || p >= len) return;  // only when cu_seqlens is malformed
  const int64_t start = static_cast<int64_t>(seq_edge0[lo]) +
                        (causal ? p * (p + 1) / 2 : p * len);
  const int64_t deg = causal ? p + 1 : len;
  if (lane_id() == 0) {
    row_ptr[row] = static_cast<I>(start);
    if (row == total - 1) row_ptr[total] = static_cast<I>(start + deg);
  }
  for (int64_t j = lane_id(); j < deg; j += kWave) col[start + j] = static_cast<I>(s + j);
}

__global__ __launch_bounds__(kBlock) void gather_rows_kernel(
    const int32_t* __restrict__ perm, const int32_t* __restrict__ erow, int64_t n,
    int32_t* __restrict__ col_t, int32_t* __restrict__ inv_perm) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  const int32_t e = perm[i];
  col_t[i] = erow[e];
  if (inv_perm) inv_perm[e] = static_cast<int32_t>(i);
}

// ---------------------------------------------------------------------------
// Degree bins.  Tile of kScanTile rows per block, rows owned in blocked order
// (thread t owns rows t*16 .. t*16+15 of the tile).
template <typename I>
__device__ __forceinline__ int degree_bin(const I* row_ptr, int64_t row,
                                          const int64_t* ub, int n_bins) {
  const int64_t d = ld_idx(row_ptr, row + 1) - ld_idx(row_ptr, row);
  int b = 0;
  while (b < n_bins - 1 && d > ub[b]) ++b;
  return b;
}

struct Bounds {
  int64_t ub[8];
};

template <typename I>
__global__ __launch_bounds__(kBlock) void bin_count_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, Bounds bounds, int n_bins,
    int nblocks, int32_t* __restrict__ counts) {
  __shared__ int c[8];
  if (threadIdx.x < 8) c[threadIdx.x] = 0;
  __syncthreads();
  int local[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  for (int k = 0; k < kScanItems; ++k) {
    int64_t row = base + k;
    if (row < n_rows) local[degree_bin(row_ptr, row, bounds.ub, n_bins)]++;
  }
  for (int b = 0; b < n_bins; ++b)
    if (local[b]) atomicAdd(&c[b], local[b]);
  __syncthreads();
  if (threadIdx.x < n_bins)
    counts[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = c[threadIdx.x];
}

template <typename I>
__global__ __launch_bounds__(kBlock) void bin_scatter_kernel(
    const I* __restrict__ row_ptr, int64_t n_rows, Bounds bounds, int n_bins,
    int nblocks, const int32_t* __restrict__ offsets, int32_t* __restrict__ rows_out) {
  __shared__ int lds4[kBlock / kWave];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  unsigned char bin[kScanItems];
  for (int k = 0; k < kScanItems; ++k) {
    int64_t row = base + k;
    bin[k] = row < n_rows ? degree_bin(row_ptr, row, bounds.ub, n_bins) : 255;
  }
  for (int b = 0; b < n_bins; ++b) {
    int cnt = 0;
    for (int k = 0; k < kScanItems; ++k) cnt += bin[k] == b;
    int total;
    int pos = block_exclusive_scan(cnt, lds4, &total);
    pos += offsets[static_cast<int64_t>(b) * nblocks + blockIdx.x];
    for (int k = 0; k < kScanItems; ++k)
      if (bin[k] == b) rows_out[pos++] = static_cast<int32_t>(base + k);
  }
}

template <typename I>
__global__ __launch_bounds__(kBlock) void split_count_kernel(
    const I* __restrict__ row_ptr, const int32_t* __restrict__ rows, int64_t n,
    int32_t chunk, int32_t* __restrict__ out) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (k >= n) return;
  const int64_t r = rows[k];
  const int64_t d = ld_idx(row_ptr, r + 1) - ld_idx(row_ptr, r);
  out[k] = static_cast<int32_t>((d + chunk - 1) / chunk);
}

}  // namespace
}  // namespace tgx

using namespace tgx;

extern "C" int tgx_destination_index(const void* row_ptr, int idx_bits, int64_t n_rows,
                                     int64_t n_edges, void* out, int out_bits,
                                     void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(out_bits == 32 || out_bits == 64, "out_bits must be 32 or 64");
  TGX_REQUIRE(n_rows >= 0 && n_edges >= 0, "negative size");
  if (n_rows == 0 || n_edges == 0) return TGX_OK;
  TGX_REQUIRE(row_ptr && out, "null pointer");
  TGX_REQUIRE(out_bits == 64 || n_rows <= INT32_MAX, "row ids overflow int32");
  const int64_t blocks = ceil_div(n_rows, kBlock / kWave);
  hipStream_t s = as_stream(stream);
  if (idx_bits == 32) {
    if (out_bits == 32)
      destination_index_kernel<<<blocks, kBlock, 0, s>>>(
          static_cast<const int32_t*>(row_ptr), n_rows, static_cast<int32_t*>(out));
    else
      destination_index_kernel<<<blocks, kBlock, 0, s>>>(
          static_cast<const int32_t*>(row_ptr), n_rows, static_cast<int64_t*>(out));
  } else {
    if (out_bits == 32)
      destination_index_kernel<<<blocks, kBlock, 0, s>>>(
          static_cast<const int64_t*>(row_ptr), n_rows, static_cast<int32_t*>(out));
    else
      destination_index_kernel<<<blocks, kBlock, 0, s>>>(
          static_cast<const int64_t*>(row_ptr), n_rows, static_cast<int64_t*>(out));
  }
  TGX_LAUNCHED("destination_index_kernel");
  return TGX_OK;
}

namespace {

// Scratch of one stable sort of n keys: two key and two payload buffers, the
// per-block digit histogram and its scan scratch.
void carve_sort(Carve& c, int64_t n) {
  const int64_t nblocks = ceil_div(n, kSortTile);
  c.take<uint32_t>(n);
  c.take<uint32_t>(n);
  c.take<int32_t>(n);
  c.take<int32_t>(n);
  c.take<int32_t>(256 * nblocks);
  c.take<int32_t>(scan_scratch_ints(256 * nblocks));
}

// Stable LSD radix sort (8-bit digits) of keys in [0, key_range) carrying the
// element index.  Writes the sorting permutation to perm and returns the
// buffer that holds the sorted keys.  Scratch is carved from c in the order
// carve_sort lays it out.
template <typename K>
uint32_t* stable_sort_by_key(const K* keys, int64_t n, int64_t key_range, int32_t* perm,
                             Carve& c, hipStream_t s, int* status) {
  const int nb = static_cast<int>(ceil_div(n, kSortTile));
  uint32_t* kbuf[2] = {c.take<uint32_t>(n), c.take<uint32_t>(n)};
  int32_t* vbuf[2] = {c.take<int32_t>(n), c.take<int32_t>(n)};
  const int64_t hist_n = 256 * static_cast<int64_t>(nb);
  int32_t* hist = c.take<int32_t>(hist_n);
  int32_t* scratch = c.take<int32_t>(scan_scratch_ints(hist_n));
  int bits = 0;
  while (bits < 32 && (static_cast<int64_t>(1) << bits) < key_range) ++bits;
  const int passes = bits == 0 ? 1 : (bits + 7) / 8;
  *status = TGX_OK;
  for (int p = 0; p < passes; ++p) {
    const int shift = 8 * p;
    uint32_t* kout = kbuf[p % 2];
    int32_t* vout = (p == passes - 1) ? perm : vbuf[p % 2];
    if (p == 0)
      radix_hist_kernel<K><<<nb, kBlock, 0, s>>>(keys, n, shift, nb, hist);
    else
      radix_hist_kernel<uint32_t><<<nb, kBlock, 0, s>>>(kbuf[(p - 1) % 2], n, shift, nb,
                                                        hist);
    if (hipGetLastError() != hipSuccess) {
      set_error("radix_hist_kernel launch failed");
      *status = TGX_INTERNAL;
      return nullptr;
    }
    *status = scan_exclusive_i32(hist, hist, hist_n, nullptr, scratch, s);
    if (*status != TGX_OK) return nullptr;
    // The first pass reads the keys in place with the element index as
    // payload; the last pass writes its payload straight into perm.
    if (p == 0)
      radix_scatter_kernel<K><<<nb, kBlock, 0, s>>>(keys, nullptr, n, shift, nb, hist,
                                                    kout, vout);
    else
      radix_scatter_kernel<uint32_t><<<nb, kBlock, 0, s>>>(
          kbuf[(p - 1) % 2], vbuf[(p - 1) % 2], n, shift, nb, hist, kout, vout);
    if (hipGetLastError() != hipSuccess) {
      set_error("radix_scatter_kernel launch failed");
      *status = TGX_INTERNAL;
      return nullptr;
    }
  }
  return kbuf[(passes - 1) % 2];
}

size_t transpose_bytes(int64_t n_edges) {
  Carve c{nullptr, 0};
  carve_sort(c, n_edges);
  c.take<int32_t>(n_edges);  // destination row per edge
  return align_up(c.used);
}

}  // namespace

extern "C" int tgx_csr_transpose_workspace(int64_t n_dst, int64_t n_src,
                                           int64_t n_edges, size_t* bytes) {
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_dst >= 0 && n_src >= 0 && n_edges >= 0, "negative size");
  *bytes = transpose_bytes(n_edges);
  return TGX_OK;
}

template <typename I>
static int transpose_impl(const I* row_ptr, const I* col, int64_t n_dst, int64_t n_src,
                          int64_t E, int32_t* row_ptr_t, int32_t* col_t,
                          int32_t* perm, int32_t* inv_perm, void* ws, size_t ws_bytes,
                          hipStream_t s) {
  const size_t need = transpose_bytes(E);
  TGX_REQUIRE(ws_bytes >= need, "workspace too small: need %zu bytes", need);
  Carve c{static_cast<char*>(ws), ws_bytes};
  int st = TGX_OK;
  const uint32_t* sorted = stable_sort_by_key(col, E, n_src, perm, c, s, &st);
  if (st != TGX_OK) return st;
  int32_t* erow = c.take<int32_t>(E);
  // row_ptr_t = lower bound of every source id in [0, n_src].
  run_end_fill_kernel<int32_t><<<ceil_div(n_src + 1, kBlock), kBlock, 0, s>>>(
      sorted, E, n_src, row_ptr_t);
  TGX_LAUNCHED("run_end_fill_kernel");
  destination_index_kernel<<<ceil_div(n_dst, kBlock / kWave), kBlock, 0, s>>>(
      row_ptr, n_dst, erow);
  TGX_LAUNCHED("destination_index_kernel");
  gather_rows_kernel<<<ceil_div(E, kBlock), kBlock, 0, s>>>(perm, erow, E, col_t, inv_perm);
  TGX_LAUNCHED("gather_rows_kernel");
  return TGX_OK;
}

extern "C" int tgx_csr_transpose(const void* row_ptr, const void* col, int idx_bits,
                                 int64_t n_dst, int64_t n_src, int64_t n_edges,
                                 int32_t* row_ptr_t, int32_t* col_t, int32_t* perm,
                                 int32_t* inv_perm, void* ws, size_t ws_bytes,
                                 void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_dst >= 0 && n_src >= 0 && n_edges >= 0, "negative size");
  TGX_REQUIRE(n_edges <= INT32_MAX && n_dst <= INT32_MAX && n_src < INT32_MAX,
              "transpose supports < 2^31 edges and nodes");
  TGX_REQUIRE(row_ptr_t, "null row_ptr_t");
  hipStream_t s = as_stream(stream);
  if (n_edges == 0) {
    TGX_HIP(hipMemsetAsync(row_ptr_t, 0, sizeof(int32_t) * (n_src + 1), s));
    return TGX_OK;
  }
  TGX_REQUIRE(row_ptr && col && col_t && perm && ws, "null pointer");
  if (idx_bits == 32)
    return transpose_impl(static_cast<const int32_t*>(row_ptr),
                          static_cast<const int32_t*>(col), n_dst, n_src, n_edges,
                          row_ptr_t, col_t, perm, inv_perm, ws, ws_bytes, s);
  return transpose_impl(static_cast<const int64_t*>(row_ptr),
                        static_cast<const int64_t*>(col), n_dst, n_src, n_edges,
                        row_ptr_t, col_t, perm, inv_perm, ws, ws_bytes, s);
}

// ---------------------------------------------------------------------------
extern "C" int tgx_plan_degree_bins_workspace(int64_t n_rows, int n_bins, size_t* bytes) {
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_rows >= 0 && n_bins >= 1 && n_bins <= 8, "n_bins must be in [1, 8]");
  const int64_t nblocks = ceil_div(n_rows, kScanTile) > 0 ? ceil_div(n_rows, kScanTile) : 1;
  Carve c{nullptr, 0};
  c.take<int32_t>(nblocks * n_bins + 64);
  c.take<int32_t>(scan_scratch_ints(nblocks * n_bins));
  *bytes = align_up(c.used);
  return TGX_OK;
}

extern "C" int tgx_plan_degree_bins(const void* row_ptr, int idx_bits, int64_t n_rows,
                                    const int64_t* upper_bounds, int n_bins,
                                    int32_t* rows_out, int64_t* bin_offsets_host,
                                    void* ws, size_t ws_bytes, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_bins >= 1 && n_bins <= 8, "n_bins must be in [1, 8]");
  TGX_REQUIRE(upper_bounds && bin_offsets_host, "null host pointer");
  TGX_REQUIRE(n_rows >= 0 && n_rows <= INT32_MAX, "n_rows must fit int32");
  for (int b = 1; b < n_bins; ++b)
    TGX_REQUIRE(upper_bounds[b] > upper_bounds[b - 1], "upper_bounds must ascend");
  if (n_rows == 0) {
    for (int b = 0; b <= n_bins; ++b) bin_offsets_host[b] = 0;
    return TGX_OK;
  }
  TGX_REQUIRE(row_ptr && rows_out && ws, "null pointer");
  size_t need = 0;
  tgx_plan_degree_bins_workspace(n_rows, n_bins, &need);
  TGX_REQUIRE(ws_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const int nblocks = static_cast<int>(ceil_div(n_rows, kScanTile));
  Carve c{static_cast<char*>(ws), ws_bytes};
  int32_t* counts = c.take<int32_t>(static_cast<int64_t>(nblocks) * n_bins + 64);
  int32_t* scratch = c.take<int32_t>(scan_scratch_ints(static_cast<int64_t>(nblocks) * n_bins));
  Bounds bd{};
  for (int b = 0; b < 8; ++b) bd.ub[b] = b < n_bins ? upper_bounds[b] : INT64_MAX;
  const int64_t cn = static_cast<int64_t>(nblocks) * n_bins;
  if (idx_bits == 32)
    bin_count_kernel<<<nblocks, kBlock, 0, s>>>(static_cast<const int32_t*>(row_ptr),
                                                n_rows, bd, n_bins, nblocks, counts);
  else
    bin_count_kernel<<<nblocks, kBlock, 0, s>>>(static_cast<const int64_t*>(row_ptr),
                                                n_rows, bd, n_bins, nblocks, counts);
  TGX_LAUNCHED("bin_count_kernel");
  // Per-bin starts are read at counts[b * nblocks] after the scan; the total
  // lands at counts[cn].
  int st = scan_exclusive_i32(counts, counts, cn, counts + cn, scratch, s);
  if (st != TGX_OK) return st;
  if (idx_bits == 32)
    bin_scatter_kernel<<<nblocks, kBlock, 0, s>>>(static_cast<const int32_t*>(row_ptr),
                                                  n_rows, bd, n_bins, nblocks, counts,
                                                  rows_out);
  else
    bin_scatter_kernel<<<nblocks, kBlock, 0, s>>>(static_cast<const int64_t*>(row_ptr),
                                                  n_rows, bd, n_bins, nblocks, counts,
                                                  rows_out);
  TGX_LAUNCHED("bin_scatter_kernel");
  std::vector<int32_t> starts(n_bins + 1);
  for (int b = 0; b < n_bins; ++b)
    TGX_HIP(hipMemcpyAsync(&starts[b], counts + static_cast<int64_t>(b) * nblocks,
                           sizeof(int32_t), hipMemcpyDeviceToHost, s));
  TGX_HIP(hipMemcpyAsync(&starts[n_bins], counts + cn, sizeof(int32_t),
                         hipMemcpyDeviceToHost, s));
  TGX_HIP(hipStreamSynchronize(s));
  for (int b = 0; b <= n_bins; ++b) bin_offsets_host[b] = starts[b];
  if (bin_offsets_host[n_bins] != n_rows) {
    set_error("row partition lost rows: %lld of %lld",
              static_cast<long long>(bin_offsets_host[n_bins]),
              static_cast<long long>(n_rows));
    return TGX_INVALID_ARGUMENT;
  }
  return TGX_OK;
}

extern "C" int tgx_plan_split_chunks(const void* row_ptr, int idx_bits,
                                     const int32_t* split_rows, int64_t n_split,
                                     int32_t chunk_edges, int32_t* chunk_offsets,
                                     int64_t* n_chunks_host, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(chunk_edges > 0, "chunk_edges must be positive");
  TGX_REQUIRE(n_chunks_host && chunk_offsets, "null pointer");
  TGX_REQUIRE(n_split >= 0 && n_split <= kScanTile * 4096LL, "too many split rows");
  hipStream_t s = as_stream(stream);
  if (n_split == 0) {
    TGX_HIP(hipMemsetAsync(chunk_offsets, 0, sizeof(int32_t), s));
    *n_chunks_host = 0;
    return TGX_OK;
  }
  TGX_REQUIRE(row_ptr && split_rows, "null pointer");
  if (idx_bits == 32)
    split_count_kernel<<<ceil_div(n_split, kBlock), kBlock, 0, s>>>(
        static_cast<const int32_t*>(row_ptr), split_rows, n_split, chunk_edges,
        chunk_offsets);
  else
    split_count_kernel<<<ceil_div(n_split, kBlock), kBlock, 0, s>>>(
        static_cast<const int64_t*>(row_ptr), split_rows, n_split, chunk_edges,
        chunk_offsets);
  TGX_LAUNCHED("split_count_kernel");
  // Up to one scan tile of split rows the device scan needs no scratch and
  // writes the total in place.  Above that (this call has no workspace
  // argument) the per-row counts come to the host, are scanned there and go
  // back; the host buffer lives until the stream has finished both copies.
  if (n_split <= kScanTile) {
    int st = scan_exclusive_i32(chunk_offsets, chunk_offsets, n_split,
                                chunk_offsets + n_split, nullptr, s);
    if (st != TGX_OK) return st;
    int32_t total = 0;
    TGX_HIP(hipMemcpyAsync(&total, chunk_offsets + n_split, sizeof(int32_t),
                           hipMemcpyDeviceToHost, s));
    TGX_HIP(hipStreamSynchronize(s));
    *n_chunks_host = total;
    return TGX_OK;
  }
  std::vector<int32_t> host(n_split + 1);
  TGX_HIP(hipMemcpyAsync(host.data(), chunk_offsets, sizeof(int32_t) * n_split,
                         hipMemcpyDeviceToHost, s));
  TGX_HIP(hipStreamSynchronize(s));
  int64_t run = 0;
  for (int64_t k = 0; k < n_split; ++k) {
    const int32_t v = host[k];
    host[k] = static_cast<int32_t>(run);
    run += v;
  }
  TGX_REQUIRE(run <= INT32_MAX, "chunk count overflows int32");
  host[n_split] = static_cast<int32_t>(run);
  TGX_HIP(hipMemcpyAsync(chunk_offsets, host.data(), sizeof(int32_t) * (n_split + 1),
                         hipMemcpyHostToDevice, s));
  TGX_HIP(hipStreamSynchronize(s));
  *n_chunks_host = run;
  return TGX_OK;
}

// ---------------------------------------------------------------------------
// Graph builders.
namespace {

size_t coo_bytes(int64_t n_edges) {
  Carve c{nullptr, 0};
  carve_sort(c, n_edges);
  c.take<int32_t>(n_edges);  // permutation when the caller does not want it
  return align_up(c.used);
}

template <typename S, typename D>
int coo_impl(const S* src, const D* dst, int64_t n_dst, int64_t E, D* row_ptr, S* col,
             int32_t* perm, void* ws, size_t ws_bytes, hipStream_t s) {
  const size_t need = coo_bytes(E);
  TGX_REQUIRE(ws_bytes >= need, "workspace too small: need %zu bytes", need);
  Carve c{static_cast<char*>(ws), ws_bytes};
  int st = TGX_OK;
  // The permutation buffer is carved after the sort scratch, so carve the
  // sort first and take the fallback permutation from what follows.
  Carve probe = c;
  carve_sort(probe, E);
  int32_t* own_perm = probe.take<int32_t>(E);
  if (!perm) perm = own_perm;
  const uint32_t* sorted = stable_sort_by_key(dst, E, n_dst, perm, c, s, &st);
  if (st != TGX_OK) return st;
  run_end_fill_kernel<D><<<ceil_div(n_dst + 1, kBlock), kBlock, 0, s>>>(sorted, E, n_dst,
                                                                          row_ptr);
  TGX_LAUNCHED("run_end_fill_kernel");
  gather_src_kernel<S><<<ceil_div(E, kBlock), kBlock, 0, s>>>(perm, src, E, col);
  TGX_LAUNCHED("gather_src_kernel");
  return TGX_OK;
}

template <typename S>
int coo_dispatch_dst(const S* src, const void* dst, int dst_bits, int64_t n_dst, int64_t E,
                     void* row_ptr, void* col, int32_t* perm, void* ws, size_t ws_bytes,
                     hipStream_t s) {
  if (dst_bits == 32)
    return coo_impl(src, static_cast<const int32_t*>(dst), n_dst, E,
                    static_cast<int32_t*>(row_ptr), static_cast<S*>(col), perm, ws,
                    ws_bytes, s);
  return coo_impl(src, static_cast<const int64_t*>(dst), n_dst, E,
                  static_cast<int64_t*>(row_ptr), static_cast<S*>(col), perm, ws, ws_bytes,
                  s);
}

size_t varlen_csr_bytes(int64_t n_seq) {
  Carve c{nullptr, 0};
  c.take<int32_t>(n_seq + 1);
  c.take<int32_t>(scan_scratch_ints(n_seq));
  return align_up(c.used);
}

template <typename I>
int varlen_csr_impl(const I* cu, int64_t n_seq, int64_t total, int64_t n_edges, int causal,
                    I* row_ptr, I* col, void* ws, size_t ws_bytes, hipStream_t s) {
  const size_t need = varlen_csr_bytes(n_seq);
  TGX_REQUIRE(ws_bytes >= need, "workspace too small: need %zu bytes", need);
  Carve c{static_cast<char*>(ws), ws_bytes};
  int32_t* edge0 = c.take<int32_t>(n_seq + 1);
  int32_t* scratch = c.take<int32_t>(scan_scratch_ints(n_seq));
  varlen_seq_edges_kernel<I><<<ceil_div(n_seq, kBlock), kBlock, 0, s>>>(cu, n_seq, causal,
                                                                         edge0);
  TGX_LAUNCHED("varlen_seq_edges_kernel");
  int st = scan_exclusive_i32(edge0, edge0, n_seq, edge0 + n_seq, scratch, s);
  if (st != TGX_OK) return st;
  int32_t got = 0;
  TGX_HIP(hipMemcpyAsync(&got, edge0 + n_seq, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  TGX_HIP(hipStreamSynchronize(s));
  TGX_REQUIRE(got == n_edges, "cu_seqlens describe %d edges, caller sized %lld", got,
              static_cast<long long>(n_edges));
  varlen_rows_kernel<I><<<ceil_div(total, kBlock / kWave), kBlock, 0, s>>>(
      cu, n_seq, edge0, causal, total, row_ptr, col);
  TGX_LAUNCHED("varlen_rows_kernel");
  return TGX_OK;
}

}  // namespace

extern "C" int tgx_coo_to_csr_workspace(int64_t n_src, int64_t n_dst, int64_t n_edges,
                                        size_t* bytes) {
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_src >= 0 && n_dst >= 0 && n_edges >= 0, "negative size");
  *bytes = coo_bytes(n_edges);
  return TGX_OK;
}

extern "C" int tgx_coo_to_csr(const void* src, int src_bits, const void* dst, int dst_bits,
                              int64_t n_src, int64_t n_dst, int64_t n_edges, void* row_ptr,
                              void* col, int32_t* perm, void* ws, size_t ws_bytes,
                              void* stream) {
  TGX_REQUIRE(src_bits == 32 || src_bits == 64, "src_bits must be 32 or 64");
  TGX_REQUIRE(dst_bits == 32 || dst_bits == 64, "dst_bits must be 32 or 64");
  TGX_REQUIRE(n_src >= 0 && n_dst >= 0 && n_edges >= 0, "negative size");
  TGX_REQUIRE(n_edges <= INT32_MAX && n_dst < INT32_MAX,
              "the device builder supports < 2^31 edges and destinations");
  TGX_REQUIRE(row_ptr, "null row_ptr");
  hipStream_t s = as_stream(stream);
  if (n_edges == 0) {
    TGX_HIP(hipMemsetAsync(row_ptr, 0, (dst_bits / 8) * (n_dst + 1), s));
    return TGX_OK;
  }
  TGX_REQUIRE(src && dst && col && ws, "null pointer");
  if (src_bits == 32)
    return coo_dispatch_dst(static_cast<const int32_t*>(src), dst, dst_bits, n_dst, n_edges,
                            row_ptr, col, perm, ws, ws_bytes, s);
  return coo_dispatch_dst(static_cast<const int64_t*>(src), dst, dst_bits, n_dst, n_edges,
                          row_ptr, col, perm, ws, ws_bytes, s);
}

extern "C" int tgx_varlen_csr_workspace(int64_t n_seq, size_t* bytes) {
  TGX_REQUIRE(bytes, "null bytes");
  TGX_REQUIRE(n_seq >= 0, "negative size");
  *bytes = varlen_csr_bytes(n_seq);
  return TGX_OK;
}

extern "C" int tgx_varlen_csr(const void* cu_seqlens, int idx_bits, int64_t n_seq,
                              int64_t total, int64_t n_edges, int causal, void* row_ptr,
                              void* col, void* ws, size_t ws_bytes, void* stream) {
  TGX_REQUIRE(idx_bits == 32 || idx_bits == 64, "idx_bits must be 32 or 64");
  TGX_REQUIRE(n_seq >= 0 && total >= 0 && n_edges >= 0, "negative size");
  TGX_REQUIRE(n_edges <= INT32_MAX, "the device builder supports < 2^31 edges");
  TGX_REQUIRE(idx_bits == 64 || total <= INT32_MAX, "positions overflow int32");
  TGX_REQUIRE(row_ptr, "null row_ptr");
  hipStream_t s = as_stream(stream);
  if (total == 0 || n_seq == 0) {
    TGX_REQUIRE(total == 0 && n_edges == 0, "no sequences but %lld positions",
                static_cast<long long>(total));
    TGX_HIP(hipMemsetAsync(row_ptr, 0, idx_bits / 8, s));
    return TGX_OK;
  }
  TGX_REQUIRE(cu_seqlens && col && ws, "null pointer");
  if (idx_bits == 32)
    return varlen_csr_impl(static_cast<const int32_t*>(cu_seqlens), n_seq, total, n_edges,
                           causal, static_cast<int32_t*>(row_ptr),
                           static_cast<int32_t*>(col), ws, ws_bytes, s);
  return varlen_csr_impl(static_cast<const int64_t*>(cu_seqlens), n_seq, total, n_edges,
                         causal, static_cast<int64_t*>(row_ptr), static_cast<int64_t*>(col),
                         ws, ws_bytes, s);
}
