/*
 * tgx.h - C ABI of libtgx_hip.so, the MI355X (gfx950) execution provider for
 * Tiga's CSR message-passing hot path.
 *
 * Conventions (kept from the reference runtime ABI, include/tiga/Runtime/
 * CAPI.h:21-35 and python/tiga/runtime/__init__.py:279-285):
 *   - every entry point returns an int status, TGX_OK == 0; a non-zero status
 *     leaves a message readable through tgx_last_error();
 *   - pointers named *_dev or documented "device" are HIP device pointers;
 *     everything else is host memory;
 *   - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream);
 *     all work is enqueued on it in order and no entry point synchronises the
 *     host unless its comment says so (planning calls copy counts back);
 *   - the library never allocates device memory: outputs, gradients and
 *     workspaces are owned by the caller (the reference allocates outputs
 *     through Torch, python/tiga/interop/torch/provider.py:170-198);
 *   - index arrays supplied by the caller (row_ptr, col_idx) are int32 or
 *     int64, selected by idx_bits (32 or 64); arrays produced by this library
 *     (transposed CSR, permutations, plans) are int32.
 *   - CSR is destination-row: row i lists the sources of destination i
 *     (reference Graph.from_csr, python/tiga/interop/torch/graph.py:153-190).
 *   - kernels trust the CSR: row_ptr must be monotonic from 0 to n_edges and
 *     every col_idx value must lie in [0, n_src); gathers are not
 *     bounds-checked on the device (the Python front end checks once per
 *     graph before the first launch, tiga/graph.py Graph._kernel_csr).
 */
#ifndef TGX_H_
#define TGX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; same meaning as GFRTStatus (CAPI.h:21-27). */
enum {
  TGX_OK = 0,
  TGX_INVALID_ARGUMENT = 1,
  TGX_UNSUPPORTED = 2,
  TGX_OUT_OF_MEMORY = 3,
  TGX_INTERNAL = 4
};

/* Element types: TGX_DTYPE_BF16 / TGX_DTYPE_F16 are raw 16-bit storage,
 * TGX_DTYPE_F32 is float.  The attention tiles take BF16 and F16; the sum
 * takes all three (its weights, partials and sums stay fp32). */
enum { TGX_DTYPE_BF16 = 0, TGX_DTYPE_F16 = 1, TGX_DTYPE_F32 = 2 };

/* Human-readable name of a status code. */
const char* tgx_status_string(int status);
/* Message recorded by the last failing call on this thread ("" if none). */
const char* tgx_last_error(void);
/* ABI version of this header (bumped on any signature change). */
int tgx_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Graph indexing                                                            */
/* ------------------------------------------------------------------------ */

/* Per-edge destination row id: out[e] = i for row_ptr[i] <= e < row_ptr[i+1].
 * Replaces Graph.destination_index (interop/torch/graph.py:1212-1222,
 * repeat_interleave(arange(num_dst), degree)).  out_bits selects int32/int64
 * output. */
int tgx_destination_index(const void* row_ptr_dev, int idx_bits, int64_t n_rows,
                          int64_t n_edges, void* out_dev, int out_bits,
                          void* stream);

/* Workspace bytes needed by tgx_csr_transpose. */
int tgx_csr_transpose_workspace(int64_t n_dst, int64_t n_src, int64_t n_edges,
                                size_t* bytes);

/* Stable transpose of a destination-row CSR into a source-row CSR.
 * Replaces Graph.transpose -> from_coo (interop/torch/graph.py:675-685 and
 * 193-231: argsort(col_idx, stable=True), bincount, cumsum).
 *   row_ptr_t_dev [n_src+1]  int32: exclusive prefix of source out-degrees
 *   col_t_dev     [n_edges]  int32: destination id of each transposed edge
 *   perm_dev      [n_edges]  int32: original edge id of each transposed edge
 *                                   (= argsort(col_idx, stable=True))
 *   inv_perm_dev  [n_edges]  int32: transposed position of each original edge
 *                                   (inv_perm[perm[k]] = k); may be NULL
 * Deterministic: output is bit-identical across runs. */
int tgx_csr_transpose(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                      int64_t n_dst, int64_t n_src, int64_t n_edges,
                      int32_t* row_ptr_t_dev, int32_t* col_t_dev,
                      int32_t* perm_dev, int32_t* inv_perm_dev,
                      void* workspace_dev, size_t workspace_bytes, void* stream);

/* Workspace bytes needed by tgx_coo_to_csr. */
int tgx_coo_to_csr_workspace(int64_t n_src, int64_t n_dst, int64_t n_edges,
                             size_t* bytes);

/* Destination-row CSR from edge lists (src[e] -> dst[e]).
 * Replaces Graph.from_coo's construction step (interop/torch/graph.py:
 * 219-227: argsort(dst, stable=True), col_idx = src[order],
 * row_ptr = [0, cumsum(bincount(dst, minlength=num_dst))]); the range checks
 * of :210-218 stay with the caller.
 *   row_ptr_dev [n_dst+1] in dst's width (dst_bits)
 *   col_dev     [n_edges] in src's width (src_bits): src in stable dst order
 *   perm_dev    [n_edges] int32: argsort(dst, stable=True); may be NULL
 * Every dst must lie in [0, n_dst).  Supports n_edges, n_dst < 2^31.
 * Deterministic: output is bit-identical across runs. */
int tgx_coo_to_csr(const void* src_dev, int src_bits, const void* dst_dev,
                   int dst_bits, int64_t n_src, int64_t n_dst, int64_t n_edges,
                   void* row_ptr_dev, void* col_dev, int32_t* perm_dev,
                   void* workspace_dev, size_t workspace_bytes, void* stream);

/* Workspace bytes needed by tgx_varlen_csr. */
int tgx_varlen_csr_workspace(int64_t n_seq, size_t* bytes);

/* Materialized block-diagonal varlen relation.  Replaces the CSR build of
 * Graph.cu_seqlens (interop/torch/graph.py:260-294): position i of sequence
 * k (cu_seqlens[k] <= i < cu_seqlens[k+1]) relates to sources
 * cu_seqlens[k]..i when causal != 0, else to its whole sequence.
 *   cu_seqlens_dev [n_seq+1] (idx_bits), starting at 0, non-decreasing,
 *                  ending at total
 *   row_ptr_dev    [total+1] (idx_bits), col_dev [n_edges] (idx_bits)
 * n_edges must equal the relation's edge count (sum of L(L+1)/2 causal, L*L
 * otherwise; checked on the device, one stream synchronisation) and be
 * < 2^31. */
int tgx_varlen_csr(const void* cu_seqlens_dev, int idx_bits, int64_t n_seq,
                   int64_t total, int64_t n_edges, int causal, void* row_ptr_dev,
                   void* col_dev, void* workspace_dev, size_t workspace_bytes,
                   void* stream);

/* ------------------------------------------------------------------------ */
/* Row partition / load balancing                                            */
/* ------------------------------------------------------------------------ */

/* Workspace bytes needed by tgx_plan_degree_bins. */
int tgx_plan_degree_bins_workspace(int64_t n_rows, int n_bins, size_t* bytes);

/* Degree-binned row worklist (reference gf_degree_reset/histogram/prefix/
 * scatter, lib/Target/Triton/Translate.cpp:4043-4187, ABI
 * include/tiga/Dialect/Task/TaskOps.td:63-82), made deterministic.
 * Bin b holds rows with upper_bounds[b-1] < degree <= upper_bounds[b]
 * (upper_bounds[-1] = -1); upper_bounds is a host array, strictly ascending,
 * and its last entry must be >= the maximum degree.
 *   rows_out_dev [n_rows] int32: row ids grouped by bin, ascending inside
 *                                 each bin (a stable partition);
 *   bin_offsets_host [n_bins+1]: start of each bin in rows_out (host).
 * Synchronises `stream` to return bin_offsets_host. */
int tgx_plan_degree_bins(const void* row_ptr_dev, int idx_bits, int64_t n_rows,
                         const int64_t* upper_bounds, int n_bins,
                         int32_t* rows_out_dev, int64_t* bin_offsets_host,
                         void* workspace_dev, size_t workspace_bytes,
                         void* stream);

/* Chunk prefix for split (hub) rows: chunk_offsets_dev[k] = sum over split
 * rows r < k of ceil(degree(rows[k]) / chunk_edges), k = 0..n_split.
 * Restates the reference row-split plan (lib/Transforms/PlanSplitRows.cpp:
 * 136-147, 64-edge partials) with a caller-chosen chunk size.
 * Synchronises `stream` to return *n_chunks_host. */
int tgx_plan_split_chunks(const void* row_ptr_dev, int idx_bits,
                          const int32_t* split_rows_dev, int64_t n_split,
                          int32_t chunk_edges, int32_t* chunk_offsets_dev,
                          int64_t* n_chunks_host, void* stream);

/* Row partition consumed by the sparse kernels: rows_dev lists the empty
 * rows, then the rows done whole by one wavefront (1..wave_max edges), then
 * the split rows (> wave_max edges) whose chunks are listed by
 * chunk_offsets_dev.  Built from tgx_plan_degree_bins with upper bounds
 * {0, wave_max, INT64_MAX} and tgx_plan_split_chunks. */
typedef struct tgx_row_plan {
  int64_t n_rows;
  int64_t n_empty;
  int64_t n_wave;
  int64_t n_split;
  int64_t n_chunks;
  int32_t wave_max;
  int32_t chunk_edges;
  const int32_t* rows_dev;
  const int32_t* chunk_offsets_dev;
} tgx_row_plan;

/* Reference planner decisions, host only (restates lib/Transforms/
 * SelectKernelSchedule.cpp:136-163 annotateLoadBalance, PlanDegreeBuckets.cpp:
 * 32-143 and PlanSplitRows.cpp:84-147).
 *   histogram: host [max_degree+1] row counts per degree, or NULL.
 *   has_node_epilogue: 1 when the kernel has a node() region.
 * Outputs (host):
 *   *plan_code: 0 row-neighbor-tile, 1 degree-bucketing (worklist),
 *               2 high-degree-tail-split, 3 provider-deferred-high-degree,
 *               4 bounded-row-preferred, 5 high-degree-tail-chunked,
 *               6 tail-split with row-split partial/finalize;
 *   *utilization_milli: padding utilization (-1 when not computed);
 *   bounds_out[*n_bounds] (capacity 64): inclusive bucket upper bounds;
 *   mapping_out[*n_bounds]: 0 worklist, 1 direct-filter, 2 worklist-chunked;
 *   rows_in_bucket_out[*n_bounds];
 *   *partials_per_row, *active_rows: row-split sizing (0 when unused). */
int tgx_plan_reference_buckets(int64_t n_rows, int64_t max_degree,
                               int64_t degree_sum, const int64_t* histogram,
                               int has_node_epilogue, int* plan_code,
                               int64_t* utilization_milli, int64_t* bounds_out,
                               int* mapping_out, int64_t* rows_in_bucket_out,
                               int* n_bounds, int64_t* partials_per_row,
                               int64_t* active_rows);

/* ------------------------------------------------------------------------ */
/* Sum reducer: out[i, :] = sum_e w[e] * x[col[e], :]                        */
/* ------------------------------------------------------------------------ */

/* Forward of the weighted-sum message (reference WeightedSumPattern,
 * python/tiga/compiler/capture.py:123-145, executed by _execute_weighted_sum,
 * interop/torch/message_passing.py:2903-3345; its eager reduce_sum keeps the
 * message dtype, interop/torch/reducer_oracle.py:44-57).
 *   x_dev [n_src, F] and out_dev [n_dst, F] (fully written) of element type
 *   dtype (TGX_DTYPE_F32, _BF16 or _F16), w_dev [n_edges] fp32 or NULL
 *   (weight 1); products and sums in fp32, one rounding per output.
 *   col_dev NULL: the columns are the edge ids, i.e. x_dev [n_edges, F] is a
 *   per-edge field summed per destination row (n_src = n_edges < 2^31; the
 *   per-edge input gradients of an edge network reduce this way).
 * F may be any positive width; widths that are multiples of 4 with
 * F*4 <= 1024 bytes take the vectorised path. */
int tgx_csr_sum_fwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                    const tgx_row_plan* plan, const void* x_dev,
                    const float* w_dev, void* out_dev, int64_t n_dst,
                    int64_t n_src, int64_t F, int dtype, float* partial_dev,
                    void* stream);

/* Bytes of partial_dev scratch the sum/attention kernels need for a plan. */
int tgx_partial_bytes(const tgx_row_plan* plan, int64_t state_floats,
                      size_t* bytes);

/* Backward of the weighted sum, no float atomics:
 *   dx[j, :] = sum over transposed edges e' of j: w[perm[e']] * dout[col_t[e'], :]
 *   dw[e]    = <dout[row(e), :], x[col[e], :]>   (written at perm[e'])
 * Replaces the reference's Torch replay (message_passing.py:378-409).
 * plan_t partitions the transposed CSR.  dx_dev / dw_dev may be NULL to skip.
 * x, dout and dx are of element type dtype; w and dw are fp32. */
int tgx_csr_sum_bwd(const int32_t* row_ptr_t_dev, const int32_t* col_t_dev,
                    const int32_t* perm_dev, const tgx_row_plan* plan_t,
                    const void* x_dev, const float* w_dev,
                    const void* dout_dev, void* dx_dev, float* dw_dev,
                    int64_t n_dst, int64_t n_src, int64_t F, int dtype,
                    float* partial_dev, void* stream);

/* Per-edge dot products in edge order over the destination-row CSR:
 *   dw[e] = <dout[row(e), :], x[col[e], :]>,  e = 0 .. n_edges-1
 * (the weight gradient of the weighted sum, written contiguously; the
 * reference's Torch replay, message_passing.py:378-409).  x [n_src, F] and
 * dout [n_dst, F] of element type dtype, dw fp32.  F <= 32 (wider rows:
 * tgx_csr_sum_bwd's dw output); others return TGX_UNSUPPORTED. */
int tgx_csr_edge_dot(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                     const tgx_row_plan* plan, const void* x_dev, const void* dout_dev,
                     float* dw_dev, int64_t n_dst, int64_t n_src, int64_t F, int dtype,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* GAT additive edge attention (fp32, bf16 or fp16 in, fp32 accumulate)     */
/*   z_e = a_src . h[j] + a_dst . h[i]   per head,  s_e = LeakyReLU(z_e)     */
/*   out[i] = sum_e softmax_i(s)_e * h[j]                                     */
/* ------------------------------------------------------------------------ */

/* Forward.  h_src [n_src, H, D] (gathered per edge) and h_dst [n_dst, H, D]
 * (the row's own features) of element type `dtype` (TGX_DTYPE_F32, _BF16 or
 * _F16); pass the same pointer twice for a homogeneous relation (then
 * n_src == n_dst).  a_src/a_dst [H, D] fp32, out [n_dst, H, D] of `dtype`.
 * Scores, softmax sums and products are fp32; out is rounded once (the
 * reference's eager path accumulates 16-bit scores in fp32 and casts back,
 * reducer_oracle.py:22-41, 137).  node_state [n_dst, H, 4] fp32 receives
 * per (node, head): [0] logsumexp of the row's scores (-inf for an empty
 * row), [1] reserved for the backward (delta = <dout, out>), [2]
 * a_dst.h_dst[i], [3] a_src.h_dst[i].
 * partial_dev: tgx_partial_bytes(plan, H*D + 2*H) bytes, or with pos_dev
 * tgx_partial_bytes(plan, 2*H*D + 3*H) (NULL if no split rows).
 * pos_dev (NULL, or 16-byte aligned fp32 [n_dst, H, D]) receives for a
 * backward the row sums over the edges whose z_e > 0 of
 * softmax_i(s)_e * (h_src[j] - out[i]) (fp32, unrounded out): with it
 * tgx_gat_bwd needs no per-edge pass over the destination rows, since a
 * row's sum of the score gradients dz_e is (1 - slope) <dout[i], pos[i]>.
 * Supported shapes: any H >= 1 with D in {4, 8, 16, 32, 64, 128, 256}
 * (others return TGX_UNSUPPORTED).  Heads run in groups of a power-of-two
 * count with at most 256 values per node (H = 8, D = 64: two groups of 4),
 * one after another on `stream`, each over its strided slice of the rows.
 * The reference evaluates this edge function with its eager oracle
 * (interop/torch/message_passing.py:2848-2894 -> reducer_oracle.py:60-137). */
int tgx_gat_fwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                const tgx_row_plan* plan, const void* h_src_dev, const void* h_dst_dev,
                const float* a_src_dev, const float* a_dst_dev,
                float negative_slope, void* out_dev, float* node_state_dev,
                int64_t n_dst, int64_t n_src, int H, int D, int dtype, float* partial_dev,
                float* pos_dev, void* stream);

/* Workspace bytes for tgx_gat_bwd with these plans and element type;
 * folded != 0 for a backward given the forward's pos (it needs no per-edge
 * buffer). */
int tgx_gat_bwd_workspace(const tgx_row_plan* plan, const tgx_row_plan* plan_t,
                          int64_t n_edges, int H, int D, int dtype, int folded,
                          size_t* bytes);

/* Fused backward from the saved logsumexp (no per-edge alpha is stored by
 * the forward and no float atomics are used): dh_src, dh_dst (of `dtype`),
 * da_src, da_dst (fp32) for loss gradient dout [n_dst, H, D].  One
 * gradient buffer (dh_src == dh_dst) declares one feature tensor for both
 * roles (then h_src == h_dst and n_src == n_dst are required) and receives
 * both roles' terms, rounded once; two buffers receive the source and the
 * destination terms separately.  Uses the transposed CSR (row_ptr_t, col_t, perm, inv_perm)
 * and its plan.  node_state slot 1 (delta) is overwritten.  pos_dev: the
 * forward's pos (then inv_perm may be NULL: the destination terms come
 * from node passes), or NULL for the per-edge destination pass over the
 * CSR, which reads each edge's score gradient through inv_perm. */
int tgx_gat_bwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                const tgx_row_plan* plan, const int32_t* row_ptr_t_dev,
                const int32_t* col_t_dev, const int32_t* perm_dev,
                const int32_t* inv_perm_dev, const tgx_row_plan* plan_t,
                const void* h_src_dev, const void* h_dst_dev, const float* a_src_dev,
                const float* a_dst_dev, float negative_slope, const void* out_dev,
                float* node_state_dev, const float* pos_dev, const void* dout_dev,
                void* dh_src_dev, void* dh_dst_dev, float* da_src_dev, float* da_dst_dev,
                int64_t n_dst, int64_t n_src, int64_t n_edges, int H, int D, int dtype,
                void* workspace_dev, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Dot-product edge attention (bf16, fp16 or fp32 in, fp32 accumulate)       */
/*   s_e = scale * (k[j] . q[i]) + bias[e]   per head,                       */
/*   out[i] = sum_e softmax_i(s)_e * v[j]                                     */
/* ------------------------------------------------------------------------ */

/* Forward.  q [n_dst, H, D], k/v [n_src, H, D], out [n_dst, H, D]: element
 * type `dtype` (TGX_DTYPE_BF16, _F16 or _F32; scores, softmax sums and
 * products in fp32, the output rounded to dtype once, as the reference's
 * eager path accumulates 16-bit inputs in fp32 and casts the result back,
 * reducer_oracle.py:22-41, 137); bias [E, H] fp32 or NULL.  ml [n_dst, H, 2] fp32 receives
 * {logsumexp (-inf for an empty row), 0}.  partial_dev:
 * tgx_partial_bytes(plan, H*D + 2*H) bytes (NULL without split rows).
 * Supported: any H >= 1 with D in {8, 16, 32, 64, 128, 256, 512}.  Heads run
 * in groups of a power-of-two count with at most 512 values per node (H = 16,
 * D = 64: two groups of 8), one after another on `stream`.
 * Replaces the eager evaluation of (src.k*dst.q).sum(-1)*scale + edge.bias
 * (interop/torch/message_passing.py:2848-2894, reducer_oracle.py:60-137). */
int tgx_dot_attn_fwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                     const tgx_row_plan* plan, const void* q_dev, const void* k_dev,
                     const void* v_dev, const float* bias_dev, float scale,
                     void* out_dev, float* ml_dev, int64_t n_dst, int64_t n_src, int H,
                     int D, int dtype, float* partial_dev, void* stream);

/* tgx_dot_attn_fwd without the partial_dev argument: the split-row partials
 * go to a static device array of 64 MiB per device (held until the process
 * ends), so the call allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  Plans whose chunks need more than
 * 64 MiB of partials ((H*D + 2*H) * 4 bytes per chunk) are rejected with
 * TGX_INVALID_ARGUMENT before any launch.  Uses the current device's array
 * (`stream` must belong to the current device); every call on one device
 * shares it.  Uncaptured calls are ordered in host call order whatever
 * their streams (a call on another stream than the last one waits for an
 * event recorded after it); calls under graph capture are not, so graph
 * replays that overlap each other or an uncaptured call on one device race.
 * No part of the array needs to start at zero: every chunk writes its
 * partial before the merge reads it. */
int tgx_dot_attn_fwd_noalloc(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                             const tgx_row_plan* plan, const void* q_dev, const void* k_dev,
                             const void* v_dev, const float* bias_dev, float scale,
                             void* out_dev, float* ml_dev, int64_t n_dst, int64_t n_src,
                             int H, int D, int dtype, void* stream);

/* Workspace bytes for tgx_dot_attn_bwd with these plans; stored_ds != 0 for
 * a backward given inv_perm (it keeps each edge's score gradient, 4*H bytes
 * per edge of the n_edges). */
int tgx_dot_attn_bwd_workspace(const tgx_row_plan* plan, const tgx_row_plan* plan_t,
                               int64_t n_edges, int H, int D, int stored_ds, size_t* bytes);

/* Fused backward from the saved logsumexp, no float atomics: dq (dtype) and
 * dbias (fp32 [E, H], may be NULL) on the destination-row CSR, dk/dv (dtype)
 * on the transposed CSR (row_ptr_t, col_t, perm) and its plan.  ml slot 1
 * (delta = <dout, out>) is overwritten.  With inv_perm_dev (the transposed
 * CSR's inverse permutation) the source pass runs first and keeps each
 * edge's ds, and the destination pass reads it through inv_perm instead of
 * recomputing it from gathered k and v rows; NULL recomputes.  n_edges is
 * the CSR's edge count. */
int tgx_dot_attn_bwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                     const tgx_row_plan* plan, const int32_t* row_ptr_t_dev,
                     const int32_t* col_t_dev, const int32_t* perm_dev,
                     const int32_t* inv_perm_dev, const tgx_row_plan* plan_t,
                     int64_t n_edges, const void* q_dev, const void* k_dev,
                     const void* v_dev, const float* bias_dev, float scale,
                     const void* out_dev, float* ml_dev, const void* dout_dev, void* dq_dev,
                     void* dk_dev, void* dv_dev, float* dbias_dev, int64_t n_dst,
                     int64_t n_src, int H, int D, int dtype, void* workspace_dev,
                     size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Dense attention tiles on MFMA over block-diagonal relations               */
/*   block k relates queries [cu_q[k], cu_q[k+1]) to keys                    */
/*   [cu_k[k], cu_k[k+1]): every pair (causal = 0) or key <= query           */
/*   (causal = 1, which needs cu_q == cu_k).  Graph.cu_seqlens(causal=...)   */
/*   passes cu_q = cu_k = cu_seqlens; Graph.dense(num_src, num_dst) one       */
/*   block [0, num_dst) x [0, num_src); Graph.triangular(n) one causal block */
/*   (interop/torch/graph.py:260-294, 535-592).                              */
/* ------------------------------------------------------------------------ */

/* Host: the work list of one attention launch, in dispatch order.  A task is
 * four int32 (block, first row, head, tile0) naming `block` rows of one
 * head, tile0 the first stored dS tile of (block, head) for
 * tgx_attn_bwd_stored (0 when tgx_attn_ds_tiles refuses the relation):
 * kind 0: query tiles (block 128, forward and dQ), work = keys seen;
 * kind 1: key tiles (block 64, dK/dV), work = queries that see the tile.
 * Every tile of one (block, head) goes to the same XCD (workgroup i runs on
 * XCD i % 8, each XCD has its own L2) and the tiles are queued together,
 * heaviest first, so they read the same key/query blocks at about the same
 * time; (block, head) groups are spread over the 8 XCDs longest first.
 * Slots past the end of a shorter XCD queue hold block -1 (skipped).
 * Call with tasks_host = NULL to get n_tasks. */
int tgx_attn_tasks(const int32_t* cu_q_host, const int32_t* cu_k_host, int n_blocks, int H,
                   int block, int kind, int causal, int32_t* tasks_host, int64_t* n_tasks);

/* Forward: out = softmax(scale * q k^T over the relation) v per head.
 * q [n_q, H, D] and k/v [n_k, H, D] (D = 32, 64 or 128, dtype TGX_DTYPE_*) have
 * element strides strides[0..3] = (q token, q head, k/v token, k/v head),
 * innermost stride 1: contiguous [n, H, D], or the reference's lane-major
 * [H, n, D] storage viewed as [n, H, D]
 * (interop/torch/message_passing.py:1944-1947); `strides` is a host array;
 * out is contiguous [n_q, H, D],
 * lse [n_q, H] fp32 natural log (-inf, and out 0, for a row without keys).
 * tasks_dev from tgx_attn_tasks (kind 0, block 128, same H and causal) on the
 * device; the kernels trust it to match cu_q/cu_k and H.
 * prune_threshold = 0 is exact softmax; in (0, 1] it is the reference's
 * block_prune_threshold (reducer/core.py:176-190): a 64-key tile is skipped
 * for a 128-query block when the tile's maximum scaled score is below the
 * block's running maximum by more than log2(threshold)
 * (lib/Target/Triton/Translate.cpp:1793-1815), a schedule-dependent
 * approximation with no gradient.  The reference's compiled tile covers
 * dense/triangular fp16 forward (Translate.cpp:1603-1912); varlen runs its
 * eager oracle (examples/varlen_causal_attention.py:46-48). */
int tgx_attn_fwd(const int32_t* cu_q_dev, const int32_t* cu_k_dev, const int32_t* tasks_dev,
                 int64_t n_tasks, int causal, int dtype, const void* q_dev,
                 const void* k_dev, const void* v_dev, const int64_t* strides,
                 float scale, float prune_threshold, void* out_dev, float* lse_dev,
                 int64_t n_q, int64_t n_k, int H, int D, void* stream);

/* Host: forward tasks with long query tiles' key ranges split, for
 * relations whose tiles are too few and too uneven to fill the GPU (one
 * causal block of a few thousand tokens: the last query tile sees all keys
 * and would alone set the launch time).  `slots` is the number of forward
 * workgroups resident at once (2 per CU).  The balanced load is the total
 * of 64-key tiles over all query tiles and heads divided by `slots` (at
 * least 8); when the longest tile sees at least 5/4 of it, every tile seeing
 * more is cut into chunks of *chunk_tiles = that many key tiles, else
 * nothing is split (*n_merge = 0: use tgx_attn_tasks kind 0 and
 * tgx_attn_fwd).  tasks_host [n_tasks, 4] = (block, first query, head,
 * code): code -1 a whole tile, else the partial slot of a chunk, chunk c =
 * slot % *max_chunks of split tile slot / *max_chunks; merge_host [n_merge,
 * 4] = (block, first query, head, chunks) per split tile, in slot order.
 * Groups (block, head) go to the XCDs as in tgx_attn_tasks, each group's
 * tasks heaviest first.  Call with tasks_host = merge_host = NULL for the
 * counts.  No counterpart in the reference, whose dense tile runs one
 * program per query block (Translate.cpp:1603-1912). */
int tgx_attn_fwd_split_tasks(const int32_t* cu_q_host, const int32_t* cu_k_host, int n_blocks,
                             int H, int causal, int slots, int32_t* tasks_host,
                             int64_t* n_tasks, int32_t* merge_host, int64_t* n_merge,
                             int32_t* chunk_tiles, int32_t* max_chunks);

/* tgx_attn_fwd (exact: no pruning) over tgx_attn_fwd_split_tasks' lists:
 * key chunks write unnormalized O, running max and sum to partial_dev
 * (n_merge * max_chunks * 128 * (D + 2) fp32), then one merge workgroup per
 * split tile combines its chunks in chunk order and writes out and lse as
 * the whole-tile epilogue does.  Same results as tgx_attn_fwd up to the
 * order of the softmax sums (chunk by chunk instead of one running sum). */
int tgx_attn_fwd_split(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                       const int32_t* tasks_dev, int64_t n_tasks, const int32_t* merge_dev,
                       int64_t n_merge, int32_t chunk_tiles, int32_t max_chunks, int causal,
                       int dtype, const void* q_dev, const void* k_dev, const void* v_dev,
                       const int64_t* strides, float scale, void* out_dev, float* lse_dev,
                       float* partial_dev, int64_t n_q, int64_t n_k, int H, int D,
                       void* stream);

/* Backward of the exact forward (no atomics): delta = <dout, out> into
 * delta_dev [n_q, H] fp32, then dK/dV over key tiles (k_tasks: kind 1,
 * block 64) and dQ over query tiles (q_tasks: kind 0, block 128).  dout, dq
 * [n_q, H, D] and dk, dv [n_k, H, D] are contiguous; q/k/v and strides (a
 * host array of four) as in the forward. */
int tgx_attn_bwd(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                 const int32_t* q_tasks_dev, int64_t n_q_tasks, const int32_t* k_tasks_dev,
                 int64_t n_k_tasks, int causal, int dtype, const void* q_dev,
                 const void* k_dev, const void* v_dev, const int64_t* strides,
                 const void* out_dev, const float* lse_dev, const void* dout_dev,
                 float scale, void* dq_dev, void* dk_dev, void* dv_dev, float* delta_dev,
                 int64_t n_q, int64_t n_k, int H, int D, void* stream);

/* Host: the stored dS tiles of a backward (64 x 64 elements of the q/k/v
 * dtype each; per (block, head) the tiles qi >= kj of a causal block, all
 * of a non-causal one).  TGX_UNSUPPORTED past 2^31 tiles. */
int tgx_attn_ds_tiles(const int32_t* cu_q_host, const int32_t* cu_k_host, int n_blocks, int H,
                      int causal, int64_t* n_tiles);

/* tgx_attn_bwd with dS stored: the dK/dV kernel also writes every dS tile
 * to ds_dev (tgx_attn_ds_tiles x 64 x 64 elements, the task lists' tile0
 * offsets), and the dQ kernel reads them back instead of recomputing S and
 * dP (one product per tile instead of three).  Same results up to the
 * rounding of S computed as Q K^T instead of K Q^T.  ds_dev is workspace:
 * the rows of keys past a block's last key are written but not meaningful
 * (the dQ kernel does not read them). */
int tgx_attn_bwd_stored(const int32_t* cu_q_dev, const int32_t* cu_k_dev,
                        const int32_t* q_tasks_dev, int64_t n_q_tasks,
                        const int32_t* k_tasks_dev, int64_t n_k_tasks, int causal, int dtype,
                        const void* q_dev, const void* k_dev, const void* v_dev,
                        const int64_t* strides, const void* out_dev, const float* lse_dev,
                        const void* dout_dev, float scale, void* dq_dev, void* dk_dev,
                        void* dv_dev, float* delta_dev, void* ds_dev, int64_t n_q, int64_t n_k,
                        int H, int D, void* stream);

/* ------------------------------------------------------------------------ */
/* nn-scored edge attention: score_e = MLP(concat of gathered fields),       */
/* out_i = sum_e softmax_i(score)_e value[col_e]                             */
/*   reference: tg.nn.trace score networks (compiler/nn_capture.py:1-33)     */
/*   evaluated by compiler/edge_nn_attention.py and                          */
/*   interop/torch/message_passing.py:2372-2577                             */
/* ------------------------------------------------------------------------ */

/* Component-wise functions between linear layers.  Derivatives follow
 * Torch's backward (at kinks too).  For log and the powers (sqrt, rsqrt,
 * square, reciprocal, pow) the padding columns of a layer are not evaluated
 * (their 0 input would give inf).  Chains that use one of the codes from
 * TGX_ACT_EXP on run on kernels built for that set, at the same interface. */
enum {
  TGX_ACT_IDENTITY = 0,
  TGX_ACT_RELU = 1,
  TGX_ACT_LEAKY_RELU = 2,   /* act_param = negative slope */
  TGX_ACT_TANH = 3,
  TGX_ACT_SIGMOID = 4,
  TGX_ACT_SILU = 5,
  TGX_ACT_GELU = 6,         /* exact (erf) form */
  TGX_ACT_ELU = 7,          /* act_param = alpha */
  TGX_ACT_HARDTANH = 8,     /* clamp to [act_param, act_param2] (relu6, clamp) */
  TGX_ACT_SOFTPLUS = 9,     /* act_param = beta, act_param2 = threshold */
  TGX_ACT_SELU = 10,
  TGX_ACT_MISH = 11,
  TGX_ACT_HARDSIGMOID = 12,
  TGX_ACT_HARDSWISH = 13,
  TGX_ACT_EXP = 14,
  TGX_ACT_LOG = 15,
  TGX_ACT_SQRT = 16,
  TGX_ACT_RSQRT = 17,
  TGX_ACT_ABS = 18,         /* derivative sign(z), 0 at 0 */
  TGX_ACT_SIN = 19,
  TGX_ACT_COS = 20,
  TGX_ACT_SQUARE = 21,
  TGX_ACT_RECIPROCAL = 22,  /* act_param / z */
  TGX_ACT_POW = 23          /* z ** act_param; derivative 0 for exponent 0 */
};

/* Row of an edge that a score-input segment is gathered from. */
enum { TGX_ROLE_SRC = 0, TGX_ROLE_DST = 1, TGX_ROLE_EDGE = 2 };

/* A score network: n_layers linear layers (1..3), the last with one output,
 * with an activation after every layer but the last, applied to the
 * concatenation of up to four fp32 input segments gathered per edge (from the
 * source row col[e], the destination row, or edge row e).  Every layer is
 * zero-padded to `width` (16, 24, 32 or 64 >= every layer's in and out size):
 * weights_dev holds n_layers blocks of [width*width weights (out-major) |
 * width biases]. */
typedef struct tgx_edge_mlp {
  int32_t n_layers;
  int32_t width;
  int32_t act[3];
  float act_param[3];
  const float* weights_dev;
  int32_t n_segments;
  int32_t seg_role[4];
  int32_t seg_width[4];
  int64_t seg_stride[4];      /* row stride in floats */
  const float* seg_dev[4];
  /* Real output width of each layer (1..width, the last one 1; 0 = width):
   * rows and columns past the real shapes are zero padding the kernels skip. */
  int32_t out_width[3];
  /* Second parameter of each activation (hardtanh's upper bound, softplus's
   * threshold; unused by the others). */
  float act_param2[3];
  /* LayerNorm over a hidden layer's real outputs before its activation
   * (nonzero = on; not on the last layer; padded widths up to 32), Torch's
   * nn.LayerNorm: (z - mean) / sqrt(var + norm_eps) * gamma + beta with the
   * biased variance.  With any layer normalized, every layer's block of
   * weights_dev (and of the weight gradients) is [width*width | width bias |
   * width gamma | width beta]. */
  int32_t norm[3];
  float norm_eps[3];
} tgx_edge_mlp;

/* scores[e] = MLP(x_e) for every edge.  dst_index_dev [n_edges] int32 is the
 * destination row of each edge (tgx_destination_index with out_bits 32). */
int tgx_edge_mlp_scores(const void* col_dev, const int32_t* dst_index_dev, int idx_bits,
                        int64_t n_edges, const tgx_edge_mlp* mlp, float* scores_dev,
                        void* stream);

/* Edge-network messages summed per destination row (the reference's
 * edge-NN tile, python/tiga/compiler/edge_nn_tile.py:1-30, dispatched by
 * interop/torch/message_passing.py:2134-2300: tg.sum() over
 * tg.nn.trace(net)(fields)).  The last Linear layer is linear, so
 *   sum_e net(x_e) = W_L (sum_e a_e) + deg(i) b_L,   a_e = the last layer's
 * input for edge e; these entry points evaluate everything before the last
 * layer, and the caller applies W_L to the row sums.  The network is given
 * as for tgx_edge_mlp_scores (the last layer's weight block is not read;
 * its out_width entry may be 1), width 16, 24 or 32.
 *
 * hidden_dev [n_edges, hidden_width] fp32 receives a_e, hidden_width being
 * the last layer's input width (the previous layer's real output width, or
 * the concatenated input width for a one-layer network). */
int tgx_edge_mlp_hidden(const void* col_dev, const int32_t* dst_index_dev, int idx_bits,
                        int64_t n_edges, const tgx_edge_mlp* mlp, float* hidden_dev,
                        int32_t hidden_width, void* stream);

/* Backward of tgx_edge_mlp_hidden given the gradient at the last layer's
 * input per destination row, seed_dev [n_dst, seed_width] (the edge e takes
 * row dst_index[e]): per-edge input-segment gradients dseg as in
 * tgx_edge_mlp_backward, and the hidden layers' weight and bias gradients
 * summed over all edges into dweights_dev (the last layer's block is
 * written as zeros).  Deterministic; workspace as
 * tgx_edge_mlp_backward_workspace. */
int tgx_edge_mlp_backward_seeded(const void* col_dev, const int32_t* dst_index_dev,
                                 int idx_bits, int64_t n_edges, const tgx_edge_mlp* mlp,
                                 const float* seed_dev, int32_t seed_width,
                                 float* dweights_dev, float* const* dseg, void* workspace_dev,
                                 size_t workspace_bytes, void* stream);

/* Segment softmax over CSR rows: alpha[e] = exp(s_e - lse_i) and lse[i]
 * (-inf for an empty row), one wave per row (reducer_oracle.py:60-137). */
int tgx_segment_softmax_fwd(const void* row_ptr_dev, int idx_bits, int64_t n_rows,
                            const float* scores_dev, float* alpha_dev, float* lse_dev,
                            void* stream);

/* Segment softmax of raw per-edge scores read where the score field lives:
 * s_e = scale * scores[col[e]] (role TGX_ROLE_SRC, a source-node table),
 * scale * scores[i] (TGX_ROLE_DST, one per destination row) or
 * scale * scores[e] (TGX_ROLE_EDGE); alpha[e] = exp(s_e - lse_i) and lse[i]
 * (-inf, no weights, for an empty row).  With tgx_csr_sum_fwd (weights
 * alpha) this is the reference's online softmax over a raw score field,
 * reducer(src.score, src.value) (reducer_oracle.py:60-137; the compiled
 * stable-weighted row tile, lib/Target/Triton/Translate.cpp:3004-3450). */
int tgx_segment_softmax_gather_fwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                                   int64_t n_rows, const float* scores_dev, int role,
                                   float scale, float* alpha_dev, float* lse_dev,
                                   void* stream);

/* The segment softmax of tgx_segment_softmax_gather_fwd (same roles, scale,
 * lse and, when alpha_dev is not NULL, alpha) and the weighted sum of the
 * value rows in the same pass: out[i] = sum_e alpha_e value[col[e]],
 * value_dev [n_src, F] and out_dev [n_rows, F] fp32, 1 <= F <= 8 (else
 * TGX_UNSUPPORTED; F = 4 or 8 needs value_dev 16-byte aligned); an empty
 * row gets 0.  TGX_ROLE_EDGE reads the per-edge
 * scores of tgx_segment_softmax_fwd.  Per row only lse and the output are
 * written: the reference's row-centric attention tile keeps (m, l) and the
 * output (compiler/edge_nn_attention.py:127-338, reducer_oracle.py:60-137),
 * and its Torch path is tgx_segment_softmax_gather_fwd + tgx_csr_sum_fwd
 * (interop/torch/message_passing.py:2579-2619). */
int tgx_segment_softmax_sum_fwd(const void* row_ptr_dev, const void* col_dev, int idx_bits,
                                int64_t n_rows, const float* scores_dev, int role, float scale,
                                const float* value_dev, int F, float* alpha_dev,
                                float* lse_dev, float* out_dev, void* stream);

/* Its backward: dscore[e] = alpha_e (dalpha_e - sum over the row of
 * alpha dalpha). */
int tgx_segment_softmax_bwd(const void* row_ptr_dev, int idx_bits, int64_t n_rows,
                            const float* alpha_dev, const float* dalpha_dev,
                            float* dscore_dev, void* stream);

/* Workspace bytes needed by tgx_edge_mlp_backward for n_edges edges. */
int tgx_edge_mlp_backward_workspace(int64_t n_edges, const tgx_edge_mlp* mlp, size_t* bytes);

/* Backward of the score network given dscore (the reference differentiates
 * the same chain with Torch autograd, interop/torch/message_passing.py:
 * 2372-2577): writes the gradient of every input segment per edge, dseg[s]
 * ([n_edges, seg_width[s]] fp32 device buffers; dseg is a host array), which
 * the caller reduces per source row over the transposed CSR and per
 * destination row over the CSR, and the weight and bias gradients summed
 * over all edges into dweights_dev, laid out as weights_dev (n_layers blocks
 * of [width*width | width], padding entries 0).  The sums are formed on the
 * device from per-block partials added in a fixed order: deterministic. */
int tgx_edge_mlp_backward(const void* col_dev, const int32_t* dst_index_dev, int idx_bits,
                          int64_t n_edges, const tgx_edge_mlp* mlp, const float* dscore_dev,
                          float* dweights_dev, float* const* dseg, void* workspace_dev,
                          size_t workspace_bytes, void* stream);

/* The backward of online-softmax attention over the network's score
 *   out[i] = sum_e softmax_i(net(fields_e)) value[col[e]]
 * from what its forward keeps per row only: lse [n_dst] (logsumexp of each
 * row's scores, tgx_segment_softmax_fwd) and out [n_dst, value_width];
 * dout [n_dst, value_width], value [n_src, value_width], all fp32 (rows of a
 * multiple of 4 floats 16-byte aligned).  Per edge the kernel replays the
 * network, recomputes alpha = exp(s - lse[i]) and forms the score gradient
 * ds = alpha (<dout[i], value[j]> - <dout[i], out[i]>) itself (no per-edge
 * score, weight or score gradient is read), then writes dseg and dweights
 * as tgx_edge_mlp_backward does, and alpha [n_edges] (fp32, edge order;
 * alpha_dev may be NULL) for the value gradient (tgx_csr_sum_bwd with alpha
 * as the weights).  fold_segment >= 0 names a source segment of width
 * value_width whose per-edge gradient rows also receive the value
 * gradient's edge term alpha_e dout[dst_e]: when the value is that source
 * field, the transposed reduction of dseg[fold_segment] is then its whole
 * gradient and the value-gradient pass is not needed; -1 folds nothing.
 * The reference's fused edge-attention backward recomputes the weights from
 * the row's (m, l) the same way (compiler/edge_nn_attention.py:344-611).
 * Workspace: tgx_edge_mlp_backward_workspace. */
int tgx_edge_mlp_attention_backward(const void* col_dev, const int32_t* dst_index_dev,
                                    int idx_bits, int64_t n_edges, const tgx_edge_mlp* mlp,
                                    const float* lse_dev, const float* out_dev,
                                    const float* dout_dev, const float* value_dev,
                                    int32_t value_width, float* alpha_dev, int fold_segment,
                                    float* dweights_dev, float* const* dseg_dev,
                                    void* workspace_dev, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Per-kernel timing (no reference counterpart; used by the benchmark)       */
/* ------------------------------------------------------------------------ */

/* Start recording a HIP event pair around every kernel this library
 * launches (clears previous totals). */
int tgx_profile_begin(void);
/* Stop recording; synchronises the recorded events and accumulates the
 * elapsed time per kernel name. */
int tgx_profile_end(void);
/* Number of distinct kernel names with accumulated time. */
int tgx_profile_count(void);
/* Entry `index`: kernel name (NUL-terminated, truncated to name_capacity),
 * number of launches and total milliseconds. */
int tgx_profile_entry(int index, char* name, int name_capacity, int64_t* launches,
                      double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* TGX_H_ */
