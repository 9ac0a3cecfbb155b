/* CPU twins of the device entry points of tgx.h.
 *
 * tgx_cpu_<name> takes the arguments of tgx_<name> with host pointers in
 * place of device pointers, without the stream and without the caller's
 * device scratch (workspace / partial buffers): a twin allocates what it
 * needs in host memory.  The twins keep the device entry points' argument
 * checks and status codes (TGX_UNSUPPORTED for the same shapes), walk the
 * same row plan (empty rows, whole rows, split rows computed chunk by chunk
 * and merged in chunk order) and add the checks a device launch cannot
 * afford: row_ptr non-decreasing from 0, every column in range, the plan's
 * rows a permutation whose bins match the degrees, chunk offsets matching
 * the split rows' degrees, the transposed CSR consistent with perm/inv_perm.
 *
 * Arithmetic is fp32 (bf16/fp16 storage converted on load, rounded to
 * nearest even on store), with fp64 for the cross-row GAT parameter
 * gradients, as on the device; results differ from the device results
 * only by summation order.  Work is spread over tgx_cpu_set_threads()
 * threads; results do not depend on the thread count.
 *
 * Same status codes as tgx.h; the last error message is tgx_last_error(). */
#ifndef TGX_CPU_H_
#define TGX_CPU_H_

#include <stddef.h>
#include <stdint.h>

#include "tgx.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Threads used by the twins (0 = the machine's hardware concurrency).
 * Returns the previous setting. */
int tgx_cpu_set_threads(int threads);

/* Twin of tgx_destination_index (reference Graph.destination_index,
 * interop/torch/graph.py:1212-1222). */
int tgx_cpu_destination_index(const void* row_ptr, int idx_bits, int64_t n_rows,
                              int64_t n_edges, void* out, int out_bits);

/* Twin of tgx_csr_transpose (reference Graph.transpose,
 * interop/torch/graph.py:675-685, 193-231); inv_perm may be NULL. */
int tgx_cpu_csr_transpose(const void* row_ptr, const void* col, int idx_bits,
                          int64_t n_dst, int64_t n_src, int64_t n_edges,
                          int32_t* row_ptr_t, int32_t* col_t, int32_t* perm,
                          int32_t* inv_perm);

/* Twin of tgx_plan_degree_bins (reference degree worklist,
 * lib/Target/Triton/Translate.cpp:4043-4187): rows grouped by bin, ascending
 * inside each bin; bin_offsets [n_bins+1].  The last bound must be at least
 * the maximum degree. */
int tgx_cpu_plan_degree_bins(const void* row_ptr, int idx_bits, int64_t n_rows,
                             const int64_t* upper_bounds, int n_bins, int32_t* rows_out,
                             int64_t* bin_offsets);

/* Twin of tgx_plan_split_chunks (reference row-split plan,
 * lib/Transforms/PlanSplitRows.cpp:136-147). */
int tgx_cpu_plan_split_chunks(const void* row_ptr, int idx_bits, const int32_t* split_rows,
                              int64_t n_split, int32_t chunk_edges, int32_t* chunk_offsets,
                              int64_t* n_chunks);

/* Twin of tgx_csr_sum_fwd (reference _execute_weighted_sum,
 * interop/torch/message_passing.py:2903-3345; reduce_sum,
 * reducer_oracle.py:44-58).  plan holds host arrays.  col may be NULL (the
 * columns are the edge ids). */
int tgx_cpu_csr_sum_fwd(const void* row_ptr, const void* col, int idx_bits,
                        const tgx_row_plan* plan, const void* x, const float* w, void* out,
                        int64_t n_dst, int64_t n_src, int64_t F, int dtype);

/* Twin of tgx_csr_sum_bwd (reference Torch replay,
 * interop/torch/message_passing.py:378-409).  dx / dw may be NULL. */
int tgx_cpu_csr_sum_bwd(const int32_t* row_ptr_t, const int32_t* col_t, const int32_t* perm,
                        const tgx_row_plan* plan_t, const void* x, const float* w,
                        const void* dout, void* dx, float* dw, int64_t n_dst, int64_t n_src,
                        int64_t F, int dtype);

/* Twin of tgx_csr_edge_dot (F <= 32). */
int tgx_cpu_csr_edge_dot(const void* row_ptr, const void* col, int idx_bits,
                         const tgx_row_plan* plan, const void* x, const void* dout, float* dw,
                         int64_t n_dst, int64_t n_src, int64_t F, int dtype);

/* Twin of tgx_gat_fwd (eager evaluation of the additive edge function,
 * interop/torch/message_passing.py:2848-2894, reducer_oracle.py:60-137).
 * Same arguments and node_state layout [n_dst, H, 4], without the device
 * entry's partial buffer, pos rows and stream. */
int tgx_cpu_gat_fwd(const void* row_ptr, const void* col, int idx_bits,
                    const tgx_row_plan* plan, const void* h_src, const void* h_dst,
                    const float* a_src, const float* a_dst, float negative_slope, void* out,
                    float* node_state, int64_t n_dst, int64_t n_src, int H, int D, int dtype);

/* Twin of tgx_gat_bwd (its per-edge destination path: no pos rows);
 * node_state slot 1 (delta) is overwritten. */
int tgx_cpu_gat_bwd(const void* row_ptr, const void* col, int idx_bits,
                    const tgx_row_plan* plan, const int32_t* row_ptr_t, const int32_t* col_t,
                    const int32_t* perm, const int32_t* inv_perm, const tgx_row_plan* plan_t,
                    const void* h_src, const void* h_dst, const float* a_src,
                    const float* a_dst, float negative_slope, const void* out,
                    float* node_state, const void* dout, void* dh_src, void* dh_dst,
                    float* da_src, float* da_dst, int64_t n_dst, int64_t n_src,
                    int64_t n_edges, int H, int D, int dtype);

/* Twin of tgx_dot_attn_fwd (q/k/v/out of element type dtype = TGX_DTYPE_BF16,
 * _F16 or _F32, fp32 bias [E, H] or NULL, ml [n_dst, H, 2]). */
int tgx_cpu_dot_attn_fwd(const void* row_ptr, const void* col, int idx_bits,
                         const tgx_row_plan* plan, const void* q, const void* k,
                         const void* v, const float* bias, float scale, void* out, float* ml,
                         int64_t n_dst, int64_t n_src, int H, int D, int dtype);

/* Twin of tgx_dot_attn_bwd (ds recomputed in the destination pass: no
 * inv_perm or edge count); ml slot 1 (delta) is overwritten. */
int tgx_cpu_dot_attn_bwd(const void* row_ptr, const void* col, int idx_bits,
                         const tgx_row_plan* plan, const int32_t* row_ptr_t,
                         const int32_t* col_t, const int32_t* perm,
                         const tgx_row_plan* plan_t, const void* q, const void* k,
                         const void* v, const float* bias, float scale, const void* out,
                         float* ml, const void* dout, void* dq, void* dk, void* dv,
                         float* dbias, int64_t n_dst, int64_t n_src, int H, int D,
                         int dtype);

/* Twin of tgx_attn_fwd over n_blocks blocks of cu_q / cu_k (host arrays of
 * n_blocks + 1) in place of the device task list.  Only exact softmax:
 * prune_threshold > 0 (a schedule-dependent approximation of the device
 * tiles) returns TGX_UNSUPPORTED. */
int tgx_cpu_attn_fwd(const int32_t* cu_q, const int32_t* cu_k, int n_blocks, int causal,
                     int dtype, const void* q, const void* k, const void* v,
                     const int64_t* strides, float scale, float prune_threshold, void* out,
                     float* lse, int64_t n_q, int64_t n_k, int H, int D);

/* Twin of tgx_attn_bwd over n_blocks blocks in place of the task lists. */
int tgx_cpu_attn_bwd(const int32_t* cu_q, const int32_t* cu_k, int n_blocks, int causal,
                     int dtype, const void* q, const void* k, const void* v,
                     const int64_t* strides, const void* out, const float* lse,
                     const void* dout, float scale, void* dq, void* dk, void* dv,
                     float* delta, int64_t n_q, int64_t n_k, int H, int D);

#ifdef __cplusplus
}
#endif

#endif /* TGX_CPU_H_ */
