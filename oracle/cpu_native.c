/*
 * The reference's native CPU forward for the sum reducer, restated in C.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): timed by bench.py as the
 * CPU baseline of the weighted sum; never linked into the product.
 *
 * Tiga's native runtime lowers csr_segment_sum(w * gather(x, col)) to a loop
 * over output elements (row, feature), each a sequential fp32 sum over the
 * row's CSR edges in stored order (lib/Transforms/LowerTensorToCPU.cpp:
 * 672-704), and splits the output elements into T contiguous chunks run on a
 * persistent thread pool, T = min(32, hardware threads) by default
 * (python_bindings/compiler_module.cpp:2048-2139, 2398-2420).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>

typedef struct {
  const int64_t* row_ptr;
  const int64_t* col;
  const float* x;
  const float* w;
  float* out;
  int64_t F;
  int64_t begin, end; /* output element range [begin, end) */
} chunk_t;

static void* run_chunk(void* arg) {
  const chunk_t* c = (const chunk_t*)arg;
  for (int64_t k = c->begin; k < c->end; ++k) {
    const int64_t row = k / c->F, f = k % c->F;
    float acc = 0.0f;
    for (int64_t e = c->row_ptr[row]; e < c->row_ptr[row + 1]; ++e)
      acc += c->w[e] * c->x[c->col[e] * c->F + f];
    c->out[k] = acc;
  }
  return NULL;
}

/* out[n_dst, F] = sum over CSR rows of w[e] * x[col[e], :]; returns 0 on success. */
int tgx_oracle_csr_sum_fwd(const int64_t* row_ptr, const int64_t* col, const float* x,
                           const float* w, float* out, int64_t n_dst, int64_t F,
                           int threads) {
  if (threads < 1) threads = 1;
  const int64_t total = n_dst * F;
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * threads);
  chunk_t* ch = (chunk_t*)malloc(sizeof(chunk_t) * threads);
  if (!tid || !ch) {
    free(tid);
    free(ch);
    return 1;
  }
  const int64_t per = (total + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    int64_t b = per * t, e = b + per;
    if (b > total) b = total;
    if (e > total) e = total;
    ch[t] = (chunk_t){row_ptr, col, x, w, out, F, b, e};
    pthread_create(&tid[t], NULL, run_chunk, &ch[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(ch);
  return 0;
}

/*
 * The same runtime's backward of w[e] * x[col[e]] summed per row, as its CPU
 * lowering emits it (lib/Transforms/LowerTensorToCPU.cpp): the message
 * gradient dmsg = csr_expand_rows(dout) finds each edge's row with a select
 * chain over every row (emitCSRExpandRows, :641-670), dx =
 * segment_sum(dmsg * w, col) scans every edge for every output element
 * (emitSegmentSum, :608-639), and dw[e] = <dmsg[e], x[col[e]]>.  Sequential
 * (one thread); O(E * N_dst * F + N_src * E * F).  dmsg_scratch holds
 * E * F floats.
 */
int tgx_oracle_csr_sum_bwd_lowered(const int64_t* row_ptr, const int64_t* col,
                                   const float* x, const float* w, const float* dout,
                                   float* dx, float* dw, float* dmsg_scratch,
                                   int64_t n_dst, int64_t n_src, int64_t F) {
  const int64_t E = row_ptr[n_dst];
  for (int64_t e = 0; e < E; ++e)
    for (int64_t f = 0; f < F; ++f) {
      int64_t src_row = 0;
      for (int64_t r = 0; r < n_dst; ++r)
        src_row = (e >= row_ptr[r] && e < row_ptr[r + 1]) ? r : src_row;
      dmsg_scratch[e * F + f] = dout[src_row * F + f];
    }
  for (int64_t j = 0; j < n_src; ++j)
    for (int64_t f = 0; f < F; ++f) {
      float acc = 0.0f;
      for (int64_t e = 0; e < E; ++e)
        acc += (col[e] == j) ? dmsg_scratch[e * F + f] * w[e] : 0.0f;
      dx[j * F + f] = acc;
    }
  for (int64_t e = 0; e < E; ++e) {
    float acc = 0.0f;
    for (int64_t f = 0; f < F; ++f) acc += dmsg_scratch[e * F + f] * x[col[e] * F + f];
    dw[e] = acc;
  }
  return 0;
}
