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
