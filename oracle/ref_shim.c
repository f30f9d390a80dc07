/* ref_shim.c -- TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's own
 * runtime/v21/src/pt_v21_host.c and runtime/v21/gen/pt_graph.c (unmodified, where they lie) into
 * oracle/_ref/libptref.so.  It gives the reference's CPU conv path a context-free entry point with
 * the oracle's signatures, so tests can check the C restatement against the reference's own code
 * and bench.py can time that code as the CPU baseline (the CPU matmul likewise, for the device
 * matmul's tests and baseline).  It also reports the reference's struct
 * pt_ctx layout, which the HIP library's own declaration must match field for field. */
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "pt_v21.h"

int ref_conv_cpu(const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy, int64_t n,
                 int cout, int K, int stride, int pad, int dil, const float *wp,
                 const float *bias, int64_t batch, int epi0, int epi1, float a0, float a1) {
  pt_ctx c;
  memset(&c, 0, sizeof c);
  return pt_v21_conv_cpu(&c, X, ldx, cin, Y, ldy, n, cout, K, stride, pad, dil, wp, bias, batch,
                         -1, -1, epi0, epi1, a0, a1);
}

int ref_convT_cpu(const float *X, int64_t ldx, int64_t cin, int64_t tin, float *Y, int64_t ldy,
                  int cout, int s, int pad, int K, const float *wp, const float *bias,
                  int64_t batch) {
  pt_ctx c;
  memset(&c, 0, sizeof c);
  return pt_v21_convT_cpu(&c, X, ldx, cin, tin, Y, ldy, cout, s, pad, K, wp, bias, batch, -1, -1);
}

int ref_matmul_cpu(const float *A, int64_t m, int64_t k, int64_t lda, const float *B, int64_t ldb,
                   int64_t n, float *C, int64_t ldc) {
  pt_ctx c;
  memset(&c, 0, sizeof c);
  return pt_v21_matmul_cpu(&c, A, m, k, lda, B, ldb, n, C, ldc);
}

/* sizeof(pt_ctx) followed by the offsets of the fields the device layer reads or writes */
int ref_ctx_layout(long *out, int n) {
  const long v[] = {
      (long) sizeof(pt_ctx),
      (long) offsetof(pt_ctx, use_cuda),       (long) offsetof(pt_ctx, n_conv),
      (long) offsetof(pt_ctx, n_convT),        (long) offsetof(pt_ctx, n_matmul),
      (long) offsetof(pt_ctx, g_alloc_ms),     (long) offsetof(pt_ctx, g_calls),
      (long) offsetof(pt_ctx, dev_bytes_weights), (long) offsetof(pt_ctx, dev_bytes_res),
      (long) offsetof(pt_ctx, devres_oom),     (long) offsetof(pt_ctx, arena_alloc_bytes),
      (long) offsetof(pt_ctx, g_weights),      (long) offsetof(pt_ctx, g_arena),
      (long) offsetof(pt_ctx, g_stream),       (long) offsetof(pt_ctx, g_arena_bytes),
      (long) offsetof(pt_ctx, g_arena_used),   (long) offsetof(pt_ctx, conv_pad_in),
      (long) offsetof(pt_ctx, conv_in_dev),    (long) offsetof(pt_ctx, conv_keep),
      (long) offsetof(pt_ctx, conv_keep_res),  (long) offsetof(pt_ctx, dev_live),
      (long) offsetof(pt_ctx, conv_out_dev),   (long) offsetof(pt_ctx, chain_mark),
      (long) offsetof(pt_ctx, devres),
  };
  const int m = (int) (sizeof v / sizeof v[0]);
  for (int i = 0; i < n && i < m; i++) out[i] = v[i];
  return m;
}
