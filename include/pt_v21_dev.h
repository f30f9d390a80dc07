/* pt_v21_dev.h -- C ABI of libptconv_hip.so, the MI355X (gfx950) device layer of the PrimeTTS
 * v2.1 runtime.
 *
 * The library replaces the reference's CUDA device object (runtime/v21/src/pt_v21_cuda.cu) at
 * link time: the reference host (pt_v21_host.c built with -DPT_V21_CUDA) calls exactly the
 * entry points declared below, with the signatures of runtime/v21/src/pt_v21.h:208-259.  The
 * "cuda" in the names is the reference's legacy naming; the implementation is native HIP.
 *
 * struct pt_ctx is the reference's per-request context (pt_v21.h:93-162).  Host and device layer
 * share it, so this declaration keeps the reference's field order and types exactly (an ABI, not
 * a design choice); tests/test_abi.py compares sizeof and every offset the device layer touches
 * against the reference header.  When the reference's own pt_v21.h is included first, it is used
 * as is and this header only adds nothing. */
#ifndef PT_V21_DEV_H_
#define PT_V21_DEV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef PT_V21_H_
struct pt_tv_;   /* the interpreter's tensor view; the device layer never dereferences it */

struct pt_ctx {
  int use_cuda;                 /* 1 = conv/convT/matmul run on the device */
  void *map;
  size_t maplen;
  char *base;
  uint32_t n_tensor;
  const char **cont_names;
  float **cont_f32;
  int *cont_isz;
  int64_t *cont_n;
  int *cont_ndim;
  char *cont_path;
  int *cont_shared;
  int64_t *cont_dims;
  int n_cont;
  struct pt_tv_ *V;
  float *wav;
  int64_t wav_n;
  int ck_n;
  const int *ck_ids;
  char ck_dir[512];
  int dev_mode;
  long n_conv, n_convT, n_matmul, n_alloc_fail;   /* calls served (the device layer counts) */
  double t_conv, t_convT, t_matmul, t_total;
  double g_alloc_ms, g_copy_ms, g_kernel_ms, g_free_ms;   /* PT_V21_CUDAPROF=1 split */
  long g_calls;
  int prof;
  int prof_node_on;
  long host_bytes_live, host_bytes_peak;
  void *pool[64];
  long pool_bytes, pool_cap;
  long host_alloc_count;
  double dev_bytes_weights, dev_bytes_arena, dev_bytes_stray;
  double dev_bytes_res;
  int devres_oom;
  size_t arena_alloc_bytes;     /* arena high-water mark */
  char *skip;
  int fuse;
  int run_from, run_to;
  int stream_inject_id;
  struct pt_tv_ *stream_inject;
  void *stream_seeds;
  int stream_nseeds;
  void *stream_state;
  double *prof_node;
  double t_ekind[96];
  long n_ekind[96];
  void *g_weights;              /* unused by the reference; unused here */
  void *g_arena;                /* device arena base (bump allocator, mark/release) */
  void *g_stream;               /* this context's hipStream_t (non-blocking) */
  size_t g_arena_bytes, g_arena_used;
  int64_t conv_pad_in;          /* >= 0: conv input rows are unpadded, pad in-kernel by this */
  const float *conv_in_dev;     /* device-resident conv input (conv chain), or NULL */
  int conv_keep;                /* 1 = leave this conv's output on the device */
  int conv_keep_res;            /* ... in the residency sub-arena (multi-consumer tensor) */
  int devadd_used;
  int dev_live;
  float *conv_out_dev;          /* set by pt_v21_conv when the output was kept */
  void *chain_mark;             /* arena mark held while a conv chain is in flight */
  void *devres;                 /* device-residency sub-arena state, NULL until first use */
};
typedef struct pt_ctx pt_ctx;
#endif /* PT_V21_H_ */

/* ---- context, stream, arena, shared weights ------------------------------------------------ */
/* pt_v21.h:209 -- creates the context's stream and arena, takes a reference on the process-wide
 * weight pool (uploading the container records once, claim-parallel across contexts), sets
 * c->use_cuda = 1.  0 / -1. */
int pt_v21_cuda_init(pt_ctx *c, int verbose);
/* pt_v21.h:213 -- once per process: creates the HIP context early.  Always 0. */
int pt_v21_cuda_prewarm(void);
/* pt_v21.h:214 -- syncs and destroys the stream, frees the arena, drops the weight reference. */
void pt_v21_cuda_shutdown(pt_ctx *c);
/* pt_v21.h:224 -- MiB of resident weights (shared by all contexts) */
double pt_v21_cuda_weights_mib(pt_ctx *c);
/* pt_v21.h:225 -- contexts inside a run (the wait policy's "could another stream use the core") */
void pt_v21_cuda_active(int delta);
/* pt_v21.h:226-228 -- clock helpers of the Nano build.  MI355X clocks are not governor-ramped by
 * load here, so keep-warm does no work and the frequencies read as unknown (-1). */
int pt_v21_cuda_keepwarm(int iters);
long pt_v21_gpu_cur_freq(void);
long pt_v21_gpu_max_freq(void);
/* pt_v21.h:230 -- 1: callers hand over unpadded rows; every kernel here pads in-kernel. */
int pt_v21_conv_pads_in_kernel(pt_ctx *c);

/* ---- the hot path -------------------------------------------------------------------------- */
/* pt_v21.h:251-253 (reference implementation pt_v21_cuda.cu:1756-1957).
 * Y[b][co][t] = epi1(epi0(bias[co] + sum_{k,ci} W[co][k][ci] * x[b][ci][t*stride + k*dil - p]))
 * W packed [cout4/4][K][cin][4]; X [batch][cin][ldx]; Y [batch][cout4][ldy], all cout4 rows.
 * p = c->conv_pad_in when >= 0 (unpadded rows), else 0 (rows already zero-padded); input columns
 * outside [0, ldx) read as 0.  wtab / btab: pool indices of resident W / bias (-1 or unknown:
 * uploaded for this call).  epi codes: 1 LeakyReLU, 2 ReLU, 3 *scalar, 4 +scalar.
 * Synchronous (Y valid on return) unless c->conv_keep: then the output stays on the device in
 * c->conv_out_dev for the next conv (c->conv_in_dev).  0 / -1. */
int pt_v21_conv(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy,
                int64_t n, int cout, int K, int stride, int pad, int dil, const float *wp,
                const float *bias, int64_t batch, int wtab, int btab, int epi0, int epi1, float a0,
                float a1);
/* pt_v21.h:255-257 (reference pt_v21_cuda.cu:2351-2491): conv_transpose1d over the packed phase
 * layout [s*cout4/4][ntap][cin][4], with the tail flush; Lout = (tin-1)*s - 2*pad + K.
 * Synchronous.  0 / -1. */
int pt_v21_convT(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, int64_t tin, float *Y,
                 int64_t ldy, int cout, int s, int pad, int K, const float *wp, const float *bias,
                 int64_t batch, int wtab, int btab);
/* pt_v21.h:258 -- C[m][nn] = A[m][k] @ B[k][nn] on the device (encoder attention; off the hot
 * path): fp32 MFMA, 64x64 blocks of C, 32x32 per wave; host buffers, synchronous.  0 / -1. */
int pt_v21_matmul(pt_ctx *c, const float *A, int64_t m, int64_t k, int64_t lda, const float *B,
                  int64_t ldb, int64_t nn, float *C, int64_t ldc);

/* ---- device residency (pt_v21.h:232-247; reference pt_v21_cuda.cu:237-454) ---------------- */
int pt_v21_devadd_run(pt_ctx *c, const float *a, const float *b, float *y, int64_t n, int epi,
                      float alpha);
int pt_v21_devleaky_run(pt_ctx *c, const float *a, float *y, int64_t n, float alpha);
float *pt_v21_dev_upload(pt_ctx *c, const void *h, int64_t n);
void pt_v21_dev_sync_host(pt_ctx *c, void *host, const void *dev, int64_t n);
void *pt_v21_dev_alloc(pt_ctx *c, size_t bytes);
void pt_v21_dev_free(pt_ctx *c, void *p);
void pt_v21_dev_reclaim(pt_ctx *c);

/* ---- imports from the host (weak: resolved when linked with the reference host) ----------- *
 * pt_v21_n_cont / pt_v21_cont / pt_v21_cont_bytes (pt_v21.h:176-180) are the weight pool's
 * source records; pt_v21_conv_cpu / pt_v21_convT_cpu / pt_v21_matmul_cpu (pt_v21.h:217-222,
 * 248-249) serve calls on a context with use_cuda == 0, as in the reference.  A library loaded
 * without a host has no CPU path: such calls fail with -1. */

#ifdef __cplusplus
}
#endif
#endif /* PT_V21_DEV_H_ */
