/* pt_dev_internal.h -- shared between the C host files of libptconv_hip.so (not installed). */
#ifndef PT_DEV_INTERNAL_H_
#define PT_DEV_INTERNAL_H_

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "pt_v21_dev.h"
#include "ptk.h"

#define PT_LOG(...)                     \
  do {                                  \
    fprintf(stderr, "pt_v21 hip: ");    \
    fprintf(stderr, __VA_ARGS__);       \
    fputc('\n', stderr);                \
  } while (0)

/* arena: per-context bump allocator, 256-byte aligned, mark / release */
void *ptdi_arena_alloc(pt_ctx *c, size_t bytes);
void *ptdi_arena_mark(pt_ctx *c);
void ptdi_arena_release(pt_ctx *c, void *mark);

/* weight pool: device pointer of record idx when it holds at least `need` bytes, else NULL */
const void *ptdi_pool_get(int idx, size_t need);
/* relaid MFMA copy of pool record idx for (M rows, K taps, cin), built once per process on the
 * caller's stream; NULL when idx is not resident */
const float *ptdi_pool_relaid(pt_ctx *c, int idx, int M, int K, int cin);
/* set the pool up from n host records (when empty) and upload the share this context claims:
 * bytes[i] = record i's fp32 size on the device, isz[i] = its source's bytes per item (4, or 2
 * for fp16 sources expanded on the device; NULL = all 4).  Sources must stay valid until return. */
int ptdi_pool_load_src(pt_ctx *c, int n, const void *const *host, const size_t *bytes,
                       const unsigned char *isz);
/* take / drop a reference on the pool (init / shutdown) */
void ptdi_pool_ref(int delta);

/* wait for the context's stream under the wait policy (PT_V21_WAIT_US); 0 / -1 */
int ptdi_wait(pt_ctx *c);
/* the wait ahead of a result copy that is followed by a stream synchronisation: the policy's
 * sleep-poll when PT_V21_WAIT_US > 0, nothing under the runtime's own wait (the synchronisation
 * after the copy waits for the kernels as well); 0 / -1 */
int ptdi_wait_before_copy(pt_ctx *c);

/* fill a conv descriptor for a plain conv over device buffers (in_op / epilogues left empty) */
void ptdi_conv_desc(ptk_conv_desc *d, const float *x, int64_t ldx, int64_t bsx, int64_t lim,
                    int cin, const float *wr, const float *bias, int nbias, int K, int stride,
                    int dil, int shift, int M, float *y, int64_t ldy, int64_t bsy, int64_t n,
                    int batch);
/* same for a convT in the phase form; returns the output length */
int64_t ptdi_convT_desc(ptk_conv_desc *d, const float *x, int64_t ldx, int64_t bsx, int64_t tin,
                        int cin, const float *wr, const float *bias, int cout, int s, int pad,
                        int K, float *y, int64_t ldy, int64_t bsy, int batch);

/* decoder layer i's packed weight size in floats (conv [C4/4][K][cin][4]; convT phase rows
 * [s*C4/4][ceil(K/s)][cin][4]) and its output channel count; -1 outside 0..PTD_DEC_NLAYER-1 */
int64_t ptdi_dec_wfloats(int i);
int ptdi_dec_cout(int i);
/* the decoder model from per-layer host sources: w[i] packed, wisz[i] bytes per item (4 fp32, 2
 * fp16 expanded on the device; wisz NULL = all fp32); the final conv's weight must be fp32 */
struct ptd_model *ptdi_model_build(pt_ctx *c, const void *const *w, const int *wisz,
                                   const float *const *b);

/* pt_v21_cuda_init with an explicit arena size */
int ptdi_ctx_init(pt_ctx *c, size_t arena_bytes, int verbose);

/* elapsed wall-clock ms since an arbitrary origin */
double ptdi_now_ms(void);

/* make / release the extra streams a context's windowed decodes split long batched runs over
 * (pt_decoder.c; made on first use when not prepared) */
void ptdi_aux_prepare(pt_ctx *c);
/* The contexts' streams remade behind 0 .. PTDI_PLACE_MAX_BALLAST idle streams (kept in ballast,
 * released by ptdi_place_release), whichever arrangement a timed probe finds spreads them most
 * evenly over the hardware queues (PTD_SERVER_PLACE=0: left as made).  Call before anything is
 * queued on them.  0, or -1 when a context is left without a stream. */
#define PTDI_PLACE_MAX_BALLAST 3
int ptdi_place_streams(pt_ctx *ctx, int n, void **ballast);
void ptdi_place_release(void **ballast);
void ptdi_aux_release(pt_ctx *c);
/* re-read the PTD_WINDOW_* knobs from the environment (otherwise read once; pt_decoder.c) */
void ptdi_decoder_knobs_reload(void);
/* The reference server's window widths (main_v21_serve.c:223-224): a first or later width below
 * 2*ctx + 8 is raised to it.  ptd_decode_windows2, its arena size and streaming queue jobs take
 * them; ptd_decode_windows (the --stream driver's form, main_v21.c:341-362) does not. */
static inline void ptdi_serve_widths(int *win_first, int *win, int ctx) {
  if (ctx >= 0 && *win_first < 2 * ctx + 8) *win_first = 2 * ctx + 8;
  if (ctx >= 0 && *win < 2 * ctx + 8) *win = 2 * ctx + 8;
}
/* windowed decode with the reference's first / later widths (taken as given); t_first != NULL:
 * window 0 is decoded alone, waited for, and its completion time stored there */
int ptdi_decode_windows(pt_ctx *c, const struct ptd_model *m, const float *z, int64_t T,
                        int win_first, int win, int ctx, float *wav, double *t_first);

#endif
