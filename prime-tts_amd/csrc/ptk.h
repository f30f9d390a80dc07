/* ptk.h -- the thin C-ABI layer between the C (gnu11) host code and the HIP side.
 *
 * Everything HIP lives behind these functions (ptk_kernels.hip): stream and memory wrappers, the
 * one-time weight relayout, and the conv / convT / elementwise / decoder-tail launchers.  The
 * host code never includes a HIP header.  All sizes are elements unless named *_bytes; every
 * pointer handed to a launcher is a device pointer.  Launchers only enqueue work on the given
 * stream; they return 0, or -1 with the reason in ptk_last_error(). */
#ifndef PTK_H_
#define PTK_H_
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- runtime wrappers */
int ptk_init(void);                                /* select device 0 once; 0 / -1 */
const char *ptk_last_error(void);
int ptk_stream_create(void **s);                   /* non-blocking stream, default priority */
int ptk_stream_destroy(void *s);
int ptk_stream_sync(void *s);
/* one single-workgroup launch of `iters` dependent ALU steps (no memory reads), for timing how
 * streams share the hardware queues */
int ptk_calib_launch(int iters, void *s);
int ptk_stream_query(void *s);                     /* 1 done, 0 busy, -1 error */
int ptk_malloc(void **p, size_t bytes);
void ptk_fail_allocs(int skip, int n);   /* tests: after skip more successes, n ptk_malloc calls fail */
int ptk_free(void *p);
int ptk_h2d_async(void *dst, const void *src, size_t bytes, void *s);
int ptk_d2h_async(void *dst, const void *src, size_t bytes, void *s);
int ptk_d2d_async(void *dst, const void *src, size_t bytes, void *s);
int ptk_fill_async(void *dst, int byte, size_t bytes, void *s);   /* not for captured streams */
/* row-strided copies: height rows of width_bytes, pitches in bytes */
int ptk_d2d_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width_bytes,
                     size_t height, void *s);
int ptk_d2h_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width_bytes,
                     size_t height, void *s);
int ptk_h2d_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width_bytes,
                     size_t height, void *s);
int ptk_event_create(void **e);
int ptk_event_destroy(void *e);
int ptk_event_record(void *e, void *s);
int ptk_stream_wait_event(void *s, void *e);
int ptk_event_elapsed_ms(float *ms, void *e0, void *e1);
int ptk_event_sync(void *e);
int ptk_device_sync(void);
/* Stream capture into a HIP graph (this thread's capture only) and replay.  ptk_capture_end ends
 * the capture in every case; with exec == NULL (the captured work failed) it discards the graph. */
int ptk_capture_begin(void *s);
int ptk_capture_end(void *s, void **exec);
int ptk_graph_launch(void *exec, void *s);
int ptk_graph_destroy(void *exec);
/* The library's static device scratch (no allocation): the current device's copy, its address
 * resolved once per device at ptk_init.  All users of one GPU share it.  0 / -1. */
#define PTK_STATIC_SCRATCH_BYTES ((size_t) 64 << 20)
int ptk_static_scratch(void **p, size_t *bytes);
/* Ordering of the scratch's users on one GPU: acquire makes stream s wait for the work of the
 * previous user (an event recorded after it; not while s is being captured), holds the device's
 * lock and stores the device index in *dev; release records the event on s when work was queued
 * (again not under capture) and drops that device's lock.  Every successful acquire is followed
 * by one release with its device index, on the same thread.  Neither allocates. */
int ptk_scratch_acquire(void *s, int *dev);
int ptk_scratch_release(void *s, int dev, int recorded_work);
/* re-read the PTK_* kernel-selection knobs from the environment (otherwise read once) */
void ptk_knobs_reload(void);

/* ---------------------------------------------------------------- conv problem descriptor
 * One implicit-GEMM problem.  Row m of the GEMM is an output channel (conv: m = co) or a phase
 * row (convT: m = r*C4 + co); column q is an output position of that row.  Reduction index
 * (k, ci): tap k, input channel ci.  Input column read for (q, k):
 *     c = q*stride + k*dil - shift          (convT phase form: stride 1, dil -1, shift 0)
 * c outside [0, lim) reads 0 (in-kernel zero padding and the convT tail flush).
 * Output for row m = r*C4 + co and column q goes to  y[b*bsy + co*ldy + (q*ys + r - ypad)]
 * when that index is in [0, Lout) (conv: C4 = M, ys = 1, ypad = 0). */
enum { PTK_IN_PLAIN = 0, PTK_IN_LEAKY = 1 };
enum {
  PTK_EPI_NONE = 0,
  PTK_EPI_LEAKY = 1,   /* v >= 0 ? v : a*v                        (reference op code 1) */
  PTK_EPI_RELU = 2,    /* v > 0 ? v : 0                            (reference op code 2) */
  PTK_EPI_MULS = 3,    /* v * a                                    (reference op code 3) */
  PTK_EPI_ADDS = 4,    /* v + a                                    (reference op code 4) */
  PTK_EPI_ADDT = 5,    /* v + t[b*bst + co*ldt + col]  (residual / branch sum; same layout as y) */
  PTK_EPI_DIVS = 6     /* v / a                                                                  */
};
#define PTK_MAX_EPI 4
#define PTK_MAX_GROUP 4

typedef struct {
  int op;
  float a;
  const float *t;
  int64_t ldt, bst;
} ptk_epi;

typedef struct {
  /* input */
  const float *x;
  int64_t ldx, bsx;           /* row stride, batch stride (elements) */
  int64_t lim;                /* valid virtual input columns [0, lim) */
  int cin;
  int in_op;
  float in_a;
  int reflect_l1;             /* virtual column 0 reads physical column 1, column c>0 reads c-1 */
  /* weights: relaid [Mp/32][K][cinp/8][64][4] (see ptk_relayout) */
  const float *w;
  /* optional: the same weights relaid for 16-row tiles [Mp/16][K][cinp/8][64][2]
     (ptk_relayout16); NULL keeps the launch on 32-row tiles */
  const float *w16;
  int cinp;
  const float *bias;
  int nbias;
  int K, dil, stride, shift;
  int M;                      /* GEMM rows (cout4 or s*cout4) */
  int C4;                     /* rows per phase (conv: M) */
  /* stride-4 convT only, 0 otherwise: the rows are interleaved by phase (row m is phase m & 3 of
     channel m >> 2; weights relaid by ptk_relayout_il / ptk_relayout16_il with il = C4), so the
     four phases of an output column sit in one lane and go to four consecutive samples */
  int phase_il;
  int64_t q0, nq;             /* output columns [q0, q0 + nq) */
  /* Per-item column ranges (overlap-save windows compute only the columns their kept samples
     depend on): batch item 0 starts ext_l columns earlier, the last item ends ext_r columns
     later (one item: both).  0, 0: every item computes [q0, q0 + nq). */
  int64_t ext_l, ext_r;
  /* columns of one item the tile shape is chosen for (0: nq).  The shape fixes the order in
     which a column's sums are added, so a launch over a sub-range of columns gives the same bits
     in those columns as the full launch when it names the full launch's column count here. */
  int64_t nq_shape;
  /* output */
  float *y;
  float *y2;                  /* optional second output: LeakyReLU(a2) of every value stored in y,
                                 same index (the next conv's pre-activated input) */
  float a2;
  int64_t ldy, bsy;
  int ys, ypad;
  int64_t Lout;
  int batch;
  int nepi;
  ptk_epi epi[PTK_MAX_EPI];
} ptk_conv_desc;

/* Relayout packed conv/convT weights [M/4][K][cin][4] into the MFMA operand layout
 * [Mp/32][K][cinp/8][64 lanes][4] (Mp = M rounded up to 32, zero rows/channels in the padding).  Returns the
 * cinp the kernels expect for this cin (ptk_conv_cinp). */
int ptk_conv_cinp(int cin);
size_t ptk_relayout_floats(int M, int K, int cin);
int ptk_relayout(float *dst, const float *wp, int M, int K, int cin, void *s);
/* the copy for 16-row tiles: [Mp/16][K][cinp/8][64][2], Mp = M rounded up to 16 */
size_t ptk_relayout16_floats(int M, int K, int cin);
int ptk_relayout16(float *dst, const float *wp, int M, int K, int cin, void *s);
/* the same two layouts with a stride-4 convT's rows interleaved by phase (il = its rows per
   phase C4, M = 4 * il): relaid row m is packed row (m & 3) * il + (m >> 2) */
int ptk_relayout_il(float *dst, const float *wp, int M, int K, int cin, int il, void *s);
int ptk_relayout16_il(float *dst, const float *wp, int M, int K, int cin, int il, void *s);
/* fp16 -> fp32 expansion of n items (bit-exact: subnormals keep their value, inf / NaN keep sign
 * and payload, nothing is quieted) */
int ptk_h2f(float *dst, const uint16_t *src, int64_t n, void *s);

/* Launch ngroup independent problems (1..PTK_MAX_GROUP) in one grid; heavy problems first.
 * Returns 0, or -1 when a shape is outside what the kernels support (ptk_last_error says why). */
int ptk_conv_launch(const ptk_conv_desc *d, int ngroup, void *s);
/* 1 when the MFMA kernel covers this problem's shape; else the caller uses the SIMT path */
int ptk_conv_mfma_ok(const ptk_conv_desc *d);

/* SIMT fallbacks over the PACKED layouts, for narrow shapes (cout4 < 16, tiny cin, huge K*dil):
 * conv: X rows of ldx with in-kernel padding by `shift`; convT: the phase/tap form.  The conv's
 * epilogue codes are PTK_EPI_* without PTK_EPI_ADDT (refused: no tensor is passed). */
int ptk_conv_simt(const float *x, int64_t ldx, int64_t bsx, int64_t lim, int cin, const float *wp,
                  const float *bias, int cout, int K, int stride, int dil, int shift, float *y,
                  int64_t ldy, int64_t bsy, int64_t n, int batch, int epi0, float a0, int epi1,
                  float a1, void *s);
int ptk_convT_simt(const float *x, int64_t ldx, int64_t bsx, int64_t tin, int cin,
                   const float *wp, const float *bias, int cout, int st, int pad, int K, float *y,
                   int64_t ldy, int64_t bsy, int64_t Lout, int batch, void *s);

/* C[m][nn] = A[m][k] @ B[k][nn], row strides lda/ldb/ldc, on fp32 MFMA: a 64 x 64 block of C per
 * workgroup, 32 x 32 per wave, k in steps of 8 (out-of-range rows, columns and k read as 0) */
int ptk_matmul(const float *A, int64_t m, int64_t k, int64_t lda, const float *B, int64_t ldb,
               int64_t nn, float *C, int64_t ldc, void *s);

/* elementwise: y = a + b (+ leaky when epi == 1), y = leaky(a) -- fp32, same ops as the host */
int ptk_add(const float *a, const float *b, float *y, int64_t n, int epi, float alpha, void *s);
int ptk_leaky(const float *a, float *y, int64_t n, float alpha, void *s);
/* y = leaky(((a + b) + c) / 3, alpha): the MRF branch average (ref/v21_graph_trace.txt:3851-3869) */
int ptk_avg3_leaky(const float *a, const float *b, const float *c, float *y, int64_t n, float alpha,
                   void *s);

/* decoder tail: conv_post output p [72][L] (row stride ldp) -> wav [16*(L-1)] (iSTFT + PQMF) */
int ptk_tail(const float *p, int64_t ldp, int64_t L, float *wav, const float *consts, void *s);
/* which samples of each batch item are stored: item i keeps local samples [lo_i, hi_i) with
 * lo_i = lo_first for i == 0 else lo, hi_i = hi_last for the last item else hi (overlap-save
 * windows keep only their interior); the rest is computed and dropped */
typedef struct {
  int64_t lo_first, lo, hi, hi_last;
} ptk_emit;
/* batched: item b reads p + b*bsp and writes wav + b*bsw */
int ptk_tail_batched(const float *p, int64_t ldp, int64_t bsp, int64_t L, float *wav, int64_t bsw,
                     int batch, const float *consts, const ptk_emit *emit, void *s);
/* the tail's table (floats): hann[16], basis_c[9*16], basis_s[9*16], the final conv's taps in
 * polyphase order hp[(band*4 + r)*16 + j] = tap 3 - r + 4j of the band (0 past tap 62; 256), and
 * its bias (1) */
#define PTK_TAIL_NCONST (16 + 144 + 144 + 256 + 1)

/* lane-layout probe of the fp32 32x32x2 MFMA builtin: d[32][32] = a[32][2] @ b[2][32] */
int ptk_mfma_probe(const float *a, const float *b, float *d, void *s);
/* and of the fp32 16x16x4 one: d[16][16] = a[16][4] @ b[4][16] */
int ptk_mfma16_probe(const float *a, const float *b, float *d, void *s);

#ifdef __cplusplus
}
#endif
#endif
