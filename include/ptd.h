/* ptd.h -- device-resident entry points of libptconv_hip.so, beside the reference ABI
 * (pt_v21_dev.h).
 *
 * The reference ABI is synchronous and host-buffer based: every pt_v21_conv/convT call copies its
 * input to the device and its output back unless a conv chain keeps it there.  These entry
 * points keep a whole MB-iSTFT decoder request on the device, the reference's PT_V21_DEVADD idea
 * (runtime/v21/src/pt_v21_host.c:2364-2543) carried through the decoder: every residual add,
 * branch sum, /3 and LeakyReLU is fused into a conv's epilogue or input staging, and the iSTFT +
 * PQMF tail is one kernel.  Same per-request model as the reference: one pt_ctx per request with
 * its own stream and arena (pt_v21_cuda_init), one shared weight pool.
 * All tensor pointers here are DEVICE pointers; calls only enqueue work on the context's stream
 * unless the name says _host or sync. */
#ifndef PTD_H_
#define PTD_H_

#include <stddef.h>
#include <stdint.h>

#include "pt_v21_dev.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Load n host records into the process-wide weight pool (one slab, 256-byte aligned records,
 * claim-parallel upload on the caller's stream), the same pool pt_v21_cuda_init fills from a
 * container.  Record i is then wtab/btab index i for pt_v21_conv/convT.  A pool that already
 * holds records keeps them and returns 0 when n matches, -1 otherwise. */
int ptd_pool_load(pt_ctx *c, int n, const void *const *host, const size_t *bytes);
/* device pointer of pool record i, or NULL */
const void *ptd_pool_record(int i);

/* ---- .ptk weight container (tools/export_v21.py:5-23, :232-274; C reader
 * runtime/v21/src/pt_v21_host.c:1086-1220, fp16 rule :653-673) ------------------------------ *
 * Header <IIIiq (magic 'PTK1', version, n_tensor, reserved, data_bytes), n records <64si4x6qqq
 * (name, ndim, dim[6], nelem, offset), 64-byte aligned payloads; bytes per item from the fp32
 * record "dtype.table" (4 fp32, 2 fp16), which must be present, as for the reference's reader.
 * The file is read whole into host memory and every range is checked: a truncated or corrupt
 * container is refused (NULL / -1 and a "pt_v21 hip: ptk:" line on stderr). */
typedef struct ptd_ptk ptd_ptk;
ptd_ptk *ptd_ptk_open(const char *path);      /* replaces the record pass of pt_v21_open */
void ptd_ptk_close(ptd_ptk *f);
int ptd_ptk_count(const ptd_ptk *f);          /* number of records */
int ptd_ptk_find(const ptd_ptk *f, const char *name);   /* first record of that name, or -1 */
/* record i: name (65 bytes, NUL-terminated), ndim, dims[6], nelem, bytes per item; 0 / -1 */
int ptd_ptk_info(const ptd_ptk *f, int i, char *name, int *ndim, int64_t *dims, int64_t *nelem,
                 int *itemsize);
const void *ptd_ptk_payload(const ptd_ptk *f, int i);   /* raw payload bytes (host), or NULL */
/* record i as fp32 on the host (n must equal its nelem): fp16 expands exactly, subnormals kept,
 * inf / NaN keep sign and payload (the reference's half2float_bits, pt_v21_host.c:653-673) */
int ptd_ptk_read_f32(const ptd_ptk *f, int i, float *out, int64_t n);
/* 0 when the container holds a v2.1 decoder this library runs: the 41 layers' dec.*.wp[#h] /
 * dec.*.b records at their packed sizes and the three fixed tail convTs (dec.ConvTranspose,
 * _1, _2) in the forms the fused tail implements; else -1 naming the first problem */
int ptd_ptk_check_decoder(const ptd_ptk *f);
/* Load the process weight pool from the container: pool record k = the record named ctab[k]
 * (the graph's constant table, gen/pt_graph.c pt_graph_ctab; NULL or absent names leave record
 * k empty).  fp16 payloads go up as fp16 and expand on the device.  Same pool and same rules as
 * ptd_pool_load; this is the container route of the reference's weights_upload
 * (pt_v21_cuda.cu:90-235), without a host fp32 copy of the model.  0 / -1. */
int ptd_pool_load_ptk(pt_ctx *c, const ptd_ptk *f, int n, const char *const *ctab);

/* ---- synthetic MB-iSTFT decoder (ref/v21_graph_trace.txt:3819-4065) ------------------------ *
 * 41 layers: 0 conv_pre, 1 ups.0, 2..19 MRF-256, 20 ups.1, 21..38 MRF-128, 39 conv_post, 40 the
 * final PQMF synthesis conv /dec/Conv (4 -> 1, K 63, packed [1][63][4][4]; bias may be NULL);
 * MRF order branch (K 3,7,11) x dilation (1,3,5) x (c1, c2).  Weights in the packed layouts. */
#define PTD_DEC_NLAYER 41
typedef struct ptd_model ptd_model;

/* Uploads the 41 layers' weights and biases once into one device slab owned by the model and
 * shared by every context, lays every conv weight out for the MFMA kernels and builds the tail's
 * table (closed-form Hann and irfft basis, layer 40's taps and bias).  Needs an initialised
 * context (its stream does the upload).  NULL on failure. */
ptd_model *ptd_model_create(pt_ctx *c, const float *const *w, const float *const *b);
/* The same model from a container's dec.* records (ptd_ptk_check_decoder must pass); fp16
 * weights expand on the device.  The container may be closed after the call.  NULL on failure. */
ptd_model *ptd_model_create_ptk(pt_ctx *c, const ptd_ptk *f);
void ptd_model_destroy(ptd_model *m);

/* Decode `batch` requests of T frames: z [batch][192][T] -> wav [batch][256*T].  Activations
 * come from the context's arena (released on return); asynchronous on the context's stream.
 * 0 / -1. */
int ptd_decode(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch, float *wav);
/* arena bytes one ptd_decode call needs */
size_t ptd_decode_arena_bytes(int64_t T, int batch);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP stream capture, serving loops that forbid hipMalloc): ptd_decode with its activations in a
 * static device scratch of the library (64 MiB per GPU, held until the process ends) instead of
 * the context's arena.  It allocates nothing.  A decode needing more than the scratch
 * (ptd_decode_arena_bytes(T, batch) > 64 MiB, e.g. batch 1 above 435 frames) is refused: -1 and a
 * stderr line, nothing queued.  Every call on one GPU shares that GPU's scratch.  Eager calls are
 * ordered on the GPU by the library: each call's kernels wait for those of the previous call on
 * that GPU, whichever context's stream ran it (an event per GPU, made at set-up), so contexts may
 * call one after another without synchronising.  A call made while its stream is being captured
 * records no such wait: replays of the graph race with any other use of the scratch that overlaps
 * them in time, and the caller orders them (one stream for all of them, or a synchronisation in
 * between).  Same output bits as ptd_decode.  Asynchronous.  0 / -1. */
int ptd_decode_noalloc(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch,
                       float *wav);
/* Same, also copying the six stage tensors (conv_pre+leaky, ups.0, MRF-256 out, ups.1, MRF-128
 * out, conv_post) of batch item 0 into the given device buffers (entries may be NULL). */
int ptd_decode_stages(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, float *wav,
                      float *const *stages);

/* The decoder tail alone, the stages after conv_post (ref/v21_graph_trace.txt:4176-4315): p is
 * conv_post's output [batch][72][L] (4 subbands x (9 log-magnitudes + 9 phase logits)), wav gets
 * [batch][16*(L-1)] samples: exp / sin / cos -> irfft (n_fft 16) -> Hann -> overlap-add (hop 4)
 * -> window-sum normalisation -> [8:-8] trim -> PQMF x4 zero-insert -> the model's 63-tap
 * synthesis conv (layer 40).  One kernel, asynchronous.  0 / -1. */
int ptd_tail(pt_ctx *c, const ptd_model *m, const float *p, int64_t L, int batch, float *wav);

/* Run decoder layer i (0..39) alone: conv (x [batch][cin][T] -> y [batch][cout4][Tout]) or convT
 * (x [batch][cin][T] -> y [batch][cout4][Lout]).  in_leaky > 0 applies LeakyReLU(in_leaky) to
 * the input as it is read; epi_leaky > 0 applies it to the output.  Asynchronous. */
int ptd_layer(pt_ctx *c, const ptd_model *m, int layer, const float *x, int64_t T, int batch,
              float *y, float in_leaky, float epi_leaky);
/* The same over a part of the GEMM columns (no counterpart in the reference): cols = {q0, nq,
 * ext_l, ext_r, nq_shape} as ptd_window_cols gives them (conv: column = output position; convT:
 * column q writes outputs q*stride - pad .. + stride - 1).  Outputs outside are not written. */
int ptd_layer_cols(pt_ctx *c, const ptd_model *m, int layer, const float *x, int64_t T, int batch,
                   float *y, float in_leaky, float epi_leaky, const int64_t *cols);
/* One MRF stack (config 3): stage 0 = MRF-256 (layers 2..19), 1 = MRF-128 (21..38);
 * x [C][T] -> out = leaky(((b0 + b1) + b2) / 3, alpha) [C][T].  Asynchronous. */
int ptd_mrf(pt_ctx *c, const ptd_model *m, int stage, const float *x, int64_t T, float alpha,
            float *out);

/* One depth j (0..2, dilation 1/3/5) of an MRF stack: the three branches' c1 convs in one
 * grouped launch (input LeakyReLU(0.1)(xin[br]): read from xin_leaky[br] when given, else applied
 * to xin[br] as it is staged; epilogue LeakyReLU(0.1) -> a[br]), then their c2 convs in one
 * grouped launch (epilogue adds the residual xin[br] -> y[br], and writes LeakyReLU(0.1) of it to
 * y_leaky[br] when y_leaky is given).  All [C][T].  Asynchronous.  Two kernel launches of
 * 2*C*C*T*(3+7+11) flops each. */
int ptd_mrf_depth(pt_ctx *c, const ptd_model *m, int stage, int depth, const float *const *xin,
                  const float *const *xin_leaky, float *const *a, float *const *y,
                  float *const *y_leaky, int64_t T);

/* Long-form request through overlap-save windows (config 5; the reference's --stream driver,
 * main_v21.c:331-370 with pt_v21_host.c:2789-2912): window k decodes frames [k*hop, k*hop + win)
 * clipped to the sequence, hop = win - 2*ctx, and keeps the samples of its frames [ctx, win - ctx)
 * (from 0 in the first window, to its end in the last).  win >= 2*ctx + 1, taken as given.  All
 * windows are independent, so they run as one batched decode.  z [192][T], wav [256*T].
 * Asynchronous. */
int ptd_decode_windows(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int win, int ctx,
                       float *wav);
size_t ptd_windows_arena_bytes(int64_t T, int win, int ctx);
/* The same with the reference's streaming schedule (main_v21_serve.c:219-257): the first window
 * win_first frames wide (fast first audio; the reference's default 48), the later ones win (its
 * default 256); a width below 2*ctx + 8 is raised to it, as the reference server does
 * (main_v21_serve.c:223-224).  The first window runs as its own decode when its width
 * differs, the evenly spaced full windows as one batched decode, a clipped last window alone.
 * Output identical to decoding the windows one at a time (ptd_decode_chunk) and keeping what the
 * reference's loop keeps.  Asynchronous.  0 / -1. */
int ptd_decode_windows2(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int win_first,
                        int win, int ctx, float *wav);
size_t ptd_windows2_arena_bytes(int64_t T, int win_first, int win, int ctx);
/* The columns a windowed decode computes (no counterpart in the reference, which decodes every
 * column of a window and drops the samples outside its interior): each conv launch covers only
 * the columns the kept samples depend on, with the tile shape of the full window, so the kept
 * samples are bit-identical to a full-window decode.  For a decode of `batch` windows of T frames
 * in which item 0 keeps samples [lo_first, hi), middle items [lo, hi) and the last item
 * [lo, hi_last) (one item: [lo_first, hi_last)), out[5*i .. 5*i + 4] receives launch i's GEMM
 * columns {q0, nq, ext_l, ext_r, nq_shape} (ptk_conv_desc: item 0 starts ext_l earlier, the last
 * item ends ext_r later), launches in decode order: conv_pre, ups.0, MRF-256 (depth, branch
 * K 3/7/11, c1 then c2: 18), ups.1, MRF-128 (18), conv_post.  Host only.  Returns 1 (columns left
 * out), 0 (every column is needed: the decode runs whole) or -1 (bad arguments).
 * PTD_WINDOW_CONE=0 in the environment makes windowed decodes compute every column. */
#define PTD_WINDOW_LAUNCHES 40
int ptd_window_cols(int64_t T, int batch, int64_t lo_first, int64_t lo, int64_t hi,
                    int64_t hi_last, int64_t *out);

/* A decode of fixed shape and buffers captured once as a HIP graph and replayed (no counterpart in
 * the reference, whose graph interpreter issues every node from the host): for a serving loop that
 * reuses its buffers, the 19 launches go to the device as one submission.  z and wav are read and
 * written in place on every replay (refill z, launch, read wav).  The graph owns its scratch
 * memory (ptd_decode_arena_bytes(T, batch)), so the context's arena is free for other work between
 * replays.  Replays run on the capturing context's stream only; destroy the graph before the
 * context and the model.  Launch is asynchronous; destroy waits for replays in flight. */
typedef struct ptd_graph ptd_graph;
ptd_graph *ptd_decode_graph(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch,
                            float *wav);
int ptd_graph_launch(pt_ctx *c, const ptd_graph *g);
void ptd_graph_destroy(ptd_graph *g);

/* One window of a sequence, for audio as it is decoded (replaces pt_v21_stream_chunk,
 * pt_v21.h:194, pt_v21_host.c:2871-2902): a < 0 reads as 0, win < 1 as 1, and the window is
 * clipped to [a, T); -1 if nothing is left.  pcm (device, >= 256*win floats) receives the whole
 * window's waveform and *n its length (256 x the clipped width); the caller keeps the interior,
 * as main_v21.c:344-362 does.  z [192][T] read in place; arena as ptd_decode_arena_bytes(win, 1).
 * Asynchronous. */
int ptd_decode_chunk(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int64_t a,
                     int64_t win, float *pcm, int64_t *n);

/* ---- concurrent serving (config 5; the reference's main_v21_par.c:59-158 model) ------------ *
 * nctx contexts (one stream + arena each, sharing the model's weights), each driven by its own
 * pthread.  ptd_serve_run hands request r to context r % nctx, runs all requests, waits for
 * all of them and returns the wall time in ms (host clock, from the first enqueue to the last
 * stream's completion).  Requests with win > 0 use the windowed path.  ptd_server_create (and
 * ptd_queue_create) time where the contexts' streams sit on HIP's hardware queues and keep the
 * most even arrangement (a few ms of single-workgroup kernels, with the device synchronised
 * between them: create servers before other work is queued on the device; PTD_SERVER_PLACE=0
 * skips it). */
typedef struct ptd_server ptd_server;
ptd_server *ptd_server_create(int nctx, size_t arena_bytes);
void ptd_server_destroy(ptd_server *s);
pt_ctx *ptd_server_ctx(ptd_server *s, int i);
typedef struct {
  const float *z;   /* device [192][T] */
  float *wav;       /* device [256*T] */
  int64_t T;
  int win, ctx;     /* win > 0: overlap-save windows */
} ptd_request;
int ptd_serve_run(ptd_server *s, const ptd_model *m, const ptd_request *req, int nreq,
                  double *wall_ms);

/* ---- queue-fed serving (the reference's server loop, main_v21_serve.c:129-160, :281-335) --- *
 * nworkers persistent workers, each with its own context (stream + arena) sharing the model,
 * created once with the queue.  Jobs are submitted with a deadline and popped earliest-deadline-
 * first (stable: equal deadlines keep submission order), as the reference's EDF queue does; the
 * queue holds at most `capacity` unfinished jobs (queued or running; the reference's MAX_QUEUE is
 * 64) and refuses more.  A job either decodes in one piece or streams: win > 0 runs the
 * overlap-save schedule of ptd_decode_windows2 with its first window decoded, and waited for, on
 * its own, so its audio (the first win_first - ctx frames) is complete at t_first, and the rest
 * batched.  All times are ptd_now_ms() values. */
typedef struct ptd_queue ptd_queue;
typedef struct {
  const float *z;        /* device [192][T], read in place; valid until the job is done */
  float *wav;            /* device [256*T] */
  int64_t T;
  int win_first, win, ctx;   /* win > 0: streaming windows; win == 0: one decode */
  double deadline_ms;    /* EDF key: smaller runs first */
} ptd_job;
typedef struct {
  int rc;                /* the job's result: 0 / -1 */
  int worker;            /* which worker ran it */
  int64_t order;         /* 0, 1, 2, ...: the order in which workers took jobs from the queue */
  double t_submit, t_start, t_first, t_end;   /* t_first: first audio complete (= t_end unless
                                                streaming) */
} ptd_job_status;
/* NULL on failure (every context released) */
ptd_queue *ptd_queue_create(const ptd_model *m, int nworkers, size_t arena_bytes, int capacity);
/* job id (>= 0), or -1 when the queue is full, closed or the job is malformed */
int64_t ptd_queue_submit(ptd_queue *q, const ptd_job *job);
/* 1 done (status filled, the job's slot released), 0 still queued or running, -1 unknown id */
int ptd_queue_poll(ptd_queue *q, int64_t id, ptd_job_status *st);
/* blocks until the job is done; 0 (status filled, slot released) or -1 unknown id */
int ptd_queue_wait(ptd_queue *q, int64_t id, ptd_job_status *st);
/* hold = 1: workers take no new job (running ones finish); 0: resume.  For a caller that submits
 * a batch of jobs and wants them ordered among themselves by deadline. */
void ptd_queue_hold(ptd_queue *q, int hold);
/* runs every queued job, joins the workers, releases the contexts */
void ptd_queue_destroy(ptd_queue *q);
double ptd_now_ms(void);   /* host clock of the job times */

/* ---- plumbing for callers without a HIP runtime of their own (tests, bench.py) ------------ */
void *ptd_malloc(size_t bytes);                 /* device memory, NULL on failure */
void ptd_free(void *p);
/* Tests of the error paths (no counterpart in the reference, whose tests force failures through
 * its env knobs only): after `skip` more device allocations of this library succeed, the next n
 * fail as if the device were out of memory.  Process-wide; n = 0 switches it off. */
void ptd_debug_fail_allocs(int skip, int n);
/* The library reads its tuning knobs (PTK_CONV_*, PTK_TAIL_*, PTD_WINDOW_*) from the environment
 * once per process, at first use.  This re-reads them, for tests that change one between calls
 * (no counterpart in the reference, whose knobs are static caches too).  The reference's operator
 * knobs (PT_V21_*) keep their read-once behaviour. */
void ptd_debug_reload_env(void);
/* Tests of what a decode reads (no counterpart in the reference): every byte of the context's
 * arena set to `byte` on its stream (0xff makes every float NaN, so a column read before any
 * launch wrote it poisons what depends on it).  Synchronous.  0 / -1. */
int ptd_debug_fill_arena(pt_ctx *c, int byte);
int ptd_h2d(pt_ctx *c, void *dst, const void *src, size_t bytes);   /* synchronous */
int ptd_d2h(pt_ctx *c, void *dst, const void *src, size_t bytes);   /* synchronous */
int ptd_sync(pt_ctx *c);                        /* wait for the context's stream */
int ptd_device_sync(void);                      /* wait for every stream of the device */
void *ptd_event_create(void);
void ptd_event_destroy(void *e);
int ptd_event_record(pt_ctx *c, void *e);       /* on the context's stream */
float ptd_event_elapsed_ms(void *e0, void *e1); /* waits for e1; negative on error */

/* fp32 32x32x2 MFMA lane-layout probe (test hook): d[32][32] = a[32][2] @ b[2][32], host
 * buffers, synchronous on the context's stream. */
int ptd_mfma_probe(pt_ctx *c, const float *a, const float *b, float *d);
/* the same for the fp32 16x16x4 MFMA builtin the 16-row conv tiles use: a[16][4], b[4][16] ->
 * d[16][16] (host buffers) */
int ptd_mfma16_probe(pt_ctx *c, const float *a, const float *b, float *d);
/* closed-form part of the tail table as the device uses it (host copy, PTD_TAIL_NCONST floats):
 * periodic Hann(16), irfft basis cos rows (9 x 16), -sin rows (9 x 16) */
#define PTD_TAIL_NCONST (16 + 144 + 144)
void ptd_tail_constants(float *out);
/* offsets of the pt_ctx fields the device layer touches (for the ABI test) */
int ptd_ctx_layout(long *out, int n);

#ifdef __cplusplus
}
#endif
#endif
