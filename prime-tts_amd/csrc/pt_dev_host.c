/* pt_dev_host.c -- C (gnu11) host side of libptconv_hip.so: the reference's device entry points
 * (runtime/v21/src/pt_v21.h:208-259) over the HIP layer in ptk_kernels.hip.
 *
 * Per request: one pt_ctx, one non-blocking HIP stream, one device arena (bump allocator with
 * mark/release; PT_V21_ARENA_MB, default 256 MiB -- the reference's 8 MiB default was sized for a
 * 4 GB Jetson, an MI355X has 288 GB).  Per process: one weight pool (a single slab, 256-byte
 * aligned records, refcounted by the contexts, uploaded once with copies claimed in parallel by
 * the contexts that arrive together), plus the MFMA relayout of each conv weight, built the first
 * time a context uses it.  Calls are synchronous as in the reference: the output is on the host
 * when pt_v21_conv returns, unless the caller asked to keep it on the device for the next conv. */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <sys/prctl.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pt_dev_internal.h"
#include "ptd.h"

/* ------------------------------------------------------------------ imports from the host
 * Weak: resolved when the library is linked into the reference host (pt_v21_host.c built with
 * -DPT_V21_CUDA), NULL when the library is loaded on its own. */
extern int pt_v21_n_cont(pt_ctx *c) __attribute__((weak));
extern const float *pt_v21_cont(pt_ctx *c, int idx) __attribute__((weak));
extern size_t pt_v21_cont_bytes(pt_ctx *c, int idx) __attribute__((weak));
extern int pt_v21_conv_cpu(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, float *Y,
                           int64_t ldy, int64_t n, int cout, int K, int stride, int pad, int dil,
                           const float *wp, const float *bias, int64_t batch, int wtab, int btab,
                           int epi0, int epi1, float a0, float a1) __attribute__((weak));
extern int pt_v21_convT_cpu(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, int64_t tin,
                            float *Y, int64_t ldy, int cout, int s, int pad, int K,
                            const float *wp, const float *bias, int64_t batch, int wtab,
                            int btab) __attribute__((weak));
extern int pt_v21_matmul_cpu(pt_ctx *c, const float *A, int64_t m, int64_t k, int64_t lda,
                             const float *B, int64_t ldb, int64_t nn, float *C,
                             int64_t ldc) __attribute__((weak));

double ptdi_now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double) ts.tv_sec * 1e3 + (double) ts.tv_nsec * 1e-6;
}

static int env_int(const char *name, int dflt) {
  const char *e = getenv(name);
  return e && *e ? atoi(e) : dflt;
}

/* PT_V21_CUDAPROF (the reference's knob, pt_v21_cuda.cu:83-87, 1781-1955): each conv / convT /
 * matmul call charges its device allocations to g_alloc_ms, its uploads to g_copy_ms, the
 * kernels with the result copy and the stream wait to g_kernel_ms, and its frees to g_free_ms,
 * synchronising the device between phases so each gets its own time.  Off, nothing is recorded
 * and nothing extra is synchronised. */
typedef struct {
  int on;
  double t;
} phase_t;
static int g_cudaprof;
static pthread_once_t g_cudaprof_once = PTHREAD_ONCE_INIT;
static void cudaprof_read(void) { g_cudaprof = getenv("PT_V21_CUDAPROF") ? 1 : 0; }
static int cudaprof(void) {
  pthread_once(&g_cudaprof_once, cudaprof_read);
  return g_cudaprof;
}
static void phase_begin(phase_t *p) {
  p->on = cudaprof();
  p->t = 0.0;
  if (p->on) {
    ptk_device_sync();
    p->t = ptdi_now_ms();
  }
}
static void phase_end(phase_t *p, double *field) {
  if (!p->on) return;
  ptk_device_sync();
  const double t = ptdi_now_ms();
  *field += t - p->t;
  p->t = t;
}

/* ================================================================== weight pool */
typedef struct {
  float *dev;
  int M, K, cin;
} relaid_t;

static struct {
  pthread_mutex_t lock;
  int ref;              /* contexts holding the pool */
  int setup;            /* slab laid out (records may still be in flight) */
  int n;
  char *slab;
  size_t slab_bytes, data_bytes;
  size_t *off, *bytes;  /* device bytes (fp32) per record */
  const void **src;     /* host sources, for the claimed copies */
  unsigned char *isz;   /* bytes per item of each source: 4 fp32, 2 fp16 (expanded on the device) */
  size_t half_max;      /* largest fp16 source in bytes (staging size of a claimant) */
  volatile int next;    /* next record to claim */
  volatile int done;    /* records whose copy has COMPLETED (counted after a stream sync) */
  volatile int fail;
  relaid_t *rl;
} P = {PTHREAD_MUTEX_INITIALIZER, 0, 0, 0, NULL, 0, 0, NULL, NULL, NULL, NULL, 0, 0, 0, 0, NULL};

/* lay the slab out and allocate it; called with P.lock held.  bytes[i] is record i's size on
 * the device (fp32); isz[i] the source's bytes per item (NULL: all 4) */
static int pool_setup_locked(int n, const void *const *src, const size_t *bytes,
                             const unsigned char *isz) {
  P.off = calloc((size_t) n, sizeof(size_t));
  P.bytes = calloc((size_t) n, sizeof(size_t));
  P.src = calloc((size_t) n, sizeof(void *));
  P.isz = calloc((size_t) n, 1);
  P.rl = calloc((size_t) n, sizeof(relaid_t));
  if (!P.off || !P.bytes || !P.src || !P.isz || !P.rl) goto oom;
  size_t total = 0, data = 0;
  P.half_max = 0;
  for (int i = 0; i < n; i++) {
    P.src[i] = src[i];
    P.bytes[i] = src[i] ? bytes[i] : 0;
    P.isz[i] = isz ? isz[i] : 4;
    if (P.isz[i] == 2 && P.bytes[i] / 2 > P.half_max) P.half_max = P.bytes[i] / 2;
    P.off[i] = total;
    total += (P.bytes[i] + 255) & ~(size_t) 255;
    data += P.bytes[i];
  }
  if (ptk_malloc((void **) &P.slab, total)) {
    PT_LOG("weight pool slab of %zu bytes failed: %s", total, ptk_last_error());
    goto oom;
  }
  P.slab_bytes = total;
  P.data_bytes = data;
  P.n = n;
  P.next = 0;
  P.done = 0;
  P.fail = 0;
  P.setup = 1;
  return 0;
oom:
  free(P.off); free(P.bytes); free(P.src); free(P.isz); free(P.rl);
  P.off = P.bytes = NULL; P.src = NULL; P.isz = NULL; P.rl = NULL;
  return -1;
}

/* Copy the records this thread claims on its own stream, sync it, publish the count, then wait
 * until every record of every claimant has completed.  Counting after the sync (not after the
 * enqueue) is what makes "done == n" mean the data is on the device. */
static int pool_claim_upload(pt_ctx *c) {
  int mine = 0;
  void *stage = NULL;   /* this claimant's fp16 staging buffer; the stream orders its reuse */
  for (;;) {
    const int i = __sync_fetch_and_add(&P.next, 1);
    if (i >= P.n) break;
    mine++;
    if (!P.bytes[i]) continue;
    int bad;
    if (P.isz[i] == 4) {
      bad = ptk_h2d_async(P.slab + P.off[i], P.src[i], P.bytes[i], c->g_stream);
    } else {
      const int64_t items = (int64_t) (P.bytes[i] / 4);
      bad = (!stage && ptk_malloc(&stage, P.half_max)) ||
            ptk_h2d_async(stage, P.src[i], (size_t) items * 2, c->g_stream) ||
            ptk_h2f((float *) (P.slab + P.off[i]), (const uint16_t *) stage, items, c->g_stream);
    }
    if (bad) __sync_bool_compare_and_swap(&P.fail, 0, 1);
  }
  if (mine && ptk_stream_sync(c->g_stream)) __sync_bool_compare_and_swap(&P.fail, 0, 1);
  ptk_free(stage);
  __sync_fetch_and_add(&P.done, mine);
  while (__sync_add_and_fetch(&P.done, 0) < P.n && !__sync_add_and_fetch(&P.fail, 0)) sched_yield();
  if (P.fail) {
    PT_LOG("weight upload failed: %s", ptk_last_error());
    return -1;
  }
  return 0;
}

static void pool_free_locked(void) {
  if (P.rl)
    for (int i = 0; i < P.n; i++) ptk_free(P.rl[i].dev);
  ptk_free(P.slab);
  free(P.off); free(P.bytes); free(P.src); free(P.isz); free(P.rl);
  P.slab = NULL; P.off = P.bytes = NULL; P.src = NULL; P.isz = NULL; P.rl = NULL;
  P.n = 0; P.setup = 0; P.slab_bytes = P.data_bytes = 0;
}

void ptdi_pool_ref(int delta) {
  pthread_mutex_lock(&P.lock);
  P.ref += delta;
  if (P.ref <= 0) {
    P.ref = 0;
    if (P.setup) pool_free_locked();
  }
  pthread_mutex_unlock(&P.lock);
}

/* PT_V21_UP_PAR (read once per process; pt_v21_cuda.cu:167-174): 1 (default) every context
 * claims records and copies them in parallel; 0 is the reference's serialised bisection endpoint,
 * where the first context copies every record while holding the pool lock and the others, once
 * they get the lock, find the copies done. */
static int g_up_par = 1;
static pthread_once_t g_up_par_once = PTHREAD_ONCE_INIT;
static void up_par_read(void) { g_up_par = env_int("PT_V21_UP_PAR", 1) != 0; }

static int pool_upload(pt_ctx *c) {
  pthread_once(&g_up_par_once, up_par_read);
  if (g_up_par) return pool_claim_upload(c);
  pthread_mutex_lock(&P.lock);
  const int r = pool_claim_upload(c);
  pthread_mutex_unlock(&P.lock);
  return r;
}

int ptdi_pool_load_src(pt_ctx *c, int n, const void *const *host, const size_t *bytes,
                       const unsigned char *isz) {
  if (!c || !c->use_cuda || n <= 0) return -1;
  pthread_mutex_lock(&P.lock);
  int r = 0;
  if (P.setup && P.n != n) {
    PT_LOG("weight pool already holds %d records (asked to load %d)", P.n, n);
    r = -1;
  } else if (!P.setup) {
    r = pool_setup_locked(n, host, bytes, isz);
  }
  pthread_mutex_unlock(&P.lock);
  if (r) return -1;
  return pool_upload(c);
}

int ptd_pool_load(pt_ctx *c, int n, const void *const *host, const size_t *bytes) {
  return ptdi_pool_load_src(c, n, host, bytes, NULL);
}

const void *ptdi_pool_get(int idx, size_t need) {
  if (!P.setup || idx < 0 || idx >= P.n || P.bytes[idx] < need || !P.bytes[idx]) return NULL;
  return P.slab + P.off[idx];
}

const void *ptd_pool_record(int i) { return ptdi_pool_get(i, 1); }

const float *ptdi_pool_relaid(pt_ctx *c, int idx, int M, int K, int cin) {
  const size_t need = (size_t) M * K * cin * sizeof(float);
  const float *src = ptdi_pool_get(idx, need);
  if (!src) return NULL;
  pthread_mutex_lock(&P.lock);
  relaid_t *r = &P.rl[idx];
  const float *out = NULL;
  if (r->dev) {
    if (r->M == M && r->K == K && r->cin == cin) out = r->dev;   /* else: geometry clash, per call */
  } else {
    float *d = NULL;
    if (!ptk_malloc((void **) &d, ptk_relayout_floats(M, K, cin) * sizeof(float)) &&
        !ptk_relayout(d, src, M, K, cin, c->g_stream) && !ptk_stream_sync(c->g_stream)) {
      r->dev = d;
      r->M = M;
      r->K = K;
      r->cin = cin;
      out = d;
    } else {
      PT_LOG("relayout of record %d failed: %s", idx, ptk_last_error());
      ptk_free(d);
    }
  }
  pthread_mutex_unlock(&P.lock);
  return out;
}

double pt_v21_cuda_weights_mib(pt_ctx *c) {
  (void) c;
  return (double) P.data_bytes / 1048576.0;
}

/* ================================================================== arena */
void *ptdi_arena_alloc(pt_ctx *c, size_t bytes) {
  const size_t off = (c->g_arena_used + 255) & ~(size_t) 255;
  if (!c->g_arena || off > c->g_arena_bytes || bytes > c->g_arena_bytes - off) return NULL;
  c->g_arena_used = off + bytes;
  if (c->g_arena_used > c->arena_alloc_bytes) c->arena_alloc_bytes = c->g_arena_used;
  return (char *) c->g_arena + off;
}
void *ptdi_arena_mark(pt_ctx *c) { return (char *) c->g_arena + c->g_arena_used; }
void ptdi_arena_release(pt_ctx *c, void *mark) {
  c->g_arena_used = (size_t) ((char *) mark - (char *) c->g_arena);
}

/* ================================================================== wait policy
 * PT_V21_WAIT_US = 0 (default): the runtime's own stream wait.  > 0: poll the stream, sleeping
 * that long between polls while another context is doing host work (the reference's policy for
 * few-core hosts, pt_v21_cuda.cu:25-57, whose default is 200), yielding otherwise;
 * PT_V21_WAIT_ADAPT=0 always sleeps.  The default differs from the reference's because an MI355X
 * host has cores to spare for the runtime's own wait. */
static int g_n_active, g_n_waiting;

void pt_v21_cuda_active(int delta) { __atomic_add_fetch(&g_n_active, delta, __ATOMIC_RELAXED); }

static int g_wait_us, g_wait_adapt;
static pthread_once_t g_wait_once = PTHREAD_ONCE_INIT;
static void wait_policy_read(void) {
  g_wait_adapt = env_int("PT_V21_WAIT_ADAPT", 1);
  g_wait_us = env_int("PT_V21_WAIT_US", 0);
}

/* Each poll interval is spent one of two ways: a short sleep, which frees the core for a context
 * that still has host work to issue, or a yield, when no context has any (every active one is
 * waiting), so the first stream to finish is noticed at once. */
static int others_issue_host_work(void) {
  return __atomic_load_n(&g_n_active, __ATOMIC_RELAXED) -
             __atomic_load_n(&g_n_waiting, __ATOMIC_RELAXED) > 0;
}

/* Short sleeps are only short with a small timer slack (Linux's default of 50 us would stretch
 * each one); set once per waiting thread unless PT_V21_SLACK0 asks to keep the default. */
static void tighten_timer_slack(void) {
  static __thread int done;
  if (done) return;
  done = 1;
  if (!getenv("PT_V21_SLACK0")) prctl(PR_SET_TIMERSLACK, 1UL, 0, 0, 0);
}

int ptdi_wait_before_copy(pt_ctx *c) {
  pthread_once(&g_wait_once, wait_policy_read);
  return g_wait_us <= 0 ? 0 : ptdi_wait(c);
}

int ptdi_wait(pt_ctx *c) {
  pthread_once(&g_wait_once, wait_policy_read);
  if (g_wait_us <= 0) return ptk_stream_sync(c->g_stream);   /* the runtime's own blocking wait */
  tighten_timer_slack();
  const struct timespec nap = {0, (long) g_wait_us * 1000L};
  __atomic_add_fetch(&g_n_waiting, 1, __ATOMIC_RELAXED);
  int state;
  for (;;) {
    state = ptk_stream_query(c->g_stream);   /* 1 done, 0 busy, -1 error */
    if (state != 0) break;
    if (g_wait_adapt && !others_issue_host_work()) sched_yield();
    else nanosleep(&nap, NULL);
  }
  __atomic_sub_fetch(&g_n_waiting, 1, __ATOMIC_RELAXED);
  return state < 0 ? -1 : 0;
}

/* ================================================================== init / shutdown */
int pt_v21_cuda_prewarm(void) {
  if (ptk_init()) PT_LOG("prewarm: %s", ptk_last_error());
  return 0;
}

int ptdi_ctx_init(pt_ctx *c, size_t arena_bytes, int verbose) {
  if (!c) return -1;
  if (ptk_init()) {
    PT_LOG("no usable device: %s", ptk_last_error());
    return -1;
  }
  if (ptk_stream_create(&c->g_stream)) {
    PT_LOG("stream create failed: %s", ptk_last_error());
    return -1;
  }
  c->g_arena = NULL;
  if (arena_bytes && ptk_malloc(&c->g_arena, arena_bytes)) {
    PT_LOG("arena of %zu MiB failed: %s", arena_bytes >> 20, ptk_last_error());
    ptk_stream_destroy(c->g_stream);
    c->g_stream = NULL;
    return -1;
  }
  c->g_arena_bytes = c->g_arena ? arena_bytes : 0;
  c->g_arena_used = 0;
  c->dev_bytes_arena = (double) c->g_arena_bytes;
  c->chain_mark = NULL;
  c->conv_in_dev = NULL;
  c->conv_out_dev = NULL;
  c->conv_keep = 0;
  c->use_cuda = 1;
  /* shared weights: the container's records when this library sits in the reference host */
  pthread_mutex_lock(&P.lock);
  P.ref++;
  int r = 0;
  const int have_cont = pt_v21_n_cont && pt_v21_cont && pt_v21_cont_bytes;
  if (!P.setup && have_cont) {
    const int n = pt_v21_n_cont(c);
    const void **src = calloc((size_t) (n > 0 ? n : 1), sizeof(void *));
    size_t *nb = calloc((size_t) (n > 0 ? n : 1), sizeof(size_t));
    if (!src || !nb) r = -1;
    for (int i = 0; r == 0 && i < n; i++) {
      src[i] = pt_v21_cont(c, i);
      nb[i] = src[i] ? pt_v21_cont_bytes(c, i) : 0;
    }
    if (r == 0 && n > 0) r = pool_setup_locked(n, src, nb, NULL);
    free(src);
    free(nb);
  }
  const int upload = P.setup;
  pthread_mutex_unlock(&P.lock);
  if (r == 0 && upload) r = pool_upload(c);
  if (r) {
    /* leave nothing behind: stream, arena and the pool reference taken above */
    pt_v21_cuda_shutdown(c);
    return -1;
  }
  c->dev_bytes_weights = (double) P.data_bytes;
  if (verbose)
    PT_LOG("context ready: %.1f MiB shared weights, %zu MiB arena",
           (double) P.data_bytes / 1048576.0, arena_bytes >> 20);
  return r;
}

int pt_v21_cuda_init(pt_ctx *c, int verbose) {
  return ptdi_ctx_init(c, (size_t) env_int("PT_V21_ARENA_MB", 256) << 20, verbose);
}

static void devres_destroy(pt_ctx *c);

void pt_v21_cuda_shutdown(pt_ctx *c) {
  if (!c) return;
  ptdi_aux_release(c);
  if (c->g_stream) {
    ptk_stream_sync(c->g_stream);
    ptk_stream_destroy(c->g_stream);
    c->g_stream = NULL;
  }
  devres_destroy(c);
  if (c->g_arena) {
    ptk_free(c->g_arena);
    c->g_arena = NULL;
  }
  c->g_arena_bytes = c->g_arena_used = 0;
  if (c->use_cuda) ptdi_pool_ref(-1);
  c->use_cuda = 0;
}

int pt_v21_cuda_keepwarm(int iters) {
  (void) iters;
  return 0;
}
long pt_v21_gpu_cur_freq(void) { return -1; }
long pt_v21_gpu_max_freq(void) { return -1; }
/* ================================================================== per-op routing
 * PT_V21_GPU=conv,convT,matmul: the reference device layer's switches for bisection
 * (pt_v21_cuda.cu:70-76).  An op whose name the value does not contain runs on the host's CPU
 * path (the same substring test: "convT" also keeps conv on the device); unset or empty, every op
 * runs on the device.  Read once per process. */
static int g_gpu_conv = 1, g_gpu_convT = 1, g_gpu_matmul = 1;
static pthread_once_t g_gpu_once = PTHREAD_ONCE_INIT;
static void gpu_ops_read(void) {
  const char *e = getenv("PT_V21_GPU");
  if (!e || !*e) return;
  g_gpu_conv = strstr(e, "conv") != NULL;
  g_gpu_convT = strstr(e, "convT") != NULL;
  g_gpu_matmul = strstr(e, "matmul") != NULL;
}
static int gpu_op(const int *flag) {
  pthread_once(&g_gpu_once, gpu_ops_read);
  return *flag;
}

/* The kernels pad rows themselves, so the host hands over unpadded rows, except when convs are
 * routed to the CPU path (which reads padded rows): then the host pads them, and never chains
 * (its chain rule needs unpadded rows, pt_v21_host.c:3341-3343). */
int pt_v21_conv_pads_in_kernel(pt_ctx *c) {
  (void) c;
  return gpu_op(&g_gpu_conv);
}

/* ================================================================== descriptors */
void ptdi_conv_desc(ptk_conv_desc *d, const float *x, int64_t ldx, int64_t bsx, int64_t lim,
                    int cin, const float *wr, const float *bias, int nbias, int K, int stride,
                    int dil, int shift, int M, float *y, int64_t ldy, int64_t bsy, int64_t n,
                    int batch) {
  memset(d, 0, sizeof *d);
  d->x = x;
  d->ldx = ldx;
  d->bsx = bsx;
  d->lim = lim;
  d->cin = cin;
  d->w = wr;
  d->cinp = ptk_conv_cinp(cin);
  d->bias = bias;
  d->nbias = nbias;
  d->K = K;
  d->dil = dil;
  d->stride = stride;
  d->shift = shift;
  d->M = M;
  d->C4 = M;
  d->q0 = 0;
  d->nq = n;
  d->y = y;
  d->ldy = ldy;
  d->bsy = bsy;
  d->ys = 1;
  d->ypad = 0;
  d->Lout = n;
  d->batch = batch;
}

/* convT phase form (pt_v21_cuda.cu:2413-2416 range): phase rows m = r*C4 + co, tap j reads
 * x[q - j] (dil -1), output q lands at q*s + r - pad; q spans every index some phase can hit */
int64_t ptdi_convT_desc(ptk_conv_desc *d, const float *x, int64_t ldx, int64_t bsx, int64_t tin,
                        int cin, const float *wr, const float *bias, int cout, int s, int pad,
                        int K, float *y, int64_t ldy, int64_t bsy, int batch) {
  const int c4 = (cout + 3) / 4 * 4, ntap = (K + s - 1) / s;
  const int64_t Lout = (tin - 1) * s - 2 * (int64_t) pad + K;
  int64_t qlo = 0;
  if (pad - (s - 1) > 0) qlo = (pad - (s - 1) + s - 1) / s;
  const int64_t qhi = (Lout - 1 + pad) / s;
  ptdi_conv_desc(d, x, ldx, bsx, tin, cin, wr, bias, cout, ntap, 1, -1, 0, s * c4, y, ldy, bsy,
                 qhi - qlo + 1, batch);
  d->C4 = c4;
  d->q0 = qlo;
  d->ys = s;
  d->ypad = pad;
  d->Lout = Lout;
  return Lout;
}

/* reference epilogue codes 1..4 map onto the same kernel codes; anything else is a no-op, as in
 * pt_epi_cpu (pt_v21_host.c:2287-2297) */
static void add_ref_epi(ptk_conv_desc *d, int op, float a) {
  if (op < 1 || op > 4) return;
  d->epi[d->nepi].op = op;
  d->epi[d->nepi].a = a;
  d->nepi++;
}

/* ================================================================== pt_v21_conv */
static int fail_oom(const char *what) {
  PT_LOG("%s: host allocation failed", what);
  return -1;
}

static int fail_cpu(const char *what) {
  PT_LOG("%s on a context without the device and no host CPU path linked", what);
  return -1;
}

/* A conv of a device context routed to the host's CPU path (PT_V21_GPU without "conv").  The CPU
 * conv reads padded rows from host memory: rows the caller handed over unpadded (conv_pad_in >= 0)
 * or left on the device (conv_in_dev) are first brought into a zero-padded host copy.  A result the
 * caller asked to keep on the device (conv_keep) also goes up into the arena, as conv_out_dev. */
static int conv_on_host(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy,
                        int64_t n, int cout, int K, int stride, int pad, int dil, const float *wp,
                        const float *bias, int64_t batch, int wtab, int btab, int epi0, int epi1,
                        float a0, float a1) {
  if (!pt_v21_conv_cpu) return fail_cpu("pt_v21_conv");
  c->conv_out_dev = NULL;
  if (n <= 0 || batch <= 0) return 0;
  const int unpadded = c->conv_pad_in >= 0 || c->conv_in_dev != NULL;
  void *mark = ptdi_arena_mark(c);
  float *xp = NULL, *rows = NULL;
  int64_t ldxp = ldx;
  int rc = -1;
  if (unpadded) {
    const int64_t T = ldx, pd = c->conv_pad_in >= 0 ? c->conv_pad_in : pad;
    const size_t nrow = (size_t) batch * (size_t) cin;
    ldxp = T + 2 * pd;
    xp = calloc(nrow * (size_t) ldxp, sizeof(float));
    if (!xp) return fail_oom("pt_v21_conv");
    const float *src = X;
    if (c->conv_in_dev) {
      rows = malloc(nrow * (size_t) T * sizeof(float));
      if (!rows || ptk_d2h_async(rows, c->conv_in_dev, nrow * (size_t) T * sizeof(float), c->g_stream) ||
          ptk_stream_sync(c->g_stream)) {
        PT_LOG("pt_v21_conv: reading the chained input: %s", rows ? ptk_last_error() : "no memory");
        goto done;
      }
      src = rows;
    }
    for (size_t r = 0; r < nrow; r++) memcpy(xp + r * ldxp + pd, src + r * T, (size_t) T * sizeof(float));
  }
  rc = pt_v21_conv_cpu(c, xp ? xp : X, ldxp, cin, Y, ldy, n, cout, K, stride, pad, dil, wp, bias,
                       batch, wtab, btab, epi0, epi1, a0, a1);
  if (rc == 0 && c->conv_keep) {
    /* a chain link, as on the device path: the arena is held from the chain's first link */
    const size_t yb = (size_t) batch * (size_t) ((cout + 3) / 4 * 4) * (size_t) ldy * sizeof(float);
    float *dy = ptdi_arena_alloc(c, yb);
    if (!dy || ptk_h2d_async(dy, Y, yb, c->g_stream) || ptk_stream_sync(c->g_stream)) {
      PT_LOG("pt_v21_conv: keeping the host result on the device failed");
      rc = -1;
    } else {
      if (!c->chain_mark) c->chain_mark = mark;
      c->conv_out_dev = dy;
      free(xp);
      free(rows);
      return 0;
    }
  }
done:
  /* the chain (if any) ends here */
  ptdi_arena_release(c, c->chain_mark ? c->chain_mark : mark);
  c->chain_mark = NULL;
  free(xp);
  free(rows);
  return rc;
}

int pt_v21_conv(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy,
                int64_t n, int cout, int K, int stride, int pad, int dil, const float *wp,
                const float *bias, int64_t batch, int wtab, int btab, int epi0, int epi1, float a0,
                float a1) {
  if (!c) return -1;
  if (!c->use_cuda) {
    if (!pt_v21_conv_cpu) return fail_cpu("pt_v21_conv");
    return pt_v21_conv_cpu(c, X, ldx, cin, Y, ldy, n, cout, K, stride, pad, dil, wp, bias, batch,
                           wtab, btab, epi0, epi1, a0, a1);
  }
  if (!gpu_op(&g_gpu_conv))
    return conv_on_host(c, X, ldx, cin, Y, ldy, n, cout, K, stride, pad, dil, wp, bias, batch,
                        wtab, btab, epi0, epi1, a0, a1);
  (void) pad;   /* the kernels read the padding from c->conv_pad_in, as the reference GEMM path */
  c->n_conv++;
  c->g_calls++;
  c->conv_out_dev = NULL;
  if (n <= 0 || batch <= 0) return 0;
  if (cin < 1 || cout < 1 || K < 1 || stride < 1 || dil < 1 || ldx < 1 || ldy < n || !Y || !wp ||
      (!X && !c->conv_in_dev) || cin > INT32_MAX || batch > 65535) {
    PT_LOG("pt_v21_conv: bad arguments (cin %lld cout %d K %d stride %d dil %d ldx %lld ldy %lld "
           "n %lld batch %lld)", (long long) cin, cout, K, stride, dil, (long long) ldx,
           (long long) ldy, (long long) n, (long long) batch);
    return -1;
  }
  const int c4 = (cout + 3) / 4 * 4;
  const int shift = c->conv_pad_in >= 0 ? (int) c->conv_pad_in : 0;
  const size_t xb = (size_t) batch * cin * ldx * sizeof(float);
  const size_t yb = (size_t) batch * c4 * n * sizeof(float);
  const size_t wb = (size_t) c4 * K * cin * sizeof(float);
  void *mark = ptdi_arena_mark(c);
  const int keep = c->conv_keep;
  void *owned[5] = {NULL, NULL, NULL, NULL, NULL};
  int nown = 0;
  phase_t ph;
  phase_begin(&ph);
#define OWN_ALLOC(ptr, bytes)                                          \
  do {                                                                 \
    if (!(ptr)) {                                                      \
      if (ptk_malloc((void **) &(ptr), (bytes))) goto fail;            \
      owned[nown++] = (void *) (ptr);                                  \
      c->dev_bytes_stray += (double) (bytes);                          \
    }                                                                  \
  } while (0)
  const float *dx = c->conv_in_dev;
  float *dxa = NULL, *dy = NULL, *dw = NULL, *db = NULL, *dwr = NULL;
  if (!dx) {
    dxa = ptdi_arena_alloc(c, xb);
    OWN_ALLOC(dxa, xb);
    phase_end(&ph, &c->g_alloc_ms);
    if (ptk_h2d_async(dxa, X, xb, c->g_stream)) goto fail;
    phase_end(&ph, &c->g_copy_ms);
    dx = dxa;
  }
  dy = (keep && c->conv_keep_res) ? pt_v21_dev_alloc(c, yb) : ptdi_arena_alloc(c, yb);
  OWN_ALLOC(dy, yb);
  phase_end(&ph, &c->g_alloc_ms);
  const float *rw = ptdi_pool_get(wtab, wb);
  const float *rb = bias ? ptdi_pool_get(btab, (size_t) cout * sizeof(float)) : NULL;
  if (bias && !rb) {
    db = ptdi_arena_alloc(c, (size_t) cout * sizeof(float));
    OWN_ALLOC(db, (size_t) cout * sizeof(float));
    phase_end(&ph, &c->g_alloc_ms);
    if (ptk_h2d_async(db, bias, (size_t) cout * sizeof(float), c->g_stream)) goto fail;
    phase_end(&ph, &c->g_copy_ms);
    rb = db;
  }
  ptk_conv_desc d;
  ptdi_conv_desc(&d, dx, ldx, (int64_t) cin * ldx, ldx, (int) cin, NULL, rb, cout, K, stride, dil,
                 shift, c4, dy, n, (int64_t) c4 * n, n, (int) batch);
  add_ref_epi(&d, epi0, a0);
  add_ref_epi(&d, epi1, a1);
  const int mfma = ptk_conv_mfma_ok(&d);
  if (!rw || mfma) {
    if (!rw) {
      dw = ptdi_arena_alloc(c, wb);
      OWN_ALLOC(dw, wb);
      phase_end(&ph, &c->g_alloc_ms);
      if (ptk_h2d_async(dw, wp, wb, c->g_stream)) goto fail;
      phase_end(&ph, &c->g_copy_ms);
      rw = dw;
    }
  }
  if (mfma) {
    const float *wr = ptdi_pool_get(wtab, wb) ? ptdi_pool_relaid(c, wtab, c4, K, (int) cin) : NULL;
    if (!wr) {
      const size_t rb_bytes = ptk_relayout_floats(c4, K, (int) cin) * sizeof(float);
      dwr = ptdi_arena_alloc(c, rb_bytes);
      OWN_ALLOC(dwr, rb_bytes);
      phase_end(&ph, &c->g_alloc_ms);
      if (ptk_relayout(dwr, rw, c4, K, (int) cin, c->g_stream)) goto fail;
      wr = dwr;
    }
    d.w = wr;
    if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  } else {
    if (ptk_conv_simt(dx, ldx, (int64_t) cin * ldx, ldx, (int) cin, rw, rb, cout, K, stride, dil,
                      shift, dy, n, (int64_t) c4 * n, n, (int) batch, epi0 >= 1 && epi0 <= 4 ? epi0 : 0,
                      a0, epi1 >= 1 && epi1 <= 4 ? epi1 : 0, a1, c->g_stream))
      goto fail;
  }
  if (keep && nown == 0) {
    /* chain link: the next conv reads dy from the arena; released when the chain ends */
    if (!c->chain_mark) c->chain_mark = mark;
    c->conv_out_dev = dy;
    phase_end(&ph, &c->g_kernel_ms);
    return 0;
  }
  if (ptdi_wait_before_copy(c)) goto fail;
  if (ldy == n) {
    if (ptk_d2h_async(Y, dy, yb, c->g_stream)) goto fail;
  } else if (ptk_d2h_2d_async(Y, (size_t) ldy * sizeof(float), dy, (size_t) n * sizeof(float),
                              (size_t) n * sizeof(float), (size_t) batch * c4, c->g_stream)) {
    goto fail;
  }
  if (ptk_stream_sync(c->g_stream)) goto fail;
  pt_v21_dev_reclaim(c);
  phase_end(&ph, &c->g_kernel_ms);
  for (int i = 0; i < nown; i++) ptk_free(owned[i]);
  phase_end(&ph, &c->g_free_ms);
  if (c->chain_mark) {
    ptdi_arena_release(c, c->chain_mark);
    c->chain_mark = NULL;
  } else {
    ptdi_arena_release(c, mark);
  }
  return 0;
fail:
  PT_LOG("pt_v21_conv failed: %s", ptk_last_error());
  ptk_stream_sync(c->g_stream);
  for (int i = 0; i < nown; i++) ptk_free(owned[i]);
  ptdi_arena_release(c, c->chain_mark ? c->chain_mark : mark);
  c->chain_mark = NULL;
  return -1;
#undef OWN_ALLOC
}

/* ================================================================== pt_v21_convT */
int pt_v21_convT(pt_ctx *c, const float *X, int64_t ldx, int64_t cin, int64_t tin, float *Y,
                 int64_t ldy, int cout, int s, int pad, int K, const float *wp, const float *bias,
                 int64_t batch, int wtab, int btab) {
  if (!c) return -1;
  if (!c->use_cuda || !gpu_op(&g_gpu_convT)) {
    if (!pt_v21_convT_cpu) return fail_cpu("pt_v21_convT");
    return pt_v21_convT_cpu(c, X, ldx, cin, tin, Y, ldy, cout, s, pad, K, wp, bias, batch, wtab, btab);
  }
  c->n_convT++;
  c->g_calls++;
  const int c4 = (cout + 3) / 4 * 4, ntap = (K + s - 1) / (s > 0 ? s : 1);
  const int64_t Lout = (tin - 1) * s - 2 * (int64_t) pad + K;
  if (Lout <= 0 || batch <= 0 || tin <= 0) return 0;
  if (cin < 1 || cout < 1 || K < 1 || s < 1 || pad < 0 || ldx < tin || ldy < Lout || !X || !Y ||
      !wp || batch > 65535) {
    PT_LOG("pt_v21_convT: bad arguments (cin %lld cout %d K %d s %d pad %d tin %lld ldx %lld "
           "ldy %lld batch %lld)", (long long) cin, cout, K, s, pad, (long long) tin,
           (long long) ldx, (long long) ldy, (long long) batch);
    return -1;
  }
  const size_t xb = (size_t) batch * cin * ldx * sizeof(float);
  const size_t yb = (size_t) batch * c4 * Lout * sizeof(float);
  const size_t wb = (size_t) s * c4 * ntap * cin * sizeof(float);
  void *mark = ptdi_arena_mark(c);
  void *owned[5] = {NULL, NULL, NULL, NULL, NULL};
  int nown = 0;
  phase_t ph;
  phase_begin(&ph);
#define OWN_ALLOC(ptr, bytes)                                          \
  do {                                                                 \
    if (!(ptr)) {                                                      \
      if (ptk_malloc((void **) &(ptr), (bytes))) goto fail;            \
      owned[nown++] = (void *) (ptr);                                  \
      c->dev_bytes_stray += (double) (bytes);                          \
    }                                                                  \
  } while (0)
  float *dx = ptdi_arena_alloc(c, xb), *dy = NULL, *dw = NULL, *db = NULL, *dwr = NULL;
  OWN_ALLOC(dx, xb);
  phase_end(&ph, &c->g_alloc_ms);
  if (ptk_h2d_async(dx, X, xb, c->g_stream)) goto fail;
  phase_end(&ph, &c->g_copy_ms);
  dy = ptdi_arena_alloc(c, yb);
  OWN_ALLOC(dy, yb);
  phase_end(&ph, &c->g_alloc_ms);
  const float *rw = ptdi_pool_get(wtab, wb);
  const float *rb = bias ? ptdi_pool_get(btab, (size_t) cout * sizeof(float)) : NULL;
  if (bias && !rb) {
    db = ptdi_arena_alloc(c, (size_t) cout * sizeof(float));
    OWN_ALLOC(db, (size_t) cout * sizeof(float));
    phase_end(&ph, &c->g_alloc_ms);
    if (ptk_h2d_async(db, bias, (size_t) cout * sizeof(float), c->g_stream)) goto fail;
    phase_end(&ph, &c->g_copy_ms);
    rb = db;
  }
  const int resident = rw != NULL;
  if (!rw) {
    dw = ptdi_arena_alloc(c, wb);
    OWN_ALLOC(dw, wb);
    phase_end(&ph, &c->g_alloc_ms);
    if (ptk_h2d_async(dw, wp, wb, c->g_stream)) goto fail;
    phase_end(&ph, &c->g_copy_ms);
    rw = dw;
  }
  ptk_conv_desc d;
  ptdi_convT_desc(&d, dx, ldx, (int64_t) cin * ldx, tin, (int) cin, NULL, rb, cout, s, pad, K, dy,
                  Lout, (int64_t) c4 * Lout, (int) batch);
  if (ptk_conv_mfma_ok(&d) && d.M >= 32) {
    const float *wr = resident ? ptdi_pool_relaid(c, wtab, s * c4, ntap, (int) cin) : NULL;
    if (!wr) {
      const size_t rbytes = ptk_relayout_floats(s * c4, ntap, (int) cin) * sizeof(float);
      dwr = ptdi_arena_alloc(c, rbytes);
      OWN_ALLOC(dwr, rbytes);
      phase_end(&ph, &c->g_alloc_ms);
      if (ptk_relayout(dwr, rw, s * c4, ntap, (int) cin, c->g_stream)) goto fail;
      wr = dwr;
    }
    d.w = wr;
    if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  } else if (ptk_convT_simt(dx, ldx, (int64_t) cin * ldx, tin, (int) cin, rw, rb, cout, s, pad, K,
                            dy, Lout, (int64_t) c4 * Lout, Lout, (int) batch, c->g_stream)) {
    goto fail;
  }
  if (ptdi_wait_before_copy(c)) goto fail;
  if (ldy == Lout) {
    if (ptk_d2h_async(Y, dy, yb, c->g_stream)) goto fail;
  } else if (ptk_d2h_2d_async(Y, (size_t) ldy * sizeof(float), dy, (size_t) Lout * sizeof(float),
                              (size_t) Lout * sizeof(float), (size_t) batch * c4, c->g_stream)) {
    goto fail;
  }
  if (ptk_stream_sync(c->g_stream)) goto fail;
  phase_end(&ph, &c->g_kernel_ms);
  for (int i = 0; i < nown; i++) ptk_free(owned[i]);
  ptdi_arena_release(c, mark);
  phase_end(&ph, &c->g_free_ms);
  return 0;
fail:
  PT_LOG("pt_v21_convT failed: %s", ptk_last_error());
  ptk_stream_sync(c->g_stream);
  for (int i = 0; i < nown; i++) ptk_free(owned[i]);
  ptdi_arena_release(c, mark);
  return -1;
#undef OWN_ALLOC
}

/* ================================================================== pt_v21_matmul */
int pt_v21_matmul(pt_ctx *c, const float *A, int64_t m, int64_t k, int64_t lda, const float *B,
                  int64_t ldb, int64_t nn, float *C, int64_t ldc) {
  if (!c) return -1;
  if (!c->use_cuda || !gpu_op(&g_gpu_matmul)) {
    if (!pt_v21_matmul_cpu) return fail_cpu("pt_v21_matmul");
    return pt_v21_matmul_cpu(c, A, m, k, lda, B, ldb, nn, C, ldc);
  }
  c->n_matmul++;
  if (m <= 0 || nn <= 0) return 0;
  if (k < 0 || lda < k || ldb < nn || ldc < nn || !A || !B || !C) {
    PT_LOG("pt_v21_matmul: bad arguments");
    return -1;
  }
  /* Tight device copies.  Only the k (A) and n (B, C) columns of each row are moved, so no byte
   * outside the matrices is read, and C's padding columns (ldc > n) are left as they are, as the
   * reference's CPU matmul leaves them (pt_v21_host.c:2635-2650).  Each matrix goes in one
   * contiguous copy; padded rows are packed / scattered on the host (a pageable 2-D copy moves
   * row by row, tens of microseconds per row). */
  const size_t f = sizeof(float);
  const size_t ab = (size_t) m * (k > 0 ? k : 1) * f, bb = (size_t) (k > 0 ? k : 1) * nn * f;
  const size_t cb = (size_t) m * nn * f;
  float *hA = NULL, *hB = NULL, *hC = NULL;   /* host staging for padded rows */
  if (k > 0 && lda != k && !(hA = malloc(ab))) return fail_oom("pt_v21_matmul");
  if (k > 0 && ldb != nn && !(hB = malloc(bb))) { free(hA); return fail_oom("pt_v21_matmul"); }
  if (ldc != nn && !(hC = malloc(cb))) { free(hA); free(hB); return fail_oom("pt_v21_matmul"); }
  for (int64_t i = 0; hA && i < m; i++) memcpy(hA + i * k, A + i * lda, (size_t) k * f);
  for (int64_t i = 0; hB && i < k; i++) memcpy(hB + i * nn, B + i * ldb, (size_t) nn * f);
  phase_t ph;
  phase_begin(&ph);
  void *mark = ptdi_arena_mark(c);
  float *dA = ptdi_arena_alloc(c, ab), *dB = ptdi_arena_alloc(c, bb), *dC = ptdi_arena_alloc(c, cb);
  int own = 0;
  if (!dA || !dB || !dC) {
    ptdi_arena_release(c, mark);
    dA = dB = dC = NULL;
    if (ptk_malloc((void **) &dA, ab) || ptk_malloc((void **) &dB, bb) || ptk_malloc((void **) &dC, cb)) {
      ptk_free(dA); ptk_free(dB); ptk_free(dC);
      free(hA); free(hB); free(hC);
      PT_LOG("pt_v21_matmul: allocation failed: %s", ptk_last_error());
      return -1;
    }
    own = 1;
  }
  phase_end(&ph, &c->g_alloc_ms);
  int r = k > 0 && (ptk_h2d_async(dA, hA ? hA : A, (size_t) m * k * f, c->g_stream) ||
                    ptk_h2d_async(dB, hB ? hB : B, (size_t) k * nn * f, c->g_stream));
  phase_end(&ph, &c->g_copy_ms);
  r = r || ptk_matmul(dA, m, k, k, dB, nn, nn, dC, nn, c->g_stream) || ptdi_wait_before_copy(c) ||
      ptk_d2h_async(hC ? hC : C, dC, cb, c->g_stream) || ptk_stream_sync(c->g_stream);
  if (!r && hC)
    for (int64_t i = 0; i < m; i++) memcpy(C + i * ldc, hC + i * nn, (size_t) nn * f);
  phase_end(&ph, &c->g_kernel_ms);
  if (r) PT_LOG("pt_v21_matmul failed: %s", ptk_last_error());
  if (own) {
    ptk_free(dA); ptk_free(dB); ptk_free(dC);
  } else {
    ptdi_arena_release(c, mark);
  }
  free(hA); free(hB); free(hC);
  phase_end(&ph, &c->g_free_ms);
  return r ? -1 : 0;
}

/* ================================================================== device residency
 * A per-context slab (PT_V21_DEVRES_MB, default 64) with a real allocator, for tensors that
 * outlive one conv chain (the reference's pt_v21_cuda.cu:237-454 contract): best-fit over free
 * blocks, neighbours merged on free, operand uploads queued and released at the chain end. */
#define DEVRES_MAXB 256
typedef struct {
  char *base;
  size_t size, top;
  int nblk;
  struct {
    size_t off, size;
    int used;
  } blk[DEVRES_MAXB];   /* sorted by offset, covering [0, top) */
  int npend;
  size_t pend[64];
} devres_t;

static void devres_destroy(pt_ctx *c) {
  devres_t *d = (devres_t *) c->devres;
  if (!d) return;
  ptk_free(d->base);
  free(d);
  c->devres = NULL;
}

void *pt_v21_dev_alloc(pt_ctx *c, size_t bytes) {
  if (!c || !c->use_cuda) return NULL;
  devres_t *d = (devres_t *) c->devres;
  if (!d) {
    d = calloc(1, sizeof *d);
    if (!d) return NULL;
    d->size = (size_t) env_int("PT_V21_DEVRES_MB", 64) << 20;
    if (ptk_malloc((void **) &d->base, d->size)) {
      free(d);
      c->devres_oom = 1;
      return NULL;
    }
    c->devres = d;
    c->dev_bytes_res = (double) d->size;
  }
  const size_t nb = (bytes + 255) & ~(size_t) 255;
  int best = -1;
  for (int i = 0; i < d->nblk; i++)
    if (!d->blk[i].used && d->blk[i].size >= nb && (best < 0 || d->blk[i].size < d->blk[best].size))
      best = i;
  if (best >= 0) {
    if (d->blk[best].size - nb >= 256 && d->nblk < DEVRES_MAXB) {   /* split, keep the tail free */
      memmove(&d->blk[best + 2], &d->blk[best + 1], (size_t) (d->nblk - best - 1) * sizeof d->blk[0]);
      d->blk[best + 1].off = d->blk[best].off + nb;
      d->blk[best + 1].size = d->blk[best].size - nb;
      d->blk[best + 1].used = 0;
      d->blk[best].size = nb;
      d->nblk++;
    }
    d->blk[best].used = 1;
    return d->base + d->blk[best].off;
  }
  if (d->top + nb > d->size || d->nblk >= DEVRES_MAXB) {
    c->devres_oom = 1;
    return NULL;
  }
  d->blk[d->nblk].off = d->top;
  d->blk[d->nblk].size = nb;
  d->blk[d->nblk].used = 1;
  d->nblk++;
  d->top += nb;
  return d->base + d->top - nb;
}

void pt_v21_dev_free(pt_ctx *c, void *p) {
  devres_t *d = c ? (devres_t *) c->devres : NULL;
  if (!d || !p || (char *) p < d->base || (char *) p >= d->base + d->size) return;   /* not ours */
  const size_t off = (size_t) ((char *) p - d->base);
  int i = 0;
  while (i < d->nblk && d->blk[i].off != off) i++;
  if (i == d->nblk || !d->blk[i].used) return;
  d->blk[i].used = 0;
  for (int k = 0; k < d->npend; k++)
    if (d->pend[k] == off) d->pend[k] = d->pend[--d->npend];
  if (i + 1 < d->nblk && !d->blk[i + 1].used) {   /* merge with the right neighbour */
    d->blk[i].size += d->blk[i + 1].size;
    memmove(&d->blk[i + 1], &d->blk[i + 2], (size_t) (d->nblk - i - 2) * sizeof d->blk[0]);
    d->nblk--;
  }
  if (i > 0 && !d->blk[i - 1].used) {   /* and with the left one */
    d->blk[i - 1].size += d->blk[i].size;
    memmove(&d->blk[i], &d->blk[i + 1], (size_t) (d->nblk - i - 1) * sizeof d->blk[0]);
    d->nblk--;
    i--;
  }
  if (i == d->nblk - 1 && !d->blk[i].used) {   /* a free block at the top returns to the top */
    d->top = d->blk[i].off;
    d->nblk--;
  }
  c->devres_oom = 0;
}

void pt_v21_dev_reclaim(pt_ctx *c) {
  devres_t *d = c ? (devres_t *) c->devres : NULL;
  if (!d) return;
  while (d->npend > 0) {
    const size_t off = d->pend[d->npend - 1];
    d->npend--;
    pt_v21_dev_free(c, d->base + off);
  }
}

float *pt_v21_dev_upload(pt_ctx *c, const void *h, int64_t n) {
  if (!c || !c->use_cuda || n <= 0) return NULL;
  float *p = pt_v21_dev_alloc(c, (size_t) n * sizeof(float));
  if (!p) return NULL;
  if (ptk_h2d_async(p, h, (size_t) n * sizeof(float), c->g_stream)) {
    pt_v21_dev_free(c, p);
    return NULL;
  }
  devres_t *d = (devres_t *) c->devres;
  if (d->npend < 64) d->pend[d->npend++] = (size_t) ((char *) p - d->base);
  return p;
}

void pt_v21_dev_sync_host(pt_ctx *c, void *host, const void *dev, int64_t n) {
  if (!c || n <= 0) return;
  if (ptdi_wait_before_copy(c) || ptk_d2h_async(host, dev, (size_t) n * sizeof(float), c->g_stream) ||
      ptk_stream_sync(c->g_stream))
    PT_LOG("pt_v21_dev_sync_host failed: %s", ptk_last_error());
}

int pt_v21_devadd_run(pt_ctx *c, const float *a, const float *b, float *y, int64_t n, int epi,
                      float alpha) {
  if (!c || !c->use_cuda) return -1;
  return ptk_add(a, b, y, n, epi == 1 ? 1 : 0, alpha, c->g_stream) ? -1 : 0;
}

int pt_v21_devleaky_run(pt_ctx *c, const float *a, float *y, int64_t n, float alpha) {
  if (!c || !c->use_cuda) return -1;
  return ptk_leaky(a, y, n, alpha, c->g_stream) ? -1 : 0;
}

/* ================================================================== plumbing */
void *ptd_malloc(size_t bytes) {
  void *p = NULL;
  if (ptk_init() || ptk_malloc(&p, bytes)) {
    PT_LOG("ptd_malloc(%zu): %s", bytes, ptk_last_error());
    return NULL;
  }
  return p;
}
void ptd_free(void *p) { ptk_free(p); }
void ptd_debug_fail_allocs(int skip, int n) { ptk_fail_allocs(skip, n); }
void ptd_debug_reload_env(void) {
  ptk_knobs_reload();
  ptdi_decoder_knobs_reload();
}
int ptd_debug_fill_arena(pt_ctx *c, int byte) {
  if (!c || !c->use_cuda || !c->g_arena) return -1;
  if (ptk_fill_async(c->g_arena, byte, c->g_arena_bytes, c->g_stream) || ptk_stream_sync(c->g_stream)) {
    PT_LOG("arena fill failed: %s", ptk_last_error());
    return -1;
  }
  return 0;
}
int ptd_h2d(pt_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !c->use_cuda) return -1;
  return (ptk_h2d_async(dst, src, bytes, c->g_stream) || ptk_stream_sync(c->g_stream)) ? -1 : 0;
}
int ptd_d2h(pt_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !c->use_cuda) return -1;
  return (ptk_d2h_async(dst, src, bytes, c->g_stream) || ptk_stream_sync(c->g_stream)) ? -1 : 0;
}
int ptd_sync(pt_ctx *c) {
  if (!c || !c->use_cuda) return -1;
  if (ptk_stream_sync(c->g_stream)) {
    PT_LOG("stream sync failed: %s", ptk_last_error());
    return -1;
  }
  return 0;
}
int ptd_device_sync(void) {
  if (ptk_device_sync()) {
    PT_LOG("device sync failed: %s", ptk_last_error());
    return -1;
  }
  return 0;
}
void *ptd_event_create(void) {
  void *e = NULL;
  return ptk_event_create(&e) ? NULL : e;
}
void ptd_event_destroy(void *e) {
  if (e) ptk_event_destroy(e);
}
int ptd_event_record(pt_ctx *c, void *e) {
  if (!c || !c->use_cuda || !e) return -1;
  return ptk_event_record(e, c->g_stream) ? -1 : 0;
}
float ptd_event_elapsed_ms(void *e0, void *e1) {
  float ms = -1.0f;
  if (ptk_event_sync(e1) || ptk_event_elapsed_ms(&ms, e0, e1)) return -1.0f;
  return ms;
}

/* ================================================================== test hooks */
int ptd_mfma_probe(pt_ctx *c, const float *a, const float *b, float *d) {
  if (!c || !c->use_cuda) return -1;
  void *mark = ptdi_arena_mark(c);
  float *da = ptdi_arena_alloc(c, 64 * sizeof(float)), *dbb = ptdi_arena_alloc(c, 64 * sizeof(float));
  float *dd = ptdi_arena_alloc(c, 1024 * sizeof(float));
  int r = !da || !dbb || !dd || ptk_h2d_async(da, a, 64 * sizeof(float), c->g_stream) ||
          ptk_h2d_async(dbb, b, 64 * sizeof(float), c->g_stream) ||
          ptk_mfma_probe(da, dbb, dd, c->g_stream) ||
          ptk_d2h_async(d, dd, 1024 * sizeof(float), c->g_stream) || ptk_stream_sync(c->g_stream);
  ptdi_arena_release(c, mark);
  return r ? -1 : 0;
}

int ptd_mfma16_probe(pt_ctx *c, const float *a, const float *b, float *d) {
  if (!c || !c->use_cuda) return -1;
  void *mark = ptdi_arena_mark(c);
  float *da = ptdi_arena_alloc(c, 64 * sizeof(float)), *dbb = ptdi_arena_alloc(c, 64 * sizeof(float));
  float *dd = ptdi_arena_alloc(c, 256 * sizeof(float));
  int r = !da || !dbb || !dd || ptk_h2d_async(da, a, 64 * sizeof(float), c->g_stream) ||
          ptk_h2d_async(dbb, b, 64 * sizeof(float), c->g_stream) ||
          ptk_mfma16_probe(da, dbb, dd, c->g_stream) ||
          ptk_d2h_async(d, dd, 256 * sizeof(float), c->g_stream) || ptk_stream_sync(c->g_stream);
  ptdi_arena_release(c, mark);
  return r ? -1 : 0;
}

int ptd_ctx_layout(long *out, int n) {
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
