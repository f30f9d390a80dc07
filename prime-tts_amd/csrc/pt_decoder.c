/* pt_decoder.c -- the synthetic MB-iSTFT decoder kept on the device, per request (C, gnu11).
 *
 * Graph (ref/v21_graph_trace.txt:3819-4065), with every host op of the reference fused:
 *   conv_pre 192->512 K7 + LeakyReLU(0.1)          one conv, epilogue leaky
 *   ups.0 convT 512->256 K16 s4 p6                  one phase-form GEMM (4 phases = 1024 rows)
 *   MRF-256: per depth j, one grouped launch of the three branches' c1 (input already
 *            LeakyReLU'd by its producer, epilogue leaky), then one of their c2 (epilogue adds the
 *            residual and, for depths 0 and 1, also writes the LeakyReLU'd copy the next depth's
 *            c1 reads)  -> 6 launches, three branch outputs left in HBM.  ups.0 / ups.1 write
 *            their output and its LeakyReLU'd copy the same way.
 *   ups.1 convT 256->128 over leaky(((b0 + b1) + b2) / 3, 0.1), formed once by one elementwise
 *            pass (cheaper than re-forming it in each of ups.1's 16 row blocks' staging)
 *   MRF-128 as above
 *   conv_post 128->72 K7 over leaky((...)/3, 0.01), formed the same way, through the (1, 0)
 *            reflection pad
 *   tail: one kernel for exp/sin/cos -> irfft basis -> Hann -> OLA / window-sum -> [8:-8] ->
 *         PQMF x4 zero-insert -> 63-tap FIR
 * 19 launches per request, no host round trip.  The weights are uploaded once into one slab
 * owned by the model and shared by every context; each context brings its own stream + arena. */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "pt_dev_internal.h"
#include "ptd.h"

static const int kMrfK[3] = {3, 7, 11};
static const int kMrfD[3] = {1, 3, 5};

typedef struct {
  int cin, cout, K, sd, pad, convT;
} layer_geo;

/* geometry of decoder layer i (spec/v21_layers.json, trace :3819-3935) */
static layer_geo dec_geo(int i) {
  layer_geo g = {0, 0, 0, 1, 0, 0};
  if (i == 0) {
    g.cin = 192; g.cout = 512; g.K = 7; g.pad = 3;
  } else if (i == 1 || i == 20) {
    g.cin = i == 1 ? 512 : 256; g.cout = i == 1 ? 256 : 128; g.K = 16; g.sd = 4; g.pad = 6; g.convT = 1;
  } else if (i == 39) {
    g.cin = 128; g.cout = 72; g.K = 7; g.pad = 3;
  } else if (i == 40) {   /* /dec/Conv after /dec/Pad 31|31: 4 -> 1, K 63 */
    g.cin = 4; g.cout = 1; g.K = 63; g.pad = 0;
  } else {
    const int base = i < 20 ? 2 : 21, C = i < 20 ? 256 : 128, o = i - base;
    const int br = o / 6, j = (o % 6) / 2, c = o % 2;
    g.cin = C; g.cout = C; g.K = kMrfK[br];
    g.sd = c == 0 ? kMrfD[j] : 1;
    g.pad = g.sd * (g.K - 1) / 2;
  }
  return g;
}

struct ptd_model {
  void *slab;                      /* relaid weights, biases, tail constants */
  const float *wr[PTD_DEC_NLAYER]; /* MFMA layout [Mp/32][K][cinp/8][64][4] */
  const float *wr16[PTD_DEC_NLAYER]; /* for 16-row tiles [Mp/16][K][cinp/8][64][2] */
  const float *b[PTD_DEC_NLAYER];
  const float *consts;             /* the tail's table: hann, basis_c, basis_s, final conv */
  layer_geo g[PTD_DEC_NLAYER];
};

static size_t al256(size_t b) { return (b + 255) & ~(size_t) 255; }

/* Closed-form constants of the tail (the reference graph folds the same values into constants):
 * periodic Hann(16); irfft basis rows w_k cos(2 pi k n / 16) / 16 and -w_k sin(...) / 16 with
 * one-sided weights w = [1, 2, ..., 2, 1]. */
void ptd_tail_constants(float *out) {
  const double pi = 3.14159265358979323846;
  float *hann = out, *bc = out + 16, *bs = out + 160;
  for (int n = 0; n < 16; n++) hann[n] = (float) (0.5 - 0.5 * cos(2.0 * pi * n / 16.0));
  for (int k = 0; k < 9; k++) {
    const double w = (k == 0 || k == 8) ? 1.0 : 2.0;
    for (int n = 0; n < 16; n++) {
      bc[k * 16 + n] = (float) (w * cos(2.0 * pi * k * n / 16.0) / 16.0);
      bs[k * 16 + n] = (float) (-w * sin(2.0 * pi * k * n / 16.0) / 16.0);
    }
  }
}

/* the final conv's taps h[band*63 + m] = W[0][band][m] out of its packed weight [1][63][4][4]
 * (row 0 of the first row block), then its bias (0 without one) */
/* The final PQMF conv's taps in polyphase order: entry ((band * 4 + r) * 16 + j) is tap
 * m = 3 - r + 4j of that band (0 for m = 63), the taps output sample 4u + r of a block multiplies
 * with y slots u + 1 + j; then the bias. */
static void tail_fir(float *dst, const float *wp, const float *bias) {
  for (int band = 0; band < 4; band++)
    for (int r = 0; r < 4; r++)
      for (int j = 0; j < 16; j++) {
        const int m = 3 - r + 4 * j;
        dst[(band * 4 + r) * 16 + j] = m < 63 ? wp[((size_t) m * 4 + band) * 4 + 0] : 0.0f;
      }
  dst[256] = bias ? bias[0] : 0.0f;
}

static void layer_gemm(const layer_geo *g, int *M, int *K) {
  const int c4 = (g->cout + 3) / 4 * 4;
  *M = g->convT ? g->sd * c4 : c4;
  *K = g->convT ? (g->K + g->sd - 1) / g->sd : g->K;
}

int64_t ptdi_dec_wfloats(int i) {
  if (i < 0 || i >= PTD_DEC_NLAYER) return -1;
  const layer_geo g = dec_geo(i);
  int M, K;
  layer_gemm(&g, &M, &K);
  return (int64_t) M * K * g.cin;
}

int ptdi_dec_cout(int i) { return i < 0 || i >= PTD_DEC_NLAYER ? -1 : dec_geo(i).cout; }

ptd_model *ptdi_model_build(pt_ctx *c, const void *const *w, const int *wisz, const float *const *b) {
  if (!c || !c->use_cuda || !w || !b) return NULL;
  ptd_model *m = calloc(1, sizeof *m);
  if (!m) return NULL;
  size_t total = 0, packed_max = 0, half_max = 0;
  size_t off_w[PTD_DEC_NLAYER], off_w16[PTD_DEC_NLAYER], off_b[PTD_DEC_NLAYER];
  int64_t wn[PTD_DEC_NLAYER];
  const int last = PTD_DEC_NLAYER - 1;
  if (!w[last] || (wisz && wisz[last] != 4)) {
    PT_LOG("decoder model: layer %d (the PQMF synthesis conv) needs an fp32 weight", last);
    free(m);
    return NULL;
  }
  for (int i = 0; i < last; i++) {
    const int isz = wisz ? wisz[i] : 4;
    if (!w[i] || !b[i] || (isz != 4 && isz != 2)) {
      PT_LOG("decoder model: layer %d has no weight or bias, or an item size other than 4 / 2", i);
      free(m);
      return NULL;
    }
    layer_geo g = dec_geo(i);
    m->g[i] = g;
    int M, K;
    layer_gemm(&g, &M, &K);
    wn[i] = (int64_t) M * K * g.cin;
    if ((size_t) wn[i] * sizeof(float) > packed_max) packed_max = (size_t) wn[i] * sizeof(float);
    if (isz == 2 && (size_t) wn[i] * 2 > half_max) half_max = (size_t) wn[i] * 2;
    off_w[i] = total;
    total += al256(ptk_relayout_floats(M, K, g.cin) * sizeof(float));
    off_w16[i] = total;
    total += al256(ptk_relayout16_floats(M, K, g.cin) * sizeof(float));
    off_b[i] = total;
    total += al256((size_t) g.cout * sizeof(float));
  }
  m->g[last] = dec_geo(last);
  const size_t off_c = total;
  total += al256(PTK_TAIL_NCONST * sizeof(float));
  float consts[PTK_TAIL_NCONST];
  ptd_tail_constants(consts);
  tail_fir(consts + PTD_TAIL_NCONST, (const float *) w[last], b[last]);
  void *tmp = NULL, *tmp16 = NULL;
  if (ptk_malloc(&m->slab, total) || ptk_malloc(&tmp, packed_max) ||
      (half_max && ptk_malloc(&tmp16, half_max)))
    goto fail;
  char *base = (char *) m->slab;
  for (int i = 0; i < last; i++) {
    const layer_geo g = m->g[i];
    int M, K;
    layer_gemm(&g, &M, &K);
    /* the packed copy goes through one staging buffer (fp16 payloads through a second one and
     * the expansion kernel); the stream orders the reuse */
    const int isz = wisz ? wisz[i] : 4;
    const int up = isz == 4
        ? ptk_h2d_async(tmp, w[i], (size_t) wn[i] * 4, c->g_stream)
        : (ptk_h2d_async(tmp16, w[i], (size_t) wn[i] * 2, c->g_stream) ||
           ptk_h2f((float *) tmp, (const uint16_t *) tmp16, wn[i], c->g_stream));
    /* the convTs' rows interleaved by phase (ptk_conv_desc.phase_il): each lane then writes its
     * column's four phases as consecutive samples */
    const int il = g.convT ? M / 4 : 0;
    if (up || ptk_relayout_il((float *) (base + off_w[i]), tmp, M, K, g.cin, il, c->g_stream) ||
        ptk_relayout16_il((float *) (base + off_w16[i]), tmp, M, K, g.cin, il, c->g_stream) ||
        ptk_h2d_async(base + off_b[i], b[i], (size_t) g.cout * sizeof(float), c->g_stream) ||
        ptk_stream_sync(c->g_stream))
      goto fail;
    m->wr[i] = (const float *) (base + off_w[i]);
    m->wr16[i] = (const float *) (base + off_w16[i]);
    m->b[i] = (const float *) (base + off_b[i]);
  }
  if (ptk_h2d_async(base + off_c, consts, sizeof consts, c->g_stream) || ptk_stream_sync(c->g_stream))
    goto fail;
  m->consts = (const float *) (base + off_c);
  ptk_free(tmp);
  ptk_free(tmp16);
  return m;
fail:
  PT_LOG("decoder model creation failed: %s", ptk_last_error());
  ptk_free(tmp);
  ptk_free(tmp16);
  ptk_free(m->slab);
  free(m);
  return NULL;
}

ptd_model *ptd_model_create(pt_ctx *c, const float *const *w, const float *const *b) {
  return ptdi_model_build(c, (const void *const *) w, NULL, b);
}

void ptd_model_destroy(ptd_model *m) {
  if (!m) return;
  ptk_device_sync();
  ptk_free(m->slab);
  free(m);
}

/* ------------------------------------------------------------------ building blocks */
static void conv_layer_desc(ptk_conv_desc *d, const ptd_model *m, int i, const float *x,
                            int64_t ldx, int64_t T, int batch, float *y, int64_t ldy) {
  const layer_geo g = m->g[i];
  const int c4 = (g.cout + 3) / 4 * 4;
  ptdi_conv_desc(d, x, ldx, (int64_t) g.cin * ldx, T, g.cin, m->wr[i], m->b[i], g.cout, g.K, 1,
                 g.sd, g.pad, c4, y, ldy, (int64_t) c4 * ldy, T, batch);
  d->w16 = m->wr16[i];
}

static void epi_push(ptk_conv_desc *d, int op, float a, const float *t, int64_t ldt, int64_t bst) {
  d->epi[d->nepi].op = op;
  d->epi[d->nepi].a = a;
  d->epi[d->nepi].t = t;
  d->epi[d->nepi].ldt = ldt;
  d->epi[d->nepi].bst = bst;
  d->nepi++;
}

/* ------------------------------------------------------------------ columns a window needs
 * An overlap-save window keeps only the samples of its interior, and each kept sample depends on
 * a bounded run of columns of every layer (its dependency cone).  Columns outside the cones of
 * the kept samples feed nothing that is stored, so a windowed decode computes each layer over the
 * union of those cones only.  Every column it computes gets the same arithmetic as in the full
 * window (the tile shape is chosen for the full width, nq_shape), so the kept samples are
 * bit-identical to those of the full-window decode.  The cones follow the graph backwards from
 * the kept samples:
 *   tail: sample s reads the PQMF input slots u in [s - 31, s + 31], nonzero only at u = 4i, and
 *         y[i] = ola[i + 8] / wsum[i + 8] overlaps frames t with 4t <= i + 8 < 4t + 16;
 *   conv (stride 1, "same" padding r = dil*(K-1)/2): column t reads [t - r, t + r];
 *   conv_post reads its (1, 0) reflection-padded input: column t reads input [t - 4, t + 2];
 *   MRF depth: x' = x + c2(leaky(c1(leaky(x)))): c2 column t reads c1 output [t - r2, t + r2] and
 *         x at t; c1 column t reads x [t - r1, t + r1] (per branch; the stage input is shared);
 *   convT phase form (stride s, pad p): GEMM column q writes outputs q*s - p .. q*s - p + s - 1,
 *         so output o comes from column floor((o + p) / s), and column q reads input
 *         [q - ntap + 1, q];
 *   the branch average and LeakyReLU passes are per column.
 * Bounds move independently, so one pass over [lo, hi) gives the middle items' columns and one
 * over [lo_first, hi_last) the first item's left and the last item's right end. */
typedef struct {
  int64_t a, b;   /* columns [a, b) */
} span;

/* the columns of one launch (ptk_conv_desc q0, nq, ext_l, ext_r, nq_shape) */
typedef struct {
  int64_t q0, nq, ext_l, ext_r, nq_shape;
} cols_t;

typedef struct {
  int on;
  cols_t pre, up0, up1, post;
  cols_t mrf[2][3][3][2];   /* [stage][depth][branch][c1, c2] */
} cone_plan;

static int64_t div_floor(int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }
static int64_t div_ceil(int64_t a, int64_t b) { return -div_floor(-a, b); }
static span span_clip(span x, int64_t lo, int64_t hi) {
  if (x.a < lo) x.a = lo;
  if (x.b > hi) x.b = hi;
  return x;
}
static span span_grow(span x, int64_t r, int64_t n) {
  x.a -= r;
  x.b += r;
  return span_clip(x, 0, n);
}
static span span_union(span x, span y) {
  if (y.a < x.a) x.a = y.a;
  if (y.b > x.b) x.b = y.b;
  return x;
}

/* convT (stride s, pad p, ntap taps, tin input columns): GEMM columns that produce outputs
 * [o.a, o.b), within [qlo, qhi] of the full launch, and the input columns they read */
static span convT_cols(span o, int s, int p, int64_t qlo, int64_t qhi) {
  span q = {div_ceil(o.a + p - s + 1, s), div_floor(o.b - 1 + p, s) + 1};
  return span_clip(q, qlo, qhi + 1);
}
static span convT_in(span q, int ntap, int64_t tin) {
  span x = {q.a - ntap + 1, q.b};
  return span_clip(x, 0, tin);
}

static void cols_set(cols_t *c, span mid, span ext, int64_t full, int batch) {
  if (batch == 1) mid = ext;
  c->q0 = mid.a;
  c->nq = mid.b - mid.a;
  c->ext_l = mid.a - ext.a;
  c->ext_r = ext.b - mid.b;
  c->nq_shape = full;
}

/* MRF stage backwards: y[2] = the columns each branch's output must hold (mid / ext); fills the
 * stage's launches and returns the stage input's columns */
static void mrf_cols(cols_t (*cols)[3][2], span ymid, span yext, int64_t T, int batch, span *xmid,
                     span *xext) {
  span um = {T, 0}, ue = {T, 0};
  for (int br = 0; br < 3; br++) {
    const int r2 = (kMrfK[br] - 1) / 2;
    span ym = ymid, ye = yext;
    for (int j = 2; j >= 0; j--) {
      const int r1 = kMrfD[j] * r2;
      const span am = span_grow(ym, r2, T), ae = span_grow(ye, r2, T);
      cols_set(&cols[j][br][1], ym, ye, T, batch);
      cols_set(&cols[j][br][0], am, ae, T, batch);
      ym = span_union(span_grow(am, r1, T), ym);
      ye = span_union(span_grow(ae, r1, T), ye);
    }
    um = span_union(um, ym);
    ue = span_union(ue, ye);
  }
  *xmid = um;
  *xext = ue;
}

/* 0 with the plan filled, -1 when no column can be left out (or the window keeps nothing) */
static int cone_plan_make(cone_plan *cp, int64_t T, int batch, const ptk_emit *em) {
  memset(cp, 0, sizeof *cp);
  const int64_t T1 = 4 * T, T2 = 16 * T, L = T2 + 1, S = 256 * T;
  span sm = {em->lo, em->hi}, se = {em->lo_first, em->hi_last};
  if (batch == 1) sm = se;
  se = span_union(se, sm);
  sm = span_clip(sm, 0, S);
  se = span_clip(se, 0, S);
  if (sm.b <= sm.a) return -1;
  if (sm.a == 0 && sm.b == S) return -1;   /* every item keeps every sample: full columns */
  span pm, pe;   /* conv_post output frames */
  {
    const span *in[2] = {&sm, &se};
    span *out[2] = {&pm, &pe};
    for (int k = 0; k < 2; k++) {
      const int64_t ilo = div_ceil(in[k]->a - 31, 4), ihi = div_floor(in[k]->b - 1 + 31, 4);
      span t = {div_ceil(ilo - 7, 4), div_floor(ihi + 8, 4) + 1};
      *out[k] = span_clip(t, 0, L);
    }
  }
  cols_set(&cp->post, pm, pe, L, batch);
  /* conv_post input (the averaged MRF-128 output), through the reflection pad */
  span ym = {pm.a - 4, pm.b + 2}, ye = {pe.a - 4, pe.b + 2};
  ym = span_clip(ym, 0, T2);
  ye = span_clip(ye, 0, T2);
  span xm, xe;
  mrf_cols(cp->mrf[1], ym, ye, T2, batch, &xm, &xe);
  /* ups.1: convT 256 -> 128, K16 s4 p6 (4 taps per phase), columns q in [1, T1 + 1] */
  span qm = convT_cols(xm, 4, 6, 1, T1 + 1), qe = convT_cols(xe, 4, 6, 1, T1 + 1);
  cols_set(&cp->up1, qm, qe, T1 + 1, batch);
  ym = convT_in(qm, 4, T1);
  ye = convT_in(qe, 4, T1);
  mrf_cols(cp->mrf[0], ym, ye, T1, batch, &xm, &xe);
  qm = convT_cols(xm, 4, 6, 1, T + 1);
  qe = convT_cols(xe, 4, 6, 1, T + 1);
  cols_set(&cp->up0, qm, qe, T + 1, batch);
  ym = convT_in(qm, 4, T);
  ye = convT_in(qe, 4, T);
  cols_set(&cp->pre, ym, ye, T, batch);
  /* a launch that would compute nothing for some item is left whole */
  const cols_t *all[4] = {&cp->pre, &cp->up0, &cp->up1, &cp->post};
  for (int k = 0; k < 4; k++)
    if (all[k]->nq <= 0) return -1;
  for (int st = 0; st < 2; st++)
    for (int j = 0; j < 3; j++)
      for (int br = 0; br < 3; br++)
        for (int k = 0; k < 2; k++)
          if (cp->mrf[st][j][br][k].nq <= 0) return -1;
  cp->on = 1;
  return 0;
}

/* Windowed-decode knobs (PTD_WINDOW_CONE, PTD_WINDOW_STREAMS, PTD_WINDOW_PARTS) and the servers'
 * stream placement (PTD_SERVER_PLACE=0: off): read once per
 * process, re-read by ptdi_decoder_knobs_reload (tests that change one between calls). */
static int g_kn_cone = 1, g_kn_streams = 0, g_kn_parts = 2, g_kn_place = 1;
static pthread_once_t g_kn_once = PTHREAD_ONCE_INIT;
static pthread_mutex_t g_kn_lock = PTHREAD_MUTEX_INITIALIZER;
static void decoder_knobs_read(void) {
  pthread_mutex_lock(&g_kn_lock);
  const char *e = getenv("PTD_WINDOW_CONE");
  __atomic_store_n(&g_kn_cone, !(e && e[0] == '0'), __ATOMIC_RELAXED);
  e = getenv("PTD_WINDOW_STREAMS");
  __atomic_store_n(&g_kn_streams, e ? atoi(e) : 0, __ATOMIC_RELAXED);
  e = getenv("PTD_WINDOW_PARTS");
  __atomic_store_n(&g_kn_parts, e ? atoi(e) : 2, __ATOMIC_RELAXED);
  e = getenv("PTD_SERVER_PLACE");
  __atomic_store_n(&g_kn_place, !(e && e[0] == '0'), __ATOMIC_RELAXED);
  pthread_mutex_unlock(&g_kn_lock);
}
static int decoder_knob(const int *k) {
  pthread_once(&g_kn_once, decoder_knobs_read);
  return __atomic_load_n(k, __ATOMIC_RELAXED);
}
void ptdi_decoder_knobs_reload(void) {
  pthread_once(&g_kn_once, decoder_knobs_read);
  decoder_knobs_read();
}

static int cone_enabled(void) { return decoder_knob(&g_kn_cone); }

static void cols_apply(ptk_conv_desc *d, const cols_t *c) {
  d->q0 = c->q0;
  d->nq = c->nq;
  d->ext_l = c->ext_l;
  d->ext_r = c->ext_r;
  d->nq_shape = c->nq_shape;
}

int ptd_window_cols(int64_t T, int batch, int64_t lo_first, int64_t lo, int64_t hi,
                    int64_t hi_last, int64_t *out) {
  if (T < 1 || batch < 1 || !out) return -1;
  const ptk_emit em = {lo_first, lo, hi, hi_last};
  cone_plan cp;
  const int on = cone_plan_make(&cp, T, batch, &em) == 0;
  const int64_t T1 = 4 * T, T2 = 16 * T, L = T2 + 1;
  const cols_t *seq[PTD_WINDOW_LAUNCHES];
  cols_t full[PTD_WINDOW_LAUNCHES];
  int n = 0;
  seq[n++] = &cp.pre;
  seq[n++] = &cp.up0;
  for (int j = 0; j < 3; j++)
    for (int br = 0; br < 3; br++)
      for (int k = 0; k < 2; k++) seq[n++] = &cp.mrf[0][j][br][k];
  seq[n++] = &cp.up1;
  for (int j = 0; j < 3; j++)
    for (int br = 0; br < 3; br++)
      for (int k = 0; k < 2; k++) seq[n++] = &cp.mrf[1][j][br][k];
  seq[n++] = &cp.post;
  for (int i = 0; i < n; i++) {
    if (!on) {   /* the full launches: every column of every item */
      const int64_t q0 = (i == 1 || i == 20) ? 1 : 0;
      const int64_t nq = i == 0 ? T : i == 1 ? T + 1 : i < 20 ? T1 : i == 20 ? T1 + 1 : i < 39 ? T2 : L;
      full[i] = (cols_t){q0, nq, 0, 0, nq};
      seq[i] = &full[i];
    }
    out[5 * i] = seq[i]->q0;
    out[5 * i + 1] = seq[i]->nq;
    out[5 * i + 2] = seq[i]->ext_l;
    out[5 * i + 3] = seq[i]->ext_r;
    out[5 * i + 4] = seq[i]->nq_shape;
  }
  return on;
}

/* One MRF depth for `batch` items: c1 group then c2 group (see ptd_mrf_depth).  xinL[br]: the
 * LeakyReLU(0.1)'d input of branch br, or NULL to apply the LeakyReLU while staging xin[br];
 * yL: when not NULL, c2 also writes LeakyReLU(0.1) of its output there. */
static int mrf_depth(pt_ctx *c, const ptd_model *m, int stage, int j, const float *const *xin,
                     const float *const *xinL, float *const *a, float *const *y,
                     float *const *yL, int64_t T, int batch, const cols_t (*cols)[2]) {
  const int base = stage == 0 ? 2 : 21, C = stage == 0 ? 256 : 128;
  ptk_conv_desc d1[3], d2[3];
  for (int br = 0; br < 3; br++) {
    const int i1 = base + br * 6 + j * 2, i2 = i1 + 1;
    conv_layer_desc(&d1[br], m, i1, xinL ? xinL[br] : xin[br], T, T, batch, a[br], T);
    if (!xinL) {
      d1[br].in_op = PTK_IN_LEAKY;
      d1[br].in_a = 0.1f;
    }
    epi_push(&d1[br], PTK_EPI_LEAKY, 0.1f, NULL, 0, 0);
    conv_layer_desc(&d2[br], m, i2, a[br], T, T, batch, y[br], T);
    epi_push(&d2[br], PTK_EPI_ADDT, 0.0f, xin[br], T, (int64_t) C * T);
    if (yL) {
      d2[br].y2 = yL[br];
      d2[br].a2 = 0.1f;
    }
    if (cols) {
      cols_apply(&d1[br], &cols[br][0]);
      cols_apply(&d2[br], &cols[br][1]);
    }
  }
  if (ptk_conv_launch(d1, 3, c->g_stream) || ptk_conv_launch(d2, 3, c->g_stream)) {
    PT_LOG("MRF depth %d failed: %s", j, ptk_last_error());
    return -1;
  }
  return 0;
}

int ptd_mrf_depth(pt_ctx *c, const ptd_model *m, int stage, int depth, const float *const *xin,
                  const float *const *xin_leaky, float *const *a, float *const *y,
                  float *const *y_leaky, int64_t T) {
  if (!c || !c->use_cuda || !m || (stage != 0 && stage != 1) || depth < 0 || depth > 2 || T < 1)
    return -1;
  return mrf_depth(c, m, stage, depth, xin, xin_leaky, a, y, y_leaky, T, 1, NULL);
}

/* MRF stack on x [batch][C][T] (xL = LeakyReLU(0.1)(x), or NULL): writes the three branch
 * outputs (before the average) */
static int mrf_run(pt_ctx *c, const ptd_model *m, int stage, const float *x, const float *xL,
                   int64_t T, int batch, float *const out[3], const cone_plan *cp) {
  const cols_t(*cols)[3][2] = cp ? cp->mrf[stage] : NULL;
  const int C = stage == 0 ? 256 : 128;
  const size_t tb = (size_t) batch * C * T * sizeof(float);
  float *a[3], *yb[3], *lb[3];
  for (int br = 0; br < 3; br++) {
    a[br] = ptdi_arena_alloc(c, tb);
    yb[br] = ptdi_arena_alloc(c, tb);
    lb[br] = ptdi_arena_alloc(c, tb);
    if (!a[br] || !yb[br] || !lb[br]) {
      PT_LOG("arena too small for the MRF stack (T %lld batch %d)", (long long) T, batch);
      return -1;
    }
  }
  /* depth 0: x -> out[] (+ lb[]); depth 1: out[] -> yb[] (+ lb[], rewritten after depth 1's c1
   * has read it: same stream); depth 2: yb[] -> out[] */
  const float *xs[3] = {x, x, x}, *xls[3] = {xL, xL, xL};
  if (mrf_depth(c, m, stage, 0, xs, xL ? xls : NULL, a, out, lb, T, batch, cols ? cols[0] : NULL))
    return -1;
  const float *p1[3] = {out[0], out[1], out[2]}, *l1[3] = {lb[0], lb[1], lb[2]};
  if (mrf_depth(c, m, stage, 1, p1, l1, a, yb, lb, T, batch, cols ? cols[1] : NULL)) return -1;
  const float *p2[3] = {yb[0], yb[1], yb[2]};
  return mrf_depth(c, m, stage, 2, p2, l1, a, out, NULL, T, batch, cols ? cols[2] : NULL);
}

int ptd_tail(pt_ctx *c, const ptd_model *m, const float *p, int64_t L, int batch, float *wav) {
  if (!c || !c->use_cuda || !m || !p || !wav || L < 2 || batch < 1) return -1;
  if (ptk_tail_batched(p, L, 72 * L, L, wav, 16 * (L - 1), batch, m->consts, NULL, c->g_stream)) {
    PT_LOG("ptd_tail failed: %s", ptk_last_error());
    return -1;
  }
  return 0;
}

size_t ptd_decode_arena_bytes(int64_t T, int batch) {
  const size_t f = sizeof(float) * (size_t) batch;
  const int64_t T1 = 4 * T, T2 = 16 * T, L = T2 + 1;
  size_t s = 0;
  s += al256(f * 512 * T) + 2 * al256(f * 256 * T1) + 3 * al256(f * 256 * T1);   /* h, x0, x0L, o[] */
  size_t mrf0 = 9 * al256(f * 256 * T1);
  size_t late = 2 * al256(f * 128 * T2) + 3 * al256(f * 128 * T2) + 9 * al256(f * 128 * T2) +
                al256(f * 72 * L) + al256(f * 256 * T1) + al256(f * 128 * T2);
  return s + (mrf0 > late ? mrf0 : late) + 4096;
}

/* Decode `batch` items of T frames.  Item b's latents are z + b*bsz with rows ldz apart (a plain
 * batch: ldz = T, bsz = 192*T; overlap-save windows read the sequence in place: ldz = the sequence
 * length, bsz = the window hop).  Item b's waveform goes to wav + b*bsw; only the samples `emit`
 * names are stored (NULL: all). */
static int decode_impl(pt_ctx *c, const ptd_model *m, const float *z, int64_t ldz, int64_t bsz,
                       int64_t T, int batch, float *wav, int64_t bsw, const ptk_emit *emit,
                       float *const *stages) {
  if (!c || !c->use_cuda || !m || !z || !wav || T < 1 || batch < 1) return -1;
  /* refuse a decode the arena cannot hold before anything is queued */
  const size_t need = ptd_decode_arena_bytes(T, batch);
  if (c->g_arena_used > c->g_arena_bytes || need > c->g_arena_bytes - c->g_arena_used) {
    PT_LOG("arena too small for a decode of T %lld x %d (need %zu MiB, %zu MiB free)",
           (long long) T, batch, need >> 20, (c->g_arena_bytes - c->g_arena_used) >> 20);
    return -1;
  }
  const int64_t T1 = 4 * T, T2 = 16 * T, L = T2 + 1;
  const size_t f = sizeof(float) * (size_t) batch;
  /* a window that keeps only part of its samples computes only the columns they depend on
   * (PTD_WINDOW_CONE=0: every column, for comparison) */
  cone_plan plan, *cp = NULL;
  if (emit && !stages && cone_enabled() && cone_plan_make(&plan, T, batch, emit) == 0) cp = &plan;
  void *mark = ptdi_arena_mark(c);
  int rc = -1;
  float *h = ptdi_arena_alloc(c, f * 512 * T);
  float *x0 = ptdi_arena_alloc(c, f * 256 * T1);
  float *x0L = ptdi_arena_alloc(c, f * 256 * T1);
  float *o0[3] = {ptdi_arena_alloc(c, f * 256 * T1), ptdi_arena_alloc(c, f * 256 * T1),
                  ptdi_arena_alloc(c, f * 256 * T1)};
  if (!h || !x0 || !x0L || !o0[0] || !o0[1] || !o0[2]) goto oom;
  ptk_conv_desc d;
  /* conv_pre + LeakyReLU */
  ptdi_conv_desc(&d, z, ldz, bsz, T, 192, m->wr[0], m->b[0], 512, 7, 1, 1, 3, 512, h, T, 512 * T, T,
                 batch);
  d.w16 = m->wr16[0];
  epi_push(&d, PTK_EPI_LEAKY, 0.1f, NULL, 0, 0);
  if (cp) cols_apply(&d, &cp->pre);
  if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  /* ups.0 */
  ptdi_convT_desc(&d, h, T, 512 * T, T, 512, m->wr[1], m->b[1], 256, 4, 6, 16, x0, T1, 256 * T1, batch);
  d.w16 = m->wr16[1];
  d.phase_il = 1;
  d.y2 = x0L;
  d.a2 = 0.1f;
  if (cp) cols_apply(&d, &cp->up0);
  if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  void *mark1 = ptdi_arena_mark(c);
  if (mrf_run(c, m, 0, x0, x0L, T1, batch, o0, cp)) goto fail;
  ptdi_arena_release(c, mark1);   /* the MRF temporaries; o0[] stay */
  float *x1 = ptdi_arena_alloc(c, f * 128 * T2);
  float *x1L = ptdi_arena_alloc(c, f * 128 * T2);
  float *o1[3] = {ptdi_arena_alloc(c, f * 128 * T2), ptdi_arena_alloc(c, f * 128 * T2),
                  ptdi_arena_alloc(c, f * 128 * T2)};
  if (!x1 || !x1L || !o1[0] || !o1[1] || !o1[2]) goto oom;
  /* ups.1 over leaky(avg(branches), 0.1) */
  float *av0 = ptdi_arena_alloc(c, f * 256 * T1);
  if (!av0 || ptk_avg3_leaky(o0[0], o0[1], o0[2], av0, (int64_t) batch * 256 * T1, 0.1f, c->g_stream)) goto fail;
  ptdi_convT_desc(&d, av0, T1, 256 * T1, T1, 256, m->wr[20], m->b[20], 128, 4, 6, 16, x1, T2,
                  128 * T2, batch);
  d.w16 = m->wr16[20];
  d.phase_il = 1;
  d.y2 = x1L;
  d.a2 = 0.1f;
  if (cp) cols_apply(&d, &cp->up1);
  if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  void *mark2 = ptdi_arena_mark(c);
  if (mrf_run(c, m, 1, x1, x1L, T2, batch, o1, cp)) goto fail;
  ptdi_arena_release(c, mark2);
  float *p = ptdi_arena_alloc(c, f * 72 * L);
  if (!p) goto oom;
  /* conv_post over reflect_pad(1,0)(leaky(avg(branches), 0.01)) */
  float *av1 = ptdi_arena_alloc(c, f * 128 * T2);
  if (!av1 || ptk_avg3_leaky(o1[0], o1[1], o1[2], av1, (int64_t) batch * 128 * T2, 0.01f, c->g_stream)) goto fail;
  ptdi_conv_desc(&d, av1, T2, 128 * T2, L, 128, m->wr[39], m->b[39], 72, 7, 1, 1, 3, 72, p, L,
                 72 * L, L, batch);
  d.w16 = m->wr16[39];
  d.reflect_l1 = 1;
  if (cp) cols_apply(&d, &cp->post);
  if (ptk_conv_launch(&d, 1, c->g_stream)) goto fail;
  if (ptk_tail_batched(p, L, 72 * L, L, wav, bsw, batch, m->consts, emit, c->g_stream)) goto fail;
  if (stages) {
    const size_t fl = sizeof(float);
    if ((stages[0] && ptk_d2d_async(stages[0], h, fl * 512 * T, c->g_stream)) ||
        (stages[1] && ptk_d2d_async(stages[1], x0, fl * 256 * T1, c->g_stream)) ||
        (stages[2] && ptk_avg3_leaky(o0[0], o0[1], o0[2], stages[2], 256 * T1, 0.1f, c->g_stream)) ||
        (stages[3] && ptk_d2d_async(stages[3], x1, fl * 128 * T2, c->g_stream)) ||
        (stages[4] && ptk_avg3_leaky(o1[0], o1[1], o1[2], stages[4], 128 * T2, 0.01f, c->g_stream)) ||
        (stages[5] && ptk_d2d_async(stages[5], p, fl * 72 * L, c->g_stream)))
      goto fail;
  }
  rc = 0;
  goto done;
oom:
  PT_LOG("arena too small for a decode of T %lld x %d (need %zu MiB)", (long long) T, batch,
         ptd_decode_arena_bytes(T, batch) >> 20);
  goto done;
fail:
  PT_LOG("decode failed: %s", ptk_last_error());
done:
  ptdi_arena_release(c, mark);   /* later work on this stream is ordered after these kernels */
  return rc;
}

int ptd_decode(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch, float *wav) {
  return decode_impl(c, m, z, T, 192 * T, T, batch, wav, 256 * T, NULL, NULL);
}

/* ptd_decode with its activations in the library's static device scratch instead of the
 * context's arena: nothing is allocated, so a caller that may not allocate device memory (inside
 * a stream capture, a serving loop that forbids it) can decode.  The scratch is shared by every
 * call on the GPU and keeps the last call's contents; every activation is written before it is
 * read, so nothing needs clearing.  Calls on one GPU are ordered there: each call's kernels wait
 * for the previous call's, whichever context's stream that ran on (ptk_scratch_acquire /
 * _release); a call under stream capture records no such wait. */
int ptd_decode_noalloc(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch,
                       float *wav) {
  if (!c || !c->use_cuda || !m || !z || !wav || T < 1 || batch < 1) return -1;
  void *base = NULL;
  size_t cap = 0;
  if (ptk_static_scratch(&base, &cap)) {
    PT_LOG("ptd_decode_noalloc: %s", ptk_last_error());
    return -1;
  }
  /* T * batch bounded first, so the size below cannot overflow */
  const size_t need = T > ((int64_t) 1 << 32) / batch ? (size_t) -1 : ptd_decode_arena_bytes(T, batch);
  if (need > cap) {
    PT_LOG("ptd_decode_noalloc: a decode of T %lld x %d needs %zu MiB of scratch; the static "
           "scratch holds %zu MiB", (long long) T, batch, need == (size_t) -1 ? need : need >> 20,
           cap >> 20);
    return -1;
  }
  int sdev = -1;
  if (ptk_scratch_acquire(c->g_stream, &sdev)) {
    PT_LOG("ptd_decode_noalloc: %s", ptk_last_error());
    return -1;
  }
  void *a0 = c->g_arena;
  const size_t b0 = c->g_arena_bytes, u0 = c->g_arena_used, h0 = c->arena_alloc_bytes;
  c->g_arena = base;
  c->g_arena_bytes = cap;
  c->g_arena_used = 0;
  int rc = ptd_decode(c, m, z, T, batch, wav);
  c->g_arena = a0;
  c->g_arena_bytes = b0;
  c->g_arena_used = u0;
  c->arena_alloc_bytes = h0;
  /* recorded even after a failure: whatever part of the decode was queued still uses the scratch */
  if (ptk_scratch_release(c->g_stream, sdev, 1)) {
    PT_LOG("ptd_decode_noalloc: %s", ptk_last_error());
    rc = -1;
  }
  return rc;
}

int ptd_decode_stages(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, float *wav,
                      float *const *stages) {
  return decode_impl(c, m, z, T, 192 * T, T, 1, wav, 256 * T, NULL, stages);
}

static int layer_run(pt_ctx *c, const ptd_model *m, int layer, const float *x, int64_t T, int batch,
                     float *y, float in_leaky, float epi_leaky, const int64_t *cols) {
  if (!c || !c->use_cuda || !m || layer < 0 || layer >= PTD_DEC_NLAYER - 1 || T < 1 || batch < 1) return -1;
  const layer_geo g = m->g[layer];
  ptk_conv_desc d;
  if (g.convT) {
    const int c4 = (g.cout + 3) / 4 * 4;
    const int64_t Lout = (T - 1) * g.sd - 2 * g.pad + g.K;
    ptdi_convT_desc(&d, x, T, (int64_t) g.cin * T, T, g.cin, m->wr[layer], m->b[layer], g.cout,
                    g.sd, g.pad, g.K, y, Lout, (int64_t) c4 * Lout, batch);
    d.w16 = m->wr16[layer];
    d.phase_il = 1;
  } else {
    conv_layer_desc(&d, m, layer, x, T, T, batch, y, T);
  }
  if (in_leaky > 0.0f) {
    d.in_op = PTK_IN_LEAKY;
    d.in_a = in_leaky;
  }
  if (epi_leaky > 0.0f) epi_push(&d, PTK_EPI_LEAKY, epi_leaky, NULL, 0, 0);
  if (cols) {
    const cols_t cc = {cols[0], cols[1], cols[2], cols[3], cols[4]};
    cols_apply(&d, &cc);
  }
  if (ptk_conv_launch(&d, 1, c->g_stream)) {
    PT_LOG("ptd_layer %d failed: %s", layer, ptk_last_error());
    return -1;
  }
  return 0;
}

int ptd_layer(pt_ctx *c, const ptd_model *m, int layer, const float *x, int64_t T, int batch,
              float *y, float in_leaky, float epi_leaky) {
  return layer_run(c, m, layer, x, T, batch, y, in_leaky, epi_leaky, NULL);
}

int ptd_layer_cols(pt_ctx *c, const ptd_model *m, int layer, const float *x, int64_t T, int batch,
                   float *y, float in_leaky, float epi_leaky, const int64_t *cols) {
  if (!cols) return -1;
  return layer_run(c, m, layer, x, T, batch, y, in_leaky, epi_leaky, cols);
}

int ptd_mrf(pt_ctx *c, const ptd_model *m, int stage, const float *x, int64_t T, float alpha,
            float *out) {
  if (!c || !c->use_cuda || !m || (stage != 0 && stage != 1) || T < 1) return -1;
  const int C = stage == 0 ? 256 : 128;
  const size_t tb = (size_t) C * T * sizeof(float);
  void *mark = ptdi_arena_mark(c);
  float *o[3] = {ptdi_arena_alloc(c, tb), ptdi_arena_alloc(c, tb), ptdi_arena_alloc(c, tb)};
  int rc = -1;
  if (o[0] && o[1] && o[2] && !mrf_run(c, m, stage, x, NULL, T, 1, o, NULL) &&
      !ptk_avg3_leaky(o[0], o[1], o[2], out, (int64_t) C * T, alpha, c->g_stream))
    rc = 0;
  else
    PT_LOG("ptd_mrf failed: %s", ptk_last_error());
  ptdi_arena_release(c, mark);
  return rc;
}

/* ------------------------------------------------------------------ overlap-save windows
 * The reference's window schedule (main_v21_serve.c:219-257): the first window is win_first
 * frames wide (fast first audio), later ones win; window at frame a covers
 * [a, a + min(width, T - a)); it emits [max(a + lo, emitted), min(a + hi, T)) with lo = ctx except
 * for the first window, hi = width - ctx except for the last; the next window starts at
 * emitted - ctx.  Windows of equal width after the first are evenly spaced (hop = win - 2*ctx)
 * and run as one batched decode. */
typedef struct {
  int64_t a, w, e0, e1;
} win_t;

static int win_schedule(int64_t T, int win_first, int win, int ctx, win_t *out, int cap) {
  int n = 0;
  int64_t a = 0, emitted = 0;
  while (emitted < T && n < cap) {
    int64_t w = a == 0 ? win_first : win;
    if (a + w > T) w = T - a;
    const int last = a + w >= T;
    const int64_t lo = a == 0 ? 0 : ctx, hi = last ? w : w - ctx;
    int64_t e0 = a + lo, e1 = a + hi;
    if (e0 < emitted) e0 = emitted;
    if (e1 > T) e1 = T;
    out[n].a = a;
    out[n].w = w;
    out[n].e0 = e0;
    out[n].e1 = e1;
    n++;
    if (e1 > emitted) emitted = e1;
    if (last) break;
    a = e1 - ctx;
    if (a <= 0) a = 1;
  }
  return n;
}

#define MAX_WIN 4096
/* most streams a batched run of windows is split over */
#define WIN_PARTS_MAX 4

/* A schedule split into the launches that run it: the first window (alone when its width differs
 * from the others, or when asked to), then a run of full-width windows at a constant hop (one
 * batched decode reading z in place with batch stride hop and writing each window's kept frames
 * to their place in wav), then at most one shorter last window. */
typedef struct {
  int n;             /* windows */
  int first_alone;   /* window 0 decoded on its own */
  int b0, nfull;     /* the batched run: windows [b0, b0 + nfull) */
  int has_last;      /* window n - 1 clipped, decoded on its own */
  int64_t hop;
  win_t w0, wl, wb0;
} win_plan;

static int win_plan_make(int64_t T, int win_first, int win, int ctx, int split_first,
                         win_plan *pl) {
  memset(pl, 0, sizeof *pl);
  if (T < 1 || ctx < 0 || win < 2 * ctx + 1 || win_first < 2 * ctx + 1) return -1;
  win_t *ws = malloc(sizeof(win_t) * MAX_WIN);
  if (!ws) return -1;
  const int n = win_schedule(T, win_first, win, ctx, ws, MAX_WIN);
  pl->n = n;
  pl->hop = win - 2 * ctx;
  pl->w0 = ws[0];
  pl->first_alone = split_first || win_first != win || ws[0].w != win;
  int i = pl->first_alone ? 1 : 0;
  pl->b0 = i;
  while (i < n && ws[i].w == win) i++;
  pl->nfull = i - pl->b0;
  pl->has_last = i < n;
  if (pl->nfull) pl->wb0 = ws[pl->b0];
  if (pl->has_last) pl->wl = ws[n - 1];
  int rc = (n < MAX_WIN && i + (pl->has_last ? 1 : 0) == n) ? 0 : -1;
  /* the invariants the batched run relies on: constant hop, kept frames [a + lo, a + win - ctx)
   * (lo = 0 only for window 0), a full last window keeps up to a + win */
  for (int k = pl->b0; rc == 0 && k < pl->b0 + pl->nfull; k++) {
    const int64_t lo = k ? ctx : 0, hi = (k + 1 == n) ? win : win - ctx;
    if (ws[k].a != pl->wb0.a + (k - pl->b0) * pl->hop || ws[k].e0 != ws[k].a + lo ||
        ws[k].e1 != ws[k].a + hi)
      rc = -1;
  }
  free(ws);
  if (rc) PT_LOG("windowed decode: unexpected window schedule (T %lld win %d/%d ctx %d)",
                 (long long) T, win_first, win, ctx);
  return rc;
}

static size_t win_plan_arena(const win_plan *pl, int win) {
  size_t b = 0, x;
  if (pl->first_alone && (x = ptd_decode_arena_bytes(pl->w0.w, 1)) > b) b = x;
  if (pl->nfull && (x = ptd_decode_arena_bytes(win, pl->nfull)) > b) b = x;
  /* the batched run split over several streams holds every part's region at once */
  for (int parts = 2; parts <= WIN_PARTS_MAX && pl->nfull >= parts; parts++) {
    x = 0;
    for (int p = 0; p < parts; p++)
      x += al256(ptd_decode_arena_bytes(win, pl->nfull / parts + (p < pl->nfull % parts ? 1 : 0)));
    if (x > b) b = x;
  }
  if (pl->has_last && (x = ptd_decode_arena_bytes(pl->wl.w, 1)) > b) b = x;
  return b + 4096;
}

/* one window decoded on its own, writing its kept frames to their place in wav */
static int win_one(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, const win_t *l,
                   float *wav) {
  const ptk_emit em = {(l->e0 - l->a) * 256, 0, (l->e1 - l->a) * 256, (l->e1 - l->a) * 256};
  return decode_impl(c, m, z + l->a, T, 0, l->w, 1, wav + l->a * 256, 0, &em, NULL);
}

/* windows [k0, k0 + nb) of the batched run of full-width windows, as one batched decode */
static int win_range(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, const win_plan *pl,
                     int k0, int nb, int win, int ctx, float *wav) {
  const int64_t a = pl->wb0.a + (int64_t) (k0 - pl->b0) * pl->hop;
  const int last = k0 + nb == pl->n;
  const ptk_emit em = {k0 == 0 ? 0 : (int64_t) ctx * 256, (int64_t) ctx * 256,
                       (int64_t) (win - ctx) * 256, (int64_t) (last ? win : win - ctx) * 256};
  return decode_impl(c, m, z + a, T, pl->hop, win, nb, wav + a * 256, pl->hop * 256, &em, NULL);
}

/* ---- a context's extra streams
 * A long batched run of windows is split in parts: the first on the context's stream, each other
 * one on an extra stream of the context, made on first use and kept until the context shuts down
 * (pt_ctx has the reference's layout, so the streams are held here, keyed by the context; a
 * context is used by one thread at a time).  Each window's samples do not depend on the batch it
 * runs in, and the parts write disjoint samples, so the output is the same.  The parts' launches
 * overlap each other's ramp-up and tail, which a long request's batched launches leave idle when
 * they run alone (in config 5, once the other requests are done). */
#define AUX_MAX 256
typedef struct {
  pt_ctx *c;
  void *s[WIN_PARTS_MAX - 1], *fork, *join[WIN_PARTS_MAX - 1];
} aux_t;
static pthread_mutex_t g_aux_lock = PTHREAD_MUTEX_INITIALIZER;
static aux_t g_aux[AUX_MAX];

static void aux_destroy(aux_t *a) {
  for (int k = 0; k < WIN_PARTS_MAX - 1; k++) {
    if (a->s[k]) {
      ptk_stream_sync(a->s[k]);
      ptk_stream_destroy(a->s[k]);
    }
    if (a->join[k]) ptk_event_destroy(a->join[k]);
  }
  if (a->fork) ptk_event_destroy(a->fork);
  memset(a, 0, sizeof *a);
}

/* The context's entry, with the streams a split in need + 1 parts uses.  Streams are made when
 * first needed, never ahead: HIP binds each new stream to the next of its hardware queues in
 * turn, so streams made early would shift the queues the contexts made after them land on (nine
 * contexts each made with three extra streams put every context stream on one queue, and the
 * queue-fed config-5 step took 5.7 against 5.0-5.25 ms).  NULL when any of them cannot be made. */
static aux_t *aux_get(pt_ctx *c, int need) {
  aux_t *r = NULL;
  pthread_mutex_lock(&g_aux_lock);
  for (int i = 0; i < AUX_MAX && !r; i++)
    if (g_aux[i].c == c) r = &g_aux[i];
  for (int i = 0; i < AUX_MAX && !r; i++) {
    if (g_aux[i].c) continue;
    if (ptk_event_create(&g_aux[i].fork)) {
      PT_LOG("extra streams of a context: %s", ptk_last_error());
      g_aux[i].fork = NULL;
      break;
    }
    g_aux[i].c = c;
    r = &g_aux[i];
  }
  if (need > WIN_PARTS_MAX - 1) need = WIN_PARTS_MAX - 1;
  for (int k = 0; r && k < need; k++)
    if ((!r->s[k] && ptk_stream_create(&r->s[k])) || (!r->join[k] && ptk_event_create(&r->join[k]))) {
      PT_LOG("extra streams of a context: %s", ptk_last_error());
      r = NULL;   /* what was made stays in the entry until the context shuts down */
    }
  pthread_mutex_unlock(&g_aux_lock);
  return r;
}

static int win_parts(int n);

/* The extra streams the default split uses, made now rather than inside the first long request
 * a context serves.  Call it once every context of a server is made (see aux_get). */
void ptdi_aux_prepare(pt_ctx *c) { (void) aux_get(c, win_parts(1 << 20) - 1); }

void ptdi_aux_release(pt_ctx *c) {
  pthread_mutex_lock(&g_aux_lock);
  for (int i = 0; i < AUX_MAX; i++)
    if (g_aux[i].c == c) aux_destroy(&g_aux[i]);
  pthread_mutex_unlock(&g_aux_lock);
}

/* Parts of a batched run of n windows: a run of 16 or more in PTD_WINDOW_PARTS parts (default
 * 2, at most 4, each at least 8 windows).  Measured on config 5 (the T = 1500 request's 22 full
 * windows beside eight other requests): 2 parts +1.0 to +2.8 % against 1 (by box), 3 and 4 parts
 * below 2.  PTD_WINDOW_STREAMS=1 never splits, =2 splits any run of two or more in two. */
static int win_parts(int n) {
  const int k = decoder_knob(&g_kn_streams);
  if (k == 1 || n < 2) return 1;
  if (k == 2) return 2;
  if (n < 16) return 1;
  int p = decoder_knob(&g_kn_parts);
  if (p > WIN_PARTS_MAX) p = WIN_PARTS_MAX;
  while (p > 2 && n / p < 8) p--;
  return p < 1 ? 1 : p;
}

/* Parts of the batched run of full-width windows this context can run at once: win_parts, as
 * long as every part's region fits in the arena (else 1), and the extra streams for them (*xo,
 * NULL for one part). */
static int win_split(pt_ctx *c, const win_plan *pl, int win, aux_t **xo) {
  *xo = NULL;
  int parts = pl->nfull ? win_parts(pl->nfull) : 1;
  if (parts > 1) {
    size_t need = 0;
    for (int p = 0; p < parts; p++)
      need += al256(ptd_decode_arena_bytes(win, pl->nfull / parts + (p < pl->nfull % parts ? 1 : 0)));
    const size_t free_b = c->g_arena_bytes > al256(c->g_arena_used)
        ? c->g_arena_bytes - al256(c->g_arena_used) : 0;
    if (need > free_b) parts = 1;
  }
  if (parts > 1 && !(*xo = aux_get(c, parts - 1))) parts = 1;
  return parts;
}

/* the extra streams start after everything queued on the context's stream so far */
static int win_fork(pt_ctx *c, aux_t *x, int parts) {
  if (ptk_event_record(x->fork, c->g_stream)) return -1;
  for (int k = 0; k < parts - 1; k++)
    if (ptk_stream_wait_event(x->s[k], x->fork)) return -1;
  return 0;
}

/* the batched run of full-width windows in `parts` parts (the extra streams already forked) */
static int win_batch(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, const win_plan *pl,
                     int win, int ctx, float *wav, int parts, aux_t *x) {
  if (parts < 2) return win_range(c, m, z, T, pl, pl->b0, pl->nfull, win, ctx, wav);
  void *s0 = c->g_stream;
  const size_t used0 = c->g_arena_used;
  size_t used = used0;
  int rc = 0, k0 = pl->b0, started = 0;
  for (int p = 0; p < parts && rc == 0; p++) {
    const int nb = pl->nfull / parts + (p < pl->nfull % parts ? 1 : 0);
    /* each part's activations after the previous parts' regions, which their kernels still use */
    c->g_arena_used = used;
    c->g_stream = p == 0 ? s0 : x->s[p - 1];
    rc = win_range(c, m, z, T, pl, k0, nb, win, ctx, wav);
    started = p + 1;
    used = al256(used) + al256(ptd_decode_arena_bytes(win, nb));
    k0 += nb;
  }
  c->g_stream = s0;
  c->g_arena_used = used0;
  /* whatever is queued on the context next (and reuses its arena) waits for every part */
  for (int p = 1; p < started; p++)
    if (ptk_event_record(x->join[p - 1], x->s[p - 1]) ||
        ptk_stream_wait_event(c->g_stream, x->join[p - 1]))
      rc = -1;
  return rc;
}

static size_t windows_arena(int64_t T, int win_first, int win, int ctx) {
  win_plan pl;
  /* the plan with the first window split off needs at least what the merged one needs */
  if (win_plan_make(T, win_first, win, ctx, 1, &pl)) return 0;
  size_t b = win_plan_arena(&pl, win);
  if (win_first == win && win_plan_make(T, win_first, win, ctx, 0, &pl) == 0) {
    const size_t b2 = win_plan_arena(&pl, win);
    if (b2 > b) b = b2;
  }
  return b;
}

size_t ptd_windows2_arena_bytes(int64_t T, int win_first, int win, int ctx) {
  ptdi_serve_widths(&win_first, &win, ctx);
  return windows_arena(T, win_first, win, ctx);
}

size_t ptd_windows_arena_bytes(int64_t T, int win, int ctx) {
  return windows_arena(T, win, win, ctx);
}

/* The windows of one sequence, in as few launches as the schedule allows.  t_first (optional):
 * window 0 is decoded alone and waited for, and the host time its audio was complete is stored
 * (the reference's fast first audio, main_v21_serve.c:219-225); the rest follows batched. */
int ptdi_decode_windows(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int win_first,
                        int win, int ctx, float *wav, double *t_first) {
  if (!c || !c->use_cuda || !m || !z || !wav) return -1;
  win_plan pl;
  if (win_plan_make(T, win_first, win, ctx, t_first != NULL, &pl)) return -1;
  int rc = 0;
  if (pl.first_alone) {
    rc = win_one(c, m, z, T, &pl.w0, wav);
    if (rc == 0 && t_first) {
      rc = ptdi_wait(c);
      *t_first = ptdi_now_ms();
    }
  }
  aux_t *x = NULL;
  const int parts = rc == 0 ? win_split(c, &pl, win, &x) : 1;
  /* The extra streams fork ahead of the shorter last window when its activations lie inside the
   * first part's region (it runs on the context's stream, before that part): the other parts then
   * start at once instead of behind it, and a stream that shares its hardware queue with other
   * requests does not hold their packets while it waits. */
  int forked = 0;
  if (rc == 0 && parts > 1 && pl.has_last &&
      ptd_decode_arena_bytes(pl.wl.w, 1) <= al256(ptd_decode_arena_bytes(win, pl.nfull / parts + (pl.nfull % parts ? 1 : 0)))) {
    rc = win_fork(c, x, parts);
    forked = 1;
  }
  /* the shorter last window before the batched run: a small decode that leaves most of the chip
   * to other streams is better early than as the tail of the request (windows write disjoint
   * samples) */
  if (rc == 0 && pl.has_last) rc = win_one(c, m, z, T, &pl.wl, wav);
  if (rc == 0 && parts > 1 && !forked) rc = win_fork(c, x, parts);
  if (rc == 0 && pl.nfull) rc = win_batch(c, m, z, T, &pl, win, ctx, wav, parts, x);
  if (rc) PT_LOG("windowed decode failed: %s", ptk_last_error());
  return rc;
}

int ptd_decode_windows(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int win, int ctx,
                       float *wav) {
  return ptdi_decode_windows(c, m, z, T, win, win, ctx, wav, NULL);
}

int ptd_decode_windows2(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int win_first,
                        int win, int ctx, float *wav) {
  ptdi_serve_widths(&win_first, &win, ctx);
  return ptdi_decode_windows(c, m, z, T, win_first, win, ctx, wav, NULL);
}

/* ------------------------------------------------------------------ captured decodes
 * A decode of fixed shape and buffers, recorded once as a HIP graph and replayed: its 19 launches
 * then go to the device as one submission.  The capture runs against a scratch region the graph
 * owns (the context's arena fields point at it for the duration), so replays never touch what the
 * context keeps in its own arena. */
struct ptd_graph {
  pt_ctx *c;
  void *exec, *scratch;
};

ptd_graph *ptd_decode_graph(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int batch,
                            float *wav) {
  if (!c || !c->use_cuda || !m || !z || !wav || T < 1 || batch < 1) return NULL;
  ptd_graph *g = calloc(1, sizeof *g);
  if (!g) return NULL;
  g->c = c;
  const size_t bytes = ptd_decode_arena_bytes(T, batch);
  if (ptk_malloc(&g->scratch, bytes)) {
    PT_LOG("ptd_decode_graph: %s", ptk_last_error());
    free(g);
    return NULL;
  }
  void *a0 = c->g_arena;
  const size_t b0 = c->g_arena_bytes, u0 = c->g_arena_used, h0 = c->arena_alloc_bytes;
  int rc = ptk_capture_begin(c->g_stream);
  if (rc == 0) {
    c->g_arena = g->scratch;
    c->g_arena_bytes = bytes;
    c->g_arena_used = 0;
    rc = ptd_decode(c, m, z, T, batch, wav);
    c->g_arena = a0;
    c->g_arena_bytes = b0;
    c->g_arena_used = u0;
    c->arena_alloc_bytes = h0;
    if (ptk_capture_end(c->g_stream, rc ? NULL : &g->exec)) rc = -1;
  }
  if (rc) {
    PT_LOG("ptd_decode_graph: capture of a decode of T %lld x %d failed: %s", (long long) T, batch,
           ptk_last_error());
    ptd_graph_destroy(g);
    return NULL;
  }
  return g;
}

int ptd_graph_launch(pt_ctx *c, const ptd_graph *g) {
  if (!c || !g || !g->exec || c != g->c) return -1;
  if (ptk_graph_launch(g->exec, c->g_stream)) {
    PT_LOG("ptd_graph_launch: %s", ptk_last_error());
    return -1;
  }
  return 0;
}

void ptd_graph_destroy(ptd_graph *g) {
  if (!g) return;
  if (g->exec || g->scratch) ptk_stream_sync(g->c->g_stream);   /* replays still running use both */
  ptk_graph_destroy(g->exec);
  ptk_free(g->scratch);
  free(g);
}

/* One window at a time, for a caller that plays audio as it arrives (pt_v21_stream_chunk,
 * pt_v21_host.c:2871-2902): the same clipping of [a, a + win) to the sequence, and the window's
 * whole waveform (256 samples a frame) to pcm.  A batch-1 decode reading z in place. */
int ptd_decode_chunk(pt_ctx *c, const ptd_model *m, const float *z, int64_t T, int64_t a,
                     int64_t win, float *pcm, int64_t *n) {
  if (n) *n = 0;
  if (!c || !m || !z || !pcm || T < 1) return -1;
  if (a < 0) a = 0;
  if (win < 1) win = 1;
  if (a + win > T) win = T - a;
  if (win < 1) return -1;
  if (decode_impl(c, m, z + a, T, 0, win, 1, pcm, 0, NULL, NULL)) return -1;
  if (n) *n = win * 256;
  return 0;
}

/* ------------------------------------------------------------------ concurrent serving */
struct ptd_server {
  int n;
  pt_ctx *ctx;
  void *ballast[PTDI_PLACE_MAX_BALLAST];   /* idle streams that set where the contexts' go */
};

/* ---- placement of a server's streams on the hardware queues
 * HIP binds each new stream to the least-used of its hardware queues (4 by default), counting
 * every stream the process holds, and a queue runs one kernel at a time.  Which of the contexts'
 * streams share a queue therefore depends on the streams made before them, which the library can
 * neither see nor choose, and a queue that carries one stream more than the others bounds a step
 * of concurrent requests (T = 226 on 8 streams: 1 / 2 / 2 / 3 streams per queue measured ~5 %
 * slower than 2 / 2 / 2 / 2).  So the servers time it: for 0 .. PTDI_PLACE_MAX_BALLAST idle
 * streams made first, the contexts' streams are made anew and each runs one bounded
 * single-workgroup kernel, all at once; they finish in (streams on the busiest queue) x (one
 * kernel's time).  The fastest arrangement is made again and kept (HIP's choice repeats for the
 * same sequence of streams).  Only where streams sit changes, not what runs on them. */
#define PLACE_ITERS 10000
static int place_make(pt_ctx *ctx, int n, void **ballast, int nb) {
  for (int i = 0; i < n; i++) {
    if (ctx[i].g_stream && ptk_stream_destroy(ctx[i].g_stream)) return -1;
    ctx[i].g_stream = NULL;
  }
  for (int k = 0; k < nb; k++)
    if (ptk_stream_create(&ballast[k])) return -1;
  for (int i = 0; i < n; i++)
    if (ptk_stream_create(&ctx[i].g_stream)) return -1;
  return 0;
}
void ptdi_place_release(void **ballast) {
  for (int k = 0; k < PTDI_PLACE_MAX_BALLAST; k++)
    if (ballast[k]) {
      ptk_stream_destroy(ballast[k]);
      ballast[k] = NULL;
    }
}
static double place_time(pt_ctx *ctx, int n) {
  double best = 1e30;
  for (int r = 0; r < 3; r++) {
    if (ptk_device_sync()) return -1.0;
    const double t0 = ptdi_now_ms();
    for (int i = 0; i < n; i++)
      if (ptk_calib_launch(PLACE_ITERS, ctx[i].g_stream)) return -1.0;
    if (ptk_device_sync()) return -1.0;
    const double t = ptdi_now_ms() - t0;
    if (t < best) best = t;
  }
  return best;
}
int ptdi_place_streams(pt_ctx *ctx, int n, void **ballast) {
  if (n < 2 || !decoder_knob(&g_kn_place)) return 0;
  double best_t = 1e30;
  int best = 0;
  for (int nb = 0; nb <= PTDI_PLACE_MAX_BALLAST; nb++) {
    if (place_make(ctx, n, ballast, nb)) goto fail;
    const double t = place_time(ctx, n);
    ptdi_place_release(ballast);
    if (t < 0.0) goto fail;
    /* fewer idle streams unless clearly faster */
    if (t < 0.9 * best_t) {
      best_t = t;
      best = nb;
    }
  }
  if (place_make(ctx, n, ballast, best) == 0) return 0;
fail:
  PT_LOG("stream placement: %s", ptk_last_error());
  ptdi_place_release(ballast);
  for (int i = 0; i < n; i++)
    if (!ctx[i].g_stream && ptk_stream_create(&ctx[i].g_stream)) return -1;
  return 0;
}

ptd_server *ptd_server_create(int nctx, size_t arena_bytes) {
  if (nctx < 1) return NULL;
  ptd_server *s = calloc(1, sizeof *s);
  if (!s) return NULL;
  s->ctx = calloc((size_t) nctx, sizeof(pt_ctx));
  if (!s->ctx) {
    free(s);
    return NULL;
  }
  for (int i = 0; i < nctx; i++) {
    if (ptdi_ctx_init(&s->ctx[i], arena_bytes, 0)) {
      s->n = i;
      ptd_server_destroy(s);
      return NULL;
    }
  }
  s->n = nctx;
  if (ptdi_place_streams(s->ctx, nctx, s->ballast)) {
    ptd_server_destroy(s);
    return NULL;
  }
  for (int i = 0; i < nctx; i++) ptdi_aux_prepare(&s->ctx[i]);   /* after every context stream */
  return s;
}

void ptd_server_destroy(ptd_server *s) {
  if (!s) return;
  for (int i = 0; i < s->n; i++) pt_v21_cuda_shutdown(&s->ctx[i]);
  ptdi_place_release(s->ballast);
  free(s->ctx);
  free(s);
}

pt_ctx *ptd_server_ctx(ptd_server *s, int i) {
  return (s && i >= 0 && i < s->n) ? &s->ctx[i] : NULL;
}

typedef struct {
  pt_ctx *c;
  const ptd_model *m;
  const ptd_request *req;
  int nreq, first, step, rc;
} worker_arg;

static void *worker(void *p) {
  worker_arg *a = (worker_arg *) p;
  pt_v21_cuda_active(1);
  a->rc = 0;
  for (int r = a->first; r < a->nreq && !a->rc; r += a->step) {
    const ptd_request *q = &a->req[r];
    a->rc = q->win > 0 ? ptd_decode_windows(a->c, a->m, q->z, q->T, q->win, q->ctx, q->wav)
                       : ptd_decode(a->c, a->m, q->z, q->T, 1, q->wav);
  }
  if (ptdi_wait(a->c)) a->rc = -1;
  pt_v21_cuda_active(-1);
  return NULL;
}

int ptd_serve_run(ptd_server *s, const ptd_model *m, const ptd_request *req, int nreq,
                  double *wall_ms) {
  if (!s || !m || !req || nreq < 1) return -1;
  const int nt = s->n < nreq ? s->n : nreq;
  pthread_t th[256];
  worker_arg args[256];
  if (nt > 256) return -1;
  const double t0 = ptdi_now_ms();
  int started = 0;
  for (int i = 0; i < nt; i++) {
    args[i] = (worker_arg){&s->ctx[i], m, req, nreq, i, s->n, 0};
    if (pthread_create(&th[i], NULL, worker, &args[i])) break;
    started++;
  }
  int rc = started == nt ? 0 : -1;
  for (int i = 0; i < started; i++) {
    pthread_join(th[i], NULL);
    if (args[i].rc) rc = -1;
  }
  if (wall_ms) *wall_ms = ptdi_now_ms() - t0;
  return rc;
}
