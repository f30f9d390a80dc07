/* pt_oracle.c -- TEST INFRASTRUCTURE ONLY (the parity checker, never the product).
 *
 * A C (gnu11) restatement of the PrimeTTS v2.1 reference CPU conv path and of the decoder graph
 * ops around it.  The product (the HIP library) never links this file; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  Citations are reference
 * file:line (paths relative to the reference repository root).
 *
 * Build: -O3 -std=gnu11 -ffp-contract=off, so every multiply and add rounds separately, as in the
 * reference's x86 host build (runtime/v21/Makefile:10 has no -mfma).
 */
#include "pt_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ conv epilogue
 * pt_v21_host.c:2287-2297: 1 LeakyReLU (v >= 0 keeps v), 2 ReLU (v > 0 keeps v), 3 multiply by a
 * scalar, 4 add a scalar; any other code leaves v alone. */
float orc_epi(float v, int op, float a) {
  switch (op) {
    case ORC_EPI_LEAKY: return v >= 0.0f ? v : a * v;
    case ORC_EPI_RELU: return v > 0.0f ? v : 0.0f;
    case ORC_EPI_MULS: return v * a;
    case ORC_EPI_ADDS: return v + a;
    default: return v;
  }
}

/* ------------------------------------------------------------------ conv1d
 * pt_v21_host.c:2299-2361.  Every output row starts at its bias (0 for the cout..cout4 padding
 * rows), then receives w*x for tap k ascending and, inside a tap, input channel ci ascending;
 * an input value of exactly 0 contributes nothing (the reference skips it).  The loop nest is
 * tap -> channel quad -> channel -> column, the reference's own order, so the per-output
 * summation order (and therefore every fp32 rounding) is the same.  Epilogue after the sums. */
int orc_conv(const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy, int64_t n, int cout,
             int K, int stride, int pad, int dil, const float *wp, const float *bias,
             int64_t batch, int epi0, int epi1, float a0, float a1) {
  (void) pad;   /* X is already padded: column t*stride + k*dil is in range */
  const int c4 = (cout + 3) / 4 * 4;
  const int nq = c4 / 4;
  for (int64_t b = 0; b < batch; b++) {
    const float *xb = X + b * cin * ldx;
    float *yb = Y + b * (int64_t) c4 * ldy;
    for (int co = 0; co < c4; co++) {
      const float bv = (bias != NULL && co < cout) ? bias[co] : 0.0f;
      float *yr = yb + (int64_t) co * ldy;
      for (int64_t t = 0; t < n; t++) yr[t] = bv;
    }
    for (int k = 0; k < K; k++) {
      const float *xk = xb + (int64_t) k * dil;
      for (int q = 0; q < nq; q++) {
        const float *wq = wp + ((int64_t) q * K + k) * cin * 4;
        float *y0 = yb + (int64_t) (4 * q) * ldy;
        float *y1 = y0 + ldy, *y2 = y1 + ldy, *y3 = y2 + ldy;
        for (int64_t ci = 0; ci < cin; ci++) {
          const float w0 = wq[4 * ci + 0], w1 = wq[4 * ci + 1];
          const float w2 = wq[4 * ci + 2], w3 = wq[4 * ci + 3];
          const float *xr = xk + ci * ldx;
          for (int64_t t = 0; t < n; t++) {
            const float xv = xr[t * stride];
            if (xv == 0.0f) continue;
            y0[t] += w0 * xv;
            y1[t] += w1 * xv;
            y2[t] += w2 * xv;
            y3[t] += w3 * xv;
          }
        }
      }
    }
    if (epi0 || epi1) {
      for (int co = 0; co < c4; co++) {
        float *yr = yb + (int64_t) co * ldy;
        for (int64_t t = 0; t < n; t++) {
          float v = yr[t];
          if (epi0) v = orc_epi(v, epi0, a0);
          if (epi1) v = orc_epi(v, epi1, a1);
          yr[t] = v;
        }
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ conv_transpose1d
 * pt_v21_host.c:2547-2593 (and docs/v21_layers.md:34-51).  Phase r, channel co, tap j:
 *   P_r[co][q] = bias[co] + sum_{j < ntap, j <= q, q-j < tin} sum_ci Wp[r][co][j][ci] * x[ci][q-j]
 *   Y[co][q*s + r - pad] = P_r[q]   for q in [0, tin + ntap - 1) (the last ntap-1 steps are the
 *   tail flush: they read only the zero tail of the delay line) and 0 <= q*s + r - pad < Lout.
 * For one output index there is exactly one (q, r), so the summation order per output is: bias,
 * then tap j ascending, then ci ascending, skipping exact-zero inputs. */
int orc_convT(const float *X, int64_t ldx, int64_t cin, int64_t tin, float *Y, int64_t ldy,
              int cout, int s, int pad, int K, const float *wp, const float *bias, int64_t batch) {
  const int ntap = (K + s - 1) / s;
  const int c4 = (cout + 3) / 4 * 4;
  const int64_t Q = tin + ntap - 1;
  const int64_t Lout = (tin - 1) * s - 2 * (int64_t) pad + K;
  for (int64_t b = 0; b < batch; b++) {
    const float *xb = X + b * cin * ldx;
    float *yb = Y + b * (int64_t) c4 * ldy;
    for (int co = 0; co < c4; co++) {
      const float bv = (bias != NULL && co < cout) ? bias[co] : 0.0f;
      for (int64_t t = 0; t < Lout; t++) yb[(int64_t) co * ldy + t] = bv;
    }
    for (int64_t q = 0; q < Q; q++) {
      for (int r = 0; r < s; r++) {
        const int64_t oi = q * s + r - pad;
        if (oi < 0 || oi >= Lout) continue;
        const float *wr = wp + (int64_t) r * (c4 / 4) * ntap * cin * 4;
        for (int qd = 0; qd < c4 / 4; qd++) {
          const float *wq = wr + (int64_t) qd * ntap * cin * 4;
          for (int j = 0; j < ntap; j++) {
            if (j > q) continue;
            const int64_t col = q - j;
            if (col >= tin) continue;
            for (int64_t ci = 0; ci < cin; ci++) {
              const float xv = xb[ci * ldx + col];
              if (xv == 0.0f) continue;
              const float *wv = wq + ((int64_t) j * cin + ci) * 4;
              for (int p = 0; p < 4; p++) yb[(int64_t) (4 * qd + p) * ldy + oi] += wv[p] * xv;
            }
          }
        }
      }
    }
  }
  return 0;
}

void orc_pad_rows(const float *X, int64_t batch, int64_t cin, int64_t T, int pad, float *out) {
  const int64_t ld = T + 2 * (int64_t) pad;
  memset(out, 0, (size_t) (batch * cin * ld) * sizeof(float));
  for (int64_t r = 0; r < batch * cin; r++)
    memcpy(out + r * ld + pad, X + r * T, (size_t) T * sizeof(float));
}

/* ------------------------------------------------------------------ elementwise (fp32) */
void orc_add(const float *a, const float *b, float *o, int64_t n) {
  for (int64_t i = 0; i < n; i++) o[i] = a[i] + b[i];
}
void orc_divs(const float *a, float s, float *o, int64_t n) {
  for (int64_t i = 0; i < n; i++) o[i] = a[i] / s;
}
void orc_muls(const float *a, float s, float *o, int64_t n) {
  for (int64_t i = 0; i < n; i++) o[i] = a[i] * s;
}
void orc_leaky(const float *a, float *o, int64_t n, float alpha) {
  for (int64_t i = 0; i < n; i++) o[i] = a[i] >= 0.0f ? a[i] : alpha * a[i];
}

/* ------------------------------------------------------------------ packing
 * tools/export_v21.py:88-94 (pack_conv) and :107-121 (pack_convtranspose), restated for the
 * tail's fixed kernels: W is ONNX [Cout][Cin][K] for a conv, [Cin][Cout][K] for a convT. */
static float *pack_conv_c(const float *W, int cout, int cin, int K) {
  const int c4 = (cout + 3) / 4 * 4;
  float *p = calloc((size_t) c4 * K * cin, sizeof(float));
  if (!p) return NULL;
  for (int co = 0; co < cout; co++)
    for (int ci = 0; ci < cin; ci++)
      for (int k = 0; k < K; k++)
        p[(((int64_t) (co / 4) * K + k) * cin + ci) * 4 + co % 4] = W[((int64_t) co * cin + ci) * K + k];
  return p;
}
static float *pack_convT_c(const float *W, int cin, int cout, int K, int s) {
  const int c4 = (cout + 3) / 4 * 4, nt = (K + s - 1) / s;
  float *ph = calloc((size_t) s * c4 * cin * nt, sizeof(float));   /* [s*C4][cin][nt] */
  if (!ph) return NULL;
  for (int r = 0; r < s; r++)
    for (int j = 0; j < nt; j++) {
      const int k = r + j * s;
      if (k >= K) continue;
      for (int co = 0; co < cout; co++)
        for (int ci = 0; ci < cin; ci++)
          ph[((int64_t) (r * c4 + co) * cin + ci) * nt + j] = W[((int64_t) ci * cout + co) * K + k];
    }
  float *p = pack_conv_c(ph, s * c4, cin, nt);
  free(ph);
  return p;
}

/* ------------------------------------------------------------------ decoder constants
 * Hann(16) periodic = 0.5 - 0.5 cos(2 pi n / 16) (trace :4009 /dec/Constant_109, whose preview
 * values it reproduces), the window-sum kernel is its square (trace :3617 onnx::ConvTranspose_5159).
 * irfft basis for n_fft 16 (trace :3607-3615): row k of the cos basis is w_k cos(2 pi k n/16)/16 and
 * of the sin basis -w_k sin(2 pi k n / 16)/16, w = [1, 2, ..., 2, 1] (k = 0..8).
 * The PQMF synthesis filter is not a closed form: it is the model constant /dec/Constant_134, the
 * weight of the final conv, and comes in as decoder layer 40 (orc_tail's wfir / bfir). */
void orc_dec_constants(float *hann16, float *basis_c, float *basis_s) {
  const double pi = 3.14159265358979323846;
  if (hann16)
    for (int n = 0; n < 16; n++) hann16[n] = (float) (0.5 - 0.5 * cos(2.0 * pi * n / 16.0));
  for (int k = 0; k < 9; k++) {
    const double w = (k == 0 || k == 8) ? 1.0 : 2.0;
    for (int n = 0; n < 16; n++) {
      if (basis_c) basis_c[k * 16 + n] = (float) (w * cos(2.0 * pi * k * n / 16.0) / 16.0);
      if (basis_s) basis_s[k * 16 + n] = (float) (-w * sin(2.0 * pi * k * n / 16.0) / 16.0);
    }
  }
}

/* ------------------------------------------------------------------ decoder geometry
 * spec/v21_layers.json + trace :3819-3935: conv_pre 192->512 K7 p3; ups.0 convT 512->256 K16 s4
 * p6; MRF convs C->C with K in {3,7,11}: c1 dilation {1,3,5}, c2 dilation 1, "same" padding
 * d*(K-1)/2; ups.1 convT 256->128; conv_post 128->72 K7 p3. */
static const int kMrfK[3] = {3, 7, 11};
static const int kMrfD[3] = {1, 3, 5};

int orc_dec_layer(int i, int *cin, int *cout, int *K, int *sd, int *pad, int *is_convT) {
  if (i < 0 || i >= ORC_DEC_NLAYER) return -1;
  *is_convT = 0;
  if (i == 0) { *cin = 192; *cout = 512; *K = 7; *sd = 1; *pad = 3; return 0; }
  if (i == 1 || i == 20) {
    *cin = i == 1 ? 512 : 256; *cout = i == 1 ? 256 : 128;
    *K = 16; *sd = 4; *pad = 6; *is_convT = 1; return 0;
  }
  if (i == 39) { *cin = 128; *cout = 72; *K = 7; *sd = 1; *pad = 3; return 0; }
  /* /dec/Conv: its input is padded by the /dec/Pad node (31|31) before it, so the conv has pad 0 */
  if (i == 40) { *cin = 4; *cout = 1; *K = 63; *sd = 1; *pad = 0; return 0; }
  const int base = i < 20 ? 2 : 21, C = i < 20 ? 256 : 128;
  const int o = i - base, b = o / 6, j = (o % 6) / 2, c = o % 2;
  *cin = C; *cout = C; *K = kMrfK[b];
  *sd = c == 0 ? kMrfD[j] : 1;
  *pad = *sd * (*K - 1) / 2;
  return 0;
}

static orc_conv_fn g_conv = orc_conv;
static orc_convT_fn g_convT = orc_convT;

void orc_set_conv_impl(orc_conv_fn conv, orc_convT_fn convT) {
  g_conv = conv ? conv : orc_conv;
  g_convT = convT ? convT : orc_convT;
}

/* ------------------------------------------------------------------ node threading
 * A batch-1 conv or convT node may be split over its output-channel quads across host threads
 * (orc_set_threads).  Every output row is then summed by one thread, in the same order as in the
 * one-thread run, through the same conv function on a slice of the packed weights (a convT's
 * phase rows r*C4/4 + q are gathered per slice), so the results are bit-identical and only the
 * wall time changes.  Tests use it to decode long sequences; the CPU baseline keeps one thread
 * per request. */
static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }
int orc_get_threads(void) { return g_threads; }

typedef struct {
  int is_convT;
  const float *x;
  int64_t ldx, cin, tin, ldy, n;
  float *y;
  int cout, K, s, pad, dil, epi0, q0, q1, nq;
  const float *w, *b;
  float a0;
  int rc;
} node_part;

static void *node_part_run(void *arg) {
  node_part *p = arg;
  const int co0 = 4 * p->q0, cout = (p->cout < 4 * p->q1 ? p->cout : 4 * p->q1) - co0;
  float *y = p->y + (int64_t) co0 * p->ldy;
  const float *b = p->b ? p->b + co0 : NULL;
  if (!p->is_convT) {
    const float *w = p->w + (int64_t) p->q0 * p->K * p->cin * 4;
    p->rc = g_conv(p->x, p->ldx, p->cin, y, p->ldy, p->n, cout, p->K, 1, p->pad, p->dil, w, b, 1,
                   p->epi0, 0, p->a0, 0.0f);
    return NULL;
  }
  const int ntap = (p->K + p->s - 1) / p->s, nqs = p->q1 - p->q0;
  const int64_t quad = (int64_t) ntap * p->cin * 4;
  float *w = malloc((size_t) (p->s * nqs * quad) * sizeof(float));
  if (!w) { p->rc = -1; return NULL; }
  for (int r = 0; r < p->s; r++)
    memcpy(w + r * nqs * quad, p->w + ((int64_t) r * p->nq + p->q0) * quad,
           (size_t) (nqs * quad) * sizeof(float));
  p->rc = g_convT(p->x, p->ldx, p->cin, p->tin, y, p->ldy, cout, p->s, p->pad, p->K, w, b, 1);
  free(w);
  return NULL;
}

/* runs the node's quads [0, nq) in up to g_threads contiguous slices; 1 when it ran, 0 when the
 * node is left to the caller (one thread, or too few quads), -1 on failure */
static int node_threads(node_part proto) {
  int parts = g_threads < proto.nq ? g_threads : proto.nq;
  if (parts < 2) return 0;
  node_part p[64];
  pthread_t th[64];
  int started = 0, rc = 1;
  for (int i = 0; i < parts; i++) {
    p[i] = proto;
    p[i].q0 = (int) ((int64_t) proto.nq * i / parts);
    p[i].q1 = (int) ((int64_t) proto.nq * (i + 1) / parts);
    p[i].rc = -1;
  }
  for (int i = 1; i < parts; i++) {
    if (pthread_create(&th[i], NULL, node_part_run, &p[i])) break;
    started = i;
  }
  node_part_run(&p[0]);
  for (int i = 1; i <= started; i++) pthread_join(th[i], NULL);
  for (int i = 0; i < parts; i++)
    if (p[i].rc != 0) rc = -1;
  return rc;
}

/* one conv node as the interpreter runs it on the CPU path: padded scratch, conv, trim */
static int conv_node(const float *x, int64_t T, int cin, int cout, int K, int pad, int dil,
                     const float *w, const float *b, int epi0, float a0, float *y, int64_t batch) {
  const int64_t ld = T + 2 * (int64_t) pad;
  const int64_t Tout = ld - (int64_t) (K - 1) * dil;
  const int c4 = (cout + 3) / 4 * 4;
  float *xp = malloc((size_t) (batch * cin * ld) * sizeof(float));
  float *yp = c4 == cout ? y : malloc((size_t) (batch * c4 * Tout) * sizeof(float));
  if (!xp || !yp) { free(xp); if (yp != y) free(yp); return -1; }
  orc_pad_rows(x, batch, cin, T, pad, xp);
  const node_part np = {.x = xp, .ldx = ld, .cin = cin, .ldy = Tout, .n = Tout, .y = yp,
                        .cout = cout, .K = K, .pad = pad, .dil = dil, .epi0 = epi0, .nq = c4 / 4,
                        .w = w, .b = b, .a0 = a0};
  const int tr = batch == 1 ? node_threads(np) : 0;
  if (tr < 0) { free(xp); if (yp != y) free(yp); return -1; }
  if (tr == 0)
    g_conv(xp, ld, cin, yp, Tout, Tout, cout, K, 1, pad, dil, w, b, batch, epi0, 0, a0, 0.0f);
  if (yp != y) {
    for (int64_t bb = 0; bb < batch; bb++)
      memcpy(y + bb * cout * Tout, yp + bb * c4 * Tout, (size_t) (cout * Tout) * sizeof(float));
    free(yp);
  }
  free(xp);
  return 0;
}

/* convT node (pt_v21_host.c:3406-3435): scratch + trim when cout4 != cout */
static int convT_node(const float *x, int64_t tin, int cin, int cout, int K, int s, int pad,
                      const float *w, const float *b, float *y, int64_t batch) {
  const int64_t Lout = (tin - 1) * s - 2 * (int64_t) pad + K;
  const int c4 = (cout + 3) / 4 * 4;
  float *yp = c4 == cout ? y : malloc((size_t) (batch * c4 * Lout) * sizeof(float));
  if (!yp) return -1;
  const node_part np = {.is_convT = 1, .x = x, .ldx = tin, .cin = cin, .tin = tin, .ldy = Lout,
                        .y = yp, .cout = cout, .K = K, .s = s, .pad = pad, .nq = c4 / 4, .w = w,
                        .b = b};
  const int tr = batch == 1 ? node_threads(np) : 0;
  if (tr < 0) { if (yp != y) free(yp); return -1; }
  if (tr == 0) g_convT(x, tin, cin, tin, yp, Lout, cout, s, pad, K, w, b, batch);
  if (yp != y) {
    for (int64_t bb = 0; bb < batch; bb++)
      memcpy(y + bb * cout * Lout, yp + bb * c4 * Lout, (size_t) (cout * Lout) * sizeof(float));
    free(yp);
  }
  return 0;
}

/* MRF stack, trace :3822-3869 (stage 1) and :3871-3918 (stage 2):
 *   l0 = leaky(x); per branch K: y = x; for d in (1,3,5):
 *     a = leaky(c1_{K,d}(j == 0 ? l0 : leaky(y)))      (conv_pre-style fused epilogue)
 *     y = c2_{K,d}(a) + y                               (host Add, conv output first)
 *   out = leaky(((y_K3 + y_K7) + y_K11) / 3, alpha). */
int orc_mrf(const float *const *wt, const float *const *bt, int C, int64_t T, const float *x,
            float alpha, float *out) {
  const int64_t n = (int64_t) C * T;
  float *l0 = malloc(n * sizeof(float)), *in = malloc(n * sizeof(float));
  float *a = malloc(n * sizeof(float)), *c = malloc(n * sizeof(float));
  float *y = malloc(n * sizeof(float)), *sum = malloc(n * sizeof(float));
  int rc = -1;
  if (!l0 || !in || !a || !c || !y || !sum) goto done;
  orc_leaky(x, l0, n, 0.1f);
  for (int br = 0; br < 3; br++) {
    const int K = kMrfK[br];
    memcpy(y, x, n * sizeof(float));
    for (int j = 0; j < 3; j++) {
      const int d = kMrfD[j], i1 = br * 6 + j * 2, i2 = i1 + 1;
      const float *src = l0;
      if (j > 0) { orc_leaky(y, in, n, 0.1f); src = in; }
      if (conv_node(src, T, C, C, K, d * (K - 1) / 2, d, wt[i1], bt[i1], ORC_EPI_LEAKY, 0.1f, a, 1)) goto done;
      if (conv_node(a, T, C, C, K, (K - 1) / 2, 1, wt[i2], bt[i2], 0, 0.0f, c, 1)) goto done;
      orc_add(c, y, y, n);
    }
    if (br == 0) memcpy(sum, y, n * sizeof(float));
    else orc_add(sum, y, sum, n);
  }
  orc_divs(sum, 3.0f, sum, n);
  orc_leaky(sum, out, n, alpha);
  rc = 0;
done:
  free(l0); free(in); free(a); free(c); free(y); free(sum);
  return rc;
}

/* iSTFT + PQMF tail, trace :3936-4065, with the reference's host-op arithmetic: Exp/Sin/Cos in
 * double rounded to fp32 (pt_v21_host.c:625-647), scalar Mul/Div/Add in fp32 (:450-494), the
 * bkt,kn->bnt einsum accumulated in double over k ascending (:1963-1995), Clip as a compare,
 * the three ConvTransposes and the final Conv through the conv/convT path with packed kernels. */
int orc_tail(const float *p, int64_t L, const float *wfir, const float *bfir, float *wav) {
  float hann[16], bc[144], bs[144];
  orc_dec_constants(hann, bc, bs);
  const int64_t Lola = (L - 1) * 4 + 16, Ly = Lola - 16, Lu = Ly * 4;
  float *mag = malloc(36 * L * sizeof(float)), *ph = malloc(36 * L * sizeof(float));
  float *re = malloc(36 * L * sizeof(float)), *im = malloc(36 * L * sizeof(float));
  float *fr = malloc(64 * L * sizeof(float)), *fi = malloc(64 * L * sizeof(float));
  double *acc = malloc(16 * L * sizeof(double));
  float *ola = malloc(4 * Lola * sizeof(float)), *ones = malloc(4 * L * sizeof(float));
  float *wsum = malloc(4 * Lola * sizeof(float)), *yv = malloc(4 * Ly * sizeof(float));
  float *u = malloc(4 * Lu * sizeof(float)), *up = malloc(4 * (Lu + 62) * sizeof(float));
  float *W = NULL, *wola = NULL, *wwin = NULL, *wup = NULL;
  int rc = -1;
  if (!mag || !ph || !re || !im || !fr || !fi || !acc || !ola || !ones || !wsum || !yv || !u || !up)
    goto done;
  /* Reshape [72][L] -> [4][18][L]; Exp of channels 0..8, Sin of 9..17 times pi (fp32 Mul) */
  for (int b = 0; b < 4; b++)
    for (int k = 0; k < 9; k++)
      for (int64_t t = 0; t < L; t++) {
        mag[(b * 9 + k) * L + t] = (float) exp((double) p[(b * 18 + k) * L + t]);
        const float sv = (float) sin((double) p[(b * 18 + 9 + k) * L + t]);
        ph[(b * 9 + k) * L + t] = sv * 3.1415927f;
      }
  for (int64_t i = 0; i < 36 * L; i++) {
    re[i] = mag[i] * (float) cos((double) ph[i]);
    im[i] = mag[i] * (float) sin((double) ph[i]);
  }
  /* the two einsums; a zero basis entry is skipped as the reference does */
  for (int pass = 0; pass < 2; pass++) {
    const float *A = pass == 0 ? re : im, *Bm = pass == 0 ? bc : bs;
    float *O = pass == 0 ? fr : fi;
    for (int b = 0; b < 4; b++) {
      for (int64_t i = 0; i < 16 * L; i++) acc[i] = 0.0;
      for (int k = 0; k < 9; k++) {
        const float *ar = A + (b * 9 + k) * L;
        for (int nn = 0; nn < 16; nn++) {
          const double bv = (double) Bm[k * 16 + nn];
          if (bv == 0.0) continue;
          for (int64_t t = 0; t < L; t++) acc[nn * L + t] += bv * (double) ar[t];
        }
      }
      for (int64_t i = 0; i < 16 * L; i++) O[b * 16 * L + i] = (float) acc[i];
    }
  }
  for (int b = 0; b < 4; b++)
    for (int nn = 0; nn < 16; nn++)
      for (int64_t t = 0; t < L; t++) {
        const int64_t i = (b * 16 + nn) * L + t;
        fr[i] = (fr[i] + fi[i]) * hann[nn];
      }
  /* OLA: ConvTranspose 16->1 K16 s4 with the delta kernel W[n][0][m] = (n == m), batch 4 */
  W = calloc(16 * 16, sizeof(float));
  if (!W) goto done;
  for (int nn = 0; nn < 16; nn++) W[nn * 16 + nn] = 1.0f;
  wola = pack_convT_c(W, 16, 1, 16, 4);
  /* window sum: ConvTranspose of ones [4][1][L] with Hann^2 */
  for (int nn = 0; nn < 16; nn++) W[nn] = hann[nn] * hann[nn];
  wwin = pack_convT_c(W, 1, 1, 16, 4);
  if (!wola || !wwin) goto done;
  if (convT_node(fr, L, 16, 1, 16, 4, 0, wola, NULL, ola, 4)) goto done;
  for (int64_t i = 0; i < 4 * L; i++) ones[i] = 1.0f;
  if (convT_node(ones, L, 1, 1, 16, 4, 0, wwin, NULL, wsum, 4)) goto done;
  /* Clip(min 1e-9), Div, Slice [8:-8] */
  for (int b = 0; b < 4; b++)
    for (int64_t i = 0; i < Ly; i++) {
      const int64_t j = b * Lola + i + 8;
      const float eps = 1e-9f;   /* the Clip min is an fp32 constant */
      const float den = wsum[j] > eps ? wsum[j] : eps;
      yv[b * Ly + i] = ola[j] / den;
    }
  /* PQMF synthesis: zero-insert x4 (ConvTranspose 4->4 K4 s4 with 4*delta), pad 31|31, conv K63 */
  float wu[64] = {0};
  for (int c = 0; c < 4; c++) wu[(c * 4 + c) * 4 + 0] = 4.0f;
  wup = pack_convT_c(wu, 4, 4, 4, 4);
  if (!wup || !wfir) goto done;
  if (convT_node(yv, Ly, 4, 4, 4, 4, 0, wup, NULL, u, 1)) goto done;
  /* /dec/Pad (constant 31|31) feeds a pad-0 conv: the conv node's scratch is that padded row */
  orc_pad_rows(u, 1, 4, Lu, 31, up);
  if (conv_node(up, Lu + 62, 4, 1, 63, 0, 1, wfir, bfir, 0, 0.0f, wav, 1)) goto done;
  rc = 0;
done:
  free(mag); free(ph); free(re); free(im); free(fr); free(fi); free(acc); free(ola); free(ones);
  free(wsum); free(yv); free(u); free(up); free(W); free(wola); free(wwin); free(wup);
  return rc;
}

int64_t orc_dec_stage_len(int stage, int64_t T) {
  switch (stage) {
    case 0: return 512 * T;
    case 1: case 2: return 256 * 4 * T;
    case 3: case 4: return 128 * 16 * T;
    case 5: return 72 * (16 * T + 1);
    default: return 0;
  }
}

/* full decoder, trace :3819-4065 */
int orc_decoder(const orc_dec_weights *W, const float *z, int64_t T, float *wav, float **stages) {
  const int64_t T1 = 4 * T, T2 = 16 * T, L = T2 + 1;
  float *h = malloc(512 * T * sizeof(float));
  float *x0 = malloc(256 * T1 * sizeof(float)), *m0 = malloc(256 * T1 * sizeof(float));
  float *x1 = malloc(128 * T2 * sizeof(float)), *m1 = malloc(128 * T2 * sizeof(float));
  float *rp = malloc(128 * L * sizeof(float)), *pp = malloc(72 * L * sizeof(float));
  int rc = -1;
  if (!h || !x0 || !m0 || !x1 || !m1 || !rp || !pp) goto done;
  /* conv_pre + its LeakyRelu (fused by the interpreter: sole consumer, pt_v21_host.c:3295-3333) */
  if (conv_node(z, T, 192, 512, 7, 3, 1, W->w[0], W->b[0], ORC_EPI_LEAKY, 0.1f, h, 1)) goto done;
  if (convT_node(h, T, 512, 256, 16, 4, 6, W->w[1], W->b[1], x0, 1)) goto done;
  if (orc_mrf(W->w + 2, W->b + 2, 256, T1, x0, 0.1f, m0)) goto done;
  if (convT_node(m0, T1, 256, 128, 16, 4, 6, W->w[20], W->b[20], x1, 1)) goto done;
  if (orc_mrf(W->w + 21, W->b + 21, 128, T2, x1, 0.01f, m1)) goto done;
  /* /dec/reflection_pad (1, 0): column 0 mirrors column 1 (pt_v21_host.c:1641-1670) */
  for (int c = 0; c < 128; c++) {
    rp[c * L] = m1[c * T2 + 1];
    memcpy(rp + c * L + 1, m1 + c * T2, T2 * sizeof(float));
  }
  if (conv_node(rp, L, 128, 72, 7, 3, 1, W->w[39], W->b[39], 0, 0.0f, pp, 1)) goto done;
  if (stages) {
    const float *src[6] = {h, x0, m0, x1, m1, pp};
    for (int s = 0; s < 6; s++)
      if (stages[s]) memcpy(stages[s], src[s], orc_dec_stage_len(s, T) * sizeof(float));
  }
  if (orc_tail(pp, L, W->w[40], W->b[40], wav)) goto done;
  rc = 0;
done:
  free(h); free(x0); free(m0); free(x1); free(m1); free(rp); free(pp);
  return rc;
}
