/* pt_oracle.h -- TEST INFRASTRUCTURE ONLY (the parity checker, never the product).
 *
 * CPU restatement, in plain C (gnu11), of the PrimeTTS v2.1 reference CPU conv path and of the
 * graph ops around it that the MB-iSTFT decoder runs.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library.  Every function cites the reference
 * file:line it follows (paths relative to the reference repository root).
 *
 * Layouts (runtime/v21/src/pt_v21_cuda.cu:3-5, tools/export_v21.py:88-121):
 *   conv   W[cout4/4][K][cin][4]        X[batch][cin][ldx]   Y[batch][cout4][ldy]
 *   convT  W[s*cout4/4][ntap][cin][4]   X[batch][cin][ldx]   Y[batch][cout4][ldy]
 */
#ifndef PT_ORACLE_H_
#define PT_ORACLE_H_
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* epilogue op codes of the fused conv epilogue (runtime/v21/src/pt_v21_host.c:2287-2297) */
enum { ORC_EPI_NONE = 0, ORC_EPI_LEAKY = 1, ORC_EPI_RELU = 2, ORC_EPI_MULS = 3, ORC_EPI_ADDS = 4 };

float orc_epi(float v, int op, float a);

/* pt_v21_conv_cpu restated (pt_v21_host.c:2299-2361): X holds ZERO-PADDED rows (the caller's
 * scratch, pt_v21_host.c:3274-3281) and n is the output length. */
int orc_conv(const float *X, int64_t ldx, int64_t cin, float *Y, int64_t ldy, int64_t n, int cout,
             int K, int stride, int pad, int dil, const float *wp, const float *bias,
             int64_t batch, int epi0, int epi1, float a0, float a1);

/* pt_v21_convT_cpu restated (pt_v21_host.c:2547-2593), including the tail flush. */
int orc_convT(const float *X, int64_t ldx, int64_t cin, int64_t tin, float *Y, int64_t ldy,
              int cout, int s, int pad, int K, const float *wp, const float *bias, int64_t batch);

/* The decoder routes its conv / convT nodes through these two pointers (default orc_conv and
 * orc_convT).  bench.py's CPU baseline points them at the reference's own pt_v21_conv_cpu /
 * pt_v21_convT_cpu (oracle/_ref), so the decoder's conv time is the reference code's. */
typedef int (*orc_conv_fn)(const float *, int64_t, int64_t, float *, int64_t, int64_t, int, int, int,
                           int, int, const float *, const float *, int64_t, int, int, float, float);
typedef int (*orc_convT_fn)(const float *, int64_t, int64_t, int64_t, float *, int64_t, int, int, int,
                            int, const float *, const float *, int64_t);
void orc_set_conv_impl(orc_conv_fn conv, orc_convT_fn convT);

/* Host threads per batch-1 conv / convT node of the decoder and MRF drivers (default 1): the
 * node's output-channel quads are split into contiguous slices, one thread each.  Each output is
 * still summed by one thread in the reference's order, so results are bit-identical to one
 * thread.  Process-wide; set it while no decoder call runs. */
void orc_set_threads(int n);
int orc_get_threads(void);

/* The interpreter's padded-row scratch for a conv node (pt_v21_host.c:3274-3281):
 * out[b][ci][pad + t] = X[b][ci][t], zero margins; out has rows of T + 2*pad. */
void orc_pad_rows(const float *X, int64_t batch, int64_t cin, int64_t T, int pad, float *out);

/* fp32 elementwise ops, bin_op fast path (pt_v21_host.c:450-494) and un_op (pt_v21_host.c:570-620) */
void orc_add(const float *a, const float *b, float *o, int64_t n);
void orc_divs(const float *a, float s, float *o, int64_t n);
void orc_muls(const float *a, float s, float *o, int64_t n);
void orc_leaky(const float *a, float *o, int64_t n, float alpha);

/* ---------------------------------------------------------------- synthetic MB-iSTFT decoder
 * Topology: ref/v21_graph_trace.txt:3819-4065 (conv_pre .. /dec/Conv).  Layer order of the
 * weight arrays (ORC_DEC_NLAYER entries): 0 conv_pre, 1 ups.0, 2..19 MRF-256, 20 ups.1,
 * 21..38 MRF-128, 39 conv_post, 40 the final PQMF synthesis conv /dec/Conv (4 -> 1, K 63, its
 * weight the model constant /dec/Constant_134; bias may be NULL).  Inside an MRF: branch b
 * (K = 3, 7, 11), dilation j (1, 3, 5), conv c (c1, c2) at index 2 + 18*stage_offset + b*6 +
 * j*2 + c. */
#define ORC_DEC_NLAYER 41
#define ORC_DEC_ZCH 192
#define ORC_DEC_STAGES 6

typedef struct {
  const float *w[ORC_DEC_NLAYER];   /* packed weights (conv or convT layout) */
  const float *b[ORC_DEC_NLAYER];   /* bias, cout entries */
} orc_dec_weights;

/* geometry of layer i: cin, cout, K, stride(convT)/dilation(conv), pad, is_convT */
int orc_dec_layer(int i, int *cin, int *cout, int *K, int *sd, int *pad, int *is_convT);

/* Fixed constants of the decoder tail that the op definitions determine: periodic Hann(16) and
 * the irfft basis (9 x 16, cos and -sin rows, one-sided weights, /16). */
void orc_dec_constants(float *hann16, float *basis_c, float *basis_s);

/* Run the decoder for z [192][T]; wav receives 256*T samples.  stages (optional, may be NULL)
 * receives copies of: 0 conv_pre+leaky [512][T], 1 ups.0 [256][4T], 2 MRF-256 output after
 * /3+leaky [256][4T], 3 ups.1 [128][16T], 4 MRF-128 output after /3+leaky [128][16T],
 * 5 conv_post [72][16T+1].  Returns 0, or -1 on OOM. */
int orc_decoder(const orc_dec_weights *W, const float *z, int64_t T, float *wav, float **stages);
int64_t orc_dec_stage_len(int stage, int64_t T);   /* floats in stage buffer */

/* MRF stack alone (config 3): x [C][T] -> leaky(((b0+b1)+b2)/3, alpha); wt/bt index 18 convs. */
int orc_mrf(const float *const *wt, const float *const *bt, int C, int64_t T, const float *x,
            float alpha, float *out);

/* Tail alone: conv_post output p [72][L] -> wav [4*4*(L-1)] (trace :3936-4065); wfir / bfir:
 * the packed weight ([1][63][4][4]) and bias (NULL: none) of the final PQMF conv. */
int orc_tail(const float *p, int64_t L, const float *wfir, const float *bfir, float *wav);

#ifdef __cplusplus
}
#endif
#endif
