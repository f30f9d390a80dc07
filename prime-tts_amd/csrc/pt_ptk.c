/* pt_ptk.c -- the .ptk weight container: reader, exact fp16 expansion, and the loaders that put a
 * container's records on the device (the process weight pool by record name, and the decoder
 * model from its dec.* records).
 *
 * Format (tools/export_v21.py:5-23, :232-274; read by runtime/v21/src/pt_v21_host.c:1086-1220):
 *   header  24 B   u32 magic 0x50544B31 'PTK1', u32 version, u32 n_tensor, i32 reserved,
 *                  i64 data_bytes
 *   records n x 136 B   char name[64] (NUL-padded), i32 ndim, 4 B pad, i64 dim[6], i64 nelem,
 *                  i64 off (relative to the data start)
 *   data    starts at the 64-byte boundary after the records; every payload is 64-byte aligned
 * A record's bytes per item come from the fp32 record "dtype.table" (one entry per record, in
 * record order: 4.0 fp32, 2.0 fp16), as the reference's C reader takes them
 * (pt_v21_host.c:1125-1146); a container without it is refused, as there.  fp16 payloads
 * (the '#h' records) expand exactly: subnormals keep their value (pt_v21_host.c:653-673).
 *
 * The file is read whole into anonymous host memory (no file-backed pointer ever reaches a HIP
 * copy), and every header field, record and payload range is checked before use: a truncated or
 * corrupt container is an error, never an out-of-bounds read. */
#define _GNU_SOURCE
#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "pt_dev_internal.h"
#include "ptd.h"

#define PTK_MAGIC 0x50544B31u
#define PTK_HDR_BYTES 24
#define PTK_REC_BYTES 136
#define PTK_NAME_BYTES 64
#define PTK_MAX_RANK 6

typedef struct {
  char name[PTK_NAME_BYTES + 1];
  int ndim, isz;
  int64_t dims[PTK_MAX_RANK], nelem, off;
} ptk_rec;

struct ptd_ptk {
  uint8_t *buf;            /* the whole file */
  size_t len;
  uint32_t version, n;
  int64_t data_bytes;
  size_t data_off;
  ptk_rec *rec;
};

static int64_t rd_i64(const uint8_t *p) { int64_t v; memcpy(&v, p, 8); return v; }
static uint32_t rd_u32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static size_t align64(size_t n) { return (n + 63) & ~(size_t) 63; }

/* binary16 -> binary32 bits (exact; the same rule as the device expansion kernel) */
static uint32_t half_to_float_bits(uint16_t h) {
  const uint32_t s = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 31u) return s | 0x7f800000u | (m << 13);
  if (e != 0u) return s | ((e + 112u) << 23) | (m << 13);
  if (m == 0u) return s;
  const uint32_t p = 31u - (uint32_t) __builtin_clz(m);   /* leading one at bit p (0..9) */
  return s | ((p + 103u) << 23) | ((m << (23u - p)) & 0x7fffffu);
}

static int read_file(const char *path, uint8_t **out, size_t *len) {
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    PT_LOG("ptk: cannot open %s: %s", path, strerror(errno));
    return -1;
  }
  struct stat st;
  if (fstat(fd, &st) || st.st_size < 0) {
    PT_LOG("ptk: cannot stat %s", path);
    close(fd);
    return -1;
  }
  const size_t n = (size_t) st.st_size;
  uint8_t *b = malloc(n ? n : 1);
  if (!b) {
    PT_LOG("ptk: no host memory for %zu bytes", n);
    close(fd);
    return -1;
  }
  size_t got = 0;
  while (got < n) {
    const ssize_t r = read(fd, b + got, n - got);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) {
      PT_LOG("ptk: read of %s failed after %zu of %zu bytes", path, got, n);
      free(b);
      close(fd);
      return -1;
    }
    got += (size_t) r;
  }
  close(fd);
  *out = b;
  *len = n;
  return 0;
}

/* parse and check everything; 0 / -1 with the reason logged */
static int parse(ptd_ptk *f, const char *path) {
  if (f->len < PTK_HDR_BYTES) {
    PT_LOG("ptk: %s is shorter than the 24-byte header", path);
    return -1;
  }
  const uint32_t magic = rd_u32(f->buf);
  if (magic != PTK_MAGIC) {
    PT_LOG("ptk: %s: bad magic 0x%x (expected PTK1)", path, magic);
    return -1;
  }
  f->version = rd_u32(f->buf + 4);
  f->n = rd_u32(f->buf + 8);
  f->data_bytes = rd_i64(f->buf + 16);
  const uint64_t table_end = PTK_HDR_BYTES + (uint64_t) PTK_REC_BYTES * f->n;
  if (table_end > f->len) {
    PT_LOG("ptk: %s: %u records run past the end of the file", path, f->n);
    return -1;
  }
  f->data_off = align64((size_t) table_end);
  if (f->data_bytes < 0 || f->data_off > f->len || (uint64_t) f->data_bytes > f->len - f->data_off) {
    PT_LOG("ptk: %s: data section (%lld bytes at %zu) does not fit the file (%zu bytes)", path,
           (long long) f->data_bytes, f->data_off, f->len);
    return -1;
  }
  f->rec = calloc(f->n ? f->n : 1, sizeof(ptk_rec));
  if (!f->rec) return -1;
  int table = -1;
  for (uint32_t i = 0; i < f->n; i++) {
    const uint8_t *r = f->buf + PTK_HDR_BYTES + (size_t) i * PTK_REC_BYTES;
    ptk_rec *q = &f->rec[i];
    memcpy(q->name, r, PTK_NAME_BYTES);
    q->name[PTK_NAME_BYTES] = 0;
    int32_t nd;
    memcpy(&nd, r + 64, 4);
    q->ndim = nd;
    for (int z = 0; z < PTK_MAX_RANK; z++) q->dims[z] = rd_i64(r + 72 + 8 * z);
    q->nelem = rd_i64(r + 120);
    q->off = rd_i64(r + 128);
    if (nd < 0 || nd > PTK_MAX_RANK || q->nelem < 0 || q->off < 0) {
      PT_LOG("ptk: %s: record %u (%s): bad ndim / nelem / offset", path, i, q->name);
      return -1;
    }
    int64_t prod = 1;
    for (int z = 0; z < nd; z++) {
      const int64_t d = q->dims[z];
      if (d < 0 || (d > 0 && prod > INT64_MAX / d)) {
        PT_LOG("ptk: %s: record %u (%s): bad dimension", path, i, q->name);
        return -1;
      }
      prod *= d;
    }
    if (prod != q->nelem) {
      PT_LOG("ptk: %s: record %u (%s): nelem %lld is not the product of its dims", path, i,
             q->name, (long long) q->nelem);
      return -1;
    }
    if (table < 0 && !strcmp(q->name, "dtype.table")) table = (int) i;
  }
  if (table < 0) {
    PT_LOG("ptk: %s: container has no dtype.table record", path);
    return -1;
  }
  /* the table itself is fp32: check its range before reading it */
  const ptk_rec *t = &f->rec[table];
  if (t->nelem < (int64_t) f->n || (uint64_t) t->off > (uint64_t) f->data_bytes ||
      (uint64_t) t->nelem * 4 > (uint64_t) f->data_bytes - (uint64_t) t->off) {
    PT_LOG("ptk: %s: dtype.table holds %lld entries for %u records, or lies outside the data",
           path, (long long) t->nelem, f->n);
    return -1;
  }
  const uint8_t *tab = f->buf + f->data_off + t->off;
  for (uint32_t i = 0; i < f->n; i++) {
    float v;
    memcpy(&v, tab + 4 * (size_t) i, 4);
    if (v != 4.0f && v != 2.0f) {
      PT_LOG("ptk: %s: dtype.table entry %u is %g (expected 4 or 2)", path, i, (double) v);
      return -1;
    }
    f->rec[i].isz = (int) v;
  }
  if (f->rec[table].isz != 4) {
    PT_LOG("ptk: %s: dtype.table describes itself as fp16", path);
    return -1;
  }
  for (uint32_t i = 0; i < f->n; i++) {
    const ptk_rec *q = &f->rec[i];
    if ((uint64_t) q->off > (uint64_t) f->data_bytes ||
        (uint64_t) q->nelem > ((uint64_t) f->data_bytes - (uint64_t) q->off) / (uint64_t) q->isz) {
      PT_LOG("ptk: %s: record %u (%s): payload of %lld x %d bytes at %lld lies outside the data",
             path, i, q->name, (long long) q->nelem, q->isz, (long long) q->off);
      return -1;
    }
  }
  return 0;
}

ptd_ptk *ptd_ptk_open(const char *path) {
  if (!path) return NULL;
  ptd_ptk *f = calloc(1, sizeof *f);
  if (!f) return NULL;
  if (read_file(path, &f->buf, &f->len) || parse(f, path)) {
    ptd_ptk_close(f);
    return NULL;
  }
  return f;
}

void ptd_ptk_close(ptd_ptk *f) {
  if (!f) return;
  free(f->rec);
  free(f->buf);
  free(f);
}

int ptd_ptk_count(const ptd_ptk *f) { return f ? (int) f->n : -1; }

int ptd_ptk_find(const ptd_ptk *f, const char *name) {
  if (!f || !name) return -1;
  for (uint32_t i = 0; i < f->n; i++)
    if (!strcmp(f->rec[i].name, name)) return (int) i;
  return -1;
}

int ptd_ptk_info(const ptd_ptk *f, int i, char *name, int *ndim, int64_t *dims, int64_t *nelem,
                 int *itemsize) {
  if (!f || i < 0 || (uint32_t) i >= f->n) return -1;
  const ptk_rec *q = &f->rec[i];
  if (name) memcpy(name, q->name, PTK_NAME_BYTES + 1);
  if (ndim) *ndim = q->ndim;
  if (dims) memcpy(dims, q->dims, sizeof q->dims);
  if (nelem) *nelem = q->nelem;
  if (itemsize) *itemsize = q->isz;
  return 0;
}

const void *ptd_ptk_payload(const ptd_ptk *f, int i) {
  if (!f || i < 0 || (uint32_t) i >= f->n) return NULL;
  return f->buf + f->data_off + f->rec[i].off;
}

int ptd_ptk_read_f32(const ptd_ptk *f, int i, float *out, int64_t n) {
  if (!f || i < 0 || (uint32_t) i >= f->n || !out || n != f->rec[i].nelem) return -1;
  const uint8_t *src = ptd_ptk_payload(f, i);
  if (f->rec[i].isz == 4) {
    memcpy(out, src, (size_t) n * 4);
  } else {
    for (int64_t k = 0; k < n; k++) {
      uint16_t h;
      memcpy(&h, src + 2 * k, 2);
      const uint32_t u = half_to_float_bits(h);
      memcpy(&out[k], &u, 4);
    }
  }
  return 0;
}

/* fp32 copy of record i (malloc'd), or NULL */
static float *read_alloc(const ptd_ptk *f, int i) {
  const int64_t n = f->rec[i].nelem;
  float *b = malloc((size_t) (n ? n : 1) * 4);
  if (b && ptd_ptk_read_f32(f, i, b, n)) {
    free(b);
    b = NULL;
  }
  return b;
}

/* ================================================================== decoder records */
/* decoder layer i's module name (spec/v21_layers.json, the dec.* packed records) */
static void dec_module(int i, char *buf, size_t cap) {
  if (i == 0) snprintf(buf, cap, "dec.conv_pre");
  else if (i == 1) snprintf(buf, cap, "dec.ups.0");
  else if (i == 20) snprintf(buf, cap, "dec.ups.1");
  else if (i == 39) snprintf(buf, cap, "dec.subband_conv_post");
  else if (i == 40) snprintf(buf, cap, "dec.Conv");
  else {
    const int base = i < 20 ? 2 : 21, o = i - base;
    snprintf(buf, cap, "dec.resblocks.%d.convs%d.%d", o / 6 + (i < 20 ? 0 : 3), o % 2 + 1,
             (o % 6) / 2);
  }
}

/* record of `module` + `suffix`, trying the fp16 name first; -1 when absent */
static int find_pair(const ptd_ptk *f, const char *module, const char *suffix) {
  char nm[PTK_NAME_BYTES * 2];
  snprintf(nm, sizeof nm, "%s%s#h", module, suffix);
  int r = ptd_ptk_find(f, nm);
  if (r < 0) {
    snprintf(nm, sizeof nm, "%s%s", module, suffix);
    r = ptd_ptk_find(f, nm);
  }
  return r;
}

/* the fixed tail convTs the fused tail kernel implements (ref/v21_graph_trace.txt:3616-3617,
 * :4044-4046): iSTFT overlap-add 16 -> 1 with the delta kernel, the window-sum 1 -> 1 with the
 * squared periodic Hann(16), and the PQMF zero-insert 4 -> 4 with 4 delta(ci, co) at tap 0 */
typedef struct {
  const char *module;
  int cin, cout, K, s;
} tail_convT;
static const tail_convT kTail[3] = {
    {"dec.ConvTranspose", 16, 1, 16, 4},
    {"dec.ConvTranspose_1", 1, 1, 16, 4},
    {"dec.ConvTranspose_2", 4, 4, 4, 4},
};

static double tail_weight(int which, int ci, int co, int k) {
  const double pi = 3.14159265358979323846;
  if (which == 0) return ci == k ? 1.0 : 0.0;
  if (which == 1) {
    const double h = 0.5 - 0.5 * cos(2.0 * pi * k / 16.0);
    return h * h;
  }
  return (ci == co && k == 0) ? 4.0 : 0.0;
}

static int check_tail(const ptd_ptk *f, int which) {
  const tail_convT *t = &kTail[which];
  const int c4 = (t->cout + 3) / 4 * 4, nt = (t->K + t->s - 1) / t->s;
  const int64_t n = (int64_t) t->s * c4 * nt * t->cin;
  const int wi = find_pair(f, t->module, ".wp"), bi = find_pair(f, t->module, ".b");
  if (wi < 0 || f->rec[wi].nelem != n) {
    PT_LOG("ptk: %s.wp is missing or does not hold %lld values", t->module, (long long) n);
    return -1;
  }
  float *w = read_alloc(f, wi), *b = bi >= 0 ? read_alloc(f, bi) : NULL;
  int bad = !w || (bi >= 0 && !b);
  /* packed convT [s*C4/4][ntap][cin][4]: ONNX tap k = r + j*s of (ci, co) sits at row r*C4 + co */
  for (int64_t e = 0; !bad && e < n; e++) {
    const int lane = (int) (e % 4), ci = (int) ((e / 4) % t->cin);
    const int64_t rest = e / 4 / t->cin;
    const int j = (int) (rest % nt), R = (int) (rest / nt) * 4 + lane;
    const int r = R / c4, co = R % c4, k = r + j * t->s;
    const double want = (co < t->cout && k < t->K) ? tail_weight(which, ci, co, k) : 0.0;
    if (fabs((double) w[e] - want) > 1e-6) bad = 1;
  }
  for (int64_t e = 0; !bad && bi >= 0 && e < f->rec[bi].nelem; e++)
    if (b[e] != 0.0f) bad = 1;
  if (bad)
    PT_LOG("ptk: %s is not the fixed form the fused decoder tail implements", t->module);
  free(w);
  free(b);
  return bad ? -1 : 0;
}

/* resolve the 41 layers' weight / bias records; 0 / -1 (logged) */
static int dec_records(const ptd_ptk *f, int *wi, int *bi) {
  for (int i = 0; i < PTD_DEC_NLAYER; i++) {
    char mod[PTK_NAME_BYTES];
    dec_module(i, mod, sizeof mod);
    wi[i] = find_pair(f, mod, ".wp");
    bi[i] = find_pair(f, mod, ".b");
    const int64_t want = ptdi_dec_wfloats(i);
    if (wi[i] < 0 || f->rec[wi[i]].nelem != want) {
      PT_LOG("ptk: %s.wp is missing or does not hold the %lld packed values of decoder layer %d",
             mod, (long long) want, i);
      return -1;
    }
    /* biases are zero-padded to cout4 by the exporter; the final conv may have none */
    if ((bi[i] < 0 && i != PTD_DEC_NLAYER - 1) ||
        (bi[i] >= 0 && f->rec[bi[i]].nelem < ptdi_dec_cout(i))) {
      PT_LOG("ptk: %s.b is missing or shorter than %d", mod, ptdi_dec_cout(i));
      return -1;
    }
  }
  for (int t = 0; t < 3; t++)
    if (check_tail(f, t)) return -1;
  return 0;
}

int ptd_ptk_check_decoder(const ptd_ptk *f) {
  if (!f) return -1;
  int wi[PTD_DEC_NLAYER], bi[PTD_DEC_NLAYER];
  return dec_records(f, wi, bi);
}

ptd_model *ptd_model_create_ptk(pt_ctx *c, const ptd_ptk *f) {
  if (!f) return NULL;
  int wi[PTD_DEC_NLAYER], bi[PTD_DEC_NLAYER];
  if (dec_records(f, wi, bi)) return NULL;
  if (!c || !c->use_cuda) return NULL;
  const void *w[PTD_DEC_NLAYER];
  const float *b[PTD_DEC_NLAYER];
  int isz[PTD_DEC_NLAYER];
  float *own[2 * PTD_DEC_NLAYER];   /* host fp32 copies: every bias and the final conv's weight */
  int nown = 0, bad = 0;
  const int last = PTD_DEC_NLAYER - 1;
  for (int i = 0; i < PTD_DEC_NLAYER; i++) {
    if (i == last) {
      float *x = read_alloc(f, wi[i]);
      own[nown++] = x;
      w[i] = x;
      isz[i] = 4;
      bad |= !x;
    } else {
      w[i] = ptd_ptk_payload(f, wi[i]);
      isz[i] = f->rec[wi[i]].isz;
    }
    b[i] = NULL;
    if (bi[i] >= 0) {
      float *x = read_alloc(f, bi[i]);
      own[nown++] = x;
      b[i] = x;
      bad |= !x;
    }
  }
  ptd_model *m = bad ? NULL : ptdi_model_build(c, w, isz, b);
  for (int k = 0; k < nown; k++) free(own[k]);
  return m;
}

/* ================================================================== weight pool */
int ptd_pool_load_ptk(pt_ctx *c, const ptd_ptk *f, int n, const char *const *ctab) {
  if (!c || !c->use_cuda || !f || !ctab || n <= 0) return -1;
  const void **src = calloc((size_t) n, sizeof(void *));
  size_t *bytes = calloc((size_t) n, sizeof(size_t));
  unsigned char *isz = calloc((size_t) n, 1);
  int r = -1;
  if (src && bytes && isz) {
    for (int k = 0; k < n; k++) {
      const int i = ctab[k] ? ptd_ptk_find(f, ctab[k]) : -1;
      isz[k] = 4;
      if (i < 0 || f->rec[i].nelem == 0) continue;   /* not in this container: empty record */
      src[k] = ptd_ptk_payload(f, i);
      bytes[k] = (size_t) f->rec[i].nelem * 4;
      isz[k] = (unsigned char) f->rec[i].isz;
    }
    r = ptdi_pool_load_src(c, n, src, bytes, isz);
  }
  free(src);
  free(bytes);
  free(isz);
  return r;
}
