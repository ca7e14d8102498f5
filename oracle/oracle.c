/*
 * oracle.c — CPU restatement of the rustCrates transformer token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Never linked into the product.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp, glibc libm).
 *
 * Citations are to the reference crate, relative to src/neural_networks/.
 * Batch semantics: at batch 1 this is the reference exactly.  At batch > 1 the
 * reference's cached decode only extends sequence 0 (masked_attention_head.rs:
 * 141-172), so the oracle defines batched decode as independent per-sequence
 * runs: sequence b caches its own lens[b] keys and decodes on its own length.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

const char* orc_last_error(void) { return g_err; }

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* num-complex 0.4.6 arithmetic                                             */
/* ------------------------------------------------------------------------ */

static inline oc64 c_add(oc64 a, oc64 b) { return (oc64){a.re + b.re, a.im + b.im}; }
static inline oc64 c_sub(oc64 a, oc64 b) { return (oc64){a.re - b.re, a.im - b.im}; }
/* impl Mul for Complex: re = a.re*b.re - a.im*b.im, im = a.re*b.im + a.im*b.re */
static inline oc64 c_mul(oc64 a, oc64 b) { return (oc64){a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re}; }
/* Complex * f64 and f64 * Complex scale both parts */
static inline oc64 c_scale(oc64 a, double t) { return (oc64){a.re * t, a.im * t}; }
/* Complex / f64 (unscale) */
static inline oc64 c_unscale(oc64 a, double t) { return (oc64){a.re / t, a.im / t}; }
/* impl Div for Complex: multiply by the conjugate over norm_sqr */
static inline oc64 c_div(oc64 a, oc64 b) {
  double n = b.re * b.re + b.im * b.im;
  double re = a.re * b.re + a.im * b.im;
  double im = a.im * b.re - a.re * b.im;
  return (oc64){re / n, im / n};
}

/* Complex::sqrt: positive-real and imaginary-axis shortcuts, else polar form
 * from_polar(sqrt(hypot), atan2/2). */
static oc64 c_sqrt(oc64 z) {
  if (z.im == 0.0) {
    if (!signbit(z.re)) return (oc64){sqrt(z.re), z.im};
    double im = sqrt(-z.re);
    return signbit(z.im) ? (oc64){0.0, -im} : (oc64){0.0, im};
  }
  if (z.re == 0.0) {
    double x = sqrt(fabs(z.im) / 2.0);
    return signbit(z.im) ? (oc64){x, -x} : (oc64){x, x};
  }
  double r = hypot(z.re, z.im);
  double theta = atan2(z.im, z.re);
  double rs = sqrt(r), th = theta / 2.0;
  return (oc64){rs * cos(th), rs * sin(th)};
}

/* Complex::tanh: (sinh 2a + i sin 2b) / (cosh 2a + cos 2b) */
static oc64 c_tanh(oc64 z) {
  double two_re = z.re + z.re, two_im = z.im + z.im;
  double den = cosh(two_re) + cos(two_im);
  return c_unscale((oc64){sinh(two_re), sin(two_im)}, den);
}

oc64 orc_cmul(oc64 a, oc64 b) { return c_mul(a, b); }
oc64 orc_cdiv(oc64 a, oc64 b) { return c_div(a, b); }
oc64 orc_csqrt(oc64 z) { return c_sqrt(z); }
oc64 orc_ctanh(oc64 z) { return c_tanh(z); }

/* gelu_complex (utils/activation.rs:195-212).  powi(3) is num-traits binary
 * exponentiation: z * (z * z). */
static oc64 gelu_c(oc64 z, int* nan_flag) {
  const double sqrt_2_over_pi = sqrt(2.0 / M_PI);
  oc64 z3 = c_mul(z, c_mul(z, z));
  oc64 f = c_scale(c_add(z, c_mul((oc64){0.044715, 0.0}, z3)), sqrt_2_over_pi);
  /* f64::max / f64::min return the non-NaN operand, like fmax / fmin */
  oc64 cl = {fmin(fmax(f.re, -30.0), 30.0), fmin(fmax(f.im, -30.0), 30.0)};
  oc64 t = c_tanh(cl);
  if (isnan(t.re) || isnan(t.im)) *nan_flag = 1; /* reference panics here */
  return c_mul(c_scale(z, 0.5), c_add((oc64){1.0, 0.0}, t));
}

oc64 orc_gelu(oc64 z, int* nan_flag) {
  int f = 0;
  oc64 r = gelu_c(z, &f);
  if (nan_flag) *nan_flag = f;
  return r;
}

/* ------------------------------------------------------------------------ */
/* L1 kernels                                                               */
/* ------------------------------------------------------------------------ */

/* One output row of multiply_complex: acc[j] = sum_k a[k] * B[k][j], each sum a
 * sequential complex fold from 0 in k order (zgemm_ alpha=1, beta=0;
 * utils/matrix.rs:16-65). */
/* 0: k ascending (default), 1: k descending, 2: k split into 8 contiguous
 * chunks, each summed ascending, the 8 partials then summed in order */
static int g_gemm_order = 0;

static void zgemm_range(uint32_t n, uint32_t k0, uint32_t k1, int desc, const oc64* a, const oc64* B, oc64* c) {
  for (uint32_t j = 0; j < n; ++j) c[j] = (oc64){0.0, 0.0};
  for (uint32_t i = k0; i < k1; ++i) {
    const uint32_t kk = desc ? k0 + k1 - 1 - i : i;
    const oc64 av = a[kk];
    const oc64* b = B + (size_t)kk * n;
    for (uint32_t j = 0; j < n; ++j) c[j] = c_add(c[j], c_mul(av, b[j]));
  }
}

static void zgemm_row(uint32_t n, uint32_t k, const oc64* a, const oc64* B, oc64* c) {
  if (g_gemm_order != 2) {
    zgemm_range(n, 0, k, g_gemm_order == 1, a, B, c);
    return;
  }
  enum { P = 8 };
  oc64* part = (oc64*)malloc(sizeof(oc64) * n);
  for (uint32_t j = 0; j < n; ++j) c[j] = (oc64){0.0, 0.0};
  const uint32_t chunk = (k + P - 1) / P;
  for (uint32_t p = 0; p < P; ++p) {
    uint32_t k0 = p * chunk, k1 = k0 + chunk < k ? k0 + chunk : k;
    if (k0 >= k1) break;
    zgemm_range(n, k0, k1, 0, a, B, part);
    for (uint32_t j = 0; j < n; ++j) c[j] = c_add(c[j], part[j]);
  }
  free(part);
}

/* Re(q . k) of one score: an entry of multiply_complex(q, transpose(K))
 * (masked_attention_head.rs:190), so it follows the zgemm order above. */
static double score_dot(uint32_t dh, const oc64* q, const oc64* k) {
  double acc = 0.0;
  if (g_gemm_order == 0) {
    for (uint32_t e = 0; e < dh; ++e) acc = acc + (q[e].re * k[e].re - q[e].im * k[e].im);
  } else if (g_gemm_order == 1) {
    for (uint32_t e = dh; e-- > 0;) acc = acc + (q[e].re * k[e].re - q[e].im * k[e].im);
  } else {
    const uint32_t chunk = (dh + 7) / 8;
    for (uint32_t e0 = 0; e0 < dh; e0 += chunk) {
      double part = 0.0;
      for (uint32_t e = e0; e < e0 + chunk && e < dh; ++e) part = part + (q[e].re * k[e].re - q[e].im * k[e].im);
      acc = acc + part;
    }
  }
  return acc;
}

/* OpenBLAS fixes no summation order for zgemm_ (its kernels block and fuse
 * differently per CPU), so any order is an equally valid restatement of
 * utils/matrix.rs:16-65.  Orders 1 and 2 exist to measure the reference's
 * own rounding noise floor: the spread between valid orders. */
void orc_set_gemm_order(int order) { g_gemm_order = (order == 1 || order == 2) ? order : 0; }

static void zgemm_serial(uint32_t m, uint32_t n, uint32_t k, const oc64* A, const oc64* B, oc64* C) {
  for (uint32_t i = 0; i < m; ++i) zgemm_row(n, k, A + (size_t)i * k, B, C + (size_t)i * n);
}

void orc_zgemm(uint32_t m, uint32_t n, uint32_t k, const oc64* A, const oc64* B, oc64* C) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)m; ++i) zgemm_row(n, k, A + (size_t)i * k, B, C + (size_t)i * n);
}

/* NormalNormLayer::normalize (norm_layer.rs:64-82) */
void orc_layernorm_row(const oc64* x, uint32_t d, double eps, const oc64* gamma, const oc64* beta, oc64* out) {
  const double len = (double)d;
  oc64 sum = {0.0, 0.0};
  for (uint32_t i = 0; i < d; ++i) sum = c_add(sum, x[i]);
  const oc64 mean = c_unscale(sum, len);
  oc64 vs = {0.0, 0.0};
  for (uint32_t i = 0; i < d; ++i) {
    oc64 t = c_sub(x[i], mean);
    vs = c_add(vs, c_mul(t, t)); /* powu(2) = t * t */
  }
  const oc64 var = c_unscale(vs, len);
  const oc64 stddev = c_sqrt(c_add(var, (oc64){eps, 0.0}));
  for (uint32_t i = 0; i < d; ++i) {
    oc64 v = c_add(c_mul(c_div(c_sub(x[i], mean), stddev), gamma[i]), beta[i]);
    out[i] = (oc64){v.re, 0.0};
  }
}

/* softmax_row_real (utils/activation.rs:431-439) */
void orc_softmax_row_real(const oc64* x, uint32_t n, double* out) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < n; ++i) mx = fmax(mx, x[i].re);
  double sum = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    out[i] = exp(x[i].re - mx);
    sum += out[i];
  }
  for (uint32_t i = 0; i < n; ++i) out[i] = out[i] / sum;
}

/* greedy_decoding (src/utils/sampling_methods.rs:5-18): Iterator::max_by with
 * partial_cmp keeps the LAST of equal maxima; a NaN makes unwrap() panic. */
int64_t orc_greedy_row(const double* row, uint32_t n) {
  if (n == 0) return 0;
  uint32_t best = 0;
  if (isnan(row[0])) return -1;
  for (uint32_t i = 1; i < n; ++i) {
    if (isnan(row[i])) return -1;
    if (row[i] >= row[best]) best = i;
  }
  return best;
}

/* apply_rotary_positional_encoding (positional_encoding_layer.rs:181-209) */
void orc_rope_row(const oc64* x, uint32_t d, double base, uint64_t position, oc64* out) {
  const uint32_t half = d / 2;
  for (uint32_t i = 0; i < half; ++i) {
    double theta = (double)position / pow(base * 1.0, 2.0 * (double)i / (double)d);
    if (theta < -1.0) theta = -1.0; /* f64::clamp */
    if (theta > 1.0) theta = 1.0;
    double s = sin(theta), c = cos(theta);
    oc64 e = x[2 * i], o = x[2 * i + 1];
    out[2 * i] = (oc64){e.re * c - o.re * s, e.im * c - o.im * s};
    out[2 * i + 1] = (oc64){e.re * s + o.re * c, e.im * s + o.im * c};
  }
}

/* ------------------------------------------------------------------------ */
/* counter generator (shared definition with the HIP path)                  */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t orc_draw(uint64_t seed, uint64_t stream, uint64_t index) {
  return mix64(mix64(mix64(seed) ^ stream) ^ index);
}

/* uniform on [-lim, lim): (2u - 1) is exact, one rounding in the product */
double orc_uniform(uint64_t seed, uint64_t stream, uint64_t index, double lim) {
  double u = (double)(orc_draw(seed, stream, index) >> 11) * 0x1.0p-53;
  return (2.0 * u - 1.0) * lim;
}

#define STREAM_PROMPT 0x7F00000000ull
#define STREAM_NORMAL 0x7E00000000ull

void orc_gen_prompts(uint64_t seed, uint32_t batch, uint32_t max_len, const uint32_t* lens, uint32_t vocab,
                     uint32_t* ids) {
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t s = 0; s < max_len; ++s) {
      uint32_t id = 1; /* PAD */
      if (!lens || s < lens[b])
        id = (uint32_t)(((unsigned __int128)orc_draw(seed, STREAM_PROMPT + b, s) * vocab) >> 64);
      ids[(size_t)b * max_len + s] = id;
    }
}

/* Box-Muller; re and im of element p are the pair drawn from (2p, 2p+1) */
void orc_gen_normal(uint64_t seed, uint64_t n, oc64* out) {
  for (uint64_t p = 0; p < n; ++p) {
    double u1 = (double)((orc_draw(seed, STREAM_NORMAL, 2 * p) >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(orc_draw(seed, STREAM_NORMAL, 2 * p + 1) >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    out[p] = (oc64){r * cos(2.0 * M_PI * u2), r * sin(2.0 * M_PI * u2)};
  }
}

/* ------------------------------------------------------------------------ */
/* network                                                                  */
/* ------------------------------------------------------------------------ */

typedef struct {
  int kind;
  uint32_t d_in, d_out;
  uint32_t vocab;
  oc64* table;
  double base;
  double eps;
  oc64 *gamma, *beta;
  uint32_t heads, dh, max_ctx;
  oc64 *wq, *wk, *wv, *bias_pos; /* [h][d][dh] x3, [h][max_ctx][max_ctx] */
  oc64 *kc, *vc;                 /* [h][cache_B][max_ctx][dh] */
  uint32_t* clen;                /* [cache_B] */
  uint32_t cache_B;
  int cache_valid;
  uint32_t hidden;
  oc64 *w1, *b1, *w2, *b2; /* Linear uses w1/b1 */
  int mode;
} orc_layer;

struct orc_net {
  orc_layer* layers;
  int n, cap;
  uint32_t train_T; /* target rows at the end of each sequence in a stateless pass (wavelet input/target split) */
};

orc_net* orc_net_create(void) { return (orc_net*)calloc(1, sizeof(orc_net)); }

static void free_cache(orc_layer* L) {
  free(L->kc);
  free(L->vc);
  free(L->clen);
  L->kc = L->vc = NULL;
  L->clen = NULL;
  L->cache_valid = 0;
  L->cache_B = 0;
}

void orc_net_destroy(orc_net* net) {
  if (!net) return;
  for (int i = 0; i < net->n; ++i) {
    orc_layer* L = &net->layers[i];
    free(L->table);
    free(L->gamma);
    free(L->beta);
    free(L->wq);
    free(L->wk);
    free(L->wv);
    free(L->bias_pos);
    free(L->w1);
    free(L->b1);
    free(L->w2);
    free(L->b2);
    free_cache(L);
  }
  free(net->layers);
  free(net);
}

int orc_num_layers(const orc_net* net) { return net ? net->n : 0; }

static orc_layer* push_layer(orc_net* net, int kind) {
  if (net->n == net->cap) {
    int cap = net->cap ? net->cap * 2 : 16;
    orc_layer* l = (orc_layer*)realloc(net->layers, sizeof(orc_layer) * cap);
    if (!l) return NULL;
    net->layers = l;
    net->cap = cap;
  }
  orc_layer* L = &net->layers[net->n++];
  memset(L, 0, sizeof *L);
  L->kind = kind;
  return L;
}

static oc64* dup_or_zero(const oc64* src, size_t n) {
  oc64* p = (oc64*)malloc(n * sizeof(oc64));
  if (!p) return NULL;
  if (src) memcpy(p, src, n * sizeof(oc64));
  else memset(p, 0, n * sizeof(oc64));
  return p;
}

static oc64* fill_const(const oc64* src, size_t n, oc64 v) {
  oc64* p = (oc64*)malloc(n * sizeof(oc64));
  if (!p) return NULL;
  for (size_t i = 0; i < n; ++i) p[i] = src ? src[i] : v;
  return p;
}

static int dwt_low_pass(uint32_t wavelet, double* lo, uint32_t* L);

int orc_add_embedding(orc_net* net, uint32_t vocab, uint32_t dim, const oc64* table) {
  if (!net || !vocab || !dim) return fail(ORC_ERR_ARG, "embedding: bad dims");
  orc_layer* L = push_layer(net, ORC_EMBEDDING);
  L->vocab = vocab;
  L->d_in = L->d_out = dim;
  L->table = dup_or_zero(table, (size_t)vocab * dim);
  return L->table ? ORC_OK : fail(ORC_ERR_NOMEM, "embedding: out of memory");
}

int orc_add_positional_encoding(orc_net* net, uint32_t dim, double base) {
  if (!net || !dim || (dim % 2)) return fail(ORC_ERR_ARG, "positional encoding: dim must be even");
  orc_layer* L = push_layer(net, ORC_POSITIONAL_ENCODING);
  L->d_in = L->d_out = dim;
  L->base = base;
  return ORC_OK;
}

int orc_add_norm(orc_net* net, uint32_t dim, double eps, const oc64* gamma, const oc64* beta) {
  if (!net || !dim) return fail(ORC_ERR_ARG, "norm: bad dims");
  orc_layer* L = push_layer(net, ORC_NORM);
  L->d_in = L->d_out = dim;
  L->eps = eps;
  L->gamma = fill_const(gamma, dim, (oc64){1.0, 0.0});
  L->beta = fill_const(beta, dim, (oc64){0.0, 0.0});
  return (L->gamma && L->beta) ? ORC_OK : fail(ORC_ERR_NOMEM, "norm: out of memory");
}

int orc_add_self_attention(orc_net* net, uint32_t heads, uint32_t dim, uint32_t max_ctx, double eps,
                           const oc64* wq, const oc64* wk, const oc64* wv, const oc64* bias_pos,
                           const oc64* gamma, const oc64* beta) {
  if (!net || !heads || !dim || dim % heads || !max_ctx) return fail(ORC_ERR_ARG, "self-attention: bad dims");
  orc_layer* L = push_layer(net, ORC_SELF_ATTENTION);
  L->heads = heads;
  L->d_in = L->d_out = dim;
  L->dh = dim / heads;
  L->max_ctx = max_ctx;
  L->eps = eps;
  size_t wn = (size_t)heads * dim * L->dh;
  L->wq = dup_or_zero(wq, wn);
  L->wk = dup_or_zero(wk, wn);
  L->wv = dup_or_zero(wv, wn);
  L->bias_pos = dup_or_zero(bias_pos, (size_t)heads * max_ctx * max_ctx);
  L->gamma = fill_const(gamma, dim, (oc64){1.0, 0.0});
  L->beta = fill_const(beta, dim, (oc64){0.0, 0.0});
  if (!L->wq || !L->wk || !L->wv || !L->bias_pos || !L->gamma || !L->beta)
    return fail(ORC_ERR_NOMEM, "self-attention: out of memory");
  return ORC_OK;
}

int orc_add_feed_forward(orc_net* net, uint32_t dim, uint32_t hidden, const oc64* w1, const oc64* b1,
                         const oc64* w2, const oc64* b2) {
  if (!net || !dim || !hidden) return fail(ORC_ERR_ARG, "feed-forward: bad dims");
  orc_layer* L = push_layer(net, ORC_FEED_FORWARD);
  L->d_in = L->d_out = dim;
  L->hidden = hidden;
  L->w1 = dup_or_zero(w1, (size_t)dim * hidden);
  L->w2 = dup_or_zero(w2, (size_t)hidden * dim);
  L->b1 = fill_const(b1, hidden, (oc64){1.0, 0.0});
  L->b2 = fill_const(b2, dim, (oc64){1.0, 0.0});
  if (!L->w1 || !L->w2 || !L->b1 || !L->b2) return fail(ORC_ERR_NOMEM, "feed-forward: out of memory");
  return ORC_OK;
}

int orc_add_linear(orc_net* net, uint32_t in, uint32_t out, const oc64* w, const oc64* b) {
  if (!net || !in || !out) return fail(ORC_ERR_ARG, "linear: bad dims");
  orc_layer* L = push_layer(net, ORC_LINEAR);
  L->d_in = in;
  L->d_out = out;
  L->w1 = dup_or_zero(w, (size_t)in * out);
  L->b1 = fill_const(b, out, (oc64){1.0, 0.0});
  if (!L->w1 || !L->b1) return fail(ORC_ERR_NOMEM, "linear: out of memory");
  return ORC_OK;
}

int orc_add_discrete_wavelet(orc_net* net, uint32_t dim, uint32_t wavelet, uint32_t mode, int is_full_mode) {
  if (!net) return fail(ORC_ERR_ARG, "null network");
  if (is_full_mode) return fail(ORC_ERR_ARG, "DiscreteWaveletLayer in full mode is not supported");
  double lo[4];
  uint32_t L;
  int rc = dwt_low_pass(wavelet, lo, &L);
  if (rc) return rc;
  if (!(mode <= 4 || mode == 6)) return fail(ORC_ERR_ARG, "wavelet mode %u is not supported", mode);
  orc_layer* Lr = push_layer(net, ORC_DISCRETE_WAVELET);
  if (!Lr) return fail(ORC_ERR_NOMEM, "out of memory");
  Lr->vocab = wavelet; /* the wavelet type */
  Lr->mode = (int)mode;
  Lr->d_in = Lr->d_out = dim;
  return ORC_OK;
}

int orc_add_softmax(orc_net* net, int operation_mode) {
  if (!net) return fail(ORC_ERR_ARG, "softmax: null net");
  orc_layer* L = push_layer(net, ORC_SOFTMAX);
  L->mode = operation_mode;
  return ORC_OK;
}

/* Xavier-uniform (utils/weights_initializer.rs:73-89) from the counter
 * generator: re from draw 2e, im from draw 2e+1, limit sqrt(6/(rows+cols)). */
static void xavier_fill(oc64* w, uint32_t rows, uint32_t cols, uint64_t seed, uint64_t stream) {
  const double lim = sqrt(6.0 / (double)((uint64_t)rows + cols));
  const int64_t n = (int64_t)rows * cols;
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < n; ++e)
    w[e] = (oc64){orc_uniform(seed, stream, 2 * (uint64_t)e, lim), orc_uniform(seed, stream, 2 * (uint64_t)e + 1, lim)};
}

static inline uint64_t stream_id(uint32_t layer, uint32_t slot) { return ((uint64_t)layer << 12) | slot; }

int orc_init_seeded(orc_net* net, uint64_t seed) {
  if (!net) return fail(ORC_ERR_ARG, "null net");
  for (int li = 0; li < net->n; ++li) {
    orc_layer* L = &net->layers[li];
    switch (L->kind) {
      case ORC_EMBEDDING: xavier_fill(L->table, L->vocab, L->d_out, seed, stream_id(li, 0)); break;
      case ORC_NORM:
        for (uint32_t i = 0; i < L->d_in; ++i) L->gamma[i] = (oc64){1.0, 0.0}, L->beta[i] = (oc64){0.0, 0.0};
        break;
      case ORC_SELF_ATTENTION: {
        size_t wn = (size_t)L->d_in * L->dh, bn = (size_t)L->max_ctx * L->max_ctx;
        for (uint32_t h = 0; h < L->heads; ++h) {
          xavier_fill(L->wq + h * wn, L->d_in, L->dh, seed, stream_id(li, 1 + 4 * h));
          xavier_fill(L->wk + h * wn, L->d_in, L->dh, seed, stream_id(li, 2 + 4 * h));
          xavier_fill(L->wv + h * wn, L->d_in, L->dh, seed, stream_id(li, 3 + 4 * h));
          xavier_fill(L->bias_pos + h * bn, L->max_ctx, L->max_ctx, seed, stream_id(li, 4 + 4 * h));
        }
        for (uint32_t i = 0; i < L->d_in; ++i) L->gamma[i] = (oc64){1.0, 0.0}, L->beta[i] = (oc64){0.0, 0.0};
        break;
      }
      case ORC_FEED_FORWARD:
        xavier_fill(L->w1, L->d_in, L->hidden, seed, stream_id(li, 1));
        xavier_fill(L->w2, L->hidden, L->d_out, seed, stream_id(li, 2));
        for (uint32_t i = 0; i < L->hidden; ++i) L->b1[i] = (oc64){1.0, 0.0};
        for (uint32_t i = 0; i < L->d_out; ++i) L->b2[i] = (oc64){1.0, 0.0};
        break;
      case ORC_LINEAR:
        xavier_fill(L->w1, L->d_in, L->d_out, seed, stream_id(li, 1));
        for (uint32_t i = 0; i < L->d_out; ++i) L->b1[i] = (oc64){1.0, 0.0};
        break;
      default: break;
    }
  }
  return ORC_OK;
}

int orc_get_tensor(const orc_net* net, uint32_t layer, uint32_t slot, oc64* out, uint64_t n) {
  if (!net || layer >= (uint32_t)net->n) return fail(ORC_ERR_ARG, "bad layer index");
  const orc_layer* L = &net->layers[layer];
  const oc64* src = NULL;
  uint64_t len = 0;
  switch (slot) {
    case 0:
      if (L->kind == ORC_EMBEDDING) src = L->table, len = (uint64_t)L->vocab * L->d_out;
      else if (L->kind == ORC_SELF_ATTENTION) src = L->wq, len = (uint64_t)L->heads * L->d_in * L->dh;
      else if (L->kind == ORC_FEED_FORWARD) src = L->w1, len = (uint64_t)L->d_in * L->hidden;
      else if (L->kind == ORC_LINEAR) src = L->w1, len = (uint64_t)L->d_in * L->d_out;
      break;
    case 1:
      if (L->kind == ORC_SELF_ATTENTION) src = L->wk, len = (uint64_t)L->heads * L->d_in * L->dh;
      else if (L->kind == ORC_FEED_FORWARD) src = L->w2, len = (uint64_t)L->hidden * L->d_out;
      break;
    case 2:
      if (L->kind == ORC_SELF_ATTENTION) src = L->wv, len = (uint64_t)L->heads * L->d_in * L->dh;
      break;
    case 3:
      if (L->kind == ORC_SELF_ATTENTION) src = L->bias_pos, len = (uint64_t)L->heads * L->max_ctx * L->max_ctx;
      break;
    case 4:
      if (L->kind == ORC_FEED_FORWARD) src = L->b1, len = L->hidden;
      else if (L->kind == ORC_LINEAR) src = L->b1, len = L->d_out;
      break;
    case 5:
      if (L->kind == ORC_FEED_FORWARD) src = L->b2, len = L->d_out;
      break;
    case 6:
      if (L->gamma) src = L->gamma, len = L->d_in;
      break;
    case 7:
      if (L->beta) src = L->beta, len = L->d_in;
      break;
  }
  if (!src) return fail(ORC_ERR_ARG, "layer %u has no tensor in slot %u", layer, slot);
  if (n != len) return fail(ORC_ERR_ARG, "tensor size %llu != %llu", (unsigned long long)n, (unsigned long long)len);
  memcpy(out, src, len * sizeof(oc64));
  return ORC_OK;
}

int orc_reset(orc_net* net) {
  if (!net) return fail(ORC_ERR_ARG, "null net");
  for (int i = 0; i < net->n; ++i)
    if (net->layers[i].kind == ORC_SELF_ATTENTION) free_cache(&net->layers[i]);
  return ORC_OK;
}


/* ------------------------------------------------------------------------ */
/* DiscreteWaveletLayer (network_types/wavelet_discrete_layer.rs:46-161)     */
/* ------------------------------------------------------------------------ */

/* Low-pass filters of DiscreteWaletetType DB1 and DB2 (wavelet_transform/
 * dwt_coeffients.rs DB_1, DB_2; dwt_type_resolver.rs:6-9): 1/sqrt(2) twice, and
 * Daubechies' closed form (1+sqrt3, 3+sqrt3, 3-sqrt3, 1-sqrt3) / (4 sqrt2),
 * evaluated in long double and rounded once to double. */
static int dwt_low_pass(uint32_t wavelet, double* lo, uint32_t* L) {
  if (wavelet == 0) {
    lo[0] = lo[1] = (double)(1.0L / sqrtl(2.0L));
    *L = 2;
    return ORC_OK;
  }
  if (wavelet == 1) {
    const long double s3 = sqrtl(3.0L), den = 4.0L * sqrtl(2.0L);
    lo[0] = (double)((1.0L + s3) / den);
    lo[1] = (double)((3.0L + s3) / den);
    lo[2] = (double)((3.0L - s3) / den);
    lo[3] = (double)((1.0L - s3) / den);
    *L = 4;
    return ORC_OK;
  }
  return fail(ORC_ERR_ARG, "wavelet type %u: only DB1 and DB2 are supported", wavelet);
}

/* get_high_pass_filter (dwt_type_resolver.rs:107-123): the low-pass filter
 * reversed, odd entries negated */
static void dwt_high_pass(const double* lo, uint32_t L, double* hi) {
  for (uint32_t i = 0; i < L; ++i) hi[i] = (i % 2 == 1) ? -lo[L - 1 - i] : lo[L - 1 - i];
}

/* one element of the padded array: source index (-1: a zero) and sign */
typedef struct {
  int32_t idx;
  double sign;
} dwt_src;

/* insert_padding_before / insert_padding_after (wavelet_transform/dwt.rs:149-293)
 * applied to the indices of n elements; *before = L - 2 elements in front */
static int dwt_padded(uint32_t n, uint32_t L, uint32_t mode, dwt_src** out, uint32_t* plen, uint32_t* before) {
  if (!(mode <= 4 || mode == 6)) return fail(ORC_ERR_ARG, "wavelet mode %u is not supported", mode);
  if (n == 0) return fail(ORC_ERR_ARG, "empty sequence");
  const uint32_t nb = L - 2;
  const uint32_t len0 = n + nb;
  const uint32_t na = (len0 % L != 0) ? L - len0 % L + 2 : L - len0 % L + 1; /* dwt.rs:50-54 */
  dwt_src* a = (dwt_src*)malloc((size_t)(n + nb + na) * sizeof(dwt_src));
  dwt_src* orig = (dwt_src*)malloc((size_t)(n + nb) * sizeof(dwt_src));
  if (!a || !orig) {
    free(a), free(orig);
    return fail(ORC_ERR_NOMEM, "dwt: out of memory");
  }
  uint32_t cur = n;
  for (uint32_t i = 0; i < n; ++i) a[i] = (dwt_src){(int32_t)i, 1.0};
  uint32_t rtmp = 0;
  for (uint32_t i = 0; i < nb; ++i) {
    dwt_src v = {-1, 1.0};
    switch (mode) {
      case 0: break;                                 /* ZERO */
      case 1: v = a[i]; break;                       /* CONSTANT: data_trans[i] */
      case 2: v = a[cur % n + i % n]; break;         /* SYMMETRIC */
      case 3: v = a[cur % n + i % n]; v.sign = -v.sign; break; /* ANTISYMMETRIC */
      case 4:                                        /* REFLECT */
        if (i > 0) rtmp = (rtmp + 2) % cur;
        if (rtmp == 0) rtmp = 1;
        v = a[rtmp];
        break;
      default: v = (dwt_src){(int32_t)(n - 1 - (i % n)), 1.0}; break; /* PERIODIC: origin_data */
    }
    memmove(a + 1, a, (size_t)cur * sizeof(dwt_src));
    a[0] = v;
    ++cur;
  }
  const uint32_t olen = cur;
  memcpy(orig, a, (size_t)olen * sizeof(dwt_src));
  for (uint32_t i = 0; i < na; ++i) {
    dwt_src v = {-1, 1.0};
    switch (mode) {
      case 0: break;
      case 1: v = a[cur - 1]; break;
      case 2: v = a[cur - (cur % olen + i % olen) - 1]; break;
      case 3: v = a[cur - (cur % olen + i % olen) - 1]; v.sign = -v.sign; break;
      case 4: v = orig[olen - ((i + 1) % olen) - 1]; break;
      default: v = orig[i % (olen - nb) + nb]; break;
    }
    a[cur++] = v;
  }
  free(orig);
  *out = a;
  *plen = cur;
  *before = nb;
  return ORC_OK;
}

/* geometry of dwt_1d (dwt.rs:36-90) on n elements: the transform length N and
 * its midpoint (the low half is [0, N/2)) */
static uint32_t dwt_len(uint32_t n, uint32_t L) {
  uint32_t N = n + (L - 2);
  if (n % 2 != 0) N += 1;
  return N;
}

int orc_dwt_1d(const double* x, uint32_t n, uint32_t wavelet, uint32_t mode, double* out, uint32_t* out_len) {
  double lo[4] = {0.0, 0.0, 0.0, 0.0}, hi[4];
  uint32_t L = 0, plen = 0, nb = 0;
  int rc = dwt_low_pass(wavelet, lo, &L);
  if (rc) return rc;
  dwt_high_pass(lo, L, hi);
  dwt_src* a;
  if ((rc = dwt_padded(n, L, mode, &a, &plen, &nb))) return rc;
  const uint32_t N = dwt_len(n, L), middle = N >> 1;
  for (uint32_t i = 0; i < N; ++i) out[i] = 0.0;
  uint32_t ind = 0;
  for (uint32_t i = 0; i < N; i += 2) {
    double vl = 0.0, vh = 0.0;
    for (uint32_t l = 0; l < L; ++l) {
      const dwt_src e = a[(i + l) % plen];
      const double v = e.idx < 0 ? 0.0 : e.sign * x[e.idx];
      vl = vl + v * lo[l];
      vh = vh + v * hi[l];
    }
    out[ind] = vl;
    out[ind + middle] = vh;
    ++ind;
  }
  free(a);
  *out_len = N;
  return ORC_OK;
}

/* compress_partial + compress_padding_mask (wavelet_discrete_layer.rs:260-281,
 * 297-313): every feature's sequence of the B x S rows becomes the low half
 * of its dwt_1d; the mask becomes the low half of dwt_1d of its 0/1 values
 * thresholded at 0.99.  Rows per sequence: *S2; lens2[b] = ones of its mask. */
static int dwt_compress(uint32_t wavelet, uint32_t mode, const oc64* x, const uint32_t* mask, uint32_t B, uint32_t S,
                        uint32_t d, oc64* out, uint32_t* mask2, uint32_t* lens2, uint32_t* S2) {
  double lo[4] = {0.0, 0.0, 0.0, 0.0};
  uint32_t L = 0, plen = 0, nb = 0;
  int rc = dwt_low_pass(wavelet, lo, &L);
  if (rc) return rc;
  dwt_src* a;
  if ((rc = dwt_padded(S, L, mode, &a, &plen, &nb))) return rc;
  const uint32_t M = dwt_len(S, L) >> 1;
  for (uint32_t b = 0; b < B; ++b) {
    const oc64* xb = x + (size_t)b * S * d;
    for (uint32_t j = 0; j < M; ++j)
      for (uint32_t c = 0; c < d; ++c) {
        oc64 v = {0.0, 0.0};
        for (uint32_t l = 0; l < L; ++l) {
          const dwt_src e = a[(2 * j + l) % plen];
          const oc64 t = e.idx < 0 ? (oc64){0.0, 0.0} : c_scale(xb[(size_t)e.idx * d + c], e.sign);
          v = c_add(v, c_scale(t, lo[l])); /* value_low + data * low_pass (dwt.rs:74-79) */
        }
        out[((size_t)b * M + j) * d + c] = v;
      }
    uint32_t ones = 0;
    for (uint32_t j = 0; j < M; ++j) {
      double v = 0.0;
      for (uint32_t l = 0; l < L; ++l) {
        const dwt_src e = a[(2 * j + l) % plen];
        const double t = e.idx < 0 ? 0.0 : e.sign * (double)mask[(size_t)b * S + e.idx];
        v = v + t * lo[l];
      }
      mask2[(size_t)b * M + j] = v > 0.99 ? 1u : 0u;
      ones += mask2[(size_t)b * M + j];
    }
    lens2[b] = ones ? ones : 1;
  }
  free(a);
  *S2 = M;
  return ORC_OK;
}

uint32_t orc_seq_out_len(const orc_net* net, uint32_t S) {
  for (int i = 0; net && i < net->n; ++i)
    if (net->layers[i].kind == ORC_DISCRETE_WAVELET) S = dwt_len(S, net->layers[i].vocab == 0 ? 2 : 4) >> 1;
  return S;
}

/* ------------------------------------------------------------------------ */
/* layer forwards                                                           */
/* ------------------------------------------------------------------------ */

/* EmbeddingLayer::forward + apply_padding_to_batch (embedding_layer.rs:112-211):
 * right-pad with PAD=1, mask 1/0; id 1 always yields the zero vector. */
static int embedding_forward(const orc_layer* L, const uint32_t* ids, const uint32_t* lens, uint32_t B, uint32_t S,
                             oc64* out, uint32_t* mask) {
  const uint32_t d = L->d_out;
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) {
      uint32_t id = s < lens[b] ? ids[(size_t)b * S + s] : 1;
      mask[(size_t)b * S + s] = s < lens[b] ? 1 : 0;
      oc64* o = out + ((size_t)b * S + s) * d;
      if (id == 1) {
        for (uint32_t i = 0; i < d; ++i) o[i] = (oc64){0.0, 0.0};
      } else {
        if (id >= L->vocab) return fail(ORC_ERR_ARG, "No token embedding found: %u", id);
        memcpy(o, L->table + (size_t)id * d, d * sizeof(oc64));
      }
    }
  return ORC_OK;
}

/* PositionalEncodingLayer::forward (positional_encoding_layer.rs:35-99):
 * position = row index, or time_step when forward_only and time_step > 0. */
static void posenc_forward(const orc_layer* L, oc64* x, uint32_t B, uint32_t S, const uint32_t* ts, int forward_only) {
  const uint32_t d = L->d_in;
  oc64* tmp = (oc64*)malloc(d * sizeof(oc64));
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) {
      uint64_t pos = s;
      uint32_t t = ts ? ts[b] : 0;
      if (forward_only && t > 0) pos = t;
      oc64* row = x + ((size_t)b * S + s) * d;
      orc_rope_row(row, d, L->base, pos, tmp);
      memcpy(row, tmp, d * sizeof(oc64));
    }
  free(tmp);
}

/* NormalNormLayer::forward (norm_layer.rs:84-130).  With `before`, the input
 * first becomes Re(x + before) + 0i (add_matrix_3d_c, utils/matrix.rs:600-613). */
static void norm_forward(double eps, const oc64* gamma, const oc64* beta, const oc64* x, const oc64* before,
                         uint64_t rows, uint32_t d, oc64* out) {
#pragma omp parallel
  {
    oc64* tmp = (oc64*)malloc(d * sizeof(oc64));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
      const oc64* xr = x + (size_t)r * d;
      if (before) {
        const oc64* br = before + (size_t)r * d;
        for (uint32_t i = 0; i < d; ++i) tmp[i] = (oc64){xr[i].re + br[i].re, 0.0};
        xr = tmp;
      }
      orc_layernorm_row(xr, d, eps, gamma, beta, out + (size_t)r * d);
    }
    free(tmp);
  }
}

/* MaskedAttentionHead::forward for all heads + SelfAttentionLayer::forward
 * (masked_attention_head.rs:122-220, self_attention_layer.rs:55-133). */
static int self_attention_forward(orc_layer* L, const oc64* x, const uint32_t* mask, const uint32_t* lens,
                                  uint32_t B, uint32_t S, int forward_only, oc64* out, oc64* concat_out) {
  const uint32_t d = L->d_in, H = L->heads, dh = L->dh, mc = L->max_ctx;
  const int decode = forward_only && L->cache_valid;
  if (decode && B != L->cache_B) return fail(ORC_ERR_STATE, "cached batch %u != %u; reset first", L->cache_B, B);
  if (S > mc) return fail(ORC_ERR_ARG, "sequence %u exceeds max context %u", S, mc);
  if (decode)
    for (uint32_t b = 0; b < B; ++b)
      if (L->clen[b] + 1 > mc) return fail(ORC_ERR_ARG, "context %u exceeds max context %u", L->clen[b] + 1, mc);
  if (forward_only && !L->cache_valid) {
    free_cache(L);
    size_t cn = (size_t)H * B * mc * dh;
    L->kc = (oc64*)calloc(cn, sizeof(oc64));
    L->vc = (oc64*)calloc(cn, sizeof(oc64));
    L->clen = (uint32_t*)calloc(B, sizeof(uint32_t));
    if (!L->kc || !L->vc || !L->clen) return fail(ORC_ERR_NOMEM, "kv cache: out of memory");
    L->cache_B = B;
  }
  const double scale = 1.0 / (1e-8 + sqrt((double)dh)); /* scale_attention_scores :453-465 */
  const size_t wn = (size_t)d * dh;
  const uint32_t T_fresh = S;
  oc64* concat = (oc64*)malloc((size_t)B * S * d * sizeof(oc64));
  oc64* knew = NULL;
  oc64* vnew = NULL;
  if (!decode) {
    knew = (oc64*)malloc((size_t)H * B * S * dh * sizeof(oc64));
    vnew = (oc64*)malloc((size_t)H * B * S * dh * sizeof(oc64));
  }
  /* K/V: all rows without a cache (:135-139), else only the last token (:140-156) */
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t h = 0; h < (int64_t)H; ++h)
    for (int64_t b = 0; b < (int64_t)B; ++b) {
      const oc64* xb = x + (size_t)b * S * d;
      if (!decode) {
        zgemm_serial(S, dh, d, xb, L->wk + h * wn, knew + ((size_t)h * B + b) * S * dh);
        zgemm_serial(S, dh, d, xb, L->wv + h * wn, vnew + ((size_t)h * B + b) * S * dh);
      } else {
        const oc64* last = xb + (size_t)(lens[b] - 1) * d;
        size_t off = (((size_t)h * B + b) * mc + L->clen[b]) * dh;
        zgemm_row(dh, d, last, L->wk + h * wn, L->kc + off);
        zgemm_row(dh, d, last, L->wv + h * wn, L->vc + off);
      }
    }
  if (decode)
    for (uint32_t b = 0; b < B; ++b) L->clen[b] += 1;
  else if (forward_only) {
    /* the cache keeps each sequence's own lens[b] rows (:159-163) */
    for (uint32_t h = 0; h < H; ++h)
      for (uint32_t b = 0; b < B; ++b) {
        size_t src = ((size_t)h * B + b) * S * dh, dst = ((size_t)h * B + b) * mc * dh;
        memcpy(L->kc + dst, knew + src, (size_t)lens[b] * dh * sizeof(oc64));
        memcpy(L->vc + dst, vnew + src, (size_t)lens[b] * dh * sizeof(oc64));
      }
    for (uint32_t b = 0; b < B; ++b) L->clen[b] = lens[b];
    L->cache_valid = 1;
  }
#pragma omp parallel
  {
    oc64* q = (oc64*)malloc((size_t)S * dh * sizeof(oc64));
    double* sc = (double*)malloc((size_t)mc * sizeof(double));
#pragma omp for collapse(2) schedule(dynamic)
    for (int64_t h = 0; h < (int64_t)H; ++h)
      for (int64_t b = 0; b < (int64_t)B; ++b) {
        const oc64* xb = x + (size_t)b * S * d;
        zgemm_serial(S, dh, d, xb, L->wq + h * wn, q); /* :132 */
        const oc64 *K, *V;
        uint32_t T;
        if (decode) {
          K = L->kc + ((size_t)h * B + b) * mc * dh;
          V = L->vc + ((size_t)h * B + b) * mc * dh;
          T = L->clen[b];
        } else {
          K = knew + ((size_t)h * B + b) * S * dh;
          V = vnew + ((size_t)h * B + b) * S * dh;
          T = T_fresh;
        }
        const oc64* bp = L->bias_pos + (size_t)h * mc * mc;
        for (uint32_t r = 0; r < S; ++r) {
          oc64* o = concat + ((size_t)b * S + r) * d + (size_t)h * dh;
          if (mask[(size_t)b * S + r] == 0) { /* softmax_complex_padding_real :369-388 */
            for (uint32_t e = 0; e < dh; ++e) o[e] = (oc64){0.0, 0.0};
            continue;
          }
          const oc64* qr = q + (size_t)r * dh;
          /* scores (:190-196): Re(q.k^T) * scale + bias_pos[r][c]; the causal
           * mask of S x S rows is applied modulo its size (:494-503) */
          for (uint32_t c = 0; c < T; ++c) {
            if ((c % S) > r) {
              sc[c] = -1e12;
              continue;
            }
            sc[c] = score_dot(dh, qr, K + (size_t)c * dh) * scale + bp[(size_t)r * mc + c].re;
          }
          double mx = -INFINITY;
          for (uint32_t c = 0; c < T; ++c) mx = fmax(mx, sc[c]);
          double sum = 0.0;
          for (uint32_t c = 0; c < T; ++c) {
            sc[c] = exp(sc[c] - mx);
            sum += sc[c];
          }
          for (uint32_t c = 0; c < T; ++c) sc[c] = sc[c] / sum;
          /* multiply_f64_complex (utils/matrix.rs:356-380) */
          for (uint32_t e = 0; e < dh; ++e) {
            oc64 acc = {0.0, 0.0};
            for (uint32_t c = 0; c < T; ++c) acc = c_add(acc, c_scale(V[(size_t)c * dh + e], sc[c]));
            o[e] = acc;
          }
        }
      }
    free(q);
    free(sc);
  }
  /* residual + LayerNorm (:101-124); the heads' output alone on request */
  if (concat_out) memcpy(concat_out, concat, (size_t)B * S * d * sizeof(oc64));
  if (out) norm_forward(L->eps, L->gamma, L->beta, concat, x, (uint64_t)B * S, d, out);
  free(concat);
  free(knew);
  free(vnew);
  return ORC_OK;
}

static int check_finite(const oc64* y, uint64_t n, const char* what) {
  for (uint64_t i = 0; i < n; ++i)
    if (!isfinite(y[i].re) || !isfinite(y[i].im)) return fail(ORC_ERR_NAN, "%s: The value is Not Valid", what);
  return ORC_OK;
}

/* FeedForwardLayer::forward (feedforward_layer.rs:56-138): Dense(GELU) with
 * pad rows zeroed (layer.rs:132-166, activation.rs:268-284), then Linear. */
static int ffn_forward(const orc_layer* L, const oc64* x, const uint32_t* mask, uint64_t rows, oc64* out) {
  const uint32_t d = L->d_in, F = L->hidden;
  int nan_flag = 0;
#pragma omp parallel
  {
    oc64* h = (oc64*)malloc((size_t)F * sizeof(oc64));
    int local_nan = 0;
#pragma omp for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
      zgemm_row(F, d, x + (size_t)r * d, L->w1, h);
      for (uint32_t j = 0; j < F; ++j) {
        oc64 z = c_add(h[j], L->b1[j]); /* add_vector */
        h[j] = (!mask || mask[r]) ? gelu_c(z, &local_nan) : (oc64){0.0, 0.0};
      }
      oc64* o = out + (size_t)r * d;
      zgemm_row(d, F, h, L->w2, o);
      for (uint32_t j = 0; j < d; ++j) o[j] = c_add(o[j], L->b2[j]);
    }
    if (local_nan) {
#pragma omp atomic write
      nan_flag = 1;
    }
    free(h);
  }
  if (nan_flag) return fail(ORC_ERR_NAN, "NaN detected in tanh(f(z))");
  return check_finite(out, rows * d, "output ffn dense"); /* transformer_network.rs:408 */
}

/* LinearLayer::forward (linear_layer.rs:55-75) */
static void linear_forward(const orc_layer* L, const oc64* x, uint64_t rows, oc64* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)rows; ++r) {
    oc64* o = out + (size_t)r * L->d_out;
    zgemm_row(L->d_out, L->d_in, x + (size_t)r * L->d_in, L->w1, o);
    for (uint32_t j = 0; j < L->d_out; ++j) o[j] = c_add(o[j], L->b1[j]);
  }
}

/* Runs one hidden-state layer in place-or-swap. */
static int run_layer(orc_layer* L, oc64** cur, oc64** nxt, uint64_t* cap, const uint32_t* mask, const uint32_t* lens,
                     uint32_t B, uint32_t S, const uint32_t* ts, int forward_only) {
  const uint64_t rows = (uint64_t)B * S;
  if (L->kind == ORC_POSITIONAL_ENCODING) {
    posenc_forward(L, *cur, B, S, ts, forward_only);
    return ORC_OK;
  }
  uint64_t need = rows * (L->d_out > L->d_in ? L->d_out : L->d_in);
  if (need > *cap) {
    free(*nxt);
    *nxt = (oc64*)malloc(need * sizeof(oc64));
    if (!*nxt) return fail(ORC_ERR_NOMEM, "activation: out of memory");
    *cap = need;
  }
  int rc = ORC_OK;
  switch (L->kind) {
    case ORC_NORM: norm_forward(L->eps, L->gamma, L->beta, *cur, NULL, rows, L->d_in, *nxt); break;
    case ORC_SELF_ATTENTION: rc = self_attention_forward(L, *cur, mask, lens, B, S, forward_only, *nxt, NULL); break;
    case ORC_FEED_FORWARD: rc = ffn_forward(L, *cur, mask, rows, *nxt); break;
    case ORC_LINEAR: linear_forward(L, *cur, rows, *nxt); break;
    default: return fail(ORC_ERR_ARG, "layer kind %d is not a hidden-state layer", L->kind);
  }
  oc64* t = *cur;
  *cur = *nxt;
  *nxt = t;
  /* both buffers must hold `need` after the swap */
  return rc;
}

static int check_lens(const uint32_t* lens, uint32_t B, uint32_t S) {
  if (!B || !S) return fail(ORC_ERR_ARG, "batch_ids is empty");
  for (uint32_t b = 0; b < B; ++b)
    if (lens[b] == 0 || lens[b] > S) return fail(ORC_ERR_ARG, "lens[%u]=%u outside [1,%u]", b, lens[b], S);
  return ORC_OK;
}

/* A wavelet layer at a prompt or stateless pass (wavelet_discrete_layer.rs:
 * 102-128): *cur [B][*S][d] becomes [B][S'][d], mask and lens follow. */
static int run_wavelet_split(const orc_layer* L, oc64** cur, oc64** nxt, uint64_t* cap, uint32_t** mask,
                             uint32_t* lens, uint32_t B, uint32_t* S, uint32_t d, uint32_t T);

/* DiscreteWaveletLayer::forward, partial mode (wavelet_discrete_layer.rs:72-161).
 * T > 0 (a stateless pass with T target rows): separate_input_target
 * (:233-279) keeps the first S - T rows as the input, whose compression is
 * followed by the T target rows unchanged, mask ones. */
static int run_wavelet(const orc_layer* L, oc64** cur, oc64** nxt, uint64_t* cap, uint32_t** mask, uint32_t* lens,
                       uint32_t B, uint32_t* S, uint32_t d, uint32_t T) {
  if (T) return run_wavelet_split(L, cur, nxt, cap, mask, lens, B, S, d, T);
  const uint32_t M = dwt_len(*S, L->vocab == 0 ? 2 : 4) >> 1;
  const uint64_t need = (uint64_t)B * (M > *S ? M : *S) * d;
  if (need > *cap) {
    oc64* c2 = (oc64*)realloc(*cur, need * sizeof(oc64));
    if (c2) *cur = c2;
    free(*nxt);
    *nxt = (oc64*)malloc(need * sizeof(oc64));
    if (!c2 || !*nxt) return fail(ORC_ERR_NOMEM, "wavelet: out of memory");
    *cap = need;
  }
  uint32_t* m2 = (uint32_t*)malloc((size_t)B * M * sizeof(uint32_t));
  if (!m2) return fail(ORC_ERR_NOMEM, "wavelet: out of memory");
  uint32_t S2 = 0;
  int rc = dwt_compress(L->vocab, (uint32_t)L->mode, *cur, *mask, B, *S, d, *nxt, m2, lens, &S2);
  if (rc) {
    free(m2);
    return rc;
  }
  free(*mask);
  *mask = m2;
  *S = S2;
  oc64* t = *cur;
  *cur = *nxt;
  *nxt = t;
  return ORC_OK;
}

static int run_wavelet_split(const orc_layer* L, oc64** cur, oc64** nxt, uint64_t* cap, uint32_t** mask,
                             uint32_t* lens, uint32_t B, uint32_t* S, uint32_t d, uint32_t T) {
  const uint32_t Sin = *S;
  if (T >= Sin) return fail(ORC_ERR_ARG, "%u target rows need more than %u rows", T, Sin);
  for (uint32_t b = 0; b < B; ++b)
    if (lens[b] != Sin)
      return fail(ORC_ERR_ARG, "target rows need unpadded sequences: separate_input_target "
                               "(wavelet_discrete_layer.rs:233-279) panics on padded ones");
  const uint32_t R = Sin - T, M = dwt_len(R, L->vocab == 0 ? 2 : 4) >> 1, S2 = M + T;
  oc64* xin = (oc64*)malloc((size_t)B * R * d * sizeof(oc64));
  oc64* comp = (oc64*)malloc((size_t)B * (M > R ? M : R) * d * sizeof(oc64));
  uint32_t* min = (uint32_t*)malloc((size_t)B * R * sizeof(uint32_t));
  uint32_t* m2 = (uint32_t*)malloc((size_t)B * S2 * sizeof(uint32_t));
  uint32_t* mc = (uint32_t*)malloc((size_t)B * M * sizeof(uint32_t));
  const uint64_t need = (uint64_t)B * (S2 > Sin ? S2 : Sin) * d;
  int rc = ORC_OK;
  if (!xin || !comp || !min || !m2 || !mc) {
    rc = fail(ORC_ERR_NOMEM, "wavelet: out of memory");
    goto done;
  }
  for (uint32_t b = 0; b < B; ++b) {
    memcpy(xin + (size_t)b * R * d, *cur + (size_t)b * Sin * d, (size_t)R * d * sizeof(oc64));
    for (uint32_t s = 0; s < R; ++s) min[(size_t)b * R + s] = 1u;
  }
  uint32_t Mo = 0;
  if ((rc = dwt_compress(L->vocab, (uint32_t)L->mode, xin, min, B, R, d, comp, mc, lens, &Mo))) goto done;
  if (need > *cap) {
    free(*nxt);
    *nxt = (oc64*)malloc(need * sizeof(oc64));
    oc64* c2 = (oc64*)realloc(*cur, need * sizeof(oc64));
    if (c2) *cur = c2;
    if (!*nxt || !c2) {
      rc = fail(ORC_ERR_NOMEM, "wavelet: out of memory");
      goto done;
    }
    *cap = need;
  }
  for (uint32_t b = 0; b < B; ++b) {
    memcpy(*nxt + (size_t)b * S2 * d, comp + (size_t)b * M * d, (size_t)M * d * sizeof(oc64));
    memcpy(*nxt + ((size_t)b * S2 + M) * d, *cur + ((size_t)b * Sin + R) * d, (size_t)T * d * sizeof(oc64));
    memcpy(m2 + (size_t)b * S2, mc + (size_t)b * M, M * sizeof(uint32_t));
    for (uint32_t t = 0; t < T; ++t) m2[(size_t)b * S2 + M + t] = 1u; /* :130-134 */
    lens[b] += T;
  }
  free(*mask);
  *mask = m2;
  m2 = NULL;
  *S = S2;
  {
    oc64* t = *cur;
    *cur = *nxt;
    *nxt = t;
  }
done:
  free(xin), free(comp), free(min), free(m2), free(mc);
  return rc;
}

void orc_set_target_rows(orc_net* net, uint32_t T) {
  if (net) net->train_T = T;
}

int orc_predict(orc_net* net, const uint32_t* ids, const uint32_t* lens_in, uint32_t B, uint32_t S_in,
                const uint32_t* time_steps, int forward_only, int out_rows, double* out, uint32_t* out_mask) {
  if (!net || !ids || !lens_in || !out) return fail(ORC_ERR_ARG, "null argument");
  int rc = check_lens(lens_in, B, S_in);
  if (rc) return rc;
  if (net->n < 2 || net->layers[0].kind != ORC_EMBEDDING || net->layers[net->n - 1].kind != ORC_SOFTMAX)
    return fail(ORC_ERR_STATE, "network must start with Embedding and end with Softmax");
  uint32_t S = S_in; /* rows per sequence: a wavelet layer compresses them */
  const uint64_t rows0 = (uint64_t)B * S;
  uint32_t dmax = 0;
  for (int i = 0; i < net->n; ++i) {
    if (net->layers[i].d_in > dmax) dmax = net->layers[i].d_in;
    if (net->layers[i].d_out > dmax) dmax = net->layers[i].d_out;
  }
  uint64_t cap = rows0 * dmax;
  oc64* cur = (oc64*)malloc(cap * sizeof(oc64));
  oc64* nxt = (oc64*)malloc(cap * sizeof(oc64));
  uint32_t* mask = (uint32_t*)malloc(rows0 * sizeof(uint32_t));
  uint32_t* lens = (uint32_t*)malloc(B * sizeof(uint32_t));
  if (!cur || !nxt || !mask || !lens) {
    free(cur), free(nxt), free(mask), free(lens);
    return fail(ORC_ERR_NOMEM, "activation: out of memory");
  }
  memcpy(lens, lens_in, B * sizeof(uint32_t));
  rc = embedding_forward(&net->layers[0], ids, lens, B, S, cur, mask);
  uint32_t d = net->layers[0].d_out;
  const int prompt_pass = !forward_only || !time_steps || time_steps[0] == 0;
  int gathered = 0; /* rows reduced to one per sequence before the vocab Linear */
  for (int li = 1; rc == ORC_OK && li < net->n - 1; ++li) {
    orc_layer* L = &net->layers[li];
    if (L->kind == ORC_DISCRETE_WAVELET) {
      if (prompt_pass) rc = run_wavelet(L, &cur, &nxt, &cap, &mask, lens, B, &S, d, forward_only ? 0 : net->train_T);
      continue; /* a cached step's row passes through (:112-128) */
    }
    if (out_rows == 1 && forward_only && L->kind == ORC_LINEAR && li == net->n - 2) {
      for (uint32_t b = 0; b < B; ++b)
        memmove(cur + (size_t)b * L->d_in, cur + ((size_t)b * S + lens[b] - 1) * L->d_in, L->d_in * sizeof(oc64));
      uint64_t need = (uint64_t)B * L->d_out;
      if (need > cap) {
        free(nxt);
        nxt = (oc64*)malloc(need * sizeof(oc64));
        oc64* c2 = (oc64*)realloc(cur, need * sizeof(oc64));
        if (!nxt || !c2) {
          rc = fail(ORC_ERR_NOMEM, "logits: out of memory");
          break;
        }
        cur = c2;
        cap = need;
      }
      linear_forward(L, cur, B, nxt);
      oc64* t = cur;
      cur = nxt;
      nxt = t;
      gathered = 1;
      continue;
    }
    if (L->kind == ORC_EMBEDDING || L->kind == ORC_SOFTMAX) {
      rc = fail(ORC_ERR_STATE, "unexpected layer kind %d inside the stack", L->kind);
      break;
    }
    rc = run_layer(L, &cur, &nxt, &cap, mask, lens, B, S, time_steps, forward_only);
    if (L->d_out) d = L->d_out;
  }
  if (rc == ORC_OK) {
    const orc_layer* SM = &net->layers[net->n - 1];
    uint32_t V = net->layers[net->n - 2].d_out;
    uint32_t out_S = gathered ? 1 : S;
    /* Softmax arm of predict (:472-489) */
    const uint32_t n_out = out_rows == 1 ? 1 : S;
    for (uint32_t b = 0; b < B; ++b) {
      for (uint32_t k = 0; k < n_out; ++k) {
        const uint32_t src_s = out_rows == 1 ? lens[b] - 1 : k; /* row in the padded batch */
        const oc64* row = gathered ? cur + (size_t)b * V : cur + ((size_t)b * out_S + src_s) * V;
        double* o = out + ((size_t)b * n_out + k) * V;
        if (forward_only) { /* convert_c_to_f64_3d (src/utils/data_converter.rs:244-256) */
          for (uint32_t v = 0; v < V; ++v) o[v] = row[v].re;
        } else if (SM->mode == ORC_TRAINING) { /* softmax_complex_padding_real */
          if (mask[(size_t)b * S + src_s] == 0)
            for (uint32_t v = 0; v < V; ++v) o[v] = 0.0;
          else
            orc_softmax_row_real(row, V, o);
        } else { /* softmax_last_row (activation.rs:409-419): only row S-1 */
          if (src_s == S - 1)
            orc_softmax_row_real(row, V, o);
          else
            for (uint32_t v = 0; v < V; ++v) o[v] = 0.0;
        }
      }
    }
    if (out_mask) memcpy(out_mask, mask, (size_t)B * S * sizeof(uint32_t));
  }
  free(cur);
  free(nxt);
  free(mask);
  free(lens);
  return rc;
}

int orc_forward_layers(orc_net* net, uint32_t first, uint32_t last, const oc64* in, const uint32_t* mask_in,
                       uint32_t B, uint32_t S, const uint32_t* time_steps, int forward_only, oc64* out) {
  /* S: rows per sequence in; a wavelet layer in the range compresses them (out [B][S'][d]) */
  if (!net || !in || !out || first >= last || last > (uint32_t)net->n) return fail(ORC_ERR_ARG, "bad layer range");
  if (!B || !S) return fail(ORC_ERR_ARG, "empty batch");
  const uint64_t rows = (uint64_t)B * S;
  uint32_t dmax = 0;
  for (uint32_t i = first; i < last; ++i) {
    if (net->layers[i].d_in > dmax) dmax = net->layers[i].d_in;
    if (net->layers[i].d_out > dmax) dmax = net->layers[i].d_out;
  }
  uint64_t cap = rows * dmax;
  oc64* cur = (oc64*)malloc(cap * sizeof(oc64));
  oc64* nxt = (oc64*)malloc(cap * sizeof(oc64));
  uint32_t* mask = (uint32_t*)malloc(rows * sizeof(uint32_t));
  uint32_t* lens = (uint32_t*)malloc(B * sizeof(uint32_t));
  int rc = ORC_OK;
  if (!cur || !nxt || !mask || !lens) rc = fail(ORC_ERR_NOMEM, "activation: out of memory");
  if (rc == ORC_OK) {
    memcpy(cur, in, rows * net->layers[first].d_in * sizeof(oc64));
    for (uint32_t b = 0; b < B; ++b) {
      lens[b] = 0;
      for (uint32_t s = 0; s < S; ++s) {
        mask[(size_t)b * S + s] = mask_in ? mask_in[(size_t)b * S + s] : 1;
        lens[b] += mask[(size_t)b * S + s] ? 1 : 0;
      }
      if (!lens[b]) lens[b] = 1;
    }
  }
  const int prompt_pass = !forward_only || !time_steps || time_steps[0] == 0;
  uint32_t d = net->layers[first].d_in;
  for (uint32_t li = first; rc == ORC_OK && li < last; ++li) {
    orc_layer* L = &net->layers[li];
    if (L->kind == ORC_DISCRETE_WAVELET) {
      if (prompt_pass) rc = run_wavelet(L, &cur, &nxt, &cap, &mask, lens, B, &S, d, forward_only ? 0 : net->train_T);
      continue;
    }
    rc = run_layer(L, &cur, &nxt, &cap, mask, lens, B, S, time_steps, forward_only);
    if (L->d_out) d = L->d_out;
  }
  if (rc == ORC_OK) memcpy(out, cur, (size_t)B * S * d * sizeof(oc64));
  free(cur);
  free(nxt);
  free(mask);
  free(lens);
  return rc;
}

int orc_generate(orc_net* net, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S,
                 uint32_t n_new, uint32_t* out_ids, double* out_logits) {
  if (!net || !prompt || !lens || !out_ids) return fail(ORC_ERR_ARG, "null argument");
  int rc = check_lens(lens, B, S);
  if (rc) return rc;
  if (n_new == 0) return ORC_OK;
  if (net->n < 2) return fail(ORC_ERR_STATE, "empty network");
  const uint32_t V = net->layers[net->n - 2].d_out;
  double* logits = (double*)malloc((size_t)B * V * sizeof(double));
  uint32_t* ids = (uint32_t*)malloc(B * sizeof(uint32_t));
  uint32_t* ones = (uint32_t*)malloc(B * sizeof(uint32_t));
  uint32_t* ts = (uint32_t*)malloc(B * sizeof(uint32_t));
  if (!logits || !ids || !ones || !ts) rc = fail(ORC_ERR_NOMEM, "generate: out of memory");
  if (rc == ORC_OK) rc = orc_reset(net); /* predict_by_text reloads the model per request (:638-652) */
  for (uint32_t t = 0; rc == ORC_OK && t < n_new; ++t) {
    if (t == 0) {
      rc = orc_predict(net, prompt, lens, B, S, NULL, 1, 1, logits, NULL);
    } else {
      for (uint32_t b = 0; b < B; ++b) {
        ones[b] = 1;
        ts[b] = lens[b] + t - 1; /* time_step of the fed token (:300-304) */
      }
      rc = orc_predict(net, ids, ones, B, 1, ts, 1, 1, logits, NULL);
    }
    if (rc) break;
    for (uint32_t b = 0; b < B; ++b) {
      int64_t id = orc_greedy_row(logits + (size_t)b * V, V);
      if (id < 0) {
        rc = fail(ORC_ERR_NAN, "greedy_decoding: NaN in logits");
        break;
      }
      ids[b] = (uint32_t)id;
      out_ids[(size_t)b * n_new + t] = (uint32_t)id;
    }
    if (out_logits) memcpy(out_logits + (size_t)t * B * V, logits, (size_t)B * V * sizeof(double));
  }
  free(logits);
  free(ids);
  free(ones);
  free(ts);
  return rc;
}

/* ======================================================================
 * The output head's training step: SoftmaxLayer::backward, LinearLayer::
 * backward and LinearLayer::update_parameters with the AdamW of
 * utils/adam_w.rs.  Parity anchors: the closed forms in
 * tests/test_oracle_pins.py (cross-entropy gradient rows summing to zero and
 * matching finite differences of the loss, the first AdamW step, the clipped
 * descent step, dW against an explicit sum of outer products).
 * ====================================================================== */

int orc_softmax_backward(const double* P, uint32_t B, uint32_t S, uint32_t V, const uint32_t* targets,
                         const uint32_t* tlens, uint32_t T, double* G) {
  if (!P || !targets || !tlens || !G || !B || !S || !V) return fail(ORC_ERR_ARG, "bad arguments");
  memset(G, 0, (size_t)B * S * V * sizeof(double));
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t tl = tlens[b];
    if (tl > T) return fail(ORC_ERR_ARG, "target length %u > %u", tl, T);
    /* seq_ind_start = len - target_len - 1 in usize (softmax_output_layer.rs:95-96) */
    if ((uint64_t)tl + 1 > S) return fail(ORC_ERR_ARG, "sequence %u: %u targets need more than %u rows", b, tl, S);
    const uint32_t start = S - tl - 1, end = S - 1;
    double unpadded = 0.0; /* targets that are not PAD (:98-103) */
    for (uint32_t t = 0; t < tl; ++t)
      if (targets[(size_t)b * T + t] != 1) unpadded += 1.0;
    const double normalizer = (double)B * unpadded;
    for (uint32_t t = 0; t < tl; ++t) {
      const uint32_t tc = targets[(size_t)b * T + t];
      if (tc >= V) return fail(ORC_ERR_ARG, "target token %u exceeds vocabulary %u", tc, V); /* :108-110 */
      if (tc == 1) continue;                                                                  /* :112-114 */
      const uint32_t s = start + t;
      if (s >= end) break; /* :118-120 */
      const double* p = P + ((size_t)b * S + s) * V;
      double* g = G + ((size_t)b * S + s) * V;
      for (uint32_t c = 0; c < V; ++c) g[c] += (c == tc ? p[c] - 1.0 : p[c]) / normalizer;
    }
  }
  return ORC_OK;
}

/* cross_entropy_loss_batch (transformer_network.rs:662-676) and
 * cross_entropy_loss (:678-711): per sequence, -ln(p + 1e-15) of each non-PAD
 * target's probability at row len - target_len - 1 + t, summed in target
 * order and divided by their count; then the sequences summed in order, as
 * Complex<f64> with im 0, divided by the batch size.  out[2] = (re, im).
 * The padding mask the reference passes is not read there (only counted). */
int orc_cross_entropy_loss_batch(const double* P, uint32_t B, uint32_t S, uint32_t V, const uint32_t* targets,
                                 const uint32_t* tlens, uint32_t T, double* out) {
  if (!P || !targets || !tlens || !out || !B || !S || !V) return fail(ORC_ERR_ARG, "bad arguments");
  double re = 0.0, im = 0.0;
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t tl = tlens[b];
    if (tl > T) return fail(ORC_ERR_ARG, "target length %u > %u", tl, T);
    /* seq_ind_start = predictions.len() - target_len - 1 in usize (:692) */
    if ((uint64_t)tl + 1 > S) return fail(ORC_ERR_ARG, "sequence %u: %u targets need more than %u rows", b, tl, S);
    const uint32_t start = S - tl - 1, end = S - 1;
    double loss = 0.0, count = 0.0;
    for (uint32_t t = 0; t < tl; ++t) {
      const uint32_t tc = targets[(size_t)b * T + t];
      if (tc == 1) continue; /* :697-699 */
      const uint32_t s = start + t;
      if (s >= end) break; /* :701-704 */
      if (tc >= V) return fail(ORC_ERR_ARG, "target token %u exceeds vocabulary %u", tc, V); /* indexing panics */
      loss += -log(P[((size_t)b * S + s) * V + tc] + 1e-15);                               /* :706-708 */
      count += 1.0;
    }
    re += loss / count; /* total_loss += f64 adds to the real part */
  }
  out[0] = re / (double)B;
  out[1] = im / (double)B;
  return ORC_OK;
}

int orc_linear_backward_c(const oc64* X, const oc64* Gin, const oc64* W, uint32_t B, uint32_t S, uint32_t d,
                          uint32_t V, oc64* dW, oc64* db, oc64* dX);

int orc_linear_backward(const oc64* X, const double* G, const oc64* W, uint32_t B, uint32_t S, uint32_t d,
                        uint32_t V, oc64* dW, oc64* db, oc64* dX) {
  if (!G || !B || !S || !V) return fail(ORC_ERR_ARG, "bad arguments");
  oc64* gc = (oc64*)malloc((size_t)B * S * V * sizeof(oc64)); /* the gradient as Complex (im 0) */
  if (!gc) return fail(ORC_ERR_NOMEM, "linear backward: out of memory");
  for (size_t i = 0; i < (size_t)B * S * V; ++i) gc[i] = (oc64){G[i], 0.0};
  const int rc = orc_linear_backward_c(X, gc, W, B, S, d, V, dW, db, dX);
  free(gc);
  return rc;
}

int orc_linear_backward_c(const oc64* X, const oc64* Gin, const oc64* W, uint32_t B, uint32_t S, uint32_t d,
                          uint32_t V, oc64* dW, oc64* db, oc64* dX) {
  if (!X || !Gin || !W || !dW || !db || !dX || !B || !S || !d || !V) return fail(ORC_ERR_ARG, "bad arguments");
  oc64* xh = (oc64*)malloc((size_t)d * S * sizeof(oc64));   /* conjugate_transpose(input_sample) */
  oc64* gc = (oc64*)malloc((size_t)S * V * sizeof(oc64));   /* one sequence's gradient */
  oc64* wh = (oc64*)malloc((size_t)V * d * sizeof(oc64));   /* conjugate_transpose(weights) */
  oc64* wg = (oc64*)malloc((size_t)d * V * sizeof(oc64));   /* one sequence's weight gradient */
  if (!xh || !gc || !wh || !wg) {
    free(xh), free(gc), free(wh), free(wg);
    return fail(ORC_ERR_NOMEM, "linear backward: out of memory");
  }
  for (uint32_t k = 0; k < d; ++k)
    for (uint32_t v = 0; v < V; ++v) {
      const oc64 w = W[(size_t)k * V + v];
      wh[(size_t)v * d + k] = (oc64){w.re, -w.im};
    }
  memset(dW, 0, (size_t)d * V * sizeof(oc64));
  memset(db, 0, (size_t)V * sizeof(oc64));
  for (uint32_t b = 0; b < B; ++b) {
    const oc64* xb = X + (size_t)b * S * d;
    for (uint32_t s = 0; s < S; ++s)
      for (uint32_t k = 0; k < d; ++k) {
        const oc64 x = xb[(size_t)s * d + k];
        xh[(size_t)k * S + s] = (oc64){x.re, -x.im};
      }
    memcpy(gc, Gin + (size_t)b * S * V, (size_t)S * V * sizeof(oc64));
    orc_zgemm(d, V, S, xh, gc, wg);                                 /* linear_layer.rs:99 */
    for (size_t i = 0; i < (size_t)d * V; ++i) dW[i] = c_add(dW[i], wg[i]); /* group_gradient_batch */
    oc64 bsum; /* bias gradient of this sequence (:101-105), then grouped */
    for (uint32_t v = 0; v < V; ++v) {
      bsum = (oc64){0.0, 0.0};
      for (uint32_t s = 0; s < S; ++s) bsum = c_add(bsum, gc[(size_t)s * V + v]);
      db[v] = c_add(db[v], bsum);
    }
    orc_zgemm(S, d, V, gc, wh, dX + (size_t)b * S * d);           /* :107 */
  }
  free(xh), free(gc), free(wh), free(wg);
  return ORC_OK;
}

/* f64::powi as compiler-rt's __powidf2: square-and-multiply over the bits */
static double powi_f64(double a, int e) {
  const int recip = e < 0;
  double r = 1.0;
  for (;;) {
    if (e & 1) r *= a;
    e /= 2;
    if (e == 0) break;
    a *= a;
  }
  return recip ? 1.0 / r : r;
}

/* clip_gradient_1d on one value (utils/matrix.rs:709-717) */
static oc64 clip1(oc64 g, double threshold) {
  const double n = hypot(g.re, g.im);
  return n > threshold ? c_scale(g, threshold / n) : g;
}

static int finite_c(oc64 z) { return isfinite(z.re) && isfinite(z.im); }

/* calculate_adam_w / calculate_adam_w_bias on one element (adam_w.rs:9-103);
 * weights take v_hat's norm at least EPSILON, the bias does not */
static oc64 adamw1(oc64 w, oc64 g, oc64* m, oc64* v, double lr, uint32_t ts, int weight) {
  const double B1 = 0.9, B2 = 0.999, EPS = 1e-8, WD = 0.01, MAX_NORM = 1.0;
  const int t = ts > 0 ? (int)ts : 1;
  const double gn = hypot(g.re, g.im);
  if (gn > MAX_NORM) g = c_scale(g, MAX_NORM / gn);
  *m = c_add(c_scale(*m, B1), c_scale(g, 1.0 - B1));
  *v = c_add(c_scale(*v, B2), c_mul(c_scale(g, 1.0 - B2), (oc64){g.re, -g.im}));
  const oc64 mh = c_unscale(*m, 1.0 - powi_f64(B1, t));
  const oc64 vh = c_unscale(*v, 1.0 - powi_f64(B2, t));
  double vn = hypot(vh.re, vh.im);
  if (weight) vn = fmax(vn, EPS);
  const double alr = lr / (sqrt(vn) + EPS);
  const oc64 decayed = c_scale(w, 1.0 - lr * WD);
  return c_sub(decayed, c_mul((oc64){alr, 0.0}, mh));
}

int orc_linear_update(oc64* W, oc64* b, uint32_t d, uint32_t V, const oc64* dW, const oc64* db, uint32_t batch,
                      oc64* mW, oc64* vW, oc64* mb, oc64* vb, int first, double lr, uint32_t time_step) {
  if (!W || !b || !dW || !db || !mW || !vW || !mb || !vb || !d || !V || !batch) return fail(ORC_ERR_ARG, "bad arguments");
  const size_t n = (size_t)d * V;
  const double bs = (double)batch;
  if (first) { /* linear_layer.rs:159-174: the clipped copies, gradient descent; the
                  moments it stores are the zeros of :141-145 (:176-180) */
    memset(mW, 0, n * sizeof(oc64));
    memset(vW, 0, n * sizeof(oc64));
    memset(mb, 0, V * sizeof(oc64));
    memset(vb, 0, V * sizeof(oc64));
    for (size_t i = 0; i < n; ++i) {
      const oc64 g = clip1(dW[i], 1.0);
      if (finite_c(g)) W[i] = c_sub(W[i], c_scale(c_unscale(g, bs), lr));
    }
    for (uint32_t j = 0; j < V; ++j) {
      const oc64 g = clip1(db[j], 1.0);
      if (finite_c(g)) b[j] = c_sub(b[j], c_scale(c_unscale(g, bs), lr));
    }
    return ORC_OK;
  }
  /* :150-158: AdamW on the grouped (unclipped) gradients */
  for (size_t i = 0; i < n; ++i) W[i] = adamw1(W[i], dW[i], &mW[i], &vW[i], lr, time_step, 1);
  for (uint32_t j = 0; j < V; ++j) b[j] = adamw1(b[j], db[j], &mb[j], &vb[j], lr, time_step, 0);
  return ORC_OK;
}

/* gelu_derivative_complex (utils/derivative.rs:48-84) */
oc64 orc_gelu_derivative(oc64 z) {
  const double s2p = sqrt(2.0 / M_PI);
  const oc64 one = {1.0, 0.0};
  const oc64 x3 = c_mul(z, c_mul(z, z)); /* powi(3) */
  const oc64 fx = c_scale(c_add(z, c_mul((oc64){0.044715, 0.0}, x3)), s2p);
  const int sat = hypot(fx.re, fx.im) > 20.0;
  const oc64 th = sat ? one : c_tanh(fx);
  const oc64 sech2 = sat ? (oc64){0.0, 0.0} : c_sub(one, c_mul(th, th)); /* 1 - tanh^2 (powi(2)) */
  const oc64 fp = c_scale(c_add(one, c_mul((oc64){0.134145, 0.0}, c_mul(z, z))), s2p);
  const oc64 d = c_add(c_mul((oc64){0.5, 0.0}, c_add(one, th)),
                       c_mul(c_mul(c_mul((oc64){0.5, 0.0}, z), sech2), fp));
  const double n = hypot(d.re, d.im);
  if (n > 1e6) return c_mul(c_unscale(d, n), (oc64){1e6, 0.0});
  if (n < 1e-12) return (oc64){1e-12, 0.0};
  return d;
}

/* Layer::backward for the Dense (GELU) layer (network_components/layer.rs:168-210):
 * prev [B][S][F] with padded rows zeroed (apply_padding_mask_batch), times
 * conj(GELU'(Z)) elementwise, then the products of the linear arm */
int orc_dense_backward(const oc64* X, const oc64* Z, const oc64* prev, const uint32_t* mask, const oc64* W,
                       uint32_t B, uint32_t S, uint32_t d, uint32_t F, oc64* dW, oc64* db, oc64* dX) {
  if (!X || !Z || !prev || !mask || !W || !B || !S || !d || !F) return fail(ORC_ERR_ARG, "bad arguments");
  const size_t n = (size_t)B * S * F;
  oc64* g = (oc64*)malloc(n * sizeof(oc64));
  if (!g) return fail(ORC_ERR_NOMEM, "dense backward: out of memory");
  for (size_t r = 0; r < (size_t)B * S; ++r)
    for (uint32_t j = 0; j < F; ++j) {
      const size_t i = r * F + j;
      if (mask[r] == 0) {
        g[i] = (oc64){0.0, 0.0};
      } else {
        const oc64 dz = orc_gelu_derivative(Z[i]);
        g[i] = c_mul(prev[i], (oc64){dz.re, -dz.im}); /* hadamard with transpose(conjugate_transpose) */
      }
    }
  const int rc = orc_linear_backward_c(X, g, W, B, S, d, F, dW, db, dX);
  free(g);
  return rc;
}

/* ======================================================================
 * The rest of backward's reverse walk (transformer_network.rs:506-636):
 * NormalNormLayer::backward, MaskedAttentionHead::backward for every head
 * under SelfAttentionLayer::backward, PositionalEncodingLayer::backward,
 * EmbeddingLayer::update_parameters, and the updates of the attention layer.
 * Parity anchors (tests/test_oracle_pins.py): the heads' gradients against
 * finite differences of a real loss in every real coordinate; RoPE's
 * backward as the adjoint of its forward; the Norm backward only through its
 * structure (real rows, linear plus quadratic in the incoming gradient), as
 * the formula is the reference's own and no closed form fixes it; the
 * embedding update through its one-hot reach and the normalized rows.
 * ====================================================================== */

/* Complex::powf (num-complex 0.4.6): from_polar(r^e, theta * e) */
static oc64 c_powf(oc64 z, double e) {
  if (e == 0.0) return (oc64){1.0, 0.0};
  const double r = pow(hypot(z.re, z.im), e), th = atan2(z.im, z.re) * e;
  return (oc64){r * cos(th), r * sin(th)};
}

/* f64 / Complex (num-complex 0.4.6): a (c - i d) / (c c + d d) */
static oc64 r_div_c(double a, oc64 z) {
  const double ns = z.re * z.re + z.im * z.im;
  return (oc64){a * z.re / ns, -a * z.im / ns};
}

/* NormalNormLayer::backward, Complex arm (norm_layer.rs:132-209), one row at a
 * time as the reference loops: x the layer's input row, its forward recomputed
 * (normalize, :64-82) for x_hat, mean and variance.  dgamma / dbeta receive
 * the row's contribution (added in, so the caller zeroes them first). */
static void norm_backward_row(const oc64* x, uint32_t n, double eps_fwd, const oc64* gamma, const oc64* beta,
                              const oc64* dout, oc64* dx, oc64* dgamma, oc64* dbeta, oc64* xhat) {
  orc_layernorm_row(x, n, eps_fwd, gamma, beta, xhat);
  const double len = (double)n;
  oc64 sum = {0.0, 0.0};
  for (uint32_t i = 0; i < n; ++i) sum = c_add(sum, x[i]);
  const oc64 mu = c_unscale(sum, len);
  oc64 vs = {0.0, 0.0};
  for (uint32_t i = 0; i < n; ++i) {
    const oc64 t = c_sub(x[i], mu);
    vs = c_add(vs, c_mul(t, t));
  }
  const oc64 var = c_add(c_unscale(vs, len), (oc64){1e-8, 0.0}); /* var_batch + eps (:158-159) */
  const oc64 std_inv = r_div_c(1.0, c_sqrt(var));
  const oc64 vpm32 = r_div_c(1.0, c_powf(var, 1.5));
  const oc64 neg_std_inv = {-std_inv.re, -std_inv.im};
  for (uint32_t j = 0; j < n; ++j) dx[j] = (oc64){0.0, 0.0};
  for (uint32_t f = 0; f < n; ++f) {
    oc64 dvar_sum = {0.0, 0.0}, dmu_sum = {0.0, 0.0}, dxmm_sum = {0.0, 0.0};
    for (uint32_t d = 0; d < n; ++d) {
      const oc64 dxm = c_sub(x[d], mu);
      dgamma[d] = c_add(dgamma[d], c_mul(dout[d], xhat[d]));
      dbeta[d] = c_add(dbeta[d], dout[d]);
      const oc64 dxhat = c_mul(dout[d], gamma[f]);
      dvar_sum = c_add(dvar_sum, c_mul(c_scale(c_mul(dxhat, dxm), -0.5), vpm32));
      dxmm_sum = c_add(dxmm_sum, c_unscale(c_scale(dxm, -2.0), len));
    }
    for (uint32_t d = 0; d < n; ++d) dmu_sum = c_add(dmu_sum, c_mul(dout[d], neg_std_inv));
    const oc64 dxhat = c_mul(dout[f], gamma[f]);
    const oc64 dmu = c_add(c_mul(dmu_sum, gamma[f]), c_mul(dvar_sum, dxmm_sum));
    const oc64 g = c_add(c_add(c_mul(dxhat, std_inv), c_mul(dvar_sum, c_unscale(c_scale(c_sub(x[f], mu), 2.0), len))),
                         c_unscale(dmu, len));
    for (uint32_t j = 0; j < n; ++j) {
      const oc64 t = c_add(c_scale(g, j == f ? 1.0 : 0.0), c_mul(g, dout[j]));
      dx[j] = c_add(dx[j], (oc64){t.re, 0.0});
    }
  }
}

int orc_norm_backward(const oc64* x, uint64_t rows, uint32_t n, double eps, const oc64* gamma, const oc64* beta,
                      const oc64* dout, oc64* dx, oc64* dgamma, oc64* dbeta) {
  if (!x || !gamma || !beta || !dout || !dx || !dgamma || !dbeta || !rows || !n) return fail(ORC_ERR_ARG, "bad arguments");
  oc64* xhat = (oc64*)malloc((size_t)n * sizeof(oc64));
  if (!xhat) return fail(ORC_ERR_NOMEM, "norm backward: out of memory");
  memset(dgamma, 0, (size_t)n * sizeof(oc64));
  memset(dbeta, 0, (size_t)n * sizeof(oc64));
  for (uint64_t r = 0; r < rows; ++r)
    norm_backward_row(x + r * n, n, eps, gamma, beta, dout + r * n, dx + r * n, dgamma, dbeta, xhat);
  free(xhat);
  return ORC_OK;
}

/* multiply_complex_with_f64 (utils/matrix.rs:328-354): complex [m][k] x real [k][n] */
static void zgemm_cr(uint32_t m, uint32_t n, uint32_t k, const oc64* A, const double* Bm, oc64* C) {
  for (uint32_t i = 0; i < m; ++i)
    for (uint32_t j = 0; j < n; ++j) {
      oc64 acc = {0.0, 0.0};
      for (uint32_t t = 0; t < k; ++t) acc = c_add(acc, c_scale(A[(size_t)i * k + t], Bm[(size_t)t * n + j]));
      C[(size_t)i * n + j] = acc;
    }
}

/* out[c][r] = conj?(in[r][c]) */
static void ztrans(uint32_t R, uint32_t C, const oc64* in, int conj, oc64* out) {
  for (uint32_t r = 0; r < R; ++r)
    for (uint32_t c = 0; c < C; ++c) {
      const oc64 v = in[(size_t)r * C + c];
      out[(size_t)c * R + r] = conj ? (oc64){v.re, -v.im} : v;
    }
}

/* MaskedAttentionHead::backward of every head for one batch of rows
 * (masked_attention_head.rs:222-345), the heads' input gradients summed in
 * head order (self_attention_layer.rs:160-190).  X [B][S][d] the layer's
 * input; Gc [B][S][d] the gradient of the heads' concatenated output, head h
 * in columns h*dh.. (split_gradient_into_heads, :232-258).  The weight and
 * bias gradients are grouped over the batch (gradient_struct.rs:400-411). */
int orc_attention_heads_backward(const oc64* X, uint32_t B, uint32_t S, const uint32_t* mask, uint32_t H, uint32_t d,
                                 uint32_t mc, const oc64* wq, const oc64* wk, const oc64* wv, const oc64* bias_pos,
                                 const oc64* Gc, oc64* dX, oc64* dwq, oc64* dwk, oc64* dwv, oc64* dbias) {
  if (!X || !mask || !wq || !wk || !wv || !bias_pos || !Gc || !dX || !dwq || !dwk || !dwv || !dbias || !B || !S || !H ||
      !d || d % H || S > mc)
    return fail(ORC_ERR_ARG, "bad arguments");
  const uint32_t dh = d / H;
  const size_t wn = (size_t)d * dh;
  const double c = 1.0 / (1e-8 + sqrt((double)dh)); /* scale_attention_scores with d_k = dh */
  const size_t SS = (size_t)S * S, Sd = (size_t)S * dh, dS = (size_t)d * S;
  oc64 *q = malloc(Sd * 16), *k = malloc(Sd * 16), *v = malloc(Sd * 16), *g = malloc(Sd * 16), *gt = malloc(Sd * 16);
  oc64 *xh = malloc(dS * 16), *grad_wv = malloc(Sd * 16), *t1 = malloc(Sd * 16), *t2 = malloc(Sd * 16);
  oc64 *ks = malloc(Sd * 16), *qs = malloc(Sd * 16), *vh = malloc(Sd * 16), *dlds = malloc(SS * 16);
  oc64 *dldq = malloc(Sd * 16), *dldk = malloc(Sd * 16), *wg = malloc(wn * 16), *wh = malloc(wn * 16);
  oc64 *dx1 = malloc(Sd > dS ? Sd * 16 : dS * 16), *dx2 = malloc(dS * 16), *dx3 = malloc(dS * 16);
  oc64* sc = malloc((size_t)S * 16);
  double *A = malloc(SS * 8), *dA = malloc(SS * 8), *dAt = malloc(SS * 8);
  int rc = ORC_OK;
  if (!q || !k || !v || !g || !gt || !xh || !grad_wv || !t1 || !t2 || !ks || !qs || !vh || !dlds || !dldq || !dldk ||
      !wg || !wh || !dx1 || !dx2 || !dx3 || !sc || !A || !dA || !dAt) {
    rc = fail(ORC_ERR_NOMEM, "attention backward: out of memory");
    goto done;
  }
  memset(dX, 0, (size_t)B * S * d * 16);
  memset(dwq, 0, (size_t)H * wn * 16);
  memset(dwk, 0, (size_t)H * wn * 16);
  memset(dwv, 0, (size_t)H * wn * 16);
  memset(dbias, 0, (size_t)H * SS * 16);
  for (uint32_t h = 0; h < H; ++h) {
    const oc64 *Wq = wq + h * wn, *Wk = wk + h * wn, *Wv = wv + h * wn, *bp = bias_pos + (size_t)h * mc * mc;
    for (uint32_t b = 0; b < B; ++b) {
      const oc64* xb = X + (size_t)b * S * d;
      const uint32_t* mk = mask + (size_t)b * S;
      zgemm_serial(S, dh, d, xb, Wq, q); /* :239-241 */
      zgemm_serial(S, dh, d, xb, Wk, k);
      zgemm_serial(S, dh, d, xb, Wv, v);
      /* the forward's attention weights (:184-205): softmax of Re over the
       * scaled, biased, causally masked scores; padded rows 0 */
      for (uint32_t r = 0; r < S; ++r) {
        double* a = A + (size_t)r * S;
        if (mk[r] == 0) {
          for (uint32_t j = 0; j < S; ++j) a[j] = 0.0;
          continue;
        }
        for (uint32_t j = 0; j < S; ++j) {
          oc64 s = {0.0, 0.0};
          for (uint32_t e = 0; e < dh; ++e) s = c_add(s, c_mul(q[(size_t)r * dh + e], k[(size_t)j * dh + e]));
          s = c_add(c_scale(s, c), bp[(size_t)r * mc + j]);
          sc[j] = j > r ? (oc64){-1e12, -1e12} : s;
        }
        orc_softmax_row_real(sc, S, a);
      }
      for (uint32_t r = 0; r < S; ++r) /* this head's slice of the gradient */
        memcpy(g + (size_t)r * dh, Gc + ((size_t)b * S + r) * d + (size_t)h * dh, dh * 16);
      ztrans(S, dh, g, 0, gt);                 /* transpose(previous_gradient) [dh][S] */
      zgemm_cr(dh, S, S, gt, A, grad_wv);      /* :276 */
      ztrans(S, d, xb, 1, xh);                 /* conjugate_transpose(input) [d][S] */
      ztrans(dh, S, grad_wv, 0, t1);           /* transpose(grad_wv) [S][dh] */
      zgemm_serial(d, dh, S, xh, t1, wg);      /* :278 */
      for (size_t i = 0; i < wn; ++i) dwv[h * wn + i] = c_add(dwv[h * wn + i], wg[i]);
      ztrans(S, dh, k, 0, ks); /* k_scaled = transpose(k) * c [dh][S] (:281) */
      for (size_t i = 0; i < Sd; ++i) ks[i] = c_scale(ks[i], c);
      for (size_t i = 0; i < Sd; ++i) qs[i] = c_scale(q[i], c); /* q_scaled [S][dh] (:282) */
      ztrans(S, dh, v, 1, vh);                 /* conjugate_transpose(v) [dh][S] */
      zgemm_serial(S, S, dh, g, vh, dlds);     /* dl_ds (:294) */
      /* backpropagate_softmax_masked_real over the row Jacobians
       * s_j (delta_jk - s_k) (utils/derivative.rs:100-131, 253-272) */
      for (uint32_t i = 0; i < S; ++i)
        for (uint32_t j = 0; j < S; ++j) {
          double acc = 0.0;
          if (mk[i] != 0) {
            const double* s = A + (size_t)i * S;
            for (uint32_t kk = 0; kk < S; ++kk) {
              const double jac = j == kk ? s[j] * (1.0 - s[j]) : -s[j] * s[kk];
              acc += jac * dlds[(size_t)i * S + kk].re;
            }
          }
          dA[(size_t)i * S + j] = acc;
        }
      for (uint32_t i = 0; i < S; ++i)
        for (uint32_t j = 0; j < S; ++j) dAt[(size_t)j * S + i] = dA[(size_t)i * S + j];
      zgemm_cr(dh, S, S, ks, dAt, dldq);       /* dl_dq [dh][S] (:301) */
      ztrans(dh, S, dldq, 1, t1);              /* conjugate_transpose(dl_dq) [S][dh] */
      zgemm_serial(d, dh, S, xh, t1, wg);      /* :305 */
      for (size_t i = 0; i < wn; ++i) dwq[h * wn + i] = c_add(dwq[h * wn + i], wg[i]);
      ztrans(S, dh, qs, 1, t2);                /* conjugate_transpose(q_scaled) [dh][S] */
      zgemm_cr(dh, S, S, t2, dA, dldk);        /* dl_dk [dh][S] (:312) */
      ztrans(dh, S, dldk, 0, t2);              /* transpose(dl_dk) [S][dh] */
      zgemm_serial(d, dh, S, xh, t2, wg);      /* :316 */
      for (size_t i = 0; i < wn; ++i) dwk[h * wn + i] = c_add(dwk[h * wn + i], wg[i]);
      ztrans(d, dh, Wq, 1, wh);                /* conjugate_transpose(weights_q) [dh][d] */
      zgemm_serial(S, d, dh, t1, wh, dx1);     /* dl_dqx (:328) */
      ztrans(d, dh, Wk, 1, wh);
      zgemm_serial(S, d, dh, t2, wh, dx2);     /* dl_dkx (:330) */
      ztrans(dh, S, grad_wv, 0, t1);
      ztrans(d, dh, Wv, 1, wh);
      zgemm_serial(S, d, dh, t1, wh, dx3);     /* dl_dvx (:332) */
      oc64* db = dbias + (size_t)h * SS;
      for (size_t i = 0; i < SS; ++i) db[i] = c_add(db[i], (oc64){dA[i], 0.0}); /* convert_to_c_f64_2d (:334) */
      oc64* dxb = dX + (size_t)b * S * d;
      for (size_t i = 0; i < dS; ++i) dxb[i] = c_add(dxb[i], c_add(c_add(dx1[i], dx2[i]), dx3[i])); /* :335-339 */
    }
  }
done:
  free(q), free(k), free(v), free(g), free(gt), free(xh), free(grad_wv), free(t1), free(t2), free(ks), free(qs);
  free(vh), free(dlds), free(dldq), free(dldk), free(wg), free(wh), free(dx1), free(dx2), free(dx3), free(sc);
  free(A), free(dA), free(dAt);
  return rc;
}

/* SelfAttentionLayer::backward (self_attention_layer.rs:135-196): the Norm's
 * backward on the layer's gradient, its input being Re(heads' output + X)
 * (the residual, add_matrix_3d_c), then the heads.  No residual gradient is
 * added: the layer returns the heads' input gradient only. */
int orc_self_attention_backward(const oc64* X, uint32_t B, uint32_t S, const uint32_t* mask, uint32_t H, uint32_t d,
                                uint32_t mc, double eps, const oc64* wq, const oc64* wk, const oc64* wv,
                                const oc64* bias_pos, const oc64* gamma, const oc64* beta, const oc64* G, oc64* dX,
                                oc64* dwq, oc64* dwk, oc64* dwv, oc64* dbias, oc64* dgamma, oc64* dbeta) {
  if (!X || !mask || !G || !B || !S || !H || !d || d % H || S > mc) return fail(ORC_ERR_ARG, "bad arguments");
  const size_t rows = (size_t)B * S;
  orc_layer L;
  memset(&L, 0, sizeof L);
  L.kind = ORC_SELF_ATTENTION;
  L.heads = H;
  L.d_in = L.d_out = d;
  L.dh = d / H;
  L.max_ctx = mc;
  L.eps = eps;
  L.wq = (oc64*)wq, L.wk = (oc64*)wk, L.wv = (oc64*)wv, L.bias_pos = (oc64*)bias_pos;
  L.gamma = (oc64*)gamma, L.beta = (oc64*)beta;
  oc64* xn = malloc(rows * d * 16);
  oc64* gn = malloc(rows * d * 16);
  uint32_t* lens = malloc((size_t)B * 4);
  int rc = ORC_OK;
  if (!xn || !gn || !lens) {
    rc = fail(ORC_ERR_NOMEM, "self-attention backward: out of memory");
    goto done;
  }
  for (uint32_t b = 0; b < B; ++b) lens[b] = S;
  /* the Norm's input: the heads' output of a stateless forward plus the
   * residual, real part only (add_matrix_3d_c) */
  rc = self_attention_forward(&L, X, mask, lens, B, S, 0, NULL, xn);
  if (rc) goto done;
  for (size_t i = 0; i < rows * d; ++i) xn[i] = (oc64){xn[i].re + X[i].re, 0.0};
  if ((rc = orc_norm_backward(xn, rows, d, eps, gamma, beta, G, gn, dgamma, dbeta))) goto done;
  rc = orc_attention_heads_backward(X, B, S, mask, H, d, mc, wq, wk, wv, bias_pos, gn, dX, dwq, dwk, dwv, dbias);
done:
  free(xn), free(gn), free(lens);
  return rc;
}

/* PositionalEncodingLayer::backward (positional_encoding_layer.rs:101-144):
 * each row's pairs rotated back by its position's angle (the row index) */
int orc_rope_backward(const oc64* G, uint32_t B, uint32_t S, uint32_t d, double base, oc64* out) {
  if (!G || !out || !B || !S || !d || d % 2) return fail(ORC_ERR_ARG, "bad arguments");
  const uint32_t half = d / 2;
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) {
      const oc64* g = G + ((size_t)b * S + s) * d;
      oc64* o = out + ((size_t)b * S + s) * d;
      for (uint32_t i = 0; i < half; ++i) {
        double theta = (double)s / pow(base * 1.0, 2.0 * (double)i / (double)d);
        if (theta < -1.0) theta = -1.0;
        if (theta > 1.0) theta = 1.0;
        const double sn = sin(theta), cs = cos(theta);
        const oc64 ge = g[2 * i], go = g[2 * i + 1];
        o[2 * i] = (oc64){ge.re * cs + go.re * sn, ge.im * cs + go.im * sn};
        o[2 * i + 1] = (oc64){-ge.re * sn + go.re * cs, -ge.im * sn + go.im * cs};
      }
    }
  return ORC_OK;
}

/* utils/normalization.rs:3-20 */
static void normalize_row(oc64* x, uint32_t n) {
  const double len = (double)n;
  oc64 sum = {0.0, 0.0};
  for (uint32_t i = 0; i < n; ++i) sum = c_add(sum, x[i]);
  const oc64 mean = c_unscale(sum, len);
  oc64 vs = {0.0, 0.0};
  for (uint32_t i = 0; i < n; ++i) {
    const oc64 t = c_sub(x[i], mean);
    vs = c_add(vs, c_mul(t, t));
  }
  const oc64 sd = c_sqrt(c_add(c_unscale(vs, len), (oc64){0.00000000001, 0.0}));
  for (uint32_t i = 0; i < n; ++i) x[i] = c_div(c_sub(x[i], mean), sd);
}

/* EmbeddingLayer::update_parameters (embedding_layer.rs:223-264): per
 * sequence, its gradient rows clipped elementwise, then for target t the
 * table row of that target id moves by lr * (row t of the gradient) / (B * V)
 * and is normalized, in order (a repeated id sees its updated row). */
int orc_embedding_update(oc64* table, uint32_t V, uint32_t d, const oc64* G, uint32_t B, uint32_t S,
                         const uint32_t* targets, const uint32_t* tlens, uint32_t T, double lr) {
  if (!table || !G || !targets || !tlens || !V || !d || !B || !S) return fail(ORC_ERR_ARG, "bad arguments");
  const double bs = (double)B * (double)V;
  oc64* g = (oc64*)malloc((size_t)S * d * sizeof(oc64));
  if (!g) return fail(ORC_ERR_NOMEM, "embedding update: out of memory");
  int rc = ORC_OK;
  for (uint32_t b = 0; b < B && !rc; ++b) {
    for (size_t i = 0; i < (size_t)S * d; ++i) g[i] = clip1(G[(size_t)b * S * d + i], 1.0);
    if (tlens[b] > T || tlens[b] > S) {
      rc = fail(ORC_ERR_ARG, "sequence %u: %u targets", b, tlens[b]);
      break;
    }
    for (uint32_t t = 0; t < tlens[b]; ++t) {
      const uint32_t id = targets[(size_t)b * T + t];
      if (id >= V) {
        rc = fail(ORC_ERR_ARG, "No token embedding found: %u", id);
        break;
      }
      oc64* row = table + (size_t)id * d;
      for (uint32_t j = 0; j < d; ++j) {
        const oc64 gj = g[(size_t)t * d + j];
        if (!finite_c(gj)) {
          rc = fail(ORC_ERR_NAN, "gradient in embedding is invalid");
          break;
        }
        row[j] = c_sub(row[j], c_scale(c_unscale(gj, bs), lr));
        if (!finite_c(row[j])) {
          rc = fail(ORC_ERR_NAN, "embedding is invalid");
          break;
        }
      }
      if (rc) break;
      normalize_row(row, d);
    }
  }
  free(g);
  return rc;
}

/* One parameter array's update_parameters arm: the first update's clipped
 * descent (lr * clip(g) / batch where finite), later ones calculate_adam_w
 * (weight = 1, EPSILON floor on v_hat's norm) or calculate_adam_w_bias
 * (weight = 0) on g as given (adam_w.rs:9-103 clip each element themselves) */
int orc_param_update(oc64* w, const oc64* g, oc64* m, oc64* v, uint64_t n, int first, double lr, double batch,
                     uint32_t time_step, int weight) {
  if (!w || !g || !m || !v) return fail(ORC_ERR_ARG, "bad arguments");
  for (uint64_t i = 0; i < n; ++i) {
    if (first) { /* the descent leaves zero moments behind it */
      m[i] = (oc64){0.0, 0.0};
      v[i] = (oc64){0.0, 0.0};
      const oc64 gc = clip1(g[i], 1.0);
      if (finite_c(gc)) w[i] = c_sub(w[i], c_scale(c_unscale(gc, batch), lr));
    } else {
      w[i] = adamw1(w[i], g[i], &m[i], &v[i], lr, time_step, weight);
    }
  }
  return ORC_OK;
}

/* inverse_dwt_1d (wavelet_transform/dwt.rs:90-124) with a DB filter of length
 * L: the inverse low pass is the low pass reversed, the inverse high pass the
 * high pass (lo reversed, odd entries negated) reversed
 * (dwt_type_resolver.rs:107-171) */
static uint32_t inverse_dwt_1d_c(const oc64* data, uint32_t n, const double* lo, uint32_t L, oc64* out) {
  double ilo[4], hp[4], ihi[4];
  for (uint32_t k = 0; k < L; ++k) ilo[k] = lo[L - 1 - k];
  for (uint32_t i = 0; i < L; ++i) hp[i] = (i & 1) ? -lo[L - 1 - i] : lo[L - 1 - i];
  for (uint32_t k = 0; k < L; ++k) ihi[k] = hp[L - 1 - k];
  const uint32_t middle = n >> 1, l = n - (L - 2);
  for (uint32_t i = 0; i < (l >> 1); ++i) {
    oc64 vl = {0.0, 0.0}, vh = {0.0, 0.0};
    for (uint32_t p = 0; p < L; p += 2) {
      const uint32_t il = (p + 1) % L, it = (p / 2 + i) % n, ih = (it + middle) % n;
      vl = c_add(c_add(vl, c_scale(data[it], ilo[il])), c_scale(data[ih], ihi[il]));
      vh = c_add(c_add(vh, c_scale(data[it], ilo[p])), c_scale(data[ih], ihi[p]));
    }
    out[2 * i] = vl;
    out[2 * i + 1] = vh;
  }
  return l;
}

/* DiscreteWaveletLayer::backward, partial mode (wavelet_discrete_layer.rs:
 * 163-207): per sequence, the gradient of the S2 - T compressed rows through
 * decompress_partial (:288-298: grad_dwt_1d_trend, dwt.rs:272-282, on every
 * feature), align_gradient_rows_complex (:318-346) when that gives another
 * row count than the S_in - T input rows, then the T target rows' gradient. */
int orc_dwt_backward(const oc64* G, uint32_t B, uint32_t S2, uint32_t S_in, uint32_t T, uint32_t wavelet, uint32_t d,
                     oc64* out) {
  if (!G || !out || !B || !d || T >= S2 || T >= S_in) return fail(ORC_ERR_ARG, "bad arguments");
  double lo[4];
  uint32_t L = 0;
  int rc = dwt_low_pass(wavelet, lo, &L);
  if (rc) return rc;
  const uint32_t M = S2 - T, R = S_in - T;
  oc64* data = (oc64*)calloc(2 * (size_t)M, sizeof(oc64));
  oc64* dec = (oc64*)malloc(2 * (size_t)M * sizeof(oc64));
  if (!data || !dec) {
    free(data), free(dec);
    return fail(ORC_ERR_NOMEM, "wavelet backward: out of memory");
  }
  for (uint32_t b = 0; b < B && !rc; ++b)
    for (uint32_t c = 0; c < d; ++c) {
      for (uint32_t j = 0; j < M; ++j) data[j] = G[((size_t)b * S2 + j) * d + c];
      for (uint32_t j = M; j < 2 * M; ++j) data[j] = (oc64){0.0, 0.0};
      const uint32_t lout = inverse_dwt_1d_c(data, 2 * M, lo, L, dec);
      if (lout < R) {
        rc = fail(ORC_ERR_STATE, "wavelet backward: %u rows for %u inputs", lout, R);
        break;
      }
      oc64* o = out + (size_t)b * S_in * d + c;
      if (lout == R) {
        for (uint32_t r = 0; r < R; ++r) o[(size_t)r * d] = dec[r];
      } else {
        for (uint32_t r = 0; r + 1 < R; ++r) o[(size_t)r * d] = dec[r];
        oc64 last = {0.0, 0.0};
        for (uint32_t i = R - 1; i < lout; ++i) last = c_add(last, dec[i]);
        o[(size_t)(R - 1) * d] = last;
      }
      for (uint32_t t = 0; t < T; ++t) o[(size_t)(R + t) * d] = G[((size_t)b * S2 + M + t) * d + c];
    }
  free(data), free(dec);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* EmbeddingLayer::create_embedding (embedding_layer.rs:65-77)               */
/* ------------------------------------------------------------------------ */

int orc_dwt_2d_full(const double* x, uint32_t rows, uint32_t cols, uint32_t wavelet, uint32_t mode, double* out,
                    uint32_t* out_rows, uint32_t* out_cols) {
  if (!x || !out || !rows || !cols) return fail(ORC_ERR_ARG, "bad arguments");
  /* dwt_2d_partial over the rows (dwt.rs:8-18) */
  double* t = (double*)malloc((size_t)rows * (cols + 4) * sizeof(double));
  double* col = (double*)malloc((size_t)(rows + 4) * 2 * sizeof(double));
  if (!t || !col) {
    free(t), free(col);
    return fail(ORC_ERR_NOMEM, "dwt_2d_full: out of memory");
  }
  uint32_t C2 = 0, R2 = 0;
  int rc = ORC_OK;
  for (uint32_t r = 0; r < rows && !rc; ++r) rc = orc_dwt_1d(x + (size_t)r * cols, cols, wavelet, mode, t + (size_t)r * (cols + 4), &C2);
  /* transpose, dwt_2d_partial over the former columns, transpose back (:27-33) */
  for (uint32_t c = 0; c < C2 && !rc; ++c) {
    double* in = col + rows + 4;
    for (uint32_t r = 0; r < rows; ++r) in[r] = t[(size_t)r * (cols + 4) + c];
    rc = orc_dwt_1d(in, rows, wavelet, mode, col, &R2);
    for (uint32_t r = 0; r < R2 && !rc; ++r) out[(size_t)r * C2 + c] = col[r];
  }
  free(t), free(col);
  if (rc) return rc;
  *out_rows = R2;
  *out_cols = C2;
  return ORC_OK;
}

/* The CMOR wavelet's cumulative integral resampled at the scale and reversed
 * (integrate_complex, utils/array_complex.rs:122-149) from wavefun_complex
 * (cwt_complex.rs:268-289): x = linspace_complex(-8, 8, 1024, true)
 * (utils/array_complex.rs:10-33: start + step added one by one, the end
 * set exactly), y = cmorl(x) (cwt_type_resolver.rs:114-123:
 * cos(2 pi fc x) E^(-x^2 / fb) / sqrt(pi fb), minus the sine likewise;
 * E.powf is pow with base e, not exp).  *klen = scale * 16 + 1 entries. */
static int cmor_kernel(double scale, double fb, double fc, oc64** kern, uint32_t* klen) {
  enum { NP = 1024 };
  static double xs[NP];
  static oc64 integral[NP];
  const double start = -8.0, end = 8.0, span = end - start;
  const double step_ls = span / ((double)NP - 1.0);
  double t = start;
  for (int i = 0; i < NP; ++i) {
    xs[i] = t;
    t = t + step_ls;
  }
  xs[NP - 1] = end;
  const double step = xs[1] - xs[0];
  for (int i = 0; i < NP; ++i) {
    const double re = xs[i];
    const double ang = 2.0 * M_PI * fc * re;
    const double g = pow(M_E, -pow(re, 2.0) / fb);
    const double den = sqrt(M_PI * fb);
    const oc64 y = {cos(ang) * g / den, -1.0 * (sin(ang) * g / den)};
    oc64 sum = {y.re * step, y.im * step};
    if (i > 0) sum = c_add(sum, integral[i - 1]);
    integral[i] = sum;
  }
  const double range = xs[NP - 1] - xs[0];
  const double a_end = scale * range + 1.0;
  const size_t K = (size_t)((a_end - 0.0) / 1.0); /* arange(0, end, 1), utils/array.rs:8-20 */
  oc64* k = (oc64*)malloc((K ? K : 1) * sizeof(oc64));
  if (!k) return fail(ORC_ERR_NOMEM, "cwt: out of memory");
  double v = 0.0;
  for (size_t j = 0; j < K; ++j) {
    const size_t idx = (size_t)(v / (scale * step));
    if (idx >= NP) {
      free(k);
      return fail(ORC_ERR_ARG, "cwt: scale %g reaches past the wavelet's integral", scale);
    }
    k[K - 1 - j] = integral[idx]; /* reversed */
    v = v + 1.0;
  }
  *kern = k;
  *klen = (uint32_t)K;
  return ORC_OK;
}

static int cwt_with_kernel(const double* x, uint32_t n, const oc64* kern, uint32_t K, double scale, oc64* out);

int orc_cwt_cmor(const double* x, uint32_t n, double scale, double fb, double fc, oc64* out) {
  if (!x || !out || !n) return fail(ORC_ERR_ARG, "bad arguments");
  oc64* kern = NULL;
  uint32_t K = 0;
  int rc = cmor_kernel(scale, fb, fc, &kern, &K);
  if (rc) return rc;
  rc = cwt_with_kernel(x, n, kern, K, scale, out);
  free(kern);
  return rc;
}

/* get_wavelet_complex's convolution and coefficients for a kernel from
 * cmor_kernel */
static int cwt_with_kernel(const double* x, uint32_t n, const oc64* kern, uint32_t K, double scale, oc64* out) {
  /* convolve_complex(data, kernel, FULL) (utils/array_complex.rs:38-94): the
   * shorter operand is reversed and slides over the longer one padded by
   * (n_out - longer) zeros on each side; each output sums in order from 0 */
  oc64* data = (oc64*)malloc((size_t)n * sizeof(oc64));
  if (!data) return fail(ORC_ERR_NOMEM, "cwt: out of memory");
  for (uint32_t i = 0; i < n; ++i) data[i] = (oc64){x[i], 0.0};
  const oc64* shortv = K < n ? kern : data;
  const oc64* longv = K < n ? data : kern;
  const uint32_t ls = K < n ? K : n, ll = K < n ? n : K;
  const uint32_t nout = n + K - 1, pad = nout - ll, flen = ll + 2 * pad;
  oc64* fp = (oc64*)calloc(flen, sizeof(oc64));
  oc64* conv = (oc64*)malloc((size_t)nout * sizeof(oc64));
  if (!fp || !conv) {
    free(data), free(fp), free(conv);
    return fail(ORC_ERR_NOMEM, "cwt: out of memory");
  }
  for (uint32_t i = 0; i < ll; ++i) fp[pad + i] = longv[i];
  for (uint32_t j = 0; j < nout; ++j) {
    oc64 sum = {0.0, 0.0};
    for (uint32_t i = 0; i < ls; ++i) sum = c_add(sum, c_mul(fp[(i + j) % flen], shortv[ls - 1 - i]));
    conv[j] = sum;
  }
  /* get_coef_complex (:154-164): -sqrt(scale) times successive differences;
   * then the centre n of them (cwt_complex.rs:205-211) */
  const double ss = -1.0 * sqrt(scale);
  const uint32_t clen = nout - 1;
  const double half = (double)(clen - n) / 2.0;
  const uint32_t down = (uint32_t)floor(half);
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t c = down + i;
    out[i] = c_scale(c_sub(conv[c + 1], conv[c]), ss);
  }
  free(data), free(fp), free(conv);
  return ORC_OK;
}

int orc_embedding_wavelet(uint64_t seed, uint64_t stream, uint32_t vocab, uint32_t src_dim, oc64* table,
                          uint32_t* dim) {
  if (!table || !dim || !vocab || src_dim < 2) return fail(ORC_ERR_ARG, "bad arguments");
  const uint32_t DB1 = 0, SYMMETRIC = 2, LEVELS = 5, MIN_WIDTH = 28; /* wavelet_network.rs:13,43-53 */
  const double SCALE0 = 2.0, FB = 1.5, FC = 1.0;                      /* the first of scales 2, 8, 16, 32 */
  oc64* kern = NULL;
  uint32_t K = 0;
  int rc = cmor_kernel(SCALE0, FB, FC, &kern, &K); /* the same for every token */
  if (rc) return rc;
  double* pix = (double*)malloc((size_t)src_dim * sizeof(double));
  double* t = (double*)malloc((size_t)(src_dim + 8) * 8 * sizeof(double));
  oc64* row = (oc64*)malloc((size_t)src_dim * sizeof(oc64));
  if (!pix || !t || !row) {
    free(kern), free(pix), free(t), free(row);
    return fail(ORC_ERR_NOMEM, "embedding: out of memory");
  }
  uint32_t width = 0;
  for (uint32_t tok = 0; tok < vocab && !rc; ++tok) {
    const double lo = -0.4, hi = 0.5;
    for (uint32_t k = 0; k < src_dim; ++k) {
      const double u = (double)(orc_draw(seed, stream, (uint64_t)tok * src_dim + k) >> 11) * 0x1.0p-53;
      pix[k] = lo + (hi - lo) * u;
    }
    /* decompose_in_wavelets (:75-120) of a one-dimensional input: one row */
    uint32_t w = src_dim;
    for (uint32_t lv = 0; lv < LEVELS && !rc; ++lv) {
      uint32_t R2 = 0, C2 = 0;
      rc = orc_dwt_2d_full(pix, 1, w, DB1, SYMMETRIC, t, &R2, &C2);
      if (rc || C2 < MIN_WIDTH) break;
      /* get_ll_hl_lh_hh (dwt.rs:379-401): the first R2/2 rows, first C2/2 columns */
      const uint32_t w2 = C2 >> 1;
      for (uint32_t k = 0; k < w2; ++k) pix[k] = t[k];
      w = w2;
    }
    if (rc) break;
    rc = cwt_with_kernel(pix, w, kern, K, SCALE0, row);
    for (uint32_t k = 0; k < w && !rc; ++k) table[(size_t)tok * w + k] = row[k];
    width = w;
  }
  free(kern), free(pix), free(t), free(row);
  if (rc) return rc;
  *dim = width;
  return ORC_OK;
}

int orc_init_embedding_wavelet(orc_net* net, uint32_t layer, uint64_t seed, uint32_t src_dim) {
  if (!net || layer >= (uint32_t)net->n) return fail(ORC_ERR_ARG, "bad layer index");
  orc_layer* L = &net->layers[layer];
  if (L->kind != ORC_EMBEDDING) return fail(ORC_ERR_ARG, "layer %u is not an Embedding", layer);
  oc64* t = (oc64*)malloc((size_t)L->vocab * src_dim * sizeof(oc64));
  if (!t) return fail(ORC_ERR_NOMEM, "embedding: out of memory");
  uint32_t dim = 0;
  int rc = orc_embedding_wavelet(seed, stream_id(layer, 0xFFF), L->vocab, src_dim, t, &dim);
  if (!rc && dim != L->d_out) rc = fail(ORC_ERR_ARG, "a %u-value draw decomposes to %u, not %u", src_dim, dim, L->d_out);
  if (!rc) memcpy(L->table, t, (size_t)L->vocab * dim * sizeof(oc64));
  free(t);
  return rc;
}
