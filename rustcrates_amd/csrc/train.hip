// train.hip — the output head's training step on gfx950: the kernels around
// the two products of LinearLayer::backward (linear_layer.rs:77-128) for the
// vocab Linear behind SoftmaxLayer::backward (softmax_output_layer.rs:67-145),
// and LinearLayer::update_parameters (linear_layer.rs:130-175) with the
// reference's AdamW (utils/adam_w.rs:9-103).
//
//   G  = softmax gradient, one row per output row; row r of sequence b
//        holds (p - [c == target]) / (B * non-PAD targets of b) when the
//        row predicts a target, else 0 (the host maps rows to targets);
//        stored as complex with im 0, the reference's Complex gradient
//   dW = conj(X)^T G and dX = G conj(W)^T: gemm() on conjugate transposes
//   db = the column sums of G
//   update: the first update descends by lr * clip(g) / B where finite; later
//        ones run AdamW on the unclipped grouped gradient (AdamW clips each
//        element to norm 1 itself), moments kept per parameter.
#include "kernels.hpp"

namespace mitok {

// one block per output row: 256 threads stream the row's probabilities
__global__ __launch_bounds__(256) void k_softmax_grad(const double* __restrict__ P, int V, const int* __restrict__ tgt,
                                                      const double* __restrict__ norm, int S, double2* __restrict__ G) {
  const long r = blockIdx.x;
  const int t = tgt[r];
  const double nz = norm[r / S];
  const double* p = P + r * V;
  double2* g = G + r * V;
  for (int c = threadIdx.x; c < V; c += 256) {
    double v = 0.0;
    if (t >= 0) v = (c == t ? p[c] - 1.0 : p[c]) / nz;  // softmax_output_layer.rs:128-135
    g[c] = make_double2(v, 0.0);
  }
}

// out[c][r] = conj(in[r][c]) for in [R][C]: 16x16 tiles through LDS
__global__ __launch_bounds__(256) void k_conj_transpose(const double2* __restrict__ in, long R, long C,
                                                        double2* __restrict__ out) {
  __shared__ double2 t[16][17];
  const long r0 = (long)blockIdx.y * 16, c0 = (long)blockIdx.x * 16;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  if (r0 + ty < R && c0 + tx < C) {
    const double2 v = in[(r0 + ty) * C + c0 + tx];
    t[ty][tx] = make_double2(v.x, -v.y);
  }
  __syncthreads();
  if (c0 + ty < C && r0 + tx < R) out[(c0 + ty) * R + r0 + tx] = t[tx][ty];
}

// db[c] = sum over sequences b of (sum over rows s of G[b][s][c]): each
// sequence's column sum in row order, then the sequences in order
// (linear_layer.rs:101-105, group_gradient_batch_bias)
__global__ __launch_bounds__(256) void k_bias_grad(const double2* __restrict__ G, int B, int S, int V,
                                                   double2* __restrict__ db) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= V) return;
  double2 acc = make_double2(0.0, 0.0);
  for (int b = 0; b < B; ++b) {
    double2 s = make_double2(0.0, 0.0);
    for (int r = 0; r < S; ++r) s = cadd(s, G[((long)b * S + r) * V + c]);
    acc = cadd(acc, s);
  }
  db[c] = acc;
}

// f64::powi as compiler-rt's __powidf2 (square and multiply over the bits)
__device__ __forceinline__ double powi_f64(double a, int e) {
  const bool recip = e < 0;
  double r = 1.0;
  for (;;) {
    if (e & 1) r *= a;
    e /= 2;
    if (e == 0) break;
    a *= a;
  }
  return recip ? 1.0 / r : r;
}

// One parameter: the first update's clipped descent (linear_layer.rs:159-174,
// clip_gradient_1d at utils/matrix.rs:709-717), or AdamW (adam_w.rs:9-103;
// `weight`: v_hat's norm at least EPSILON, which the bias arm omits).  This
// file is built with -ffp-contract=off: every multiply and add rounds on its
// own, as the Rust expressions do.
__device__ __forceinline__ double2 update1(double2 w, double2 g, double2* m, double2* v, const TrainStep& ts,
                                           bool weight) {
  if (ts.first) {
    const double n = hypot(g.x, g.y);
    if (n > 1.0) g = cscale(g, 1.0 / n);
    if (!(isfinite(g.x) && isfinite(g.y))) return w;
    return csub(w, cscale(cunscale(g, ts.batch), ts.lr));
  }
  const double B1 = 0.9, B2 = 0.999, EPS = 1e-8, WD = 0.01, MAX_NORM = 1.0;
  const int t = ts.time_step > 0 ? ts.time_step : 1;
  const double gn = hypot(g.x, g.y);
  if (gn > MAX_NORM) g = cscale(g, MAX_NORM / gn);
  const double2 mm = cadd(cscale(*m, B1), cscale(g, 1.0 - B1));
  const double2 vv = cadd(cscale(*v, B2), cmul(cscale(g, 1.0 - B2), make_double2(g.x, -g.y)));
  *m = mm;
  *v = vv;
  const double2 mh = cunscale(mm, 1.0 - powi_f64(B1, t));
  const double2 vh = cunscale(vv, 1.0 - powi_f64(B2, t));
  double vn = hypot(vh.x, vh.y);
  if (weight) vn = fmax(vn, EPS);
  const double alr = ts.lr / (sqrt(vn) + EPS);
  return csub(cscale(w, 1.0 - ts.lr * WD), cmul(make_double2(alr, 0.0), mh));
}

__global__ __launch_bounds__(256) void k_linear_update(double2* __restrict__ W, const double2* __restrict__ dW,
                                                       double2* __restrict__ mW, double2* __restrict__ vW, long n,
                                                       double2* __restrict__ b, const double2* __restrict__ db,
                                                       double2* __restrict__ mb, double2* __restrict__ vb, int V,
                                                       TrainStep ts) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) W[i] = update1(W[i], dW[i], &mW[i], &vW[i], ts, true);
  if (i < V) b[i] = update1(b[i], db[i], &mb[i], &vb[i], ts, false);
}

// gelu_derivative_complex (utils/derivative.rs:48-84): powi(3) = z (z z),
// powi(2) = t t; saturated beyond |f(z)| = 20; the result kept to norms in
// [1e-12, 1e6]
__device__ __forceinline__ double2 gelu_deriv(double2 z) {
  const double s2p = sqrt(2.0 / M_PI);
  const double2 one = make_double2(1.0, 0.0);
  const double2 x3 = cmul(z, cmul(z, z));
  const double2 fx = cscale(cadd(z, cmul(make_double2(0.044715, 0.0), x3)), s2p);
  const bool sat = hypot(fx.x, fx.y) > 20.0;
  const double2 th = sat ? one : ctanh_nc(fx);
  const double2 sech2 = sat ? make_double2(0.0, 0.0) : csub(one, cmul(th, th));
  const double2 fp = cscale(cadd(one, cmul(make_double2(0.134145, 0.0), cmul(z, z))), s2p);
  const double2 d = cadd(cmul(make_double2(0.5, 0.0), cadd(one, th)),
                         cmul(cmul(cmul(make_double2(0.5, 0.0), z), sech2), fp));
  const double n = hypot(d.x, d.y);
  if (n > 1e6) return cmul(cunscale(d, n), make_double2(1e6, 0.0));
  if (n < 1e-12) return make_double2(1e-12, 0.0);
  return d;
}

// Dense (GELU) backward's elementwise step (layer.rs:181-192): the gradient
// of the activated output, its padded rows zeroed (apply_padding_mask_batch),
// times conj(GELU'(Z)) of the pre-activation Z
__global__ __launch_bounds__(256) void k_gelu_backward(const double2* __restrict__ dH, const double2* __restrict__ Z,
                                                       const uint32_t* __restrict__ mask, long rows, int F,
                                                       double2* __restrict__ G) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * F) return;
  const long r = i / F;
  double2 g = make_double2(0.0, 0.0);
  if (!mask || mask[r] != 0) {
    const double2 dz = gelu_deriv(Z[i]);
    g = cmul(dH[i], make_double2(dz.x, -dz.y));
  }
  G[i] = g;
}

void gelu_backward(hipStream_t st, const double2* dH, const double2* Z, const uint32_t* mask, long rows, int F,
                   double2* G) {
  const long n = rows * F;
  if (n > 0) MITOK_LAUNCH(k_gelu_backward, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dH, Z, mask, rows, F, G);
}

void softmax_grad(hipStream_t st, const double* P, int rows, int V, const int* tgt, const double* norm, int S,
                  double2* G) {
  if (rows > 0) MITOK_LAUNCH(k_softmax_grad, dim3(rows), dim3(256), 0, st, P, V, tgt, norm, S, G);
}

void conj_transpose(hipStream_t st, const double2* in, long R, long C, double2* out) {
  const dim3 grid((unsigned)((C + 15) / 16), (unsigned)((R + 15) / 16));
  if (R > 0 && C > 0) MITOK_LAUNCH(k_conj_transpose, grid, dim3(256), 0, st, in, R, C, out);
}

void bias_grad(hipStream_t st, const double2* G, int B, int S, int V, double2* db) {
  if (V > 0) MITOK_LAUNCH(k_bias_grad, dim3((V + 255) / 256), dim3(256), 0, st, G, B, S, V, db);
}

void linear_update(hipStream_t st, double2* W, const double2* dW, double2* mW, double2* vW, long n, double2* b,
                   const double2* db, double2* mb, double2* vb, int V, const TrainStep& ts) {
  const long work = std::max<long>(n, V);
  if (work > 0)
    MITOK_LAUNCH(k_linear_update, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st, W, dW, mW, vW, n, b, db, mb,
                 vb, V, ts);
}

}  // namespace mitok
