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
// (linear_layer.rs:101-105, group_gradient_batch_bias).  Two launches: one
// thread per (sequence, column) sums its rows (eight loads in flight), then
// one per column adds the sequences' sums, times `mult`.
__global__ __launch_bounds__(256) void k_seq_colsum(const double2* __restrict__ G, int B, int S, int V,
                                                    double2* __restrict__ part) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long)B * V) return;
  const int c = (int)(t % V), b = (int)(t / V);
  const double2* g = G + (long)b * S * V + c;
  double2 s = make_double2(0.0, 0.0);
  int r = 0;
  for (; r + 8 <= S; r += 8) {
    double2 u[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) u[q] = g[(long)(r + q) * V];
#pragma unroll
    for (int q = 0; q < 8; ++q) s = cadd(s, u[q]);
  }
  for (; r < S; ++r) s = cadd(s, g[(long)r * V]);
  part[t] = s;
}
__global__ __launch_bounds__(256) void k_seq_sum(const double2* __restrict__ part, int B, int V, double mult,
                                                 double2* __restrict__ out) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= V) return;
  double2 acc = make_double2(0.0, 0.0);
  for (int b = 0; b < B; ++b) acc = cadd(acc, part[(long)b * V + c]);
  out[c] = mult == 1.0 ? acc : cscale(acc, mult);
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
    // the descent stores zero moments for the AdamW that follows it
    // (linear_layer.rs:141-145,176-180): after reset_previous_gradient too
    *m = make_double2(0.0, 0.0);
    *v = make_double2(0.0, 0.0);
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

// cross_entropy_loss_batch (transformer_network.rs:662-711) on the softmax
// output P [B][S][V].  Block b: its targets' terms -ln(p + 1e-15), p at row
// S - tl - 1 + t, are formed in parallel into LDS (PAD targets, id 1, marked
// skipped), then one thread sums them in target order and divides by their
// count (cross_entropy_loss, :674-711; no target is left out by its
// `seq_ind >= end_ind` break, since the rows end at S - 2).  part[b] holds it.
__global__ __launch_bounds__(256) void k_ce_seq(const double* __restrict__ P, int S, int V,
                                                const uint32_t* __restrict__ tgt, const uint32_t* __restrict__ tlen,
                                                int T, double* __restrict__ part) {
  extern __shared__ double lp[];  // [T]
  const int b = blockIdx.x, tl = (int)tlen[b];
  const int start = S - tl - 1;
  for (int t = threadIdx.x; t < tl; t += 256) {
    const uint32_t tc = tgt[(long)b * T + t];
    lp[t] = tc == 1u ? NAN : -log(P[((long)b * S + start + t) * V + tc] + 1e-15);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double loss = 0.0, count = 0.0;
    for (int t = 0; t < tl; ++t)
      if (tgt[(long)b * T + t] != 1u) {
        loss += lp[t];
        count += 1.0;
      }
    part[b] = loss / count;
  }
}

// the batch: sum of the sequences' losses in order, divided by B, as the
// complex (sum / B, 0 / B) the reference returns
__global__ void k_ce_batch(const double* __restrict__ part, int B, double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double re = 0.0;
  for (int b = 0; b < B; ++b) re += part[b];
  out[0] = re / (double)B;
  out[1] = 0.0 / (double)B;
}

void cross_entropy(hipStream_t st, const double* P, int B, int S, int V, const uint32_t* tgt, const uint32_t* tlen,
                   int T, double* part, double* out) {
  if (B <= 0) return;
  MITOK_LAUNCH(k_ce_seq, dim3(B), dim3(256), (size_t)T * sizeof(double), st, P, S, V, tgt, tlen, T, part);
  MITOK_LAUNCH(k_ce_batch, dim3(1), dim3(64), 0, st, part, B, out);
}

void conj_transpose(hipStream_t st, const double2* in, long R, long C, double2* out) {
  const dim3 grid((unsigned)((C + 15) / 16), (unsigned)((R + 15) / 16));
  if (R > 0 && C > 0) MITOK_LAUNCH(k_conj_transpose, grid, dim3(256), 0, st, in, R, C, out);
}

void bias_grad(hipStream_t st, const double2* G, int B, int S, int V, double2* ws, double2* db) {
  colsum(st, G, B, S, V, 1.0, ws, db);
}

void linear_update(hipStream_t st, double2* W, const double2* dW, double2* mW, double2* vW, long n, double2* b,
                   const double2* db, double2* mb, double2* vb, int V, const TrainStep& ts) {
  const long work = std::max<long>(n, V);
  if (work > 0)
    MITOK_LAUNCH(k_linear_update, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st, W, dW, mW, vW, n, b, db, mb,
                 vb, V, ts);
}

// ---------------------------------------------------------------------------
// the rest of backward's reverse walk (transformer_network.rs:506-636)
// ---------------------------------------------------------------------------

// sum over a 256-thread block through LDS; every thread gets the total
__device__ double2 block_sum2(double2 v, double2* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] = cadd(sh[threadIdx.x], sh[threadIdx.x + w]);
    __syncthreads();
  }
  const double2 r = sh[0];
  __syncthreads();
  return r;
}
__device__ double block_max1(double v, double* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] = fmax(sh[threadIdx.x], sh[threadIdx.x + w]);
    __syncthreads();
  }
  const double r = sh[0];
  __syncthreads();
  return r;
}

// f64 / Complex and Complex::powf (num-complex 0.4.6: from_polar(r^e, theta e))
__device__ __forceinline__ double2 rdivc(double a, double2 z) {
  const double ns = z.x * z.x + z.y * z.y;
  return make_double2(a * z.x / ns, -a * z.y / ns);
}
__device__ __forceinline__ double2 cpowf(double2 z, double e) {
  const double r = pow(hypot(z.x, z.y), e), th = atan2(z.y, z.x) * e;
  return make_double2(r * cos(th), r * sin(th));
}

// NormalNormLayer::backward, Complex arm (norm_layer.rs:132-209), one block per
// row.  The row's input is x, or Re(x + resid) + 0i for the Norm inside a
// SelfAttention layer (add_matrix_3d_c); its forward (normalize, :64-82) is
// recomputed for x_hat, mean and variance.  The reference's f-loop is
// collapsed: with t_d = x_d - mu and the row sums P = sum dout_d t_d,
// D = sum dout_d, M = sum -2 t_d / n, element f's gradient is
//   g_f = dout_f gamma_f / sqrt(v) + gamma_f P (-1/2) v^-3/2 (2 t_f / n)
//         + (-D gamma_f / sqrt(v) + gamma_f P (-1/2) v^-3/2 M) / n,
// v = variance + 1e-8, and the row's input gradient is Re(g_j + (sum_f g_f) dout_j).
// pg[r][j] = dout_j x_hat_j feeds gamma's gradient (n copies per row).
__global__ __launch_bounds__(256) void k_norm_backward(const double2* __restrict__ x, const double2* __restrict__ resid,
                                                       int n, double eps, const double2* __restrict__ gamma,
                                                       const double2* __restrict__ beta,
                                                       const double2* __restrict__ dout, double2* __restrict__ dx,
                                                       double2* __restrict__ pg) {
  __shared__ double2 sh[256];
  const long r = blockIdx.x;
  const double2* xr = x + r * n;
  const double2* gr = dout + r * n;
  const double len = (double)n;
  auto xin = [&](int j) {
    if (!resid) return xr[j];
    return make_double2(xr[j].x + resid[r * n + j].x, 0.0);
  };
  double2 s = make_double2(0.0, 0.0);
  for (int j = threadIdx.x; j < n; j += 256) s = cadd(s, xin(j));
  const double2 mu = cunscale(block_sum2(s, sh), len);
  s = make_double2(0.0, 0.0);
  for (int j = threadIdx.x; j < n; j += 256) {
    const double2 t = csub(xin(j), mu);
    s = cadd(s, cmul(t, t));
  }
  const double2 var = cunscale(block_sum2(s, sh), len);
  const double2 sd = csqrt_nc(cadd(var, make_double2(eps, 0.0)));
  const double2 vb = cadd(var, make_double2(1e-8, 0.0));
  const double2 std_inv = rdivc(1.0, csqrt_nc(vb));
  const double2 vpm32 = rdivc(1.0, cpowf(vb, 1.5));
  double2 P = make_double2(0.0, 0.0), D = P, M = P;
  for (int j = threadIdx.x; j < n; j += 256) {
    const double2 t = csub(xin(j), mu);
    P = cadd(P, cmul(gr[j], t));
    D = cadd(D, gr[j]);
    M = cadd(M, cunscale(cscale(t, -2.0), len));
  }
  P = block_sum2(P, sh);
  D = block_sum2(D, sh);
  M = block_sum2(M, sh);
  const double2 dmu_sum = cmul(D, make_double2(-std_inv.x, -std_inv.y));
  const double2 pv = cmul(cscale(P, -0.5), vpm32);
  double2 gs = make_double2(0.0, 0.0);
  for (int j = threadIdx.x; j < n; j += 256) {
    const double2 t = csub(xin(j), mu);
    const double2 dvar = cmul(gamma[j], pv);
    const double2 dmu = cadd(cmul(dmu_sum, gamma[j]), cmul(dvar, M));
    const double2 g = cadd(cadd(cmul(cmul(gr[j], gamma[j]), std_inv), cmul(dvar, cunscale(cscale(t, 2.0), len))),
                           cunscale(dmu, len));
    gs = cadd(gs, g);
    dx[r * n + j] = g;  // held until the row total is known
    const double2 xh = cadd(cmul(cdiv(t, sd), gamma[j]), beta[j]);
    pg[r * n + j] = cmul(gr[j], make_double2(xh.x, 0.0));
  }
  gs = block_sum2(gs, sh);
  for (int j = threadIdx.x; j < n; j += 256) {
    const double2 g = dx[r * n + j];
    dx[r * n + j] = make_double2(g.x + cmul(gs, gr[j]).x, 0.0);
  }
}


// One query row of one head (grid: S x H x B): the forward's attention
// weights A (masked_attention_head.rs:184-205: Re of the scaled scores plus
// Re(bias_pos), the causal mask, softmax_complex_padding_real) and
// dl_da = backpropagate_softmax_masked_real of dl_ds = G conj(V)^T over the
// row Jacobian s_j (delta_jk - s_k) (utils/derivative.rs:100-131, 253-272):
// dA_j = s_j (r_j - sum_k s_k r_k), r_k = Re(dl_ds_k); padded rows 0.
__global__ __launch_bounds__(256) void k_attn_probs_grad(const double2* __restrict__ qkv, const double* __restrict__ bias_re,
                                                         int mc, const uint32_t* __restrict__ mask,
                                                         const double2* __restrict__ G, int S, int H, int dh, double c,
                                                         double* __restrict__ A, double* __restrict__ dA) {
  extern __shared__ double dyn[];
  double* sc = dyn;       // [S] scores, then weights
  double* rr = dyn + S;   // [S] Re(dl_ds)
  __shared__ double2 qs[256], gs[256];  // the row's q and gradient (dh <= 256)
  __shared__ double shm[256];
  __shared__ double2 sh2[256];
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int d = H * dh, ld = 3 * d;
  const long row = (long)b * S + i;
  double* Ar = A + (((long)b * H + h) * S + i) * S;
  double* dAr = dA + (((long)b * H + h) * S + i) * S;
  if (mask[row] == 0) {
    for (int j = tid; j < S; j += 256) Ar[j] = dAr[j] = 0.0;
    return;
  }
  for (int m = tid; m < dh; m += 256) {
    qs[m] = qkv[row * ld + (long)h * dh + m];
    gs[m] = G[row * d + (long)h * dh + m];
  }
  __syncthreads();
  // 16 lanes per key (a key's row read in contiguous 16-lane runs), 16 keys per pass
  const double* bp = bias_re + ((long)h * mc + i) * mc;
  const int sub = tid & 15, kq = tid >> 4;
  for (int j0 = 0; j0 < S; j0 += 16) {
    const int j = j0 + kq;
    double s = 0.0, rv = 0.0;
    if (j < S) {
      const double2* k = qkv + ((long)b * S + j) * ld + d + (long)h * dh;
      const double2* v = k + d;
      for (int m = sub; m < dh; m += 16) {
        const double2 kk = k[m], vv = v[m];
        s = s + (qs[m].x * kk.x - qs[m].y * kk.y);
        rv = rv + (gs[m].x * vv.x + gs[m].y * vv.y);
      }
    }
    s = row16_sum(s);
    rv = row16_sum(rv);
    if (j < S && sub == 0) {
      sc[j] = j > i ? -1e12 : s * c + bp[j];
      rr[j] = rv;
    }
  }
  __syncthreads();
  double mx = -INFINITY;
  for (int j = tid; j < S; j += 256) mx = fmax(mx, sc[j]);
  mx = block_max1(mx, shm);
  double2 acc = make_double2(0.0, 0.0);
  for (int j = tid; j < S; j += 256) {
    sc[j] = exp(sc[j] - mx);
    acc.x += sc[j];
  }
  const double sum = block_sum2(acc, sh2).x;
  acc = make_double2(0.0, 0.0);
  for (int j = tid; j < S; j += 256) {
    sc[j] = sc[j] / sum;
    acc.x += sc[j] * rr[j];
  }
  const double sr = block_sum2(acc, sh2).x;
  for (int j = tid; j < S; j += 256) {
    Ar[j] = sc[j];
    dAr[j] = sc[j] * (rr[j] - sr);
  }
}

// The three small products of MaskedAttentionHead::backward per (sequence,
// head), one output element each (masked_attention_head.rs:276-316):
//   dV = A^T G,  dQ = dA conj(K) c,  dK = dA^T conj(Q) c
// written as the gradient of the packed [q | k | v] row (head h at h*dh).
__global__ __launch_bounds__(256) void k_attn_dqkv(const double2* __restrict__ qkv, const double* __restrict__ A,
                                                   const double* __restrict__ dA, const double2* __restrict__ G, int B,
                                                   int S, int H, int dh, double c, double2* __restrict__ dqkv) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = (long)B * H * S * dh;
  if (t >= total) return;
  const int m = (int)(t % dh);
  const int i = (int)((t / dh) % S);
  const int h = (int)((t / ((long)dh * S)) % H);
  const int b = (int)(t / ((long)dh * S * H));
  const int d = H * dh, ld = 3 * d;
  const double* Ab = A + ((long)b * H + h) * S * S;
  const double* dAb = dA + ((long)b * H + h) * S * S;
  const double2* base = qkv + (long)b * S * ld + (long)h * dh + m;
  const double2* gb = G + (long)b * S * d + (long)h * dh + m;
  double2 dq = make_double2(0.0, 0.0), dk = dq, dv = dq;
  for (int j = 0; j < S; ++j) {
    const double2 kj = base[(long)j * ld + d];     // K[j][m]
    const double2 qj = base[(long)j * ld];         // Q[j][m]
    const double a = dAb[(long)i * S + j];         // dA[i][j]
    const double at = dAb[(long)j * S + i];        // dA[j][i]
    dq = cadd(dq, make_double2(a * kj.x, -a * kj.y));
    dk = cadd(dk, make_double2(at * qj.x, -at * qj.y));
    dv = cadd(dv, cscale(gb[(long)j * d], Ab[(long)j * S + i]));
  }
  double2* o = dqkv + ((long)b * S + i) * ld + (long)h * dh + m;
  o[0] = cscale(dq, c);
  o[d] = cscale(dk, c);
  o[2 * d] = dv;
}

// bias_pos's update on its S x S slice (masked_attention_head.rs:387-393,
// 427-434): the gradient dl_da summed over the sequences (group_gradient_batch),
// clipped; the first update descends, later ones run AdamW from zero moments
// (the reference never reloads prev_m/v_bias_pos).  Only Re(bias_pos) reaches
// the scores, and its update does not depend on the imaginary part.
__global__ __launch_bounds__(256) void k_attn_bias_update(double* __restrict__ bias_re, int mc,
                                                          const double* __restrict__ dA, int B, int H, int S,
                                                          TrainStep ts) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long)H * S * S) return;
  const int j = (int)(t % S), i = (int)((t / S) % S), h = (int)(t / ((long)S * S));
  double g = 0.0;
  for (int b = 0; b < B; ++b) g += dA[(((long)b * H + h) * S + i) * S + j];
  double* w = bias_re + ((long)h * mc + i) * mc + j;
  double2 m0 = make_double2(0.0, 0.0), v0 = m0;
  *w = update1(make_double2(*w, 0.0), make_double2(g, 0.0), &m0, &v0, ts, true).x;
}

// one parameter array: update1 on every element
__global__ __launch_bounds__(256) void k_param_update(double2* __restrict__ w, const double2* __restrict__ g,
                                                      double2* __restrict__ m, double2* __restrict__ v, long n,
                                                      int weight, TrainStep ts) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) w[i] = update1(w[i], g[i], &m[i], &v[i], ts, weight != 0);
}

// PositionalEncodingLayer::backward (positional_encoding_layer.rs:101-144):
// the pairs of row s rotated back by the forward's angle at position s
// (cs: the forward's (cos, sin) table)
__global__ __launch_bounds__(256) void k_rope_backward(const double2* __restrict__ G, long rows, int S, int d,
                                                       const double2* __restrict__ cs, double2* __restrict__ out) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const int half = d / 2;
  if (t >= rows * half) return;
  const long r = t / half;
  const int i = (int)(t % half);
  const int pos = (int)(r % S);
  const double2 w = cs[(long)pos * half + i];  // (cos, sin)
  const double2 ge = G[r * d + 2 * i], go = G[r * d + 2 * i + 1];
  out[r * d + 2 * i] = make_double2(ge.x * w.x + go.x * w.y, ge.y * w.x + go.y * w.y);
  out[r * d + 2 * i + 1] = make_double2(-ge.x * w.y + go.x * w.x, -ge.y * w.y + go.y * w.x);
}

// EmbeddingLayer::update_parameters (embedding_layer.rs:223-264): one block
// per distinct target id, its occurrences in the reference's order: the row
// moves by lr * clip(g) / (B V) (g: the gradient row at the target's index),
// then is normalized (utils/normalization.rs:3-20).  A non-finite gradient or
// row raises the error word (the reference panics).
__global__ __launch_bounds__(256) void k_embedding_update(double2* __restrict__ table, int d,
                                                          const uint32_t* __restrict__ ids,
                                                          const int* __restrict__ start, const int* __restrict__ occ,
                                                          const double2* __restrict__ G, double lr, double bs,
                                                          uint32_t* __restrict__ err) {
  __shared__ double2 sh[256];
  double2* row = table + (long)ids[blockIdx.x] * d;
  const double len = (double)d;
  bool bad = false;
  for (int k = start[blockIdx.x]; k < start[blockIdx.x + 1]; ++k) {
    const double2* g = G + (long)occ[k] * d;
    double2 s = make_double2(0.0, 0.0);
    for (int j = threadIdx.x; j < d; j += 256) {
      double2 gj = g[j];
      const double gn = hypot(gj.x, gj.y);
      if (gn > 1.0) gj = cscale(gj, 1.0 / gn);
      if (!(isfinite(gj.x) && isfinite(gj.y))) bad = true;
      const double2 w = csub(row[j], cscale(cunscale(gj, bs), lr));
      if (!(isfinite(w.x) && isfinite(w.y))) bad = true;
      row[j] = w;
      s = cadd(s, w);
    }
    __syncthreads();
    const double2 mean = cunscale(block_sum2(s, sh), len);
    s = make_double2(0.0, 0.0);
    for (int j = threadIdx.x; j < d; j += 256) {
      const double2 t = csub(row[j], mean);
      s = cadd(s, cmul(t, t));
    }
    const double2 sd = csqrt_nc(cadd(cunscale(block_sum2(s, sh), len), make_double2(0.00000000001, 0.0)));
    for (int j = threadIdx.x; j < d; j += 256) row[j] = cdiv(csub(row[j], mean), sd);
    __syncthreads();
  }
  if (bad) atomicOr(err, (uint32_t)EB_TRAIN_NONFINITE);
}

void norm_backward(hipStream_t st, const double2* x, const double2* resid, long rows, int n, double eps,
                   const double2* gamma, const double2* beta, const double2* dout, double2* dx, double2* pg) {
  if (rows > 0) MITOK_LAUNCH(k_norm_backward, dim3((unsigned)rows), dim3(256), 0, st, x, resid, n, eps, gamma, beta, dout, dx, pg);
}

void colsum(hipStream_t st, const double2* X, int B, int S, int n, double mult, double2* ws, double2* out) {
  if (n <= 0 || B <= 0) return;
  MITOK_LAUNCH(k_seq_colsum, dim3((unsigned)(((long)B * n + 255) / 256)), dim3(256), 0, st, X, B, S, n, ws);
  MITOK_LAUNCH(k_seq_sum, dim3((n + 255) / 256), dim3(256), 0, st, ws, B, n, mult, out);
}

void attn_probs_grad(hipStream_t st, const double2* qkv, const double* bias_re, int mc, const uint32_t* mask,
                     const double2* G, int B, int S, int H, int dh, double c, double* A, double* dA) {
  MITOK_LAUNCH(k_attn_probs_grad, dim3(S, H, B), dim3(256), (size_t)2 * S * sizeof(double), st, qkv, bias_re, mc, mask,
               G, S, H, dh, c, A, dA);
}

void attn_dqkv(hipStream_t st, const double2* qkv, const double* A, const double* dA, const double2* G, int B, int S,
               int H, int dh, double c, double2* dqkv) {
  const long total = (long)B * H * S * dh;
  if (total > 0)
    MITOK_LAUNCH(k_attn_dqkv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, qkv, A, dA, G, B, S, H, dh, c, dqkv);
}

void attn_bias_update(hipStream_t st, double* bias_re, int mc, const double* dA, int B, int H, int S, const TrainStep& ts) {
  const long total = (long)H * S * S;
  if (total > 0)
    MITOK_LAUNCH(k_attn_bias_update, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, bias_re, mc, dA, B, H, S, ts);
}

void param_update(hipStream_t st, double2* w, const double2* g, double2* m, double2* v, long n, bool weight,
                  const TrainStep& ts) {
  if (n > 0)
    MITOK_LAUNCH(k_param_update, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, g, m, v, n, weight ? 1 : 0, ts);
}

void rope_backward(hipStream_t st, const double2* G, long rows, int S, int d, const double2* cs, double2* out) {
  const long total = rows * (d / 2);
  if (total > 0)
    MITOK_LAUNCH(k_rope_backward, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, G, rows, S, d, cs, out);
}

void embedding_update(hipStream_t st, double2* table, int d, const uint32_t* ids, int n_ids, const int* start,
                      const int* occ, const double2* G, double lr, double bs, uint32_t* err) {
  if (n_ids > 0)
    MITOK_LAUNCH(k_embedding_update, dim3(n_ids), dim3(256), 0, st, table, d, ids, start, occ, G, lr, bs, err);
}

// DiscreteWaveletLayer::backward, partial mode (wavelet_discrete_layer.rs:
// 163-207): input row r of sequence b gets sum_k w[r][k] G[b][src[r][k]]
// (four taps at most, src -1: none).  The host builds the table from
// decompress_partial (grad_dwt_1d_trend, dwt.rs:272-282: the low-pass filter
// transposed over the compressed rows), align_gradient_rows_complex (:318-346)
// and the target rows, whose gradient passes through (weight 1).
__global__ __launch_bounds__(256) void k_dwt_backward(const double2* __restrict__ G, int B, int S2, int Sin, int d,
                                                      const int* __restrict__ src, const double* __restrict__ w,
                                                      double2* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * Sin * d) return;
  const int c = (int)(i % d);
  const long br = i / d;
  const int r = (int)(br % Sin), b = (int)(br / Sin);
  double2 v = make_double2(0.0, 0.0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int s = src[r * 4 + k];
    if (s >= 0) v = cadd(v, cscale(G[((long)b * S2 + s) * d + c], w[r * 4 + k]));
  }
  out[i] = v;
}

void dwt_backward(hipStream_t st, const double2* G, int B, int S2, int Sin, int d, const int* src, const double* w,
                  double2* out) {
  const long n = (long)B * Sin * d;
  if (n > 0) MITOK_LAUNCH(k_dwt_backward, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, G, B, S2, Sin, d, src, w, out);
}

}  // namespace mitok
