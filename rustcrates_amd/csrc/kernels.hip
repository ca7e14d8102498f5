// kernels.hip — row kernels of the complex-f64 transformer token loop on gfx950
// (embedding, RoPE, LayerNorm, argmax, softmax, initialisation).  The products
// are in gemm.hip, attention in attention.hip.
//
// All tensors are row-major complex f64 (double2).  Wavefronts are 64 lanes.
// Reference math is cited per kernel (paths relative to src/neural_networks/).
#include <algorithm>

#include "kernels.hpp"

namespace mitok {

static inline int cdiv_i(long a, long b) { return (int)((a + b - 1) / b); }

// ===========================================================================
// Row kernels
// ===========================================================================
// EmbeddingLayer::forward (embedding_layer.rs:158-211): PAD id 1 -> zeros.
__global__ void k_embed(const double2* __restrict__ table, int V, int d, const uint32_t* __restrict__ ids, int rows,
                        double2* __restrict__ out, uint32_t* err) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * d) return;
  int r = (int)(i / d), c = (int)(i - (long)r * d);
  uint32_t id = ids[r];
  double2 v = make_double2(0.0, 0.0);
  if (id != 1) {
    if (id >= (uint32_t)V) {
      if (c == 0) atomicOr(err, (uint32_t)EB_BAD_TOKEN);
    } else {
      v = table[(long)id * d + c];
    }
  }
  out[i] = v;
}

void embed(hipStream_t st, const double2* table, int V, int d, const uint32_t* ids, int rows, double2* out,
           uint32_t* err) {
  long n = (long)rows * d;
  hipLaunchKernelGGL(k_embed, dim3(cdiv_i(n, 256)), dim3(256), 0, st, table, V, d, ids, rows, out, err);
}

// apply_rotary_positional_encoding (positional_encoding_layer.rs:181-209) with
// (cos, sin) of the clamped angle tabulated on the host with libm.  Without
// explicit positions, row r (one per sequence) sits at kv_len[r] + off[r].
__global__ void k_rope(double2* __restrict__ x, int rows, int d, const double2* __restrict__ cs, int max_pos,
                       const int* __restrict__ pos, const int* __restrict__ kv_len, const int* __restrict__ off,
                       uint32_t* err) {
  const int half = d / 2;
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * half) return;
  int r = (int)(i / half), k = (int)(i - (long)r * half);
  int p = pos ? pos[r] : kv_len[r] + (off ? off[r] : 0);
  if (p >= max_pos) {
    atomicOr(err, (uint32_t)EB_CTX_OVERFLOW);
    return;
  }
  double2 t = cs[(long)p * half + k];  // (cos, sin)
  double2* xr = x + (long)r * d;
  double2 e = xr[2 * k], o = xr[2 * k + 1];
  xr[2 * k] = make_double2(e.x * t.x - o.x * t.y, e.y * t.x - o.y * t.y);
  xr[2 * k + 1] = make_double2(e.x * t.y + o.x * t.x, e.y * t.y + o.y * t.x);
}

void rope(hipStream_t st, double2* x, int rows, int d, const double2* cs_table, int max_pos, const int* pos,
          const int* kv_len, const int* off, uint32_t* err) {
  long n = (long)rows * (d / 2);
  hipLaunchKernelGGL(k_rope, dim3(cdiv_i(n, 256)), dim3(256), 0, st, x, rows, d, cs_table, max_pos, pos, kv_len, off,
                     err);
}

// DiscreteWaveletLayer at a prompt pass (wavelet_discrete_layer.rs:102-128,
// compress_partial :260-266): feature c of output row j of sequence b is the
// low half of dwt_1d (wavelet_transform/dwt.rs:36-90) along the sequence,
//   v = 0 + t_0 lo[0] + ... + t_(L-1) lo[L-1],   t_l = sgn_l x[b][src_l][c],
// summed in that order (src -1: a padding zero; src[j][0] = -2 - r: row j is
// input row r unchanged, a target row of a stateless pass).  The tap table
// [S2][L] restates the reference's sequence padding on the host.
__global__ void k_dwt_rows(const double2* __restrict__ x, int B, int S, int d, const int* __restrict__ src,
                           const double* __restrict__ sgn, const double* __restrict__ lo, int L, int S2,
                           double2* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * S2 * d) return;
  const int c = (int)(i % d);
  const long bj = i / d;
  const int j = (int)(bj % S2), b = (int)(bj / S2);
  double2 v = make_double2(0.0, 0.0);
  const int s0 = src[j * L];
  if (s0 <= -2) {  // a target row of a stateless pass, passed through
    out[i] = x[((long)b * S + (-2 - s0)) * d + c];
    return;
  }
  for (int l = 0; l < L; ++l) {
    const int s = src[j * L + l];
    const double g = sgn[j * L + l];
    double2 t = make_double2(0.0, 0.0);
    if (s >= 0) {
      const double2 xv = x[((long)b * S + s) * d + c];
      t = make_double2(xv.x * g, xv.y * g);
    }
    v.x = v.x + t.x * lo[l];
    v.y = v.y + t.y * lo[l];
  }
  out[i] = v;
}

void dwt_rows(hipStream_t st, const double2* x, int B, int S, int d, const int* src, const double* sgn,
              const double* lo, int L, int S2, double2* out) {
  const long n = (long)B * S2 * d;
  if (n) hipLaunchKernelGGL(k_dwt_rows, dim3(cdiv_i(n, 256)), dim3(256), 0, st, x, B, S, d, src, sgn, lo, L, S2, out);
}

// NormalNormLayer::forward/normalize (norm_layer.rs:64-130): one wave per row,
// the row held in registers.  With `before`: x = Re(x + before) + 0i first.
template <int NPL>
__global__ __launch_bounds__(256) void k_layernorm(const double2* __restrict__ x, const double2* __restrict__ before,
                                                   double2* __restrict__ out, int rows, int d, double eps,
                                                   const double2* __restrict__ gamma, const double2* __restrict__ beta) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const double2* xr = x + (long)row * d;
  const double2* br = before ? before + (long)row * d : nullptr;
  double2 v[NPL];
  double sre = 0.0, sim = 0.0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = make_double2(0.0, 0.0);
    if (c < d) {
      double2 t = xr[c];
      if (br) t = make_double2(t.x + br[c].x, 0.0);  // add_matrix_3d_c (utils/matrix.rs:600-613)
      v[i] = t;
      sre += t.x;
      sim += t.y;
    }
  }
  sre = wave_sum(sre);
  sim = wave_sum(sim);
  const double len = (double)d;
  const double2 mean = make_double2(sre / len, sim / len);
  double vre = 0.0, vim = 0.0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + 64 * i;
    if (c < d) {
      double2 t = csub(v[i], mean);
      double2 tt = cmul(t, t);  // powu(2)
      vre += tt.x;
      vim += tt.y;
    }
  }
  vre = wave_sum(vre);
  vim = wave_sum(vim);
  const double2 var = make_double2(vre / len, vim / len);
  const double2 sd = csqrt_nc(make_double2(var.x + eps, var.y + 0.0));
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + 64 * i;
    if (c < d) {
      double2 o = cadd(cmul(cdiv(csub(v[i], mean), sd), gamma[c]), beta[c]);
      out[(long)row * d + c] = make_double2(o.x, 0.0);
    }
  }
}

void layernorm(hipStream_t st, const double2* x, const double2* before, double2* out, int rows, int d, double eps,
               const double2* gamma, const double2* beta) {
  dim3 grid(cdiv_i(rows, 4)), blk(256);
  const int npl = cdiv_i(d, 64);
  if (npl <= 1) hipLaunchKernelGGL(k_layernorm<1>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
  else if (npl <= 2) hipLaunchKernelGGL(k_layernorm<2>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
  else if (npl <= 4) hipLaunchKernelGGL(k_layernorm<4>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
  else if (npl <= 8) hipLaunchKernelGGL(k_layernorm<8>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
  else if (npl <= 12) hipLaunchKernelGGL(k_layernorm<12>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
  else hipLaunchKernelGGL(k_layernorm<16>, grid, blk, 0, st, x, before, out, rows, d, eps, gamma, beta);
}

__global__ void k_gather_rows(const double2* __restrict__ src, int S, int d, const uint32_t* __restrict__ lens, int B,
                              double2* __restrict__ dst) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * d) return;
  int b = (int)(i / d), c = (int)(i - (long)b * d);
  dst[i] = src[((long)b * S + (lens[b] - 1)) * d + c];
}

void gather_rows(hipStream_t st, const double2* src, int S, int d, const uint32_t* lens, int B, double2* dst) {
  hipLaunchKernelGGL(k_gather_rows, dim3(cdiv_i((long)B * d, 256)), dim3(256), 0, st, src, S, d, lens, B, dst);
}

// greedy_decoding (src/utils/sampling_methods.rs:5-18) on host-provided
// logits: max_by keeps the last of equal maxima; a NaN is an error
// (partial_cmp().unwrap() panics).  The token loop fuses this into the vocab
// GEMM instead (gemm.hip).
__global__ __launch_bounds__(256) void k_argmax(const double* __restrict__ logits, int V, uint32_t* __restrict__ ids,
                                                uint32_t* err) {
  __shared__ double sv[4];
  __shared__ int si[4];
  __shared__ int snan;
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) snan = 0;
  __syncthreads();
  const double* row = logits + (long)b * V;
  double bv = -INFINITY;
  int bi = -1;
  bool nan = false;
  for (int i = tid; i < V; i += 256) {
    const double v = row[i];
    if (isnan(v)) nan = true;
    else argmax_combine(bv, bi, v, i);
  }
  if (nan) snan = 1;
  wave_argmax(bv, bi);
  if ((tid & 63) == 0) sv[tid >> 6] = bv, si[tid >> 6] = bi;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_combine(bv, bi, sv[w], si[w]);
    if (snan || bi < 0) {
      atomicOr(err, (uint32_t)EB_ARGMAX_NAN);
      bi = 0;
    }
    ids[b] = (uint32_t)bi;
  }
}

void argmax_rows(hipStream_t st, const double* logits, int rows, int V, uint32_t* ids, uint32_t* err) {
  hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(256), 0, st, logits, V, ids, err);
}

// SoftmaxLayer::forward (softmax_output_layer.rs:40-64): TRAINING = every
// unpadded row, PRODUCTION = softmax_last_row (row S-1 only; activation.rs:409-419).
__global__ __launch_bounds__(256) void k_softmax_rows(const double2* __restrict__ lg, int S, int V,
                                                      const uint32_t* __restrict__ mask, int mode,
                                                      double* __restrict__ out) {
  __shared__ double red[8];
  const int row = blockIdx.x, tid = threadIdx.x;
  const double2* x = lg + (long)row * V;
  double* o = out + (long)row * V;
  const int s = row % S;
  const bool active = mode == 0 ? (mask[row] != 0) : (s == S - 1);
  if (!active) {
    for (int i = tid; i < V; i += 256) o[i] = 0.0;
    return;
  }
  double mx = -INFINITY;
  for (int i = tid; i < V; i += 256) mx = fmax(mx, x[i].x);
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
  double sum = 0.0;
  for (int i = tid; i < V; i += 256) {
    double e = exp(x[i].x - mx);
    o[i] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = sum;
  __syncthreads();
  sum = (red[4] + red[5]) + (red[6] + red[7]);
  for (int i = tid; i < V; i += 256) o[i] = o[i] / sum;
}

void softmax_rows(hipStream_t st, const double2* logits, int rows, int S, int V, const uint32_t* row_mask, int mode,
                  double* out) {
  hipLaunchKernelGGL(k_softmax_rows, dim3(rows), dim3(256), 0, st, logits, S, V, row_mask, mode, out);
}

// ===========================================================================
// Initialisation
// ===========================================================================
// Xavier-uniform (utils/weights_initializer.rs:73-89) from the counter generator.
__global__ void k_fill_seeded(double2* __restrict__ dst, int rows, int cols, long ld, uint64_t key, double lim) {
  long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * cols) return;
  long r = e / cols, c = e - r * cols;
  dst[r * ld + c] = make_double2(uniform_from_key(key, 2 * (uint64_t)e, lim), uniform_from_key(key, 2 * (uint64_t)e + 1, lim));
}
__global__ void k_fill_seeded_re(double* __restrict__ dst, int rows, int cols, long ld, uint64_t key, double lim) {
  long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * cols) return;
  long r = e / cols, c = e - r * cols;
  dst[r * ld + c] = uniform_from_key(key, 2 * (uint64_t)e, lim);
}
__global__ void k_fill_const(double2* __restrict__ dst, size_t n, double2 v) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = v;
}
__global__ void k_fill_int(int* __restrict__ dst, size_t n, int v) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = v;
}
__global__ void k_fill_u32(uint32_t* __restrict__ dst, size_t n, uint32_t v) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = v;
}

void fill_seeded(hipStream_t st, double2* dst, int rows, int cols, long ld, uint64_t key, double lim) {
  hipLaunchKernelGGL(k_fill_seeded, dim3(cdiv_i((long)rows * cols, 256)), dim3(256), 0, st, dst, rows, cols, ld, key, lim);
}
void fill_seeded_re(hipStream_t st, double* dst, int rows, int cols, long ld, uint64_t key, double lim) {
  hipLaunchKernelGGL(k_fill_seeded_re, dim3(cdiv_i((long)rows * cols, 256)), dim3(256), 0, st, dst, rows, cols, ld, key, lim);
}
void fill_const(hipStream_t st, double2* dst, size_t n, double2 v) {
  if (n) hipLaunchKernelGGL(k_fill_const, dim3(cdiv_i((long)n, 256)), dim3(256), 0, st, dst, n, v);
}
void fill_int(hipStream_t st, int* dst, size_t n, int v) {
  if (n) hipLaunchKernelGGL(k_fill_int, dim3(cdiv_i((long)n, 256)), dim3(256), 0, st, dst, n, v);
}
void fill_u32(hipStream_t st, uint32_t* dst, size_t n, uint32_t v) {
  if (n) hipLaunchKernelGGL(k_fill_u32, dim3(cdiv_i((long)n, 256)), dim3(256), 0, st, dst, n, v);
}

}  // namespace mitok
