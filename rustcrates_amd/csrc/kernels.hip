// kernels.hip — gfx950 (CDNA4) kernels of the complex-f64 transformer token loop.
//
// All tensors are row-major complex f64 (double2).  Wavefronts are 64 lanes.
// Reference math is cited per kernel (paths relative to src/neural_networks/).
#include <algorithm>

#include "kernels.hpp"

namespace mitok {

typedef double v4d __attribute__((ext_vector_type(4)));

static inline int cdiv_i(long a, long b) { return (int)((a + b - 1) / b); }

// ===========================================================================
// GEMM epilogue (shared by the MFMA kernel, the GEMV reduce and split-K reduce)
// ===========================================================================
__device__ __forceinline__ void apply_epi(const Epi& ep, int m, int n, double2 v) {
  if (ep.bias) v = cadd(v, ep.bias[n]);  // add_vector (utils/matrix.rs:615-625)
  switch (ep.mode) {
    case EPI_STORE:
      if (ep.check_finite && !(isfinite(v.x) && isfinite(v.y))) atomicOr(ep.err, (uint32_t)EB_FFN_NONFINITE);
      ep.out[(long)m * ep.ldo + n] = v;
      break;
    case EPI_GELU: {
      bool nan = false;
      if (ep.row_mask && ep.row_mask[m] == 0) v = make_double2(0.0, 0.0);  // activation.rs:268-284
      else v = gelu_nc(v, &nan);
      if (nan) atomicOr(ep.err, (uint32_t)EB_GELU_NAN);
      ep.out[(long)m * ep.ldo + n] = v;
      break;
    }
    case EPI_RE: ep.out_re[(long)m * ep.ldo + n] = v.x; break;
    case EPI_QKV: {
      if (n < ep.d) {
        ep.out[(long)m * ep.ldo + n] = v;
        break;
      }
      const int part = n < 2 * ep.d ? 1 : 2;
      const int c = n - part * ep.d;
      const int h = c / ep.dh, e = c - h * ep.dh;
      const int b = m / ep.S, s = m - b * ep.S;
      if (ep.kv_row && ep.kv_row[b] != s) break;  // decode branch: only the last token (masked_attention_head.rs:140-156)
      const int pos = (ep.kv_base ? ep.kv_base[b] : 0) + (ep.kv_row ? 0 : s);
      if (pos >= ep.ctx) {
        atomicOr(ep.err, (uint32_t)EB_CTX_OVERFLOW);
        break;
      }
      double2* dst = part == 1 ? ep.kc : ep.vc;
      dst[(((long)b * ep.heads + h) * ep.ctx + pos) * ep.dh + e] = v;
      break;
    }
  }
}

// ===========================================================================
// GEMV for M <= 8 rows: HBM-bound weight stream.  Block = 4 waves x 64 columns;
// each wave walks its own kw rows of W with 8 loads in flight per lane, the
// four waves are summed in LDS, and blockIdx.y's partial goes to ws[y][m][n].
// ===========================================================================
template <int MR, bool RE>
__global__ __launch_bounds__(256) void k_gemv(const double2* __restrict__ X, long ldx, int M,
                                              const double2* __restrict__ W, long ldw, int N, int K, int kw,
                                              void* __restrict__ ws) {
  extern __shared__ double2 xs[];  // [MR][4*kw]
  __shared__ double2 red[3][MR][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KB = 4 * kw;
  const int kb0 = blockIdx.y * KB;
  for (int i = threadIdx.x; i < MR * KB; i += 256) {
    int m = i / KB, kk = i - m * KB, k = kb0 + kk;
    xs[i] = (m < M && k < K) ? X[(long)m * ldx + k] : make_double2(0.0, 0.0);
  }
  __syncthreads();
  const int n = blockIdx.x * 64 + lane;
  double2 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = make_double2(0.0, 0.0);
  const int k0 = kb0 + wave * kw;
  const int kmax = min(kw, K - k0);
  if (n < N && kmax > 0) {
    const double2* wp = W + (long)k0 * ldw + n;
    const double2* xw = xs + wave * kw;
    int kk = 0;
    for (; kk + 8 <= kmax; kk += 8) {
      double2 w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = wp[(long)(kk + u) * ldw];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          double2 x = xw[m * KB + kk + u];
          if (RE) acc[m].x += x.x * w[u].x - x.y * w[u].y;
          else acc[m] = cadd(acc[m], cmul(x, w[u]));
        }
    }
    for (; kk < kmax; ++kk) {
      double2 w = wp[(long)kk * ldw];
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        double2 x = xw[m * KB + kk];
        if (RE) acc[m].x += x.x * w.x - x.y * w.y;
        else acc[m] = cadd(acc[m], cmul(x, w));
      }
    }
  }
  if (wave > 0)
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave - 1][m][lane] = acc[m];
  __syncthreads();
  if (wave == 0 && n < N) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) break;
      double2 v = acc[m];
      v = cadd(v, red[0][m][lane]);
      v = cadd(v, red[1][m][lane]);
      v = cadd(v, red[2][m][lane]);
      long o = ((long)blockIdx.y * M + m) * N + n;
      if (RE) ((double*)ws)[o] = v.x;
      else ((double2*)ws)[o] = v;
    }
  }
}

// Sum of the P split-K partials, then the epilogue.
__global__ __launch_bounds__(256) void k_reduce_epi(const double2* __restrict__ ws, int P, int M, int N, Epi ep) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * N) return;
  int m = (int)(i / N), n = (int)(i - (long)m * N);
  double2 v = ws[i];
  for (int p = 1; p < P; ++p) v = cadd(v, ws[(long)p * M * N + i]);
  apply_epi(ep, m, n, v);
}

__global__ __launch_bounds__(256) void k_reduce_epi_re(const double* __restrict__ ws, int P, int M, int N, Epi ep) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * N) return;
  int m = (int)(i / N), n = (int)(i - (long)m * N);
  double v = ws[i];
  for (int p = 1; p < P; ++p) v += ws[(long)p * M * N + i];
  if (ep.bias) v += ep.bias[n].x;
  ep.out_re[(long)m * ep.ldo + n] = v;
}

// ===========================================================================
// MFMA complex GEMM.  Block tile 64x64 (4 waves of 32x32), K step 16, operands
// de-interleaved into re/im planes in LDS (double-buffered).  Per 16x16x4 step
// a wave issues 4 v_mfma_f64_16x16x4_f64 per output tile:
//     Cr += Ar*Br;  Cr += (-Ai)*Bi;  Ci += Ar*Bi;  Ci += Ai*Br
// Lane layout of v_mfma_f64_16x16x4_f64 (wave64): A[i][k] at lane i+16k,
// B[k][j] at lane j+16k, D[i][j] at lane j+16*(i%4), element i/4 (unlike the
// f32 16x16x4 form, consecutive output rows sit in consecutive lane groups).
// ===========================================================================
constexpr int GBM = 64, GBN = 64, GBK = 16, GPAD = 4;

__global__ __launch_bounds__(256) void k_zgemm_mfma(const double2* __restrict__ A, long lda,
                                                       const double2* __restrict__ Bm, long ldb, int M, int N, int K,
                                                       int kchunk, Epi ep, double2* __restrict__ ws) {
  __shared__ double As[2][2][GBK][GBM + GPAD];
  __shared__ double Bs[2][2][GBK][GBN + GPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int a_row = tid >> 2, a_k = (tid & 3) * 4;
  const int b_k = tid >> 4, b_n = (tid & 15) * 4;

  double2 ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int m = m0 + a_row, k = k0 + a_k + i;
      ra[i] = (m < M && k < kend) ? A[(long)m * lda + k] : make_double2(0.0, 0.0);
      int kb = k0 + b_k, n = n0 + b_n + i;
      rb[i] = (kb < kend && n < N) ? Bm[(long)kb * ldb + n] : make_double2(0.0, 0.0);
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      As[st][0][a_k + i][a_row] = ra[i].x;
      As[st][1][a_k + i][a_row] = ra[i].y;
      Bs[st][0][b_k][b_n + i] = rb[i].x;
      Bs[st][1][b_k][b_n + i] = rb[i].y;
    }
  };

  v4d cr[2][2], ci[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) cr[i][j] = ci[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

  const int nk = kend > kbeg ? (kend - kbeg + GBK - 1) / GBK : 0;
  if (nk > 0) {
    gload(kbeg);
    sstore(0);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int st = it & 1;
    if (it + 1 < nk) gload(kbeg + (it + 1) * GBK);
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 4) {
      const int kr = kk + (lane >> 4);
      double ar[2], ai[2], br[2], bi[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ar[i] = As[st][0][kr][wm + 16 * i + (lane & 15)];
        ai[i] = As[st][1][kr][wm + 16 * i + (lane & 15)];
        br[i] = Bs[st][0][kr][wn + 16 * i + (lane & 15)];
        bi[i] = Bs[st][1][kr][wn + 16 * i + (lane & 15)];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          cr[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[i], br[j], cr[i][j], 0, 0, 0);
          ci[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[i], bi[j], ci[i][j], 0, 0, 0);
          cr[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(-ai[i], bi[j], cr[i][j], 0, 0, 0);
          ci[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ai[i], br[j], ci[i][j], 0, 0, 0);
        }
    }
    if (it + 1 < nk) sstore(st ^ 1);
    __syncthreads();
  }

  const bool split = gridDim.z > 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + 16 * i + (lane >> 4) + 4 * r;
        const int n = n0 + wn + 16 * j + (lane & 15);
        if (m < M && n < N) {
          double2 v = make_double2(cr[i][j][r], ci[i][j][r]);
          if (split) ws[((long)blockIdx.z * M + m) * N + n] = v;
          else apply_epi(ep, m, n, v);
        }
      }
}

// ---- GEMM dispatch --------------------------------------------------------
struct GemvPlan {
  int mr, kw, P, ncb;
};
static GemvPlan plan_gemv(int M, int N, int K) {
  GemvPlan p;
  p.mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  p.ncb = cdiv_i(N, 64);
  int P = std::max(1, cdiv_i(1024, p.ncb));
  int kw = std::max(8, cdiv_i(cdiv_i(K, 4 * P), 8) * 8);
  p.kw = kw;
  p.P = cdiv_i(K, 4 * kw);
  return p;
}
struct MfmaPlan {
  int P, kchunk, mt, nt;
};
static MfmaPlan plan_mfma(int M, int N, int K) {
  MfmaPlan p;
  p.mt = cdiv_i(M, GBM);
  p.nt = cdiv_i(N, GBN);
  int tiles = p.mt * p.nt;
  int P = 1;
  if (tiles < 512) P = std::min(cdiv_i(512, tiles), std::max(1, K / 64));
  p.kchunk = cdiv_i(cdiv_i(K, P), GBK) * GBK;
  p.P = cdiv_i(K, p.kchunk);
  return p;
}

size_t gemm_ws_bytes(int M, int N, int K, int mode) {
  if (M <= 8) {
    GemvPlan p = plan_gemv(M, N, K);
    return (size_t)p.P * M * N * (mode == EPI_RE ? sizeof(double) : sizeof(double2));
  }
  MfmaPlan p = plan_mfma(M, N, K);
  return p.P > 1 ? (size_t)p.P * M * N * sizeof(double2) : 0;
}

template <int MR>
static void launch_gemv(hipStream_t st, const GemvPlan& p, const double2* A, long lda, int M, const double2* B, long ldb,
                        int N, int K, bool re, void* ws) {
  dim3 grid(p.ncb, p.P);
  size_t shm = (size_t)MR * 4 * p.kw * sizeof(double2);
  if (re) hipLaunchKernelGGL((k_gemv<MR, true>), grid, dim3(256), shm, st, A, lda, M, B, ldb, N, K, p.kw, ws);
  else hipLaunchKernelGGL((k_gemv<MR, false>), grid, dim3(256), shm, st, A, lda, M, B, ldb, N, K, p.kw, ws);
}

void gemm(hipStream_t st, int M, int N, int K, const double2* A, long lda, const double2* B, long ldb, const Epi& ep,
          void* ws) {
  if (M <= 0 || N <= 0) return;
  const long total = (long)M * N;
  if (M <= 8) {
    GemvPlan p = plan_gemv(M, N, K);
    const bool re = ep.mode == EPI_RE;
    switch (p.mr) {
      case 1: launch_gemv<1>(st, p, A, lda, M, B, ldb, N, K, re, ws); break;
      case 2: launch_gemv<2>(st, p, A, lda, M, B, ldb, N, K, re, ws); break;
      case 4: launch_gemv<4>(st, p, A, lda, M, B, ldb, N, K, re, ws); break;
      default: launch_gemv<8>(st, p, A, lda, M, B, ldb, N, K, re, ws); break;
    }
    if (re) hipLaunchKernelGGL(k_reduce_epi_re, dim3(cdiv_i(total, 256)), dim3(256), 0, st, (const double*)ws, p.P, M, N, ep);
    else hipLaunchKernelGGL(k_reduce_epi, dim3(cdiv_i(total, 256)), dim3(256), 0, st, (const double2*)ws, p.P, M, N, ep);
    return;
  }
  MfmaPlan p = plan_mfma(M, N, K);
  dim3 grid(p.nt, p.mt, p.P);
  hipLaunchKernelGGL(k_zgemm_mfma, grid, dim3(256), 0, st, A, lda, B, ldb, M, N, K, p.kchunk, ep, (double2*)ws);
  if (p.P > 1)
    hipLaunchKernelGGL(k_reduce_epi, dim3(cdiv_i(total, 256)), dim3(256), 0, st, (const double2*)ws, p.P, M, N, ep);
}

// ===========================================================================
// Attention, one block per (query row, head, sequence).
// MaskedAttentionHead::forward (masked_attention_head.rs:184-208): scores are
// Re(q.k) * 1/(1e-8 + sqrt(dh)) + Re(bias_pos[r][c]); the S x S causal mask is
// applied modulo its size (:494-503) so key c is visible iff (c % S) <= r;
// masked entries are -1e12; softmax of the real part (activation.rs:431-439);
// padded query rows give 0 (:369-388); out = sum_c p_c * v_c (matrix.rs:356-380).
// ===========================================================================
__global__ __launch_bounds__(256) void k_attention_rows(Attn a) {
  extern __shared__ double smem[];
  const int r = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const long row = (long)b * a.S + r;
  double2* out = a.out + row * a.ldo + (long)h * a.dh;
  if (a.row_mask && a.row_mask[row] == 0) {
    for (int e = tid; e < a.dh; e += 256) out[e] = make_double2(0.0, 0.0);
    return;
  }
  const int T = a.kv_len ? a.kv_len[b] + a.T_add : a.T_const;
  double* sc = smem;                                  // [T_max]
  double2* qs = (double2*)(smem + a.T_max);          // [dh]
  double2* pv = qs + a.dh;                           // [256]
  double* wred = (double*)(pv + 256);                // [8]
  for (int e = tid; e < a.dh; e += 256) qs[e] = a.q[row * a.ldq + (long)h * a.dh + e];
  __syncthreads();
  const double2* K = a.kc + ((long)b * a.H + h) * a.ctx * a.dh;
  const double2* V = a.vc + ((long)b * a.H + h) * a.ctx * a.dh;
  const double* bp = a.bias_re + ((long)h * a.mc + r) * a.mc;
  double lmax = -INFINITY;
  for (int c = tid; c < T; c += 256) {
    double s;
    if ((c % a.S) > r) {
      s = -1e12;
    } else {
      const double2* kr = K + (long)c * a.dh;
      double acc = 0.0;
      for (int e = 0; e < a.dh; ++e) {
        double2 kv = kr[e], qv = qs[e];
        acc += qv.x * kv.x - qv.y * kv.y;
      }
      s = acc * a.scale + bp[c];
    }
    sc[c] = s;
    lmax = fmax(lmax, s);
  }
  lmax = wave_max(lmax);
  if ((tid & 63) == 0) wred[tid >> 6] = lmax;
  __syncthreads();
  const double mx = fmax(fmax(wred[0], wred[1]), fmax(wred[2], wred[3]));
  __syncthreads();
  double lsum = 0.0;
  for (int c = tid; c < T; c += 256) {
    double e = exp(sc[c] - mx);
    sc[c] = e;
    lsum += e;
  }
  lsum = wave_sum(lsum);
  if ((tid & 63) == 0) wred[4 + (tid >> 6)] = lsum;
  __syncthreads();
  const double sum = (wred[4] + wred[5]) + (wred[6] + wred[7]);
  const int G = 256 / a.dh;
  const int e = tid % a.dh, g = tid / a.dh;
  double2 acc = make_double2(0.0, 0.0);
  if (g < G)
    for (int c = g; c < T; c += G) {
      double p = sc[c] / sum;
      double2 v = V[(long)c * a.dh + e];
      acc.x += p * v.x;
      acc.y += p * v.y;
    }
  pv[tid] = acc;
  __syncthreads();
  if (tid < a.dh) {
    double2 s = pv[tid];
    for (int gg = 1; gg < G; ++gg) s = cadd(s, pv[gg * a.dh + tid]);
    out[tid] = s;
  }
}

void attention_rows(hipStream_t st, const Attn& a) {
  size_t shm = (size_t)a.T_max * sizeof(double) + (size_t)(a.dh + 256) * sizeof(double2) + 8 * sizeof(double);
  hipLaunchKernelGGL(k_attention_rows, dim3(a.S, a.H, a.B), dim3(256), shm, st, a);
}

// ---- split-key decode attention (one query row per sequence) ----
constexpr int DEC_CHUNK = 16;  // keys per block

__global__ __launch_bounds__(256) void k_attention_decode_part(Attn a, double* __restrict__ pm,
                                                               double* __restrict__ pl, double2* __restrict__ po,
                                                               int nsplit) {
  __shared__ double sc[DEC_CHUNK];
  __shared__ double2 pv[256];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.kv_len ? a.kv_len[b] + a.T_add : a.T_const;
  const int c0 = split * DEC_CHUNK;
  const long pidx = ((long)b * a.H + h) * nsplit + split;
  if (c0 >= T) return;  // the combine reads only ceil(T / DEC_CHUNK) splits
  const int nc = min(DEC_CHUNK, T - c0);
  const long row = b;  // S == 1
  const double2* qrow = a.q + row * a.ldq + (long)h * a.dh;
  const double2* K = a.kc + ((long)b * a.H + h) * a.ctx * a.dh;
  const double2* V = a.vc + ((long)b * a.H + h) * a.ctx * a.dh;
  // wave w scores keys c0 + w, c0 + w + 4, ...; lanes split the head dim
  for (int j = wave; j < nc; j += 4) {
    const double2* kr = K + (long)(c0 + j) * a.dh;
    double acc = 0.0;
    for (int e = lane; e < a.dh; e += 64) {
      double2 kv = kr[e], qv = qrow[e];
      acc += qv.x * kv.x - qv.y * kv.y;
    }
    acc = wave_sum(acc);
    if (lane == 0) sc[j] = acc * a.scale + a.bias_re[(long)h * a.mc * a.mc + c0 + j];  // bias_pos row 0
  }
  __syncthreads();
  double mloc = -INFINITY;
  for (int j = 0; j < nc; ++j) mloc = fmax(mloc, sc[j]);
  const int G = 256 / a.dh;
  const int e = tid % a.dh, g = tid / a.dh;
  double2 acc = make_double2(0.0, 0.0);
  double lsum = 0.0;
  if (g < G) {
    for (int j = g; j < nc; j += G) {
      double p = exp(sc[j] - mloc);
      double2 v = V[(long)(c0 + j) * a.dh + e];
      acc.x += p * v.x;
      acc.y += p * v.y;
    }
  }
  if (tid == 0)
    for (int j = 0; j < nc; ++j) lsum += exp(sc[j] - mloc);
  pv[tid] = acc;
  __syncthreads();
  if (tid < a.dh) {
    double2 s = pv[tid];
    for (int gg = 1; gg < G; ++gg) s = cadd(s, pv[gg * a.dh + tid]);
    po[pidx * a.dh + tid] = s;
  }
  if (tid == 0) {
    pm[pidx] = mloc;
    pl[pidx] = lsum;
  }
}

__global__ __launch_bounds__(256) void k_attention_decode_combine(Attn a, const double* __restrict__ pm,
                                                                  const double* __restrict__ pl,
                                                                  const double2* __restrict__ po, int nsplit) {
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int T = a.kv_len ? a.kv_len[b] + a.T_add : a.T_const;
  const int ns = (T + DEC_CHUNK - 1) / DEC_CHUNK;
  const long base = ((long)b * a.H + h) * nsplit;
  double2* out = a.out + (long)b * a.ldo + (long)h * a.dh;
  if (a.row_mask && a.row_mask[b] == 0) {
    for (int e = tid; e < a.dh; e += 256) out[e] = make_double2(0.0, 0.0);
    return;
  }
  double m = -INFINITY;
  for (int s = 0; s < ns; ++s) m = fmax(m, pm[base + s]);
  double L = 0.0;
  for (int s = 0; s < ns; ++s) L += pl[base + s] * exp(pm[base + s] - m);
  for (int e = tid; e < a.dh; e += 256) {
    double2 o = make_double2(0.0, 0.0);
    for (int s = 0; s < ns; ++s) {
      double w = exp(pm[base + s] - m);
      double2 v = po[(base + s) * a.dh + e];
      o.x += v.x * w;
      o.y += v.y * w;
    }
    out[e] = make_double2(o.x / L, o.y / L);
  }
}

size_t attention_decode_ws_bytes(int B, int H, int dh, int T_max) {
  int ns = cdiv_i(T_max, DEC_CHUNK);
  return (size_t)B * H * ns * (2 * sizeof(double) + dh * sizeof(double2));
}

void attention_decode(hipStream_t st, const Attn& a, void* ws) {
  const int ns = cdiv_i(a.T_max, DEC_CHUNK);
  double* pm = (double*)ws;
  double* pl = pm + (long)a.B * a.H * ns;
  double2* po = (double2*)(pl + (long)a.B * a.H * ns);
  hipLaunchKernelGGL(k_attention_decode_part, dim3(ns, a.H, a.B), dim3(256), 0, st, a, pm, pl, po, ns);
  hipLaunchKernelGGL(k_attention_decode_combine, dim3(a.H, a.B), dim3(256), 0, st, a, pm, pl, po, ns);
}

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
// (cos, sin) of the clamped angle tabulated on the host with libm.
__global__ void k_rope(double2* __restrict__ x, int rows, int d, const double2* __restrict__ cs, int max_pos,
                       const int* __restrict__ pos, const int* __restrict__ kv_len, uint32_t* err) {
  const int half = d / 2;
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * half) return;
  int r = (int)(i / half), k = (int)(i - (long)r * half);
  int p = pos ? pos[r] : kv_len[r];
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
          const int* kv_len, uint32_t* err) {
  long n = (long)rows * (d / 2);
  hipLaunchKernelGGL(k_rope, dim3(cdiv_i(n, 256)), dim3(256), 0, st, x, rows, d, cs_table, max_pos, pos, kv_len, err);
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

// greedy_decoding (src/utils/sampling_methods.rs:5-18): max_by keeps the last
// of equal maxima; a NaN is an error (partial_cmp().unwrap() panics).
__global__ __launch_bounds__(256) void k_argmax(const double* __restrict__ logits, int V, uint32_t* __restrict__ ids,
                                                uint32_t* hist, int hist_stride, int* hist_cnt, int* kv_len,
                                                int advance_kv, uint32_t* err) {
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
    double v = row[i];
    if (isnan(v)) nan = true;
    else if (bi < 0 || v >= bv) bv = v, bi = i;
  }
  if (nan) snan = 1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    double ov = __shfl_xor(bv, o, 64);
    int oi = __shfl_xor(bi, o, 64);
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) bv = ov, bi = oi;
  }
  if ((tid & 63) == 0) sv[tid >> 6] = bv, si[tid >> 6] = bi;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      if (si[w] >= 0 && (bi < 0 || sv[w] > bv || (sv[w] == bv && si[w] > bi))) bv = sv[w], bi = si[w];
    if (snan || bi < 0) {
      atomicOr(err, (uint32_t)EB_ARGMAX_NAN);
      bi = 0;
    }
    ids[b] = (uint32_t)bi;
    if (hist) {
      int t = hist_cnt[b];
      hist[(long)b * hist_stride + t] = (uint32_t)bi;
      hist_cnt[b] = t + 1;
    }
    if (advance_kv) kv_len[b] += 1;
  }
}

void argmax_rows(hipStream_t st, const double* logits, int rows, int V, uint32_t* ids, uint32_t* hist, int hist_stride,
                 int* hist_cnt, int* kv_len, int advance_kv, uint32_t* err) {
  hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(256), 0, st, logits, V, ids, hist, hist_stride, hist_cnt, kv_len,
                     advance_kv, err);
}

__global__ void k_store_logits(const double* __restrict__ logits, long n, double* __restrict__ hist,
                               const int* __restrict__ hist_cnt) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  hist[(long)hist_cnt[0] * n + i] = logits[i];
}

void store_logits(hipStream_t st, const double* logits, int rows, int V, double* hist, const int* hist_cnt) {
  long n = (long)rows * V;
  hipLaunchKernelGGL(k_store_logits, dim3(cdiv_i(n, 256)), dim3(256), 0, st, logits, n, hist, hist_cnt);
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
__global__ void k_copy_re(const double2* __restrict__ src, double* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i].x;
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
void copy_re(hipStream_t st, const double2* src, double* dst, size_t n) {
  if (n) hipLaunchKernelGGL(k_copy_re, dim3(cdiv_i((long)n, 256)), dim3(256), 0, st, src, dst, n);
}

}  // namespace mitok
