// gemm.hip — complex-f64 products of the token loop on gfx950.
//
// multiply_complex (utils/matrix.rs:16-65) is zgemm with alpha 1, beta 0 on
// row-major [in][out] weights.  Here every product is fused with what the
// reference does around it:
//   prologue  the row transform of the layers before it: embedding gather
//             (embedding_layer.rs:158-211), RoPE (positional_encoding_layer.rs:
//             181-209), residual Re(x + before) (utils/matrix.rs:600-613) and
//             NormalNormLayer (norm_layer.rs:64-130)   [GEMV only]
//   epilogue  bias (utils/matrix.rs:615-625), GELU with pad rows zeroed
//             (layer.rs:132-166, activation.rs:195-212,268-284), KV-cache append
//             (masked_attention_head.rs:135-178), Re-logits
//             (data_converter.rs:244-256) and greedy_decoding
//             (src/utils/sampling_methods.rs:5-18).
// Split-K partials are finished inside the same launch by the block that
// arrives last (arrive_last), summed in split order so results do not depend
// on arrival order.
#include <algorithm>

#include "kernels.hpp"

namespace mitok {

typedef double v4d __attribute__((ext_vector_type(4)));

static inline int cdiv_i(long a, long b) { return (int)((a + b - 1) / b); }

// ===========================================================================
// epilogue: returns Re of the stored value (used by the fused argmax)
// ===========================================================================
__device__ __forceinline__ double apply_epi(const Epi& ep, int M, int N, int m, int n, double2 v) {
  if (ep.bias) v = cadd(v, ep.bias[n]);
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
    case EPI_RE:
      ep.out_re[(long)m * ep.ldo + n] = v.x;
      if (ep.hist_re) ep.hist_re[((long)ep.hist_cnt[0] * M + m) * N + n] = v.x;
      break;
    case EPI_QKV: {
      if (n < ep.d) {
        ep.out[(long)m * ep.ldo + n] = v;
        break;
      }
      const int part = n < 2 * ep.d ? 1 : 2;
      const int c = n - part * ep.d;
      const int h = c / ep.dh, e = c - h * ep.dh;
      const int b = m / ep.S, s = m - b * ep.S;
      if (ep.kv_row && ep.kv_row[b] != s) break;  // cached branch: only the last token (masked_attention_head.rs:140-156)
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
  return v.x;
}

// greedy_decoding finish: one block per row reduces that row's per-tile
// (max, last index) partials, then stores the id, appends it to the history
// and advances the sequence's KV length.
__global__ __launch_bounds__(256) void k_argmax_finalize(Argmax am, int tiles) {
  __shared__ double sv[4];
  __shared__ int si[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double bv = -INFINITY;
  int bi = -1;
  for (int t = tid; t < tiles; t += 256) argmax_combine(bv, bi, am.part_v[(long)m * tiles + t], am.part_i[(long)m * tiles + t]);
  wave_argmax(bv, bi);
  if (lane == 0) sv[wave] = bv, si[wave] = bi;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_combine(bv, bi, sv[w], si[w]);
    if (bi < 0) {  // every logit was NaN (the reference panics)
      atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
      bi = 0;
    }
    am.ids[m] = (uint32_t)bi;
    if (am.hist) {
      const int t = am.hist_cnt[m];
      am.hist[(long)m * am.hist_stride + t] = (uint32_t)bi;
      am.hist_cnt[m] = t + 1;
    }
    if (am.advance_kv) am.kv_len[m] += 1;
  }
}

// ===========================================================================
// prologue (row transform) on the fly
// ===========================================================================
__device__ __forceinline__ double2 ro_raw(const RowOps& r, int m, int k, int K) {
  if (r.table) {
    const uint32_t id = r.ids[m];
    if (id == 1u || id >= (uint32_t)r.vocab) return make_double2(0.0, 0.0);  // PAD; bad ids flagged by ro_check
    return r.table[(long)id * K + k];
  }
  return r.x[(long)m * r.ldx + k];
}

// source element with RoPE (pairs (2i, 2i+1) rotate by the tabulated angle)
__device__ __forceinline__ double2 ro_source(const RowOps& r, int m, int k, int K) {
  if (!r.rope_cs) return ro_raw(r, m, k, K);
  const int p = min(r.rope_pos[m], r.rope_max - 1);  // overflow flagged by ro_check
  const int i = k >> 1;
  const double2 t = r.rope_cs[(long)p * (K >> 1) + i];
  const double2 e = ro_raw(r, m, 2 * i, K), o = ro_raw(r, m, 2 * i + 1, K);
  return (k & 1) ? make_double2(e.x * t.y + o.x * t.x, e.y * t.y + o.y * t.x)
                 : make_double2(e.x * t.x - o.x * t.y, e.y * t.x - o.y * t.y);
}

__device__ __forceinline__ double2 ro_value(const RowOps& r, int m, int k, int K) {
  double2 v = ro_source(r, m, k, K);
  if (r.resid) v = make_double2(v.x + r.resid[(long)m * r.ldr + k].x, 0.0);
  return v;
}

__device__ __forceinline__ void ro_check(const RowOps& r, int m) {
  if (r.table && r.ids[m] != 1u && r.ids[m] >= (uint32_t)r.vocab) atomicOr(r.err, (uint32_t)EB_BAD_TOKEN);
  if (r.rope_cs && r.rope_pos[m] >= r.rope_max) atomicOr(r.err, (uint32_t)EB_CTX_OVERFLOW);
}

// normalize (norm_layer.rs:77): Re(((x - mean) / sd) * gamma + beta) + 0i
__device__ __forceinline__ double2 ln_apply(double2 v, double2 mean, double2 sd, double2 g, double2 b) {
  const double2 o = cadd(cmul(cdiv(csub(v, mean), sd), g), b);
  return make_double2(o.x, 0.0);
}

// LayerNorm statistics of rows m0 .. m0+M-1 (M <= MR) over K elements:
// mean = sum(x) / K, var = sum((x - mean)^2) / K (complex square),
// sd = csqrt(var + eps) (norm_layer.rs:64-80).  Block-wide; all threads call it.
template <int MR>
__device__ void ro_stats(const RowOps& r, int m0, int M, int K, double2* mean_s, double2* sd_s) {
  __shared__ double red_s[4][2 * MR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double a[2 * MR];
  const double len = (double)K;
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = 0.0;
  for (int k = tid; k < K; k += 256)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) {
        const double2 v = ro_value(r, m0 + m, k, K);
        a[2 * m] += v.x;
        a[2 * m + 1] += v.y;
      }
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = wave_sum(a[j]);
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < 2 * MR; ++j) red_s[wave][j] = a[j];
  __syncthreads();
  if (tid < M) {
    const double sre = (red_s[0][2 * tid] + red_s[1][2 * tid]) + (red_s[2][2 * tid] + red_s[3][2 * tid]);
    const double sim = (red_s[0][2 * tid + 1] + red_s[1][2 * tid + 1]) + (red_s[2][2 * tid + 1] + red_s[3][2 * tid + 1]);
    mean_s[tid] = make_double2(sre / len, sim / len);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = 0.0;
  for (int k = tid; k < K; k += 256)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) {
        const double2 t = csub(ro_value(r, m0 + m, k, K), mean_s[m]);
        const double2 tt = cmul(t, t);
        a[2 * m] += tt.x;
        a[2 * m + 1] += tt.y;
      }
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = wave_sum(a[j]);
  __syncthreads();  // red_s reuse
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < 2 * MR; ++j) red_s[wave][j] = a[j];
  __syncthreads();
  if (tid < M) {
    const double vre = (red_s[0][2 * tid] + red_s[1][2 * tid]) + (red_s[2][2 * tid] + red_s[3][2 * tid]);
    const double vim = (red_s[0][2 * tid + 1] + red_s[1][2 * tid + 1]) + (red_s[2][2 * tid + 1] + red_s[3][2 * tid + 1]);
    sd_s[tid] = csqrt_nc(make_double2(vre / len + r.eps, vim / len + 0.0));
  }
  __syncthreads();
}

// ===========================================================================
// GEMV for M <= 8 rows: HBM-bound weight stream.  A block owns C columns and a
// K range of 4*kw rows; lane (r, c) = (lane / C, lane % C) reads row r of each
// group of 64/C rows, so one wave instruction covers 64/C rows x C columns.
// The first 8 weight loads per lane are in flight while the prologue builds
// the block's input rows in LDS.  Lanes of a column are summed by shuffles,
// the 4 waves through LDS; blockIdx.y splits K (at most 8 ways, so few blocks
// meet at each completion counter).
// ===========================================================================
constexpr int GEMV_MAX_SPLIT = 8;
constexpr int SKINNY_MAX_SPLIT = 8;

template <int MR, int C>
__global__ __launch_bounds__(256) void k_gemv(RowOps ro, int M, const double2* __restrict__ W, long ldw, int N, int K,
                                              int kw, Epi ep, Argmax am, double2* __restrict__ ws,
                                              uint32_t* __restrict__ cnt) {
  constexpr int RPW = 64 / C;  // rows per wave instruction
  extern __shared__ double2 xs[];  // [MR][4*kw]
  __shared__ double2 red[3][MR][C];
  __shared__ double2 st_mean[MR], st_sd[MR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane / C, c = lane - (lane / C) * C;
  const int KB = 4 * kw;
  const int kb0 = blockIdx.y * KB;
  const int n = blockIdx.x * C + c;
  const bool col_ok = n < N;
  const int k0 = kb0 + wave * kw;
  const int kmax = max(0, min(kw, K - k0));
  const int nu = kmax > r ? (kmax - r + RPW - 1) / RPW : 0;  // rows k0 + r + u*RPW, u < nu
  const double2* wp = W + (long)(k0 + r) * ldw + n;
  const long wstep = (long)RPW * ldw;

  double2 w[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) w[u] = (col_ok && u < nu) ? wp[u * wstep] : make_double2(0.0, 0.0);

  if (ro.ln) ro_stats<MR>(ro, 0, M, K, st_mean, st_sd);
  if (blockIdx.x == 0 && blockIdx.y == 0 && tid < M) ro_check(ro, tid);
  for (int i = tid; i < MR * KB; i += 256) {
    const int m = i / KB, kk = i - m * KB, k = kb0 + kk;
    double2 v = make_double2(0.0, 0.0);
    if (m < M && k < K) {
      v = ro_value(ro, m, k, K);
      if (ro.ln) v = ln_apply(v, st_mean[m], st_sd[m], ro.gamma[k], ro.beta[k]);
      if (ro.save && blockIdx.x == 0) ro.save[(long)m * ro.ldsave + k] = v;
    }
    xs[i] = v;
  }
  __syncthreads();

  double2 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = make_double2(0.0, 0.0);
  if (col_ok) {
    const double2* xw = xs + wave * kw + r;  // row u of this lane: xw[m * KB + u * RPW]
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < nu)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * KB + u * RPW], w[u]));
    int u0 = 8;
    for (; u0 + 8 <= nu; u0 += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = wp[(u0 + u) * wstep];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * KB + (u0 + u) * RPW], w[u]));
    }
    for (; u0 < nu; ++u0) {
      const double2 wv = wp[u0 * wstep];
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * KB + u0 * RPW], wv));
    }
  }
  // lanes of one column (same c, r = 0 .. RPW-1) -> r = 0
#pragma unroll
  for (int o = C; o < 64; o <<= 1)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      acc[m].x += __shfl_xor(acc[m].x, o, 64);
      acc[m].y += __shfl_xor(acc[m].y, o, 64);
    }
  if (wave > 0 && lane < C)
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave - 1][m][lane] = acc[m];
  __syncthreads();
  const bool owner = wave == 0 && lane < C;  // lane c of wave 0 owns column n
  if (owner)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = cadd(cadd(cadd(acc[m], red[0][m][lane]), red[1][m][lane]), red[2][m][lane]);

  const int P = gridDim.y;
  if (P > 1) {
    if (owner && col_ok)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) st_dev(&ws[((long)blockIdx.y * M + m) * N + n], acc[m]);
    if (!arrive_last(&cnt[blockIdx.x], (uint32_t)P)) return;
    if (owner && col_ok)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) {
          double2 pv[GEMV_MAX_SPLIT];  // all loads in flight, then summed in split order
#pragma unroll
          for (int p = 0; p < GEMV_MAX_SPLIT; ++p)
            pv[p] = p < P ? ld_dev(&ws[((long)p * M + m) * N + n]) : make_double2(0.0, 0.0);
          double2 v = pv[0];
#pragma unroll
          for (int p = 1; p < GEMV_MAX_SPLIT; ++p)
            if (p < P) v = cadd(v, pv[p]);
          acc[m] = v;
        }
  }

  double re[MR];
  if (owner && col_ok)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) re[m] = apply_epi(ep, M, N, m, n, acc[m]);
  if (!am.part_v || wave != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m)
    if (m < M) {
      double bv = -INFINITY;
      int bi = -1;
      if (lane < C && col_ok) {
        if (isnan(re[m])) atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
        else bv = re[m], bi = n;
      }
      wave_argmax(bv, bi);
      if (lane == 0) {
        am.part_v[(long)m * gridDim.x + blockIdx.x] = bv;
        am.part_i[(long)m * gridDim.x + blockIdx.x] = bi;
      }
    }
}

// The prologue alone, one block per row.
__global__ __launch_bounds__(256) void k_rowops(RowOps ro, int K, double2* __restrict__ out, long ldo) {
  __shared__ double2 st_mean[1], st_sd[1];
  const int m = blockIdx.x;
  if (ro.ln) ro_stats<1>(ro, m, 1, K, st_mean, st_sd);
  if (threadIdx.x == 0) ro_check(ro, m);
  for (int k = threadIdx.x; k < K; k += 256) {
    double2 v = ro_value(ro, m, k, K);
    if (ro.ln) v = ln_apply(v, st_mean[0], st_sd[0], ro.gamma[k], ro.beta[k]);
    out[(long)m * ldo + k] = v;
    if (ro.save) ro.save[(long)m * ro.ldsave + k] = v;
  }
}

void rowops_apply(hipStream_t st, int M, int K, const RowOps& ro, double2* out, long ldo) {
  if (M > 0) hipLaunchKernelGGL(k_rowops, dim3(M), dim3(256), 0, st, ro, K, out, ldo);
}

// ===========================================================================
// MFMA complex GEMM.  Block tile 64x64 (4 waves of 32x32), K step 16, operands
// de-interleaved into re/im planes in LDS (double-buffered).  Per 16x16x4 step
// a wave issues 4 v_mfma_f64_16x16x4_f64 per output tile:
//     Cr += Ar*Br;  Cr += (-Ai)*Bi;  Ci += Ar*Bi;  Ci += Ai*Br
// Lane layout of v_mfma_f64_16x16x4_f64 (wave64): A[i][k] at lane i+16k,
// B[k][j] at lane j+16k, D[i][j] at lane j+16*(i%4), element i/4 (unlike the
// f32 16x16x4 form, consecutive output rows sit in consecutive lane groups).
// blockIdx.z splits K; the last block of a tile sums the partials.
// ===========================================================================
constexpr int GBM = 64, GBN = 64, GBK = 16, GPAD = 4;

__global__ __launch_bounds__(256) void k_zgemm_mfma(const double2* __restrict__ A, long lda,
                                                       const double2* __restrict__ Bm, long ldb, int M, int N, int K,
                                                       int kchunk, Epi ep, Argmax am, double2* __restrict__ ws,
                                                       uint32_t* __restrict__ cnt) {
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

  // Re values of the tile for the fused argmax, staged in the (now idle) As buffer
  double* stage = &As[0][0][0][0];  // [64][65]
  const bool argmax = am.part_v != nullptr;
  if (gridDim.z == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ml = wm + 16 * i + (lane >> 4) + 4 * r, nl = wn + 16 * j + (lane & 15);
          const int m = m0 + ml, n = n0 + nl;
          if (m < M && n < N) {
            const double re = apply_epi(ep, M, N, m, n, make_double2(cr[i][j][r], ci[i][j][r]));
            if (argmax) stage[ml * 65 + nl] = re;
          }
        }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + (lane >> 4) + 4 * r;
          const int n = n0 + wn + 16 * j + (lane & 15);
          if (m < M && n < N) st_dev(&ws[((long)blockIdx.z * M + m) * N + n], make_double2(cr[i][j][r], ci[i][j][r]));
        }
    if (!arrive_last(&cnt[blockIdx.y * gridDim.x + blockIdx.x], gridDim.z)) return;
    // thread t owns tile elements t + 256 i (row t/64 + 4i, column t%64); the
    // splits are summed in order, 16 independent loads in flight per split
    const int P = gridDim.z;
    const int nl = tid & 63, n = n0 + nl;
    double2 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = make_double2(0.0, 0.0);
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + (tid >> 6) + 4 * i;
        if (m < M && n < N) v[i] = cadd(v[i], ld_dev(&ws[((long)p * M + m) * N + n]));
      }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ml = (tid >> 6) + 4 * i, m = m0 + ml;
      if (m < M && n < N) {
        const double re = apply_epi(ep, M, N, m, n, v[i]);
        if (argmax) stage[ml * 65 + nl] = re;
      }
    }
  }
  if (!argmax) return;
  __syncthreads();
  // per-row (max, last index) over the tile's columns: wave w takes rows w, w+4, ...
  for (int ml = wave; ml < GBM; ml += 4) {
    const int m = m0 + ml, n = n0 + lane;
    if (m >= M) break;
    double bv = -INFINITY;
    int bi = -1;
    if (n < N) {
      const double v = stage[ml * 65 + lane];
      if (isnan(v)) atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
      else bv = v, bi = n;
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
      am.part_v[(long)m * gridDim.x + blockIdx.x] = bv;
      am.part_i[(long)m * gridDim.x + blockIdx.x] = bi;
    }
  }
}

// ===========================================================================
// Skinny MFMA GEMM for 9 <= M <= 64 rows (batched decode): a block owns all M
// rows (RT tiles of 16) and 16 columns; its K range is split over the 4 waves,
// each accumulating the whole 16RT x 16 tile with v_mfma_f64_16x16x4_f64 from
// operands loaded straight from global memory (A: row i, k offset lane/16;
// B: column i, k offset lane/16).  Waves are summed through LDS, blockIdx.y
// splits K at most 8 ways.
// ===========================================================================
template <int RT>
__global__ __launch_bounds__(256) void k_zgemm_skinny(const double2* __restrict__ X, long ldx, int M,
                                                        const double2* __restrict__ W, long ldw, int N, int K, int kc,
                                                        Epi ep, Argmax am, double2* __restrict__ ws,
                                                        uint32_t* __restrict__ cnt) {
  __shared__ double2 red[4][16 * RT][16];
  __shared__ double stage[16 * RT][17];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * 16, n = n0 + i;
  const int kb0 = blockIdx.y * kc, kb1 = min(K, kb0 + kc);
  const int q = kc / 4;  // multiple of 16
  const int ka = kb0 + wave * q, kz = min(kb1, ka + q);

  v4d cr[RT], ci[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) cr[t] = ci[t] = v4d{0.0, 0.0, 0.0, 0.0};

  constexpr int U = 4;  // k-steps of 4 per batch
  for (int k = ka; k < kz; k += 4 * U) {
    double2 b[U], a[RT][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + 4 * u + kq;
      b[u] = (kk < kz && n < N) ? W[(long)kk * ldw + n] : make_double2(0.0, 0.0);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const int m = 16 * t + i;
        a[t][u] = (kk < kz && m < M) ? X[(long)m * ldx + kk] : make_double2(0.0, 0.0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[t][u].x, b[u].x, cr[t], 0, 0, 0);
        ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[t][u].x, b[u].y, ci[t], 0, 0, 0);
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[t][u].y, b[u].y, cr[t], 0, 0, 0);
        ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[t][u].y, b[u].x, ci[t], 0, 0, 0);
      }
  }
  // D[i][j] of row tile t at lane j + 16*(i%4), element i/4
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][16 * t + 4 * e + kq][i] = make_double2(cr[t][e], ci[t][e]);
  __syncthreads();
  // thread tid owns tile elements tid + 256 j: row (tid >> 4) + 16 j, column tid & 15
  const int col = tid & 15, n1 = n0 + col;
  double2 v[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const int row = (tid >> 4) + 16 * j;
    v[j] = cadd(cadd(cadd(red[0][row][col], red[1][row][col]), red[2][row][col]), red[3][row][col]);
  }
  const int P = gridDim.y;
  if (P > 1) {
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int m = (tid >> 4) + 16 * j;
      if (m < M && n1 < N) st_dev(&ws[((long)blockIdx.y * M + m) * N + n1], v[j]);
    }
    if (!arrive_last(&cnt[blockIdx.x], (uint32_t)P)) return;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int m = (tid >> 4) + 16 * j;
      if (m < M && n1 < N) {
        double2 pv[SKINNY_MAX_SPLIT];
#pragma unroll
        for (int p = 0; p < SKINNY_MAX_SPLIT; ++p)
          pv[p] = p < P ? ld_dev(&ws[((long)p * M + m) * N + n1]) : make_double2(0.0, 0.0);
        double2 s = pv[0];
#pragma unroll
        for (int p = 1; p < SKINNY_MAX_SPLIT; ++p)
          if (p < P) s = cadd(s, pv[p]);
        v[j] = s;
      }
    }
  }
  const bool argmax = am.part_v != nullptr;
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const int row = (tid >> 4) + 16 * j;
    if (row < M && n1 < N) {
      const double re = apply_epi(ep, M, N, row, n1, v[j]);
      if (argmax) stage[row][col] = re;
    }
  }
  if (!argmax) return;
  __syncthreads();
  // per row over the 16 columns: 16-lane groups, (max, last index)
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const int row = (tid >> 4) + 16 * j;
    double bv = -INFINITY;
    int bi = -1;
    if (row < M && n1 < N) {
      const double x = stage[row][col];
      if (isnan(x)) atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
      else bv = x, bi = n1;
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      const double ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      argmax_combine(bv, bi, ov, oi);
    }
    if (col == 0 && row < M) {
      am.part_v[(long)row * gridDim.x + blockIdx.x] = bv;
      am.part_i[(long)row * gridDim.x + blockIdx.x] = bi;
    }
  }
}

// ---- planning and dispatch ------------------------------------------------
// GEMV: C columns per block (16, or 64 for wide outputs), K split so that the
// grid has about 512 blocks, at most GEMV_MAX_SPLIT ways.
struct GemvPlan {
  int mr, C, kw, P, ncb;
};
static GemvPlan plan_gemv(int M, int N, int K) {
  GemvPlan p;
  p.mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  p.C = cdiv_i(N, 64) >= 256 ? 64 : 16;
  const int rpw = 64 / p.C;
  p.ncb = cdiv_i(N, p.C);
  int P = std::min(GEMV_MAX_SPLIT, std::max(1, cdiv_i(512, p.ncb)));
  // rows per block: a multiple of 4 waves x rpw, and its input rows fit 64 KB of LDS
  const int unit = 4 * rpw;
  int KB = cdiv_i(cdiv_i(K, P), unit) * unit;
  const int kb_max = std::max(unit, (65536 / (16 * p.mr)) / unit * unit);
  KB = std::min(KB, kb_max);
  p.kw = KB / 4;
  p.P = cdiv_i(K, KB);
  return p;
}
// skinny MFMA: 16 columns per block, K split in chunks that are multiples of
// 64 (16 per wave), about 512 blocks, at most SKINNY_MAX_SPLIT ways
struct SkinnyPlan {
  int rt, ncb, kc, P;
};
static SkinnyPlan plan_skinny(int M, int N, int K) {
  SkinnyPlan p;
  p.rt = cdiv_i(M, 16);
  p.ncb = cdiv_i(N, 16);
  const int P = std::min(SKINNY_MAX_SPLIT, std::max(1, cdiv_i(512, p.ncb)));
  p.kc = cdiv_i(cdiv_i(K, P), 64) * 64;
  p.P = cdiv_i(K, p.kc);
  return p;
}
struct MfmaPlan {
  int P, kchunk, mt, nt;
};
static MfmaPlan plan_mfma(int M, int N, int K) {
  MfmaPlan p;
  p.mt = cdiv_i(M, GBM);
  p.nt = cdiv_i(N, GBN);
  const int tiles = p.mt * p.nt;
  int P = 1;
  if (tiles < 512) P = std::min(cdiv_i(512, tiles), std::max(1, K / 64));
  p.kchunk = cdiv_i(cdiv_i(K, P), GBK) * GBK;
  p.P = cdiv_i(K, p.kchunk);
  return p;
}

constexpr int SKINNY_MAX_M = 64;

size_t gemm_ws_bytes(int M, int N, int K) {
  int P;
  if (M <= 8) P = plan_gemv(M, N, K).P;
  else if (M <= SKINNY_MAX_M) P = plan_skinny(M, N, K).P;
  else P = plan_mfma(M, N, K).P;
  return P > 1 ? (size_t)P * M * N * sizeof(double2) : 0;
}

// argmax partials: one per row and 16-column tile covers every product shape
size_t argmax_part_elems(int M, int N) { return (size_t)M * cdiv_i(N, 16); }

template <int MR, int C>
static void launch_gemv(hipStream_t st, const GemvPlan& p, const RowOps& ro, int M, const double2* W, long ldw, int N,
                        int K, const Epi& ep, const Argmax& am, const Sync& sy) {
  dim3 grid(p.ncb, p.P);
  const size_t shm = (size_t)MR * 4 * p.kw * sizeof(double2);
  hipLaunchKernelGGL((k_gemv<MR, C>), grid, dim3(256), shm, st, ro, M, W, ldw, N, K, p.kw, ep, am, (double2*)sy.ws,
                     sy.counters);
}
template <int MR>
static void launch_gemv_c(hipStream_t st, const GemvPlan& p, const RowOps& ro, int M, const double2* W, long ldw, int N,
                          int K, const Epi& ep, const Argmax& am, const Sync& sy) {
  if (p.C == 64) launch_gemv<MR, 64>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
  else launch_gemv<MR, 16>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
}

int gemm(hipStream_t st, int M, int N, int K, const RowOps& ro, const double2* W, long ldw, const Epi& ep,
         const Argmax* amp, const Sync& sy) {
  if (M <= 0 || N <= 0) return OK;
  const Argmax am = amp ? *amp : Argmax();
  if (gemm_ws_bytes(M, N, K) > sy.ws_bytes) return ERR_STATE;
  int tiles = 0;  // column tiles of the argmax partials
  if (M <= 8) {
    const GemvPlan p = plan_gemv(M, N, K);
    if (p.ncb >= SYNC_COUNTERS) return ERR_ARG;
    switch (p.mr) {
      case 1: launch_gemv_c<1>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      case 2: launch_gemv_c<2>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      case 4: launch_gemv_c<4>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      default: launch_gemv_c<8>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
    }
    tiles = p.ncb;
  } else {
    if (!ro.plain()) return ERR_ARG;  // the MFMA paths read plain rows; materialise the prologue first
    if (M <= SKINNY_MAX_M) {
      const SkinnyPlan p = plan_skinny(M, N, K);
      if (p.ncb >= SYNC_COUNTERS) return ERR_ARG;
      dim3 grid(p.ncb, p.P);
      switch (p.rt) {
        case 1: hipLaunchKernelGGL((k_zgemm_skinny<1>), grid, dim3(256), 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, (double2*)sy.ws, sy.counters); break;
        case 2: hipLaunchKernelGGL((k_zgemm_skinny<2>), grid, dim3(256), 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, (double2*)sy.ws, sy.counters); break;
        case 3: hipLaunchKernelGGL((k_zgemm_skinny<3>), grid, dim3(256), 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, (double2*)sy.ws, sy.counters); break;
        default: hipLaunchKernelGGL((k_zgemm_skinny<4>), grid, dim3(256), 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, (double2*)sy.ws, sy.counters); break;
      }
      tiles = p.ncb;
    } else {
      const MfmaPlan p = plan_mfma(M, N, K);
      if (p.P > 1 && (long)p.mt * p.nt >= SYNC_COUNTERS) return ERR_ARG;
      dim3 grid(p.nt, p.mt, p.P);
      hipLaunchKernelGGL(k_zgemm_mfma, grid, dim3(256), 0, st, ro.x, ro.ldx, W, ldw, M, N, K, p.kchunk, ep, am,
                         (double2*)sy.ws, sy.counters);
      tiles = p.nt;
    }
  }
  if (am.part_v) hipLaunchKernelGGL(k_argmax_finalize, dim3(M), dim3(256), 0, st, am, tiles);
  return OK;
}

}  // namespace mitok
