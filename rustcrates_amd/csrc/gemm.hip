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

#include "epilogue.hpp"

namespace mitok {

static inline int cdiv_i(long a, long b) { return (int)((a + b - 1) / b); }

// greedy_decoding finish: one block per row reduces that row's per-tile
// (max, last index) partials, then stores the id, appends it to the history
// and advances the sequence's KV length.
__global__ __launch_bounds__(256) void k_argmax_finalize(Argmax am, int tiles) {
  __shared__ double sv[4];
  __shared__ int si[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double bv = -INFINITY;
  int bi = -1;
  constexpr int U = 8;  // partials per thread requested together (one memory round trip up to 2048 tiles)
  for (int t0 = tid; t0 < tiles; t0 += 256 * U) {
    double v[U];
    int ix[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + 256 * u;
      v[u] = t < tiles ? am.part_v[(long)m * tiles + t] : -INFINITY;
      ix[u] = t < tiles ? am.part_i[(long)m * tiles + t] : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) argmax_combine(bv, bi, v[u], ix[u]);
  }
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
// GEMV for M <= 8 rows: HBM-bound weight stream.  A block owns C columns and a
// K range of 4*kw rows; lane (r, c) = (lane / C, lane % C) reads row r of each
// group of 64/C rows, so one wave instruction covers 64/C rows x C columns.
// The first 16 weight loads per lane -- every row of the lane for the layer
// products of config 3 -- are in flight while the prologue builds the block's
// input rows in LDS; longer ranges then take 8 rows at a time.  Every lane
// issues every load (rows past its range read a zero constant), so each wait
// covers only the loads it needs.  Lanes of a column are summed by shuffles,
// the 4 waves through LDS; blockIdx.y splits K (at most 8 ways, so few blocks
// meet at each completion counter).
// PRE: the input rows are plain (x[m][k] as stored, the decode products of 2-8
// sequences), at most GEMV_PRE elements per thread.  They are requested before
// the weights: a wave's loads return in order, so a prologue whose loads go
// out after the weights' waits for the whole weight stream, and the
// multiply-adds only start after it.  Requested first, the rows are in LDS
// when the first weights arrive.
// ===========================================================================
constexpr int GEMV_PRE = 16;
constexpr int GEMV_MAX_SPLIT = 8;
__device__ const double2 gemv_zero2 = {0.0, 0.0};  // what a load past a lane's rows reads
// w[u] <- rows u0 + u of the lane's column, u < 8 (zero past its nu rows)
__device__ __forceinline__ void gemv_rows(double2 (&w)[8], const double2* wp, long wstep, int u0, int nu) {
#pragma unroll
  for (int u = 0; u < 8; ++u) w[u] = ld_stream(u0 + u < nu ? wp + (u0 + u) * wstep : &gemv_zero2);
}
// acc[m] += x[m][row u0 + u] * w[u], u < 8; rows past nu (zero weights) read
// the lane's first row, so they add exact zeros
template <int MR>
__device__ __forceinline__ void gemv_fma(double2 (&acc)[MR], const double2* xw, int RL, int RPW, int u0, int nu,
                                         const double2 (&w)[8]) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int iu = u0 + u < nu ? u0 + u : 0;
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * RL + iu * RPW], w[u]));
  }
}
constexpr int SKINNY_MAX_SPLIT = 8;

template <int MR, int C, bool PRE>
__global__ __launch_bounds__(256) void k_gemv(RowOps ro, int M, const double2* __restrict__ W, long ldw, int N, int K,
                                              int kw, Epi ep, Argmax am, double2* __restrict__ ws,
                                              uint32_t* __restrict__ cnt) {
  constexpr int RPW = 64 / C;  // rows per wave instruction
  extern __shared__ double2 lds2[];  // input rows [MR][RL], then the attention-combine weights
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
  // a LayerNorm needs the whole row in LDS; otherwise the block's K range
  const int ka = ro.ln ? 0 : kb0, RL = ro.ln ? K : KB;
  RoLds L;
  L.wts = (double*)(lds2 + MR * RL);
  L.lsum = L.wts + (ro.att.po ? (size_t)M * ro.att.H * ro.att.nsplit : 0);
  L.m0 = 0;

  const int nuc = col_ok ? nu : 0;  // rows this lane loads
  const int nu_max = (kw + RPW - 1) / RPW;  // the most rows of any lane (block-uniform)
  double2 xr[PRE ? GEMV_PRE : 1];
  if constexpr (PRE) {  // element i = m * RL + (k - kb0) of the block's rows, before any weight
#pragma unroll
    for (int j = 0; j < GEMV_PRE; ++j) {
      const int i = tid + 256 * j, m = i / RL, k = kb0 + (i - m * RL);
      xr[j] = ld_glb((i < MR * RL && m < M && k < K) ? ro.x + (long)m * ro.ldx + k : &gemv_zero2);
    }
  }
  double2 w0[8], w1[8];
  gemv_rows(w0, wp, wstep, 0, nuc);
  gemv_rows(w1, wp, wstep, 8, nuc);

  if constexpr (PRE) {
#pragma unroll
    for (int j = 0; j < GEMV_PRE; ++j)
      if (tid + 256 * j < MR * RL) lds2[tid + 256 * j] = xr[j];
    __syncthreads();
  } else {
    ro_prepare(ro, M, L);
    ro_build<MR>(ro, M, K, ka, RL, kb0, min(K, kb0 + KB), lds2, L, st_mean, st_sd);
  }
  if (blockIdx.x == 0 && blockIdx.y == 0 && tid < M) ro_check(ro, tid);
  const double2* xs = lds2 + (kb0 - ka);  // row m of the block's range at xs[m * RL]
  if (ro.save && blockIdx.x == 0)
    for (int i = tid; i < MR * KB; i += 256) {
      const int m = i / KB, k = kb0 + (i - m * KB);
      if (m < M && k < K) ro.save[(long)m * ro.ldsave + k] = xs[m * RL + (k - kb0)];
    }

  double2 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = make_double2(0.0, 0.0);
  {
    // row u of this lane: xw[m * RL + u * RPW]; a row past the lane's range
    // has a zero weight and reads the lane's first row (a lane with no rows:
    // the block's first), so it adds an exact zero
    const double2* xw = xs + (nuc > 0 ? wave * kw + r : 0);
    gemv_fma<MR>(acc, xw, RL, RPW, 0, nuc, w0);
    gemv_fma<MR>(acc, xw, RL, RPW, 8, nuc, w1);
    // rows past the first 16 (the wide vocab product, config 5's products), 8 at a time
    for (int u0 = 16; u0 < nu_max; u0 += 8) {
      gemv_rows(w0, wp, wstep, u0, nuc);
      gemv_fma<MR>(acc, xw, RL, RPW, u0, nuc, w0);
    }
  }
  // lanes of one column (same c, r = 0 .. RPW-1) -> r = 0
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m].x = col_sum<C>(acc[m].x);
    acc[m].y = col_sum<C>(acc[m].y);
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
  if (ep.mode == EPI_PART) {  // the consumer sums the partials and applies what follows
    if (owner && col_ok)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) ep.out[((long)blockIdx.y * M + m) * N + n] = acc[m];
    return;
  }
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

  // the epilogue, one output per lane of wave 0 rather than MR per column
  // owner (a GELU is a chain of transcendentals: eight in one lane take eight
  // times as long); the Re values come back to the owners for the argmax
  double re[MR];
  if (MR == 1) {
    if (owner && col_ok) re[0] = apply_epi(ep, M, N, 0, n, acc[0]);
  } else {
    if (owner)
#pragma unroll
      for (int m = 0; m < MR; ++m) red[0][m][lane] = acc[m];
    __builtin_amdgcn_wave_barrier();
    __shared__ double epi_re[MR][C];
    if (wave == 0)
      for (int i = lane; i < MR * C; i += 64) {
        const int m = i / C, cc = i - (i / C) * C, nn = blockIdx.x * C + cc;
        if (m < M && nn < N) epi_re[m][cc] = apply_epi(ep, M, N, m, nn, red[0][m][cc]);
      }
    __builtin_amdgcn_wave_barrier();
    if (owner)
#pragma unroll
      for (int m = 0; m < MR; ++m) re[m] = epi_re[m][lane];
  }
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

// The attention-combine row transform (chunk combine, residual, LayerNorm) of
// row m with its two memory round trips overlapped: this thread's chunk
// outputs (the first RO_ATT_CH chunks of each of its columns) and residuals
// are requested before ro_prepare asks for the chunks' (max, sum).  The sums
// run in ro_base's order and the LayerNorm is ro_build's (ro_ln), so the row
// is the one ro_build would give.
constexpr int RO_ATT_CH = 8, RO_ATT_EPT = 4;
__device__ __forceinline__ bool rowops_att_ok(const RowOps& ro, int K) {
  return ro.att.po && !ro.table && !ro.rope_cs && !ro.bias && !ro.gelu && !ro.finite_check && K <= 256 * RO_ATT_EPT;
}
__device__ void rowops_att(const RowOps& ro, int K, int m, double2* buf, const RoLds& L, double2* st_mean,
                           double2* st_sd) {
  const AttnSplit& a = ro.att;
  const int tid = threadIdx.x;
  const int ns = (a.kv_len[m] + 1 + a.CH - 1) / a.CH;
  double2 gpre[LN_PRE], bpre[LN_PRE];
#pragma unroll
  for (int j = 0; j < LN_PRE; ++j) {
    const int k = tid + 256 * j;
    const bool ok = ro.ln && k < K;
    gpre[j] = ok ? ro.gamma[k] : make_double2(0.0, 0.0);
    bpre[j] = ok ? ro.beta[k] : make_double2(0.0, 0.0);
  }
  double2 t[RO_ATT_EPT][RO_ATT_CH], rs[RO_ATT_EPT];
#pragma unroll
  for (int j = 0; j < RO_ATT_EPT; ++j) {
    const int k = tid + 256 * j;
    const bool ok = k < K;
    const int h = k / a.dh, e = k - h * a.dh;
    const long base = ((long)m * a.H + h) * a.nsplit;
#pragma unroll
    for (int q = 0; q < RO_ATT_CH; ++q) t[j][q] = (ok && q < ns) ? a.po[(base + q) * a.dh + e] : make_double2(0.0, 0.0);
    rs[j] = (ok && ro.resid) ? ro.resid[(long)m * ro.ldr + k] : make_double2(0.0, 0.0);
  }
  ro_prepare(ro, 1, L);
#pragma unroll
  for (int j = 0; j < RO_ATT_EPT; ++j) {
    const int k = tid + 256 * j;
    if (k >= K) continue;
    const int h = k / a.dh, e = k - h * a.dh;
    const long base = ((long)m * a.H + h) * a.nsplit;
    const double* w = L.wts + (long)h * a.nsplit;
    double2 o = make_double2(0.0, 0.0);
#pragma unroll
    for (int q = 0; q < RO_ATT_CH; ++q)
      if (q < ns) {
        o.x += t[j][q].x * w[q];
        o.y += t[j][q].y * w[q];
      }
    for (int s0 = RO_ATT_CH; s0 < ns; s0 += 8) {  // longer caches: the rest, eight loads in flight
      double2 u[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) u[q] = s0 + q < ns ? a.po[(base + s0 + q) * a.dh + e] : make_double2(0.0, 0.0);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (s0 + q < ns) {
          o.x += u[q].x * w[s0 + q];
          o.y += u[q].y * w[s0 + q];
        }
    }
    const double l = L.lsum[h];
    double2 v = make_double2(o.x / l, o.y / l);
    if (ro.resid) v = make_double2(v.x + rs[j].x, 0.0);
    buf[k] = v;
  }
  __syncthreads();
  if (ro.ln) ro_ln<1>(ro, 1, K, K, 0, K, buf, st_mean, st_sd, gpre, bpre);
}

// The prologue alone, one block per row.
__global__ __launch_bounds__(256) void k_rowops(RowOps ro, int K, double2* __restrict__ out, long ldo) {
  extern __shared__ double2 lds2[];  // the row [K], then the attention-combine weights
  __shared__ double2 st_mean[1], st_sd[1];
  const int m = blockIdx.x;
  RoLds L;
  L.wts = (double*)(lds2 + K);
  L.lsum = L.wts + (ro.att.po ? (size_t)ro.att.H * ro.att.nsplit : 0);
  L.m0 = m;
  if (rowops_att_ok(ro, K)) {
    rowops_att(ro, K, m, lds2, L, st_mean, st_sd);
  } else {
    ro_prepare(ro, 1, L);
    ro_build<1>(ro, 1, K, 0, K, 0, K, lds2, L, st_mean, st_sd);
  }
  if (threadIdx.x == 0) ro_check(ro, m);
  for (int k = threadIdx.x; k < K; k += 256) {
    const double2 v = lds2[k];
    out[(long)m * ldo + k] = v;
    if (ro.save) ro.save[(long)m * ro.ldsave + k] = v;
  }
}

// The chunk combine alone for long caches, one 64-lane block per (row,
// head): out[m][h*dh + e] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// The weights and their sum are ro_prepare's (same lanes, same reductions)
// and each element sums its chunks in order, so the rows equal those
// rowops_att forms; there one block per row requests its chunks eight at a
// time, which at thousands of keys (64 chunks per head) is eight dependent
// round trips in one CU.
constexpr int COMBINE_BATCH = 16;
__global__ __launch_bounds__(64) void k_attn_combine(AttnSplit a, double2* __restrict__ out, long ldo) {
  __shared__ double wts[256];  // nsplit <= 256
  const int m = blockIdx.x / a.H, h = blockIdx.x - m * a.H;
  const int lane = threadIdx.x;
  const int ns = (a.kv_len[m] + 1 + a.CH - 1) / a.CH;
  const long base = ((long)m * a.H + h) * a.nsplit;
  double vm[4], vl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int sidx = lane + 64 * j;
    const bool in = sidx < a.nsplit;
    vm[j] = in ? a.pm[base + sidx] : -INFINITY;
    vl[j] = in ? a.pl[base + sidx] : 0.0;
  }
  double mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane + 64 * j < ns) mx = fmax(mx, vm[j]);
  mx = wave_max(mx);
  double l = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int sidx = lane + 64 * j;
    if (sidx < ns) {
      const double w = exp(vm[j] - mx);
      wts[sidx] = w;
      l += vl[j] * w;
    }
  }
  l = wave_sum(l);
  __syncthreads();
  for (int e = lane; e < a.dh; e += 64) {
    double2 o = make_double2(0.0, 0.0);
    for (int s0 = 0; s0 < ns; s0 += COMBINE_BATCH) {
      double2 t[COMBINE_BATCH];
#pragma unroll
      for (int q = 0; q < COMBINE_BATCH; ++q) t[q] = a.po[(base + min(s0 + q, ns - 1)) * a.dh + e];
#pragma unroll
      for (int q = 0; q < COMBINE_BATCH; ++q)
        if (s0 + q < ns) {
          o.x += t[q].x * wts[s0 + q];
          o.y += t[q].y * wts[s0 + q];
        }
    }
    out[(long)m * ldo + (long)h * a.dh + e] = make_double2(o.x / l, o.y / l);
  }
}

void rowops_apply(hipStream_t st, int M, int K, const RowOps& ro, double2* out, long ldo) {
  if (M <= 0) return;
  if (ro.att.po && ro.att.nsplit > RO_ATT_CH && ro.att.nsplit <= 256 && !ro.table && !ro.rope_cs && !ro.bias &&
      !ro.gelu && !ro.finite_check && ro.att.H * ro.att.dh == K) {
    // long caches: combine per (row, head) into `out`, then residual and
    // LayerNorm on those rows in place (k_rowops reads a row whole before
    // writing it)
    MITOK_LAUNCH(k_attn_combine, dim3(M * ro.att.H), dim3(64), 0, st, ro.att, out, ldo);
    RowOps r = ro;
    r.att = AttnSplit();
    r.x = out;
    r.ldx = ldo;
    r.npart = 0;
    MITOK_LAUNCH(k_rowops, dim3(M), dim3(256), (size_t)K * sizeof(double2), st, r, K, out, ldo);
    return;
  }
  const size_t shm = (size_t)K * sizeof(double2) + (ro.att.po ? (size_t)ro.att.H * (ro.att.nsplit + 1) * sizeof(double) : 0);
  MITOK_LAUNCH(k_rowops, dim3(M), dim3(256), shm, st, ro, K, out, ldo);
}


template <int RT, bool RE>
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

  constexpr int U = 4;  // k-steps of 4 per batch, double-buffered
  double2 b[2][U], a[2][RT][U];
  auto load = [&](int buf, int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + 4 * u + kq;
      b[buf][u] = (kk < kz && n < N) ? W[(long)kk * ldw + n] : make_double2(0.0, 0.0);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const int m = 16 * t + i;
        a[buf][t][u] = (kk < kz && m < M) ? X[(long)m * ldx + kk] : make_double2(0.0, 0.0);
      }
    }
  };
  // the tiles' first products before their second ones: two MFMAs on one
  // accumulator are never adjacent
  auto mma = [&](int buf) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].x, b[buf][u].x, cr[t], 0, 0, 0);
        if (!RE) ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].x, b[buf][u].y, ci[t], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[buf][t][u].y, b[buf][u].y, cr[t], 0, 0, 0);
        if (!RE) ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].y, b[buf][u].x, ci[t], 0, 0, 0);
      }
    }
  };
  constexpr int KS = 4 * U;  // unrolled by two: both buffer indices are constants
  if (ka < kz) load(0, ka);
  for (int k = ka; k < kz; k += 2 * KS) {
    if (k + KS < kz) load(1, k + KS);
    mma(0);
    if (k + KS >= kz) break;
    if (k + 2 * KS < kz) load(0, k + 2 * KS);
    mma(1);
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
  if (ep.mode == EPI_PART) {  // the next launch sums the partials and applies what follows
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int m = (tid >> 4) + 16 * j;
      if (m < M && n1 < N) ep.out[((long)blockIdx.y * M + m) * N + n1] = v[j];
    }
    return;
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
    row16_argmax(bv, bi);
    if (col == 0 && row < M) {
      am.part_v[(long)row * gridDim.x + blockIdx.x] = bv;
      am.part_i[(long)row * gridDim.x + blockIdx.x] = bi;
    }
  }
}

// ===========================================================================
// Row-tile skinny variant (9 <= M <= 64, layer-wide outputs).  Block (bx, by,
// bz) owns CT column tiles of 16 at bx, the 16-row tile by and K range bz of
// 16*nkw; its 4 waves split that range, nkw k-steps of 4 each.  Per k-step a
// wave loads one activation fragment and CT weight fragments and issues 4*CT
// v_mfma_f64_16x16x4_f64 (A: row i, k offset lane/16; B: column i).  Three
// batches of 4 k-steps are in flight ahead of the one being multiplied.  The
// waves' tiles are summed through LDS in wave order.  One row tile per block
// gives two or more blocks per column tile, so an output as wide as the FFN's
// hidden layer fills the chip without a K split and its epilogue (GELU) runs
// in the same block; EPI_PART leaves gridDim.z partials for the consumer.
// D[i][j] sits at lane j + 16*(i%4), element i/4.
// ===========================================================================
template <int CT>
__global__ __launch_bounds__(256) void k_zgemm_skinny_rows(const double2* __restrict__ X, long ldx, int M,
                                                         const double2* __restrict__ W, long ldw, int N, int K,
                                                         int nkw, Epi ep) {
  constexpr int U = 4;  // k-steps per batch
  __shared__ double2 red[4][16][16 * CT + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * 16 * CT, m = blockIdx.y * 16 + i;
  const int ka = (blockIdx.z * 4 + wave) * 4 * nkw, kz = min(K, ka + 4 * nkw);
  double2 a[3][U], b[3][U][CT];
  auto load = [&](int s, int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + 4 * u + kq;
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int n = n0 + 16 * c + i;
        b[s][u][c] = (kk < kz && n < N) ? W[(long)kk * ldw + n] : make_double2(0.0, 0.0);
      }
      a[s][u] = (kk < kz && m < M) ? X[(long)m * ldx + kk] : make_double2(0.0, 0.0);
    }
  };
  v4d cr[CT], ci[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) cr[c] = ci[c] = v4d{0.0, 0.0, 0.0, 0.0};
  // the real-part products of the batch before its imaginary-part ones: two
  // MFMAs on one accumulator are never adjacent
  auto mma = [&](int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        cr[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u][c].x, cr[c], 0, 0, 0);
        ci[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u][c].y, ci[c], 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        cr[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[s][u].y, b[s][u][c].y, cr[c], 0, 0, 0);
        ci[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].y, b[s][u][c].x, ci[c], 0, 0, 0);
      }
    }
  };
  constexpr int KS = 4 * U;  // k per batch; the loop is unrolled by three so buffer indices are constants
  load(0, ka);
  load(1, ka + KS);
  load(2, ka + 2 * KS);
  for (int k = ka; k < kz; k += 3 * KS) {
    mma(0);
    if (k + 3 * KS < kz) load(0, k + 3 * KS);
    if (k + KS >= kz) break;
    mma(1);
    if (k + 4 * KS < kz) load(1, k + 4 * KS);
    if (k + 2 * KS >= kz) break;
    mma(2);
    if (k + 5 * KS < kz) load(2, k + 5 * KS);
  }
#pragma unroll
  for (int c = 0; c < CT; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][4 * e + kq][16 * c + i] = make_double2(cr[c][e], ci[c][e]);
  __syncthreads();
  for (int idx = tid; idx < 16 * 16 * CT; idx += 256) {
    const int row = idx / (16 * CT), col = idx - row * 16 * CT;
    const double2 v = cadd(cadd(cadd(red[0][row][col], red[1][row][col]), red[2][row][col]), red[3][row][col]);
    const int n = n0 + col, mm = blockIdx.y * 16 + row;
    if (mm >= M || n >= N) continue;
    if (ep.mode == EPI_PART) ep.out[((long)blockIdx.z * M + mm) * N + n] = v;
    else apply_epi(ep, M, N, mm, n, v);
  }
}

// ===========================================================================
// Row-tile variant with 16 waves per block: as k_zgemm_skinny_rows (CT = 1),
// but the block's K range of 64*nkw is split over 16 waves, four per SIMD, so
// each SIMD interleaves four waves' loads and MFMAs.  With one wave per SIMD
// a wave of ~128 MFMAs cannot hide its own load latency (the 4-wave kernel ran
// at 22-28% MFMA busy); here each wave has a quarter of the work and the
// SIMD's other waves compute while it waits.  Two batches of 4 k-steps per
// wave are requested ahead of the one being multiplied (the register budget at
// four waves per SIMD).  The 16 waves' tiles are summed through LDS in wave
// order, so results repeat bit for bit.
// ===========================================================================
constexpr int ROWS16_WAVES = 16;
constexpr size_t ROWS16_LDS = (size_t)ROWS16_WAVES * 16 * 16 * sizeof(double2);  // 64 KB

__global__ __launch_bounds__(1024) void k_zgemm_rows16(const double2* __restrict__ X, long ldx, int M,
                                                     const double2* __restrict__ W, long ldw, int N, int K, int nkw,
                                                     Epi ep) {
  constexpr int U = 4, NW = ROWS16_WAVES, LD = 16;
  extern __shared__ double2 red16[];  // [NW][16][LD]: lanes write and read whole 1 KB rows, no bank conflicts
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kq = lane >> 4;
  const int n = blockIdx.x * 16 + i, m = blockIdx.y * 16 + i;
  const int ka = (blockIdx.z * NW + wave) * 4 * nkw, kz = min(K, ka + 4 * nkw);
  double2 a[2][U], b[2][U];
  auto load = [&](int s, int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + 4 * u + kq;
      b[s][u] = (kk < kz && n < N) ? W[(long)kk * ldw + n] : make_double2(0.0, 0.0);
      a[s][u] = (kk < kz && m < M) ? X[(long)m * ldx + kk] : make_double2(0.0, 0.0);
    }
  };
  v4d cr = {0.0, 0.0, 0.0, 0.0}, ci = {0.0, 0.0, 0.0, 0.0};
  // each batch's real-part products before its imaginary-part ones, so two
  // MFMAs on one accumulator are never adjacent
  auto mma = [&](int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      cr = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u].x, cr, 0, 0, 0);
      ci = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u].y, ci, 0, 0, 0);
      cr = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[s][u].y, b[s][u].y, cr, 0, 0, 0);
      ci = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].y, b[s][u].x, ci, 0, 0, 0);
    }
  };
  constexpr int KS = 4 * U;  // k per batch; unrolled by two so buffer indices are constants
  load(0, ka);
  load(1, ka + KS);
  for (int k = ka; k < kz; k += 2 * KS) {
    mma(0);
    if (k + 2 * KS < kz) load(0, k + 2 * KS);
    if (k + KS >= kz) break;
    mma(1);
    if (k + 3 * KS < kz) load(1, k + 3 * KS);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red16[(wave * 16 + 4 * e + kq) * LD + i] = make_double2(cr[e], ci[e]);
  __syncthreads();
  if (tid < 256) {
    const int row = tid >> 4, col = tid & 15;
    double2 v = red16[row * LD + col];
#pragma unroll
    for (int w = 1; w < NW; ++w) v = cadd(v, red16[(w * 16 + row) * LD + col]);
    const int nn = blockIdx.x * 16 + col, mm = blockIdx.y * 16 + row;
    if (mm < M && nn < N) {
      if (ep.mode == EPI_PART) ep.out[((long)blockIdx.z * M + mm) * N + nn] = v;
      else apply_epi(ep, M, N, mm, nn, v);
    }
  }
}

// The same product for the planned shapes of 8 or 12 k-steps (32 or 48 of K)
// per wave, as straight-line code (12: config 4's FFN Dense, K 768 whole in
// the block; 729 -> 725 ms of decode per call against k_zgemm_rows16): the
// loads of all NB 8-k batches go out first, an
// out-of-range operand lane reading a zero constant instead (no branch), so
// the compiler waits for each batch's own loads (in-order vmcnt) and the
// first batch's MFMAs run while the later batches are still in flight.  In
// k_zgemm_rows16 the guarded loads are branches, and the loop waits for every
// load before its first MFMA.  The MFMA sequence on each accumulator (k-steps
// in ascending order) is the same as there, so the results are identical.
__device__ const double2 rows16s_zero = {0.0, 0.0};  // what an out-of-range operand lane reads

template <int NB>  // batches of 2 k-steps: 4 (32 of K per wave, 512 per block) or 6 (48, 768)
__global__ __launch_bounds__(1024) void k_zgemm_rows16s(const double2* __restrict__ X, long ldx, int M,
                                                      const double2* __restrict__ W, long ldw, int N, int K, Epi ep) {
  constexpr int U = 2, NW = ROWS16_WAVES, LD = 16;
  extern __shared__ double2 red16[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kq = lane >> 4;
  const int n = blockIdx.x * 16 + i, m = blockIdx.y * 16 + i;
  const int ka = (blockIdx.z * NW + wave) * 8 * NB;
  const long nc = min(n, N - 1), mc = min(m, M - 1);
  const bool nok = n < N, mok = m < M;
  double2 a[NB][U], b[NB][U];
#pragma unroll
  for (int s = 0; s < NB; ++s)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // the address, not the value, is selected: every lane loads, so no
      // load sits under a branch
      const int kk = ka + 8 * s + 4 * u + kq;
      const long kc = min(kk, K - 1);
      const bool ok = kk < K;
      b[s][u] = ld_glb((ok && nok) ? W + kc * ldw + nc : &rows16s_zero);
      a[s][u] = ld_glb((ok && mok) ? X + mc * ldx + kc : &rows16s_zero);
    }
  v4d cr = {0.0, 0.0, 0.0, 0.0}, ci = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int s = 0; s < NB; ++s)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      cr = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u].x, cr, 0, 0, 0);
      ci = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].x, b[s][u].y, ci, 0, 0, 0);
      cr = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[s][u].y, b[s][u].y, cr, 0, 0, 0);
      ci = __builtin_amdgcn_mfma_f64_16x16x4f64(a[s][u].y, b[s][u].x, ci, 0, 0, 0);
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) red16[(wave * 16 + 4 * e + kq) * LD + i] = make_double2(cr[e], ci[e]);
  __syncthreads();
  if (tid < 256) {
    const int row = tid >> 4, col = tid & 15;
    double2 v = red16[row * LD + col];
#pragma unroll
    for (int w = 1; w < NW; ++w) v = cadd(v, red16[(w * 16 + row) * LD + col]);
    const int nn = blockIdx.x * 16 + col, mm = blockIdx.y * 16 + row;
    if (mm < M && nn < N) {
      if (ep.mode == EPI_PART) ep.out[((long)blockIdx.z * M + mm) * N + nn] = v;
      else apply_epi(ep, M, N, mm, nn, v);
    }
  }
}

// ===========================================================================
// Wide skinny variant (vocab-wide outputs): a block owns all M rows (RT
// tiles of 16) and 16*CW columns; its 4 waves are CW column groups x (4/CW) K
// groups.  Each wave accumulates its 16RT x 16 tile with v_mfma_f64_16x16x4_f64
// (A: row i, k offset lane/16; B: column i, k offset lane/16), double-buffered.
// With CW = 4 (the planned shape) the activation rows come from LDS, staged
// once per block; otherwise both operands are loaded from global memory and
// waves sharing columns are summed through LDS.  blockIdx.y splits K at most 8
// ways: EPI_PART leaves the partials, other modes complete in the last block
// to arrive.  RE: only the real part is formed.
// D[i][j] of row tile t sits at lane j + 16*(i%4), element i/4.
// ===========================================================================
template <int RT, bool RE, int CW, int U = 4>
__global__ __launch_bounds__(256) void k_zgemm_skinny_cols(const double2* __restrict__ X, long ldx, int M,
                                                        const double2* __restrict__ W, long ldw, int N, int K, int kc,
                                                        Epi ep, Argmax am, double2* __restrict__ ws,
                                                        uint32_t* __restrict__ cnt) {
  constexpr int KG = 4 / CW;  // K groups
  __shared__ double2 red[KG > 1 ? KG - 1 : 1][CW][RT * 4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cg = wave % CW, kg = wave / CW;
  const int i = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * 16 * CW + 16 * cg, n = n0 + i;
  const int kb0 = blockIdx.y * kc, kb1 = min(K, kb0 + kc);
  const int q = kc / KG;  // multiple of 16
  const int ka = kb0 + kg * q, kz = min(kb1, ka + q);

  v4d cr[RT], ci[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) cr[t] = ci[t] = v4d{0.0, 0.0, 0.0, 0.0};

  // U k-steps of 4 per batch: two batches (8U weight and 8U*RT activation
  // loads per lane) in flight cover the load latency of the MFMAs of one
  double2 b[2][U], a[2][RT][U];
  auto load = [&](int buf, int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + 4 * u + kq;
      b[buf][u] = ld_glb((kk < kz && n < N) ? W + (long)kk * ldw + n : &rows16s_zero);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const int m = 16 * t + i;
        a[buf][t][u] = ld_glb((kk < kz && m < M) ? X + (long)m * ldx + kk : &rows16s_zero);
      }
    }
  };
  // Cr += Ar*Br + (-Ai)*Bi; Ci += Ar*Bi + Ai*Br (only Cr when the real part is
  // all that is used).  The tiles' first products go before their second ones,
  // so two MFMAs on one accumulator are never adjacent (each would wait for
  // the previous result).
  auto mma = [&](int buf) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].x, b[buf][u].x, cr[t], 0, 0, 0);
        if (!RE) ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].x, b[buf][u].y, ci[t], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        cr[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(-a[buf][t][u].y, b[buf][u].y, cr[t], 0, 0, 0);
        if (!RE) ci[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[buf][t][u].y, b[buf][u].x, ci[t], 0, 0, 0);
      }
    }
  };
  constexpr int KS = 4 * U;
  if constexpr (KG == 1) {
    // All four waves walk the same K range, so the activation rows are staged
    // through LDS once per block (coalesced loads of CK-wide chunks, the next
    // chunk in registers while this one is used) instead of being read by
    // every wave: that was 2 B of L2 traffic per weight byte and kept the
    // texture path about 2/3 busy.  The weights stay a register stream.
    constexpr int CK = RT <= 1 ? 128 : RT == 2 ? 64 : 32;  // k per chunk
    constexpr int NR = 16 * RT;                            // rows staged
    constexpr int PT = NR * CK / 256;                      // elements per thread per chunk
    static_assert(CK % (2 * KS) == 0 && (NR * CK) % 256 == 0, "chunk shape");
    __shared__ double2 As[2][NR][CK + 1];
    const int tid = threadIdx.x;
    double2 st[PT];
    auto fetch = [&](int k0) {
#pragma unroll
      for (int j = 0; j < PT; ++j) {
        const int e = tid + 256 * j, m = e / CK, kk = k0 + (e - m * CK);
        st[j] = ld_glb((m < M && kk < kz) ? X + (long)m * ldx + kk : &rows16s_zero);
      }
    };
    auto stage = [&](int buf) {
#pragma unroll
      for (int j = 0; j < PT; ++j) {
        const int e = tid + 256 * j, m = e / CK;
        As[buf][m][e - m * CK] = st[j];
      }
    };
    auto loadw = [&](int buf, int k) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k + 4 * u + kq;
        b[buf][u] = ld_glb((kk < kz && n < N) ? W + (long)kk * ldw + n : &rows16s_zero);
      }
    };
    auto frag = [&](int abuf, int wbuf, int kl) {  // a[wbuf] <- the chunk's rows at local k kl
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < RT; ++t) a[wbuf][t][u] = As[abuf][16 * t + i][kl + 4 * u + kq];
    };
    const int nch = (kz - ka + CK - 1) / CK;
    if (nch > 0) {
      fetch(ka);
      stage(0);
      loadw(0, ka);
    }
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
      const int kc0 = ka + c * CK;
      if (c + 1 < nch) fetch(kc0 + CK);
      const int ab = c & 1;
#pragma unroll
      for (int bi = 0; bi < CK / KS; bi += 2) {  // two batches per pass: constant buffer indices
        const int k = kc0 + bi * KS;
        if (k < kz) {
          loadw(1, k + KS);
          frag(ab, 0, bi * KS);
          mma(0);
          loadw(0, k + 2 * KS);
          frag(ab, 1, (bi + 1) * KS);
          mma(1);
        }
      }
      if (c + 1 < nch) stage(ab ^ 1);
      __syncthreads();
    }
  } else {
    // double buffer unrolled by two so both buffer indices are constants (registers, not scratch)
    if (ka < kz) load(0, ka);
    for (int k = ka; k < kz; k += 2 * KS) {
      if (k + KS < kz) load(1, k + KS);
      mma(0);
      if (k + KS >= kz) break;
      if (k + 2 * KS < kz) load(0, k + 2 * KS);
      mma(1);
    }
  }

  // K groups of a column group -> the kg == 0 wave, in group order
  if (KG > 1) {
    if (kg > 0)
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[kg - 1][cg][t * 4 + e][lane] = make_double2(cr[t][e], ci[t][e]);
    __syncthreads();
    if (kg == 0)
#pragma unroll
      for (int g = 0; g < KG - 1; ++g)
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const double2 v = red[g][cg][t * 4 + e][lane];
            cr[t][e] += v.x;
            ci[t][e] += v.y;
          }
  }
  const bool owner = kg == 0;
  if (ep.mode == EPI_PART) {  // the next launch sums the partials and applies what follows
    if (owner)
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * t + 4 * e + kq;
          if (m < M && n < N) ep.out[((long)blockIdx.y * M + m) * N + n] = make_double2(cr[t][e], ci[t][e]);
        }
    return;
  }
  const int P = gridDim.y;
  if (P > 1) {
    if (owner)
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * t + 4 * e + kq;
          if (m < M && n < N) st_dev(&ws[((long)blockIdx.y * M + m) * N + n], make_double2(cr[t][e], ci[t][e]));
        }
    if (!arrive_last(&cnt[blockIdx.x], (uint32_t)P)) return;
    if (owner)
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * t + 4 * e + kq;
          if (m < M && n < N) {
            double2 pv[SKINNY_MAX_SPLIT];  // all loads in flight, then summed in split order
#pragma unroll
            for (int p = 0; p < SKINNY_MAX_SPLIT; ++p)
              pv[p] = p < P ? ld_dev(&ws[((long)p * M + m) * N + n]) : make_double2(0.0, 0.0);
            double2 s = pv[0];
#pragma unroll
            for (int p = 1; p < SKINNY_MAX_SPLIT; ++p)
              if (p < P) s = cadd(s, pv[p]);
            cr[t][e] = s.x;
            ci[t][e] = s.y;
          }
        }
  }
  if (!owner) return;
  const bool argmax = am.part_v != nullptr;
  const int tiles16 = (N + 15) / 16;
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * t + 4 * e + kq;
      double re = 0.0;
      if (m < M && n < N) re = apply_epi(ep, M, N, m, n, make_double2(cr[t][e], ci[t][e]));
      if (argmax) {  // (max, last index) of row m over this wave's 16 columns
        double bv = -INFINITY;
        int bi = -1;
        if (m < M && n < N) {
          if (isnan(re)) atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
          else bv = re, bi = n;
        }
        row16_argmax(bv, bi);
        if (i == 0 && m < M) {
          am.part_v[(long)m * tiles16 + n0 / 16] = bv;
          am.part_i[(long)m * tiles16 + n0 / 16] = bi;
        }
      }
    }
}

// ---- planning and dispatch ------------------------------------------------
// GEMV: C columns per block (16, or 64 for wide outputs), K split so that the
// grid has about 512 blocks, at most GEMV_MAX_SPLIT ways.
struct GemvPlan {
  int mr, C, kw, P, ncb;
};
// part: EPI_PART (no completion, the consumer sums): 8-column blocks and a
// split that brings the grid to about 256 blocks -- the fastest shapes of a
// sweep over columns {4, 8, 16, 64} x splits {1, 2, 4, 8} at config 3.
// Otherwise 16 columns (64 for wide outputs) and a completion counter.
// narrow: a final output without the fused argmax (whose partials are one
// per 16 columns) takes 8-column blocks once they alone fill the chip, so no
// K split and no completion in the last block: measured on MI355X, decode
// per step 497 -> 476 us at config 3 with 4 sequences, 710 -> 683 with 8,
// 1647 -> 1599 at config 5
static GemvPlan plan_gemv(int M, int N, int K, bool part, bool narrow = false) {
  GemvPlan p;
  p.mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const bool wide = cdiv_i(N, 64) >= 256;
  p.C = wide ? 64 : (part || (narrow && cdiv_i(N, 8) >= 256) ? 8 : 16);
  const int rpw = 64 / p.C;
  p.ncb = cdiv_i(N, p.C);
  // K splits for a grid of about 256 blocks; with 5-8 rows about 192 (config 3
  // with 8 sequences: QKV without a split, FFN Linear in 3, 447 -> 433 us per
  // step; no change with 2-4 rows)
  int P = std::min(GEMV_MAX_SPLIT, std::max(1, cdiv_i(M > 4 ? 192 : 256, p.ncb)));
  // the vocab product of 5-8 rows splits K in two: each lane's weight rows
  // come 8 per memory round trip after the first 16, with eight rows of
  // multiply-adds between, so halving them per lane pays for the completion.
  // Decode per step at config 3 with 8 sequences 482 -> 449 us (4 splits:
  // 460); with 4 rows the split measured slower (357 -> 369) and 16-column
  // blocks slower for both (386, 500)
  if (wide && M > 4) P = std::max(P, 2);
  // a split product takes as many splits as keep every lane's range within
  // 24 weight rows, the 16 k_gemv requests before its prologue and one batch
  // of 8 (config 5's FFN Linear: 4 splits of 768 rows, not 3 of 1024; 6
  // splits of 512, 16 rows per lane, measured no faster)
  if (part && !wide) P = std::min(GEMV_MAX_SPLIT, std::max(P, cdiv_i(K, 4 * 24 * rpw)));
  // rows per block: a multiple of 4 waves x rpw, and its input rows fit 64 KB of LDS
  const int unit = 4 * rpw;
  int KB = cdiv_i(cdiv_i(K, P), unit) * unit;
  const int kb_max = std::max(unit, (65536 / (16 * p.mr)) / unit * unit);
  KB = std::min(KB, kb_max);
  p.kw = KB / 4;
  p.P = cdiv_i(K, KB);
  if (!part && p.P > GEMV_MAX_SPLIT) p.P = -1;  // not reachable for the supported widths
  return p;
}
// skinny MFMA: wide outputs take 64-column blocks whose 4 waves share the A
// rows (no K split); the rest 16-column blocks, K split over the waves and in
// chunks of multiples of 64 over blocks (about 512 blocks, at most
// SKINNY_MAX_SPLIT ways)
struct SkinnyPlan {
  int rt, cw, ncb, kc, P;  // cw 4: the wide variant
  int rows = 0, ct = 1, nkw = 0;  // rows: the row-tile variant, CT column tiles, nkw k-steps per wave
  int w16 = 0;                    // rows with 16 waves per block (k_zgemm_rows16)
};
// outputs at least this wide take the wide variant (a grid of 256 blocks
// without a K split); measured at config 3, batch 32, the layer products
// (1536 and 2048 columns) were slower in it with 8-way K splits than in the
// narrow variant, whose partials are fewer
constexpr int SKINNY_WIDE_N = 64 * 256;
// K splits of the narrow variant: about this many blocks.  Measured at
// config 3, batch 32 (layer products per generate call): 128 -> 39.4 ms,
// 512 -> 32.7 ms, 1024 -> 34.9 ms (more partials for the consumers)
constexpr int SKINNY_TARGET_BLOCKS = 512;
// Row-tile variant: about this many MFMAs per wave.  Measured alone on MI355X
// at config 3, batch 32 (weights streamed from HBM), against the narrow
// variant: QKV (2 splits, CT 2) 10.4 -> 8.7 us; FFN Dense with no split
// (GELU in the block) 10.3 -> 9.1 us before the narrow variant's split
// completion; FFN Linear (4 splits) 10.2 -> 9.2 us with half the partials.
// 64 and 256 MFMAs per wave measured slower.
constexpr int SKINNY_ROWS_MFMA = 128;
// the 16-wave row-tile kernel from this inner dimension up (a block's K range
// covers 16 waves of 4-step batches)
constexpr int ROWS16_MIN_K = 256;
constexpr int SKINNY_ROWS_MAX_NKW = 64;     // k-steps per wave of a product that may not split K
constexpr int SKINNY_ROWS_MIN_BLOCKS = 128;  // fewer: the chip is less than half busy
// argmax: the fused greedy id needs per-tile partials, which only the narrow
// and wide variants leave
static SkinnyPlan plan_skinny(int M, int N, int K, bool part, bool argmax) {
  SkinnyPlan p;
  p.rt = cdiv_i(M, 16);
  if (N >= SKINNY_WIDE_N) {
    // 64 columns per block, activation rows shared through LDS; K split over
    // blocks for a grid of about 256 (one split for outputs that fill it)
    p.cw = 4;
    p.ncb = cdiv_i(N, 64);
    const int P = std::min(SKINNY_MAX_SPLIT, std::max(1, cdiv_i(256, p.ncb)));
    p.kc = cdiv_i(cdiv_i(K, P), 64) * 64;
    p.P = cdiv_i(K, p.kc);
    return p;
  }
  p.cw = 0;
  if (!argmax && K >= ROWS16_MIN_K) {
    // 16 waves per block, 512 of K per block (32 per wave): the layer products
    // of config 3 and up fill the chip with one K range per block (FFN Dense,
    // QKV) or four (FFN Linear, K 2048)
    SkinnyPlan r = p;
    r.rows = 1;
    r.w16 = 1;
    r.ct = 1;
    r.ncb = cdiv_i(N, 16);
    r.nkw = 8;
    int P = cdiv_i(K, 64 * r.nkw);
    if (!part) {
      r.nkw = cdiv_i(K, 64);
      P = 1;
    } else if (P > SKINNY_MAX_SPLIT) {
      r.nkw = cdiv_i(K, 64 * SKINNY_MAX_SPLIT);
      P = cdiv_i(K, 64 * r.nkw);
    }
    r.P = P;
    r.kc = 64 * r.nkw;
    if (r.nkw <= SKINNY_ROWS_MAX_NKW) return r;
  }
  if (!argmax) {
    SkinnyPlan r = p;
    const int tiles = cdiv_i(N, 16) * p.rt;  // 16x16 output tiles
    r.rows = 1;
    r.ct = (part && tiles >= 128) ? 2 : 1;
    r.ncb = cdiv_i(N, 16 * r.ct);
    r.nkw = SKINNY_ROWS_MFMA / (4 * r.ct);
    int P = cdiv_i(K, 16 * r.nkw);
    if (part) {
      // at most SKINNY_MAX_SPLIT partials; more splits (shorter waves) for a
      // grid that would leave most of the chip idle
      const int fill = std::min(SKINNY_MAX_SPLIT, cdiv_i(192, r.ncb * p.rt));
      P = std::min(SKINNY_MAX_SPLIT, std::max(P, fill));
      r.nkw = std::max(4, cdiv_i(cdiv_i(K, 16 * P), 4) * 4);
      P = cdiv_i(K, 16 * r.nkw);
    } else if (P > 1) {
      r.nkw = std::max(4, cdiv_i(cdiv_i(K, 16), 4) * 4);
      P = 1;
    }
    r.P = P;
    r.kc = 16 * r.nkw;
    if (r.nkw <= SKINNY_ROWS_MAX_NKW && (part || (long)r.ncb * p.rt >= SKINNY_ROWS_MIN_BLOCKS)) return r;
  }
  p.ncb = cdiv_i(N, 16);
  const int P = std::min(SKINNY_MAX_SPLIT, std::max(1, cdiv_i(SKINNY_TARGET_BLOCKS, p.ncb)));
  p.kc = cdiv_i(cdiv_i(K, P), 64) * 64;
  p.P = cdiv_i(K, p.kc);
  return p;
}
struct MfmaPlan {
  int P, kchunk, mt, nt;
};
constexpr int MFMA_MAX_SPLIT = 8;
static MfmaPlan plan_mfma(int M, int N, int K) {
  MfmaPlan p;
  p.mt = cdiv_i(M, GBM);
  p.nt = cdiv_i(N, GBN);
  const int tiles = p.mt * p.nt;
  int P = 1;
  // at most MFMA_MAX_SPLIT ways: at config 3, batch 1 (128 prompt rows) FFN
  // Linear split 32 ways took 199 us, FFN Dense split 8 ways 92 us for the
  // same flops
  if (tiles < 512) P = std::min({cdiv_i(512, tiles), std::max(1, K / 64), MFMA_MAX_SPLIT});
  p.kchunk = cdiv_i(cdiv_i(K, P), GBK) * GBK;
  p.P = cdiv_i(K, p.kchunk);
  return p;
}

constexpr int SKINNY_MAX_M = 64;

int gemm_parts(int M, int N, int K) {
  if (M <= 8) return plan_gemv(M, N, K, true).P;
  if (M <= SKINNY_MAX_M) {
    const SkinnyPlan p = plan_skinny(M, N, K, true, false);
    return p.P;
  }
  return 0;
}

size_t gemm_ws_bytes(int M, int N, int K) {
  int P;
  if (M <= 8) P = std::max(plan_gemv(M, N, K, false).P, plan_gemv(M, N, K, false, true).P);
  else if (M <= SKINNY_MAX_M) P = plan_skinny(M, N, K, false, true).P;  // the largest split workspace
  else P = plan_mfma(M, N, K).P;
  return P > 1 ? (size_t)P * M * N * sizeof(double2) : 0;
}

// argmax partials: one per row and 16-column tile covers every product shape
size_t argmax_part_elems(int M, int N) { return (size_t)M * cdiv_i(N, 16); }

static size_t gemv_lds_bytes(const GemvPlan& p, const RowOps& ro, int M, int K) {
  const size_t rl = ro.ln ? (size_t)K : (size_t)4 * p.kw;
  return (size_t)p.mr * rl * sizeof(double2) +
         (ro.att.po ? (size_t)M * ro.att.H * (ro.att.nsplit + 1) * sizeof(double) : 0);
}

template <int MR, int C>
static void launch_gemv(hipStream_t st, const GemvPlan& p, const RowOps& ro, int M, const double2* W, long ldw, int N,
                        int K, const Epi& ep, const Argmax& am, const Sync& sy) {
  dim3 grid(p.ncb, p.P);
  const size_t shm = gemv_lds_bytes(p, ro, M, K);
  // plain rows that fit the staging registers are requested before the weights
  if (ro.plain() && (long)MR * 4 * p.kw <= 256L * GEMV_PRE)
    MITOK_LAUNCH((k_gemv<MR, C, true>), grid, dim3(256), shm, st, ro, M, W, ldw, N, K, p.kw, ep, am, (double2*)sy.ws,
                 sy.counters);
  else
    MITOK_LAUNCH((k_gemv<MR, C, false>), grid, dim3(256), shm, st, ro, M, W, ldw, N, K, p.kw, ep, am, (double2*)sy.ws,
                 sy.counters);
}
template <int MR>
static void launch_gemv_c(hipStream_t st, const GemvPlan& p, const RowOps& ro, int M, const double2* W, long ldw, int N,
                          int K, const Epi& ep, const Argmax& am, const Sync& sy) {
  if (p.C == 64) launch_gemv<MR, 64>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
  else if (p.C == 16) launch_gemv<MR, 16>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
  else launch_gemv<MR, 8>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
}

template <bool RE>
static void launch_skinny(hipStream_t st, const SkinnyPlan& p, const RowOps& ro, int M, const double2* W, long ldw,
                          int N, int K, const Epi& ep, const Argmax& am, const Sync& sy) {
  const dim3 grid(p.ncb, p.P), blk(256);
  double2* ws = (double2*)sy.ws;
  if (p.rows) {  // EPI_PART, or one K range per block (no argmax: not a vocab-wide output)
    const dim3 g3(p.ncb, p.rt, p.P);
    if (p.w16) {
      if (p.nkw == 8) MITOK_LAUNCH(k_zgemm_rows16s<4>, g3, dim3(64 * ROWS16_WAVES), ROWS16_LDS, st, ro.x, ro.ldx, M, W, ldw, N, K, ep);
      else if (p.nkw == 12) MITOK_LAUNCH(k_zgemm_rows16s<6>, g3, dim3(64 * ROWS16_WAVES), ROWS16_LDS, st, ro.x, ro.ldx, M, W, ldw, N, K, ep);
      else MITOK_LAUNCH(k_zgemm_rows16, g3, dim3(64 * ROWS16_WAVES), ROWS16_LDS, st, ro.x, ro.ldx, M, W, ldw, N, K, p.nkw, ep);
      return;
    }
    if (p.ct == 2) MITOK_LAUNCH(k_zgemm_skinny_rows<2>, g3, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.nkw, ep);
    else MITOK_LAUNCH(k_zgemm_skinny_rows<1>, g3, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.nkw, ep);
    return;
  }
  if (p.cw == 4) {
    switch (p.rt) {
      case 1: MITOK_LAUNCH((k_zgemm_skinny_cols<1, RE, 4>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
      case 2: MITOK_LAUNCH((k_zgemm_skinny_cols<2, RE, 4>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
      case 3: MITOK_LAUNCH((k_zgemm_skinny_cols<3, RE, 4>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
      default: MITOK_LAUNCH((k_zgemm_skinny_cols<4, RE, 4>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
    }
    return;
  }
  switch (p.rt) {
    case 1: MITOK_LAUNCH((k_zgemm_skinny<1, RE>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
    case 2: MITOK_LAUNCH((k_zgemm_skinny<2, RE>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
    case 3: MITOK_LAUNCH((k_zgemm_skinny<3, RE>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
    default: MITOK_LAUNCH((k_zgemm_skinny<4, RE>), grid, blk, 0, st, ro.x, ro.ldx, M, W, ldw, N, K, p.kc, ep, am, ws, sy.counters); break;
  }
}

int gemm(hipStream_t st, int M, int N, int K, const RowOps& ro, const double2* W, long ldw, const Epi& ep,
         const Argmax* amp, const Sync& sy) {
  if (M <= 0 || N <= 0) return OK;
  if (K <= 0) return ERR_ARG;  // no product has an empty inner dimension
  const Argmax am = amp ? *amp : Argmax();
  if (ep.mode != EPI_PART && gemm_ws_bytes(M, N, K) > sy.ws_bytes) return ERR_STATE;
  int tiles = 0;  // column tiles of the argmax partials
  if (M <= 8) {
    const bool part = ep.mode == EPI_PART;
    const GemvPlan p = plan_gemv(M, N, K, part, am.part_v == nullptr);
    if (p.P < 1 || p.ncb >= SYNC_COUNTERS || (part && am.part_v)) return ERR_ARG;
    if (gemv_lds_bytes(p, ro, M, K) > 120 * 1024) return ERR_ARG;
    switch (p.mr) {
      case 1: launch_gemv_c<1>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      case 2: launch_gemv_c<2>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      case 4: launch_gemv_c<4>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
      default: launch_gemv_c<8>(st, p, ro, M, W, ldw, N, K, ep, am, sy); break;
    }
    tiles = p.ncb;
  } else {
    if (!ro.plain()) return ERR_ARG;  // the MFMA paths read plain rows
    if (M <= SKINNY_MAX_M) {
      const SkinnyPlan p = plan_skinny(M, N, K, ep.mode == EPI_PART, am.part_v != nullptr);
      if (p.ncb >= SYNC_COUNTERS) return ERR_ARG;
      if (ep.mode == EPI_PART && am.part_v) return ERR_ARG;
      if (ep.mode == EPI_RE) launch_skinny<true>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
      else launch_skinny<false>(st, p, ro, M, W, ldw, N, K, ep, am, sy);
      tiles = cdiv_i(N, 16);  // argmax partials per 16 columns
    } else {
      if (ep.mode == EPI_PART) return ERR_ARG;
      const MfmaPlan p = plan_mfma(M, N, K);
      if (p.P > 1 && (long)p.mt * p.nt >= SYNC_COUNTERS) return ERR_ARG;
      dim3 grid(p.nt, p.mt, p.P);
      if (launch_zgemm_mfma(st, grid, ro.x, ro.ldx, W, ldw, M, N, K, p.kchunk, ep, am, (double2*)sy.ws, sy.counters) != OK)
        return ERR_ARG;
      tiles = p.nt;
    }
  }
  if (am.part_v) MITOK_LAUNCH(k_argmax_finalize, dim3(M), dim3(256), 0, st, am, tiles);
  return OK;
}

}  // namespace mitok
