// rowops.hpp — the row transform a product applies to its input rows on the
// fly (RowOps in kernels.hpp): device functions shared by the GEMV prologue and
// the stand-alone materialisation kernel.
//
// Reference operations restated here (paths relative to src/neural_networks/):
//   embedding gather, PAD id 1 -> 0         embedding_layer.rs:158-211
//   RoPE on (even, odd) pairs               positional_encoding_layer.rs:181-209
//   bias add                                 utils/matrix.rs:615-625
//   gelu_complex, pad rows -> 0             utils/activation.rs:195-212,268-284
//   residual Re(x + before) + 0i            utils/matrix.rs:600-613
//   NormalNormLayer                         network_components/norm_layer.rs:64-130
//   decode attention combine over chunks    masked_attention_head.rs:184-208
#pragma once

#include "kernels.hpp"

namespace mitok {

// Per-block state of an attention-combine source: for local row lm and head h,
// wts[(lm*H + h)*nsplit + s] = e^(m_s - M) and lsum[lm*H + h] = sum_s l_s e^(m_s - M).
struct RoLds {
  double* wts = nullptr;
  double* lsum = nullptr;
  int m0 = 0;  // global index of local row 0
};

__device__ __forceinline__ size_t ro_lds_doubles(const RowOps& r, int M) {
  return r.att.po ? (size_t)M * r.att.H * (r.att.nsplit + 1) : 0;
}

// Block-wide; all threads call it.  One wave per two (row, head) pairs: the
// KV lengths and every chunk's (max, sum) of both pairs are requested
// together (chunks past the sequence's length are read and then masked; the
// buffer holds nsplit of them), so the weights cost one memory round trip.
template <class Acc = AccPlain>
__device__ inline void ro_prepare(const RowOps& r, int M, const RoLds& L) {
  if (!r.att.po) return;
  const AttnSplit& a = r.att;
  constexpr int SL = 4;  // chunk slots per lane: nsplit <= 256
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int mh0 = wave; mh0 < M * a.H; mh0 += 8) {
    double vm[2][SL], vl[2][SL];
    int ns[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int mh = mh0 + 4 * q;
      const bool valid = mh < M * a.H;
      const int lm = valid ? mh / a.H : 0, h = valid ? mh - lm * a.H : 0;
      ns[q] = valid ? (Acc::kv(a.kv_len, L.m0 + lm) + 1 + a.CH - 1) / a.CH : 0;
      const long base = ((long)(L.m0 + lm) * a.H + h) * a.nsplit;
#pragma unroll
      for (int j = 0; j < SL; ++j) {
        const int sidx = lane + 64 * j;
        const bool in = valid && sidx < a.nsplit;
        vm[q][j] = in ? Acc::ld(a.pm + base + sidx) : -INFINITY;
        vl[q][j] = in ? Acc::ld(a.pl + base + sidx) : 0.0;
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int mh = mh0 + 4 * q;
      if (mh >= M * a.H) continue;  // uniform over the wave
      double mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < SL; ++j)
        if (lane + 64 * j < ns[q]) mx = fmax(mx, vm[q][j]);
      mx = wave_max(mx);
      double l = 0.0;
#pragma unroll
      for (int j = 0; j < SL; ++j) {
        const int sidx = lane + 64 * j;
        if (sidx < ns[q]) {
          const double w = exp(vm[q][j] - mx);
          L.wts[(long)mh * a.nsplit + sidx] = w;
          l += vl[q][j] * w;
        }
      }
      l = wave_sum(l);
      if (lane == 0) L.lsum[mh] = l;
    }
  }
  __syncthreads();
}

// source element (m global row) + bias -> finite check -> GELU.  Loads of
// partials and attention chunks are unrolled by 8 so they are in flight together.
template <class Acc = AccPlain>
__device__ __forceinline__ double2 ro_base(const RowOps& r, int m, int k, int K, const RoLds& L) {
  double2 v;
  if (r.table) {
    const uint32_t id = Acc::id(r.ids, m);
    if (id == 1u || id >= (uint32_t)r.vocab) v = make_double2(0.0, 0.0);  // PAD; bad ids flagged by ro_check
    else v = Acc::c(r.table + (long)id * K + k);
  } else if (r.att.po) {
    const AttnSplit& a = r.att;
    const int h = k / a.dh, e = k - h * a.dh;
    const int lm = m - L.m0;
    const int T = Acc::kv(a.kv_len, m) + 1;
    const int ns = (T + a.CH - 1) / a.CH;
    const long base = ((long)m * a.H + h) * a.nsplit;
    const double* w = L.wts + ((long)lm * a.H + h) * a.nsplit;
    double2 o = make_double2(0.0, 0.0);
    for (int s0 = 0; s0 < ns; s0 += 8) {
      double2 t[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) t[q] = s0 + q < ns ? Acc::ld(a.po + (base + s0 + q) * a.dh + e) : make_double2(0.0, 0.0);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (s0 + q < ns) {
          o.x += t[q].x * w[s0 + q];
          o.y += t[q].y * w[s0 + q];
        }
    }
    const double l = L.lsum[lm * a.H + h];
    v = make_double2(o.x / l, o.y / l);
  } else {
    const double2* p = r.x + (long)m * r.ldx + k;
    if (r.npart <= 1) {
      v = Acc::ld(p);
    } else {
      double2 t[8];  // npart <= 8 (the GEMV splits at most 8 ways)
#pragma unroll
      for (int q = 0; q < 8; ++q) t[q] = q < r.npart ? Acc::ld(p + q * r.part_stride) : make_double2(0.0, 0.0);
      v = t[0];
#pragma unroll
      for (int q = 1; q < 8; ++q)
        if (q < r.npart) v = cadd(v, t[q]);
    }
  }
  if (r.bias) v = cadd(v, Acc::c(r.bias + k));
  if (r.finite_check && !(isfinite(v.x) && isfinite(v.y))) atomicOr(r.err, (uint32_t)EB_FFN_NONFINITE);
  if (r.gelu) {
    if (r.row_mask && Acc::c(r.row_mask + m) == 0) {
      v = make_double2(0.0, 0.0);
    } else {
      bool nan = false;
      v = gelu_nc(v, &nan);
      if (nan) atomicOr(r.err, (uint32_t)EB_GELU_NAN);
    }
  }
  return v;
}

// position of row m for RoPE: its table entry, plus the row's offset when the
// prompt pass compressed the sequence (a wavelet layer: decode positions count
// the uncompressed prompt, transformer_network.rs:300-304)
template <class Acc = AccPlain>
__device__ __forceinline__ int ro_pos(const RowOps& r, int m) {
  return Acc::kv(r.rope_pos, m) + (r.rope_off ? Acc::c(r.rope_off + m) : 0);
}

// with RoPE: pairs (2i, 2i+1) rotate by the tabulated angle of the row's position
template <class Acc = AccPlain>
__device__ __forceinline__ double2 ro_source(const RowOps& r, int m, int k, int K, const RoLds& L) {
  if (!r.rope_cs) return ro_base<Acc>(r, m, k, K, L);
  const int p = min(ro_pos<Acc>(r, m), r.rope_max - 1);  // overflow flagged by ro_check
  const int i = k >> 1;
  const double2 t = Acc::c(r.rope_cs + (long)p * (K >> 1) + i);
  const double2 e = ro_base<Acc>(r, m, 2 * i, K, L), o = ro_base<Acc>(r, m, 2 * i + 1, K, L);
  return (k & 1) ? make_double2(e.x * t.y + o.x * t.x, e.y * t.y + o.y * t.x)
                 : make_double2(e.x * t.x - o.x * t.y, e.y * t.x - o.y * t.y);
}

template <class Acc = AccPlain>
__device__ __forceinline__ double2 ro_value(const RowOps& r, int m, int k, int K, const RoLds& L) {
  double2 v = ro_source<Acc>(r, m, k, K, L);
  if (r.resid) v = make_double2(v.x + Acc::ld(r.resid + (long)m * r.ldr + k).x, 0.0);
  return v;
}

template <class Acc = AccPlain>
__device__ __forceinline__ void ro_check(const RowOps& r, int m) {
  if (r.table) {
    const uint32_t id = Acc::id(r.ids, m);
    if (id != 1u && id >= (uint32_t)r.vocab) atomicOr(r.err, (uint32_t)EB_BAD_TOKEN);
  }
  if (r.rope_cs && ro_pos<Acc>(r, m) >= r.rope_max) atomicOr(r.err, (uint32_t)EB_CTX_OVERFLOW);
}

constexpr int LN_PRE = 4;  // gamma/beta columns per thread requested up front (rows up to 1024 wide)

// normalize (norm_layer.rs:77): Re(((x - mean) / sd) * gamma + beta) + 0i
__device__ __forceinline__ double2 ln_apply(double2 v, double2 mean, double2 sd, double2 g, double2 b) {
  const double2 o = cadd(cmul(cdiv(csub(v, mean), sd), g), b);
  return make_double2(o.x, 0.0);
}

// LayerNorm statistics of rows L.m0 .. L.m0+M-1 (M <= MR) over K elements:
// mean = sum(x) / K, var = sum((x - mean)^2) / K (complex square),
// sd = csqrt(var + eps) (norm_layer.rs:64-80).  Block-wide; all threads call it.
template <int MR, class Acc = AccPlain>
__device__ void ro_stats(const RowOps& r, int M, int K, const RoLds& L, double2* mean_s, double2* sd_s) {
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
        const double2 v = ro_value<Acc>(r, L.m0 + m, k, K, L);
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
        const double2 t = csub(ro_value<Acc>(r, L.m0 + m, k, K, L), mean_s[m]);
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


// Builds the transformed input rows m < M (M <= MR; local row m is global row
// L.m0 + m) into LDS: buf[m * RL + (k - ka)] for k in [ka, ka + RL).  With a
// LayerNorm the range must be the whole row (ka = 0, RL = K) and only
// [n0, n1) is normalised; RoPE pairs must not straddle the range (ka even).
// Every source element is loaded once; statistics are taken from LDS.
// Block-wide; all threads call it; ends with a barrier.
// The LayerNorm of rows m < M (M <= MR) held in LDS at buf[m * RL + k]
// (the whole row: ka = 0, RL = K), normalising columns [n0, n1) in place.
// gpre/bpre: gamma and beta of this thread's first LN_PRE columns, requested
// by the caller with the source rows.  Block-wide; ends with a barrier.
template <int MR, class Acc = AccPlain>
__device__ __forceinline__ void ro_ln(const RowOps& r, int M, int K, int RL, int n0, int n1, double2* buf, double2* st_mean,
                      double2* st_sd, const double2 (&gpre)[LN_PRE], const double2 (&bpre)[LN_PRE]) {
  __shared__ double red_s[4][2 * MR], red_v[4][2 * MR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const double len = (double)K;
  double a[2 * MR];
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = 0.0;
  for (int k = tid; k < K; k += 256)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) {
        const double2 v = buf[m * RL + k];
        a[2 * m] += v.x;
        a[2 * m + 1] += v.y;
      }
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = wave_sum(a[j]);
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < 2 * MR; ++j) red_s[wave][j] = a[j];
  __syncthreads();
  // one row: every thread forms the mean (same operands, same order, same
  // bits); more rows: one thread per row, through LDS
  double2 mean0 = make_double2(0.0, 0.0);
  if (MR == 1) {
    const double sre = (red_s[0][0] + red_s[1][0]) + (red_s[2][0] + red_s[3][0]);
    const double sim = (red_s[0][1] + red_s[1][1]) + (red_s[2][1] + red_s[3][1]);
    mean0 = make_double2(sre / len, sim / len);
  } else {
    if (tid < M) {
      const double sre = (red_s[0][2 * tid] + red_s[1][2 * tid]) + (red_s[2][2 * tid] + red_s[3][2 * tid]);
      const double sim = (red_s[0][2 * tid + 1] + red_s[1][2 * tid + 1]) + (red_s[2][2 * tid + 1] + red_s[3][2 * tid + 1]);
      st_mean[tid] = make_double2(sre / len, sim / len);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = 0.0;
  for (int k = tid; k < K; k += 256)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) {
        const double2 t = csub(buf[m * RL + k], MR == 1 ? mean0 : st_mean[m]);
        const double2 tt = cmul(t, t);
        a[2 * m] += tt.x;
        a[2 * m + 1] += tt.y;
      }
#pragma unroll
  for (int j = 0; j < 2 * MR; ++j) a[j] = wave_sum(a[j]);
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < 2 * MR; ++j) red_v[wave][j] = a[j];
  __syncthreads();
  if (MR == 1) {
    // one row: every thread takes the square root itself rather than waiting
    // at another barrier for one thread's
    const double vre = (red_v[0][0] + red_v[1][0]) + (red_v[2][0] + red_v[3][0]);
    const double vim = (red_v[0][1] + red_v[1][1]) + (red_v[2][1] + red_v[3][1]);
    const double2 sd = csqrt_nc(make_double2(vre / len + r.eps, vim / len + 0.0));
    if (tid == 0) st_mean[0] = mean0, st_sd[0] = sd;
#pragma unroll
    for (int j = 0; j < LN_PRE; ++j) {
      const int k = n0 + tid + 256 * j;
      if (k < n1) buf[k] = ln_apply(buf[k], mean0, sd, gpre[j], bpre[j]);
    }
    for (int k = n0 + tid + 256 * LN_PRE; k < n1; k += 256)
      buf[k] = ln_apply(buf[k], mean0, sd, Acc::c(r.gamma + k), Acc::c(r.beta + k));
  } else {
    if (tid < M) {
      const double vre = (red_v[0][2 * tid] + red_v[1][2 * tid]) + (red_v[2][2 * tid] + red_v[3][2 * tid]);
      const double vim = (red_v[0][2 * tid + 1] + red_v[1][2 * tid + 1]) + (red_v[2][2 * tid + 1] + red_v[3][2 * tid + 1]);
      st_sd[tid] = csqrt_nc(make_double2(vre / len + r.eps, vim / len + 0.0));
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < LN_PRE; ++j) {
      const int k = n0 + tid + 256 * j;
      if (k < n1)
        for (int m = 0; m < M; ++m) buf[m * RL + k] = ln_apply(buf[m * RL + k], st_mean[m], st_sd[m], gpre[j], bpre[j]);
    }
    for (int k = n0 + tid + 256 * LN_PRE; k < n1; k += 256) {
      const double2 g = Acc::c(r.gamma + k), b = Acc::c(r.beta + k);
      for (int m = 0; m < M; ++m) buf[m * RL + k] = ln_apply(buf[m * RL + k], st_mean[m], st_sd[m], g, b);
    }
  }
  __syncthreads();
}

template <int MR, class Acc = AccPlain>
__device__ void ro_build(const RowOps& r, int M, int K, int ka, int RL, int n0, int n1, double2* buf, const RoLds& L,
                         double2* st_mean, double2* st_sd) {
  const int tid = threadIdx.x;
  // the LayerNorm's gamma and beta of this thread's first columns are
  // requested with the source rows, not after the statistics
  double2 gpre[LN_PRE], bpre[LN_PRE];
#pragma unroll
  for (int j = 0; j < LN_PRE; ++j) {
    const int k = n0 + tid + 256 * j;
    const bool ok = r.ln && k < n1;
    gpre[j] = ok ? Acc::c(r.gamma + k) : make_double2(0.0, 0.0);
    bpre[j] = ok ? Acc::c(r.beta + k) : make_double2(0.0, 0.0);
  }
  // pass 1: every source element once, four per thread with their loads in
  // flight together; without RoPE the residual joins here
  const bool res1 = r.resid && !r.rope_cs;
  const int tot = MR * RL;
  for (int i0 = tid; i0 < tot; i0 += 4 * 256) {
    double2 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * 256;
      const int m = i / RL, k = ka + (i - m * RL);
      const bool ok = i < tot && m < M && k < K;
      v[u] = ok ? ro_base<Acc>(r, L.m0 + m, k, K, L) : make_double2(0.0, 0.0);
      if (res1 && ok) v[u] = make_double2(v[u].x + Acc::ld(r.resid + (long)(L.m0 + m) * r.ldr + k).x, 0.0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + u * 256 < tot) buf[i0 + u * 256] = v[u];
  }
  __syncthreads();
  if (r.rope_cs) {
    const int half = (RL + 1) / 2;
    for (int i = tid; i < MR * half; i += 256) {
      const int m = i / half, j = i - m * half, k = ka + 2 * j;
      if (m >= M || k >= K) continue;
      const int gm = L.m0 + m;
      const bool pair = 2 * j + 1 < RL && k + 1 < K;  // always true with RoPE (even K, even range)
      double2 e = buf[m * RL + 2 * j], o = pair ? buf[m * RL + 2 * j + 1] : make_double2(0.0, 0.0);
      if (r.rope_cs) {
        const int p = min(ro_pos<Acc>(r, gm), r.rope_max - 1);  // overflow flagged by ro_check
        const double2 t = Acc::c(r.rope_cs + (long)p * (K >> 1) + (k >> 1));
        const double2 e2 = make_double2(e.x * t.x - o.x * t.y, e.y * t.x - o.y * t.y);
        const double2 o2 = make_double2(e.x * t.y + o.x * t.x, e.y * t.y + o.y * t.x);
        e = e2;
        o = o2;
      }
      if (r.resid) {
        e = make_double2(e.x + Acc::ld(r.resid + (long)gm * r.ldr + k).x, 0.0);
        if (pair) o = make_double2(o.x + Acc::ld(r.resid + (long)gm * r.ldr + k + 1).x, 0.0);
      }
      buf[m * RL + 2 * j] = e;
      if (pair) buf[m * RL + 2 * j + 1] = o;
    }
    __syncthreads();
  }
  if (!r.ln) return;
  ro_ln<MR, Acc>(r, M, K, RL, n0, n1, buf, st_mean, st_sd, gpre, bpre);
}

}  // namespace mitok
