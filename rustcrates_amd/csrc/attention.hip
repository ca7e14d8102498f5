// attention.hip — MaskedAttentionHead::forward (masked_attention_head.rs:122-220)
// on gfx950: scores Re(q.k) * 1/(1e-8 + sqrt(dh)) + Re(bias_pos[r][c]), causal
// mask -1e12, softmax of the real part (activation.rs:431-439), pad query rows
// 0 (:369-388), out = sum_c p_c v_c (utils/matrix.rs:356-380).
#include <algorithm>

#include "kernels.hpp"

namespace mitok {

static inline int cdiv_i(long a, long b) { return (int)((a + b - 1) / b); }

// ===========================================================================
// One block per (query row, head, sequence).  The S x S causal mask is applied
// modulo its size (masked_attention_head.rs:494-503), so key c is visible iff
// (c % S) <= r; bias_pos row r (decode of several rows keeps the reference's
// top-left slice, :193-194).
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
  double* sc = smem;                          // [T_max]
  double2* qs = (double2*)(smem + a.T_max);  // [dh]
  double2* pv = qs + a.dh;                   // [256]
  double* wred = (double*)(pv + 256);        // [8]
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
        const double2 kv = kr[e], qv = qs[e];
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
    const double e = exp(sc[c] - mx);
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
      const double p = sc[c] / sum;
      const double2 v = V[(long)c * a.dh + e];
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
  const size_t shm = (size_t)a.T_max * sizeof(double) + (size_t)(a.dh + 256) * sizeof(double2) + 8 * sizeof(double);
  hipLaunchKernelGGL(k_attention_rows, dim3(a.S, a.H, a.B), dim3(256), shm, st, a);
}

// ===========================================================================
// Decode (one query row per sequence, masked_attention_head.rs:135-208 with
// the cache): keys are split in chunks of CH, one block per (chunk, head,
// sequence).  No causal mask in this branch; bias_pos row 0.  A block scores
// its chunk (16 lanes per key, 4 keys per wave), keeps the chunk's max m,
// sum l of exp(s - m) and o = sum exp(s - m) v, and the last chunk of each
// (sequence, head) to finish rescales the chunks to the common max, in
// chunk order: out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// ===========================================================================
constexpr int DEC_LPK = 16;          // lanes per key in the score phase
constexpr int DEC_MAX_SPLITS = 256;  // key chunks per (sequence, head)

static int decode_chunk(int B, int H) { return B * H <= 64 ? 32 : 64; }

__global__ __launch_bounds__(256) void k_attention_decode(Attn a, int CH, int nsplit, double* __restrict__ pm,
                                                          double* __restrict__ pl, double2* __restrict__ po,
                                                          uint32_t* __restrict__ cnt) {
  __shared__ double sc[64];
  __shared__ double2 pv[256];
  __shared__ double stat[2];
  __shared__ double cw[DEC_MAX_SPLITS], cl[DEC_MAX_SPLITS];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.kv_len ? a.kv_len[b] + a.T_add : a.T_const;
  const int c0 = split * CH;
  if (c0 >= T) return;  // not part of this sequence's split count
  const int nc = min(CH, T - c0);
  const int ns = (T + CH - 1) / CH;
  const long bh = (long)b * a.H + h;
  const double2* qrow = a.q + (long)b * a.ldq + (long)h * a.dh;
  const double2* K = a.kc + bh * a.ctx * a.dh;
  const double2* V = a.vc + bh * a.ctx * a.dh;
  const double* bias0 = a.bias_re + (long)h * a.mc * a.mc;  // bias_pos row 0

  // scores: key j = it + 4*w + (lane / 16) of the chunk, lanes j%16 split the head dim
  const int sub = lane & (DEC_LPK - 1), kw = lane / DEC_LPK;
  for (int j0 = 0; j0 < nc; j0 += 16) {
    const int j = j0 + wave * 4 + kw;
    double acc = 0.0;
    if (j < nc) {
      const double2* kr = K + (long)(c0 + j) * a.dh;
      for (int e = sub; e < a.dh; e += DEC_LPK) {
        const double2 kv = kr[e], qv = qrow[e];
        acc += qv.x * kv.x - qv.y * kv.y;
      }
    }
#pragma unroll
    for (int o = DEC_LPK / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (j < nc && sub == 0) sc[j] = acc * a.scale + bias0[c0 + j];
  }
  __syncthreads();
  if (wave == 0) {
    const double s = lane < nc ? sc[lane] : -INFINITY;
    const double m = wave_max(s);
    const double p = lane < nc ? exp(s - m) : 0.0;
    const double l = wave_sum(p);
    if (lane < nc) sc[lane] = p;
    if (lane == 0) stat[0] = m, stat[1] = l;
  }
  __syncthreads();
  const int G = 256 / a.dh;
  const int e = tid % a.dh, g = tid / a.dh;
  double2 acc = make_double2(0.0, 0.0);
  if (g < G)
    for (int j = g; j < nc; j += G) {
      const double p = sc[j];
      const double2 v = V[(long)(c0 + j) * a.dh + e];
      acc.x += p * v.x;
      acc.y += p * v.y;
    }
  pv[tid] = acc;
  __syncthreads();
  const long pidx = bh * nsplit + split;
  if (tid < a.dh) {
    double2 s = pv[tid];
    for (int gg = 1; gg < G; ++gg) s = cadd(s, pv[gg * a.dh + tid]);
    st_dev(&po[pidx * a.dh + tid], s);
  }
  if (tid == 0) {
    st_dev(&pm[pidx], stat[0]);
    st_dev(&pl[pidx], stat[1]);
  }
  if (!arrive_last(&cnt[bh], (uint32_t)ns)) return;

  double2* out = a.out + (long)b * a.ldo + (long)h * a.dh;
  if (a.row_mask && a.row_mask[b] == 0) {
    for (int t = tid; t < a.dh; t += 256) out[t] = make_double2(0.0, 0.0);
    return;
  }
  const long base = bh * nsplit;
  // chunk statistics through LDS: cw[s] = e^(m_s - M), L = sum_s l_s cw[s] in chunk order
  if (tid < ns) cw[tid] = ld_dev(&pm[base + tid]);
  __syncthreads();
  double M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmax(M, cw[s]);
  __syncthreads();
  if (tid < ns) {
    const double w = exp(cw[tid] - M);
    cw[tid] = w;
    cl[tid] = ld_dev(&pl[base + tid]) * w;
  }
  __syncthreads();
  double L = 0.0;
  for (int s = 0; s < ns; ++s) L += cl[s];
  for (int t = tid; t < a.dh; t += 256) {
    double2 o = make_double2(0.0, 0.0);
    int s = 0;
    for (; s + 4 <= ns; s += 4) {
      const double2 v0 = ld_dev(&po[(base + s) * a.dh + t]);
      const double2 v1 = ld_dev(&po[(base + s + 1) * a.dh + t]);
      const double2 v2 = ld_dev(&po[(base + s + 2) * a.dh + t]);
      const double2 v3 = ld_dev(&po[(base + s + 3) * a.dh + t]);
      o.x += v0.x * cw[s], o.y += v0.y * cw[s];
      o.x += v1.x * cw[s + 1], o.y += v1.y * cw[s + 1];
      o.x += v2.x * cw[s + 2], o.y += v2.y * cw[s + 2];
      o.x += v3.x * cw[s + 3], o.y += v3.y * cw[s + 3];
    }
    for (; s < ns; ++s) {
      const double2 v = ld_dev(&po[(base + s) * a.dh + t]);
      o.x += v.x * cw[s];
      o.y += v.y * cw[s];
    }
    out[t] = make_double2(o.x / L, o.y / L);
  }
}

size_t attention_decode_ws_bytes(int B, int H, int dh, int T_max) {
  const int ns = cdiv_i(T_max, decode_chunk(B, H));
  return (size_t)B * H * ns * (2 * sizeof(double) + dh * sizeof(double2));
}

int attention_decode(hipStream_t st, const Attn& a, const Sync& sy) {
  const int CH = decode_chunk(a.B, a.H);
  const int ns = cdiv_i(a.T_max, CH);
  if (attention_decode_ws_bytes(a.B, a.H, a.dh, a.T_max) > sy.ws_bytes) return ERR_STATE;
  if ((long)a.B * a.H >= SYNC_COUNTERS - 1 || a.dh > 256 || a.S != 1 || ns > DEC_MAX_SPLITS) return ERR_ARG;
  double* pm = (double*)sy.ws;
  double* pl = pm + (long)a.B * a.H * ns;
  double2* po = (double2*)(pl + (long)a.B * a.H * ns);
  hipLaunchKernelGGL(k_attention_decode, dim3(ns, a.H, a.B), dim3(256), 0, st, a, CH, ns, pm, pl, po, sy.counters);
  return OK;
}

}  // namespace mitok
