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
  MITOK_LAUNCH(k_attention_rows, dim3(a.S, a.H, a.B), dim3(256), shm, st, a);
}

// ===========================================================================
// Decode (one query row per sequence, masked_attention_head.rs:135-208 with
// the cache): keys are split in chunks of CH, one block per (chunk, head,
// sequence).  No causal mask in this branch; bias_pos row 0.  A block scores
// its chunk (16 lanes per key, 4 keys per wave) and leaves the chunk's max m,
// sum l of exp(s - m) and o = sum exp(s - m) v; the rows are finished by the
// row transform (rowops.hpp), which rescales the chunks to the common max:
// out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M), then the residual and
// LayerNorm of the attention layer.  No block waits for another.
// ===========================================================================
constexpr int DEC_LPK = 16;          // lanes per key in the score phase
constexpr int DEC_MAX_SPLITS = 256;  // key chunks per (sequence, head)

// keys per chunk: 32 reads the cache at ~7 TB/s where 64 reached under 4
// (the same bytes, fewer blocks in flight); 16 when there are few heads in all
constexpr int DEC_MAX_CHUNK = 32;
static int decode_chunk(int B, int H) { return B * H <= 16 ? 16 : 32; }

// q is the sum of npart partials (row b at q + b * ldq, partial stride
// pstride).  With `append`, the partials hold [q | k | v] of the new token
// (the fused decode plan): the chunk of position T-1 sums that token's k and
// v, appends them to the cache and uses them directly.
// DH > 0: head dim known at compile time; every key, value and bias_pos
// load of the chunk is issued at entry, before q is summed, so the chunk
// costs one memory round trip.  DH == 0: any head dim up to 256.
template <int DH>
__device__ __forceinline__ void attn_chunk(const Attn& a, const double2* __restrict__ qkv, long ldq, int npart,
                                           long pstride, int append, const AttnSplit& o, int split, int h, int b) {
  constexpr int NP = DEC_MAX_CHUNK / 16;  // score passes (16 keys each)
  __shared__ double sc[DEC_MAX_CHUNK];
  __shared__ double2 pv[256];
  __shared__ double2 qs[256], kn[256], vn[256];
  __shared__ double stat[2];
  const int dh = DH > 0 ? DH : a.dh;
  // the thread index goes through an empty asm: the compact grid's item loop
  // then recomputes the per-lane offsets for every chunk instead of holding
  // them (hoisted) across the loop.  With the q sums spread over the waves
  // and no load under a branch, DH 64 takes 93 VGPRs (5 blocks per CU) where
  // it took 160 (3); the decode step measured the same either way, so the
  // kernel is not bound by its resident blocks
  int tid_o = threadIdx.x;
  asm volatile("" : "+v"(tid_o));
  const int tid = tid_o, lane = tid & 63, wave = tid >> 6;
  const int T = a.kv_len[b] + 1;
  const int CH = o.CH;
  const int c0 = split * CH;
  if (c0 >= T) return;  // the consumer reads only this sequence's chunks
  const int nc = min(CH, T - c0);
  const bool has_new = append && c0 + nc == T;  // chunk of the new token, position T-1, still to append
  const int d = a.H * dh;
  const long bh = (long)b * a.H + h;
  const double2* K = a.kc + bh * a.ctx * dh;
  const double2* V = a.vc + bh * a.ctx * dh;
  const double* bias0 = a.bias_re + (long)h * a.mc * a.mc;  // bias_pos row 0

  // score lanes: 16 per key, 4 keys per wave and pass
  const int sub = lane & (DEC_LPK - 1), kq = lane / DEC_LPK;
  constexpr int EPL = DH > 0 ? (DH + DEC_LPK - 1) / DEC_LPK : 1;
  // value lanes: element e, key group g of G
  const int G = 256 / dh;
  const int e = tid % dh, g = tid / dh;
  constexpr int VG = 256 / (DH > 0 ? DH : 256);
  constexpr int VU = DH > 0 ? (DEC_MAX_CHUNK + VG - 1) / VG : 1;  // keys per value lane
  // keys and bias rows are in flight while q is summed
  double2 kv[NP][EPL];
  double bj[NP];
  if (DH > 0) {
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      // keys past the chunk load its last key (every load is issued, none
      // under a branch); their scores are never stored
      const int j = min(pass * 16 + wave * 4 + kq, nc - 1);
      const double2* kr = K + (long)(c0 + j) * dh + sub;
#pragma unroll
      for (int t = 0; t < EPL; ++t) kv[pass][t] = kr[t * DEC_LPK];
      bj[pass] = bias0[c0 + j];
    }
  }

  // q, and for the chunk of the new token k and v, each summed over the npart
  // partials in order; thread i takes vector i / dh (q, k, v) at element
  // i % dh, so the three sums run in different waves
  const double2* row = qkv + (long)b * ldq + (long)h * dh;
  const int nvec = has_new ? 3 : 1;
  for (int i = tid; i < nvec * dh; i += 256) {
    const int vec = i / dh, ee = i - vec * dh;
    const double2* src = row + (long)vec * d + ee;
    double2 s = make_double2(0.0, 0.0);
    for (int p0 = 0; p0 < npart; p0 += 4) {  // four loads in flight; past npart they repeat the last
      double2 t[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) t[p] = src[(long)min(p0 + p, npart - 1) * pstride];
#pragma unroll
      for (int p = 0; p < 4; ++p)
        if (p0 + p < npart) s = (p0 + p == 0) ? t[p] : cadd(s, t[p]);
    }
    if (vec == 0) {
      qs[ee] = s;
    } else {
      (vec == 1 ? kn : vn)[ee] = s;
      if (T - 1 < a.ctx)  // append (masked_attention_head.rs:159-178)
        (vec == 1 ? a.kc_w : a.vc_w)[(bh * a.ctx + (T - 1)) * dh + ee] = s;
      else if (vec == 1 && ee == 0)
        atomicOr(a.err, (uint32_t)EB_CTX_OVERFLOW);
    }
  }
  __syncthreads();

  if (DH > 0) {
    if (has_new) {  // the new token's row from LDS (its cache row was written just above)
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        const int j = pass * 16 + wave * 4 + kq;
#pragma unroll
        for (int t = 0; t < EPL; ++t) {
          const int ee = sub + t * DEC_LPK;
          if (c0 + j == T - 1 && ee < dh) kv[pass][t] = kn[ee];
        }
      }
    }
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int j = pass * 16 + wave * 4 + kq;
      double acc = 0.0;
#pragma unroll
      for (int t = 0; t < EPL; ++t) {
        const int ee = sub + t * DEC_LPK;
        if (ee < dh) acc += qs[ee].x * kv[pass][t].x - qs[ee].y * kv[pass][t].y;
      }
      acc = row16_sum(acc);  // the 16 lanes of key j
      if (j < nc && sub == 0) sc[j] = acc * a.scale + bj[pass];
    }
  } else {
    for (int j0 = 0; j0 < nc; j0 += 16) {
      const int j = j0 + wave * 4 + kq;
      double acc = 0.0;
      if (j < nc) {
        const bool is_new = has_new && c0 + j == T - 1;
        const double2* kr = K + (long)(c0 + j) * dh;
        for (int ee = sub; ee < dh; ee += DEC_LPK) {
          const double2 k2 = is_new ? kn[ee] : kr[ee], qv = qs[ee];
          acc += qv.x * k2.x - qv.y * k2.y;
        }
      }
      acc = row16_sum(acc);  // the 16 lanes of key j
      if (j < nc && sub == 0) sc[j] = acc * a.scale + bias0[c0 + j];
    }
  }
  __syncthreads();
  if (wave == 0) {  // nc <= 32 < 64 lanes
    const double s = lane < nc ? sc[lane] : -INFINITY;
    const double m = wave_max(s);
    const double p = lane < nc ? exp(s - m) : 0.0;
    const double l = wave_sum(p);
    if (lane < nc) sc[lane] = p;
    if (lane == 0) stat[0] = m, stat[1] = l;
  }
  __syncthreads();
  // out[e] over the chunk's keys: group g takes keys g, g + G, ...
  double2 acc = make_double2(0.0, 0.0);
  if (DH > 0) {
    // the values are requested after the softmax: loading them with the keys
    // (one memory round trip per chunk instead of two, 126 VGPRs) measured no
    // faster in the decode step
    double2 vv[VU];
#pragma unroll
    for (int u = 0; u < VU; ++u) vv[u] = V[(long)(c0 + min(g + u * G, nc - 1)) * dh + e];  // past nc: not summed
    if (has_new)
#pragma unroll
      for (int u = 0; u < VU; ++u)
        if (g < G && c0 + g + u * G == T - 1) vv[u] = vn[e];
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int j = g + u * G;
      if (g < G && j < nc) {
        const double p = sc[j];
        acc.x += p * vv[u].x;
        acc.y += p * vv[u].y;
      }
    }
  } else if (g < G) {
    for (int j = g; j < nc; j += G) {
      const double p = sc[j];
      const double2 v = (has_new && c0 + j == T - 1) ? vn[e] : V[(long)(c0 + j) * dh + e];
      acc.x += p * v.x;
      acc.y += p * v.y;
    }
  }
  pv[tid] = acc;
  __syncthreads();
  const long pidx = bh * o.nsplit + split;
  if (tid < dh) {
    double2 s = pv[tid];
    for (int gg = 1; gg < G; ++gg) s = cadd(s, pv[gg * dh + tid]);
    ((double2*)o.po)[pidx * dh + tid] = s;
  }
  if (tid == 0) {
    ((double*)o.pm)[pidx] = stat[0];
    ((double*)o.pl)[pidx] = stat[1];
  }
}

// The grid covers at most the blocks resident on the chip at once (and at most
// DEC_MAX_BLOCKS) whatever the cache length the launch was sized for: the
// blocks walk the chunks the sequences have now, item = (sequence, head,
// chunk) in that order, so no block starts only to find its chunk empty (a
// graph replays one grid while the caches grow).  Up to 256 sequences; with
// more, one block per (chunk, head, sequence) of the launch's maximum.
constexpr int DEC_MAX_BLOCKS = 2048;
constexpr int DEC_COMPACT_MAX_B = 256;

template <int DH>
__global__ __launch_bounds__(256) void k_attention_split(Attn a, const double2* __restrict__ qkv, long ldq, int npart,
                                                         long pstride, int append, AttnSplit o, int compact) {
  if (!compact) {
    attn_chunk<DH>(a, qkv, ldq, npart, pstride, append, o, blockIdx.x, blockIdx.y, blockIdx.z);
    return;
  }
  __shared__ int s_off[DEC_COMPACT_MAX_B + 1];  // first item of sequence b
  __shared__ int s_ns[DEC_COMPACT_MAX_B];
  const int tid = threadIdx.x;
  const int ns = tid < a.B ? (a.kv_len[tid] + 1 + o.CH - 1) / o.CH : 0;
  if (tid < DEC_COMPACT_MAX_B) s_ns[tid] = ns;
  // inclusive scan of H * ns over the 256 threads
  s_off[tid + 1] = a.H * ns;
  if (tid == 0) s_off[0] = 0;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int v = tid + 1 > off ? s_off[tid + 1 - off] : 0;
    __syncthreads();
    s_off[tid + 1] += v;
    __syncthreads();
  }
  // the item's coordinates are the same in every lane: held in scalar
  // registers, so the chunk's addresses are scalar too (as in a grid launch)
  const int total = __builtin_amdgcn_readfirstlane(s_off[a.B]);
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    int lo = 0, hi = a.B - 1;  // the sequence whose range holds item
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_off[mid] <= item) lo = mid;
      else hi = mid - 1;
    }
    lo = __builtin_amdgcn_readfirstlane(lo);
    const int r = __builtin_amdgcn_readfirstlane(item - s_off[lo]), nsb = __builtin_amdgcn_readfirstlane(s_ns[lo]);
    attn_chunk<DH>(a, qkv, ldq, npart, pstride, append, o, r % nsb, r / nsb, lo);
    __syncthreads();  // the chunk's LDS is reused by the next item
  }
}

// Blocks of k_attention_split<DH> resident on the device at once (occupancy x
// CUs, at most DEC_MAX_BLOCKS): a compact grid no larger runs in one round.
// Asked once per head-dim variant; the query enqueues nothing, so it is safe
// while a graph is being captured.
static int split_resident_blocks(int dh) {
  static int cached[5] = {0, 0, 0, 0, 0};
  const int slot = dh == 16 ? 0 : dh == 32 ? 1 : dh == 64 ? 2 : dh == 128 ? 3 : 4;
  if (cached[slot] > 0) return cached[slot];
  const void* k = slot == 0 ? (const void*)k_attention_split<16>
                : slot == 1 ? (const void*)k_attention_split<32>
                : slot == 2 ? (const void*)k_attention_split<64>
                : slot == 3 ? (const void*)k_attention_split<128>
                            : (const void*)k_attention_split<0>;
  int dev = 0, cus = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, 256, 0) != hipSuccess || cus <= 0 || occ <= 0)
    return DEC_MAX_BLOCKS;
  cached[slot] = std::min(DEC_MAX_BLOCKS, occ * cus);
  return cached[slot];
}

AttnSplit attention_split_plan(const Attn& a) {
  AttnSplit o;
  o.H = a.H;
  o.dh = a.dh;
  o.CH = decode_chunk(a.B, a.H);
  o.nsplit = cdiv_i(a.T_max, o.CH);
  o.kv_len = a.kv_len;
  return o;
}

size_t attention_split_ws_bytes(int B, int H, int dh, int T_max) {
  const int ns = cdiv_i(T_max, decode_chunk(B, H));
  return (size_t)B * H * ns * (2 * sizeof(double) + dh * sizeof(double2));
}

int attention_decode_split(hipStream_t st, const Attn& a, const double2* q, long ldq, int npart, long part_stride,
                           bool append, const AttnSplit& o) {
  if (a.S != 1 || a.dh > 256 || o.nsplit > DEC_MAX_SPLITS || o.CH > DEC_MAX_CHUNK || !a.kv_len || npart > 8 ||
      npart < 1)
    return ERR_ARG;
  if (append && (!a.kc_w || !a.vc_w)) return ERR_ARG;
  const long items = (long)o.nsplit * a.H * a.B;
  const int compact = a.B <= DEC_COMPACT_MAX_B ? 1 : 0;
  const dim3 grid = compact ? dim3((unsigned)std::min<long>(items, split_resident_blocks(a.dh))) : dim3(o.nsplit, a.H, a.B);
  const int ap = append ? 1 : 0;
  switch (a.dh) {
    case 16: MITOK_LAUNCH(k_attention_split<16>, grid, dim3(256), 0, st, a, q, ldq, npart, part_stride, ap, o, compact); break;
    case 32: MITOK_LAUNCH(k_attention_split<32>, grid, dim3(256), 0, st, a, q, ldq, npart, part_stride, ap, o, compact); break;
    case 64: MITOK_LAUNCH(k_attention_split<64>, grid, dim3(256), 0, st, a, q, ldq, npart, part_stride, ap, o, compact); break;
    case 128: MITOK_LAUNCH(k_attention_split<128>, grid, dim3(256), 0, st, a, q, ldq, npart, part_stride, ap, o, compact); break;
    default: MITOK_LAUNCH(k_attention_split<0>, grid, dim3(256), 0, st, a, q, ldq, npart, part_stride, ap, o, compact); break;
  }
  return OK;
}

// ===========================================================================
// Prefill (keys = the S rows of the call, T == S): flash-style, one block per
// (query tile of 16*NW rows, head, sequence), 32-key tiles up to the tile's
// causal limit.  Re(q.k) = sum_e (qr kr - qi ki) is a real dot product of
// length 2*dh: keys are staged in LDS as [kr | -ki], queries held as MFMA A
// operands [qr | qi], and v_mfma_f64_16x16x4_f64 forms 16x16 score tiles.
// Scores get the scale and Re(bias_pos[r][c]); keys c > r get -1e12
// (masked_attention_head.rs:189-203).  The softmax runs online (running row
// max m and sum l, the partial output rescaled by e^(m_old - m_new)); the
// first tile always holds key 0, so m is a real score from then on and masked
// keys contribute exactly 0.  P goes through LDS to become the A operand of
// the P.V MFMAs (values staged in LDS).  out = acc / l; pad rows give 0.
// D[i][j] of a 16x16 tile sits at lane j + 16*(i%4), element i/4.
// ===========================================================================
template <int DH, int NW>
__global__ __launch_bounds__(64 * NW) void k_attention_prefill(Attn a) {
  constexpr int KT = 32;          // keys per tile
  constexpr int KD = 2 * DH;      // real dot length
  constexpr int KSTR = KD + 1;    // LDS row stride of the key tile (doubles)
  constexpr int NTH = 64 * NW;
  constexpr int ET = DH / 16;     // 16-column tiles of the head dim
  __shared__ double Ks[KT * KSTR];
  __shared__ double2 Vs[KT * DH];
  __shared__ double Ps[NW][16][KT + 1];
  const int h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kq = lane >> 4;
  const int S = a.S, T = a.T_const;
  const int q0 = blockIdx.x * 16 * NW;  // block's first query row
  const int r0 = q0 + 16 * wave;         // wave's first query row
  const long rowbase = (long)b * S;
  const double2* Kc = a.kc + ((long)b * a.H + h) * a.ctx * DH;
  const double2* Vc = a.vc + ((long)b * a.H + h) * a.ctx * DH;
  const double* bias = a.bias_re + (long)h * a.mc * a.mc;

  // A operand of the scores: u[i][k] = k < DH ? qr[k] : qi[k - DH], k = 4s + kq
  double uq[KD / 4];
  {
    const int r = r0 + i;
    const double2* qrow = a.q + (rowbase + (r < S ? r : 0)) * a.ldq + (long)h * DH;
#pragma unroll
    for (int s2 = 0; s2 < KD / 4; ++s2) {
      const int k = 4 * s2 + kq;
      const double2 qv = r < S ? qrow[k % DH] : make_double2(0.0, 0.0);
      uq[s2] = k < DH ? qv.x : qv.y;
    }
  }
  v4d o_re[ET], o_im[ET];
#pragma unroll
  for (int t = 0; t < ET; ++t) o_re[t] = o_im[t] = v4d{0.0, 0.0, 0.0, 0.0};
  double m[4], l[4];  // rows r0 + 4e + kq
#pragma unroll
  for (int e = 0; e < 4; ++e) m[e] = -INFINITY, l[e] = 0.0;

  const int kend = min(T, q0 + 16 * NW);  // keys any row of the block can see
  for (int c0 = 0; c0 < kend; c0 += KT) {
    __syncthreads();  // the previous tile is consumed
    for (int idx = tid; idx < KT * DH; idx += NTH) {
      const int key = idx / DH, e = idx - key * DH, c = c0 + key;
      const double2 kv = c < T ? Kc[(long)c * DH + e] : make_double2(0.0, 0.0);
      const double2 vv = c < T ? Vc[(long)c * DH + e] : make_double2(0.0, 0.0);
      Ks[key * KSTR + e] = kv.x;
      Ks[key * KSTR + DH + e] = -kv.y;
      Vs[key * DH + e] = vv;
    }
    __syncthreads();
    // scores of 16 rows x 32 keys
    v4d sc[2] = {v4d{0.0, 0.0, 0.0, 0.0}, v4d{0.0, 0.0, 0.0, 0.0}};
#pragma unroll
    for (int s2 = 0; s2 < KD / 4; ++s2)
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
        sc[jt] = __builtin_amdgcn_mfma_f64_16x16x4f64(uq[s2], Ks[(16 * jt + i) * KSTR + 4 * s2 + kq], sc[jt], 0, 0, 0);
    // scale, bias, causal mask; online softmax per row
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + 4 * e + kq;
      double v[2];
      double mt = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const int c = c0 + 16 * jt + i;
        if (c > r || r >= S) v[jt] = -1e12;
        else v[jt] = sc[jt][e] * a.scale + bias[(long)r * a.mc + c];
        mt = fmax(mt, v[jt]);
      }
      mt = row16_max(mt);
      const double mn = fmax(m[e], mt);
      const double alpha = exp(m[e] - mn);
      double ls = 0.0;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const double p = exp(v[jt] - mn);
        Ps[wave][4 * e + kq][16 * jt + i] = p;
        ls += p;
      }
      ls = row16_sum(ls);
      l[e] = l[e] * alpha + ls;
      m[e] = mn;
#pragma unroll
      for (int t = 0; t < ET; ++t) o_re[t][e] *= alpha, o_im[t][e] *= alpha;
    }
    __syncthreads();  // P of every wave written
    // out += P . V: A = P[row i][key 4s + kq], B = V[key 4s + kq][16t + i]
#pragma unroll
    for (int s2 = 0; s2 < KT / 4; ++s2) {
      const double pa = Ps[wave][i][4 * s2 + kq];
#pragma unroll
      for (int t = 0; t < ET; ++t) {
        const double2 vb = Vs[(4 * s2 + kq) * DH + 16 * t + i];
        o_re[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(pa, vb.x, o_re[t], 0, 0, 0);
        o_im[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(pa, vb.y, o_im[t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = r0 + 4 * e + kq;
    if (r >= S) continue;
    const long row = rowbase + r;
    const bool pad = a.row_mask && a.row_mask[row] == 0;
    double2* out = a.out + row * a.ldo + (long)h * DH;
#pragma unroll
    for (int t = 0; t < ET; ++t)
      out[16 * t + i] = pad ? make_double2(0.0, 0.0) : make_double2(o_re[t][e] / l[e], o_im[t][e] / l[e]);
  }
}

bool attention_prefill(hipStream_t st, const Attn& a) {
  if (a.kv_len || a.T_const != a.S || a.S <= 0) return false;
  const auto launch = [&](auto kern, int nw) {
    MITOK_LAUNCH(kern, dim3(cdiv_i(a.S, 16 * nw), a.H, a.B), dim3(64 * nw), 0, st, a);
  };
  switch (a.dh) {
    case 16: launch(k_attention_prefill<16, 8>, 8); return true;
    case 32: launch(k_attention_prefill<32, 8>, 8); return true;
    case 64: launch(k_attention_prefill<64, 8>, 8); return true;
    case 128: launch(k_attention_prefill<128, 4>, 4); return true;
    default: return false;
  }
}

}  // namespace mitok
