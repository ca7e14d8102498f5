// resident.hpp — device code of the resident decode loop (resident.hip): the
// decode loop of mitok_generate for up to 8 sequences as one cooperative
// launch that stays resident for every step.  Each resident_k<MR>.hip
// instantiates the kernel for one row count, so the variants compile in
// parallel.
//
// At batch 1 the decode step is a chain of small dependent products (QKV ->
// attention -> FFN Dense -> FFN Linear per layer, then the vocab product and
// the greedy id): each moves a few MB of weights, so as separate launches
// every link pays a launch and a ramp-up and the HBM stream stalls between
// them.  Here one block per CU runs a program of operations (ROp) for all
// steps: the blocks share each operation's work items and meet at a grid
// barrier between operations.  The barrier is a flag per block, each written
// with a device-coherent store and polled by every block in one load per
// lane (about 1.2 us for 256 blocks on MI355X, below one kernel boundary).
//
// Coherence: the XCDs' L2 caches are not coherent with each other, and an
// agent-scope fence (L2 write-back + invalidate) measured 18-40 us per
// barrier.  So every value one block leaves for another inside the launch —
// activations, split partials, the KV rows appended this step, ids, KV
// lengths — is stored and loaded at device coherence (COH = true in
// rowops.hpp / epilogue.hpp, ld_dev / st_dev).  Weights and tables, which
// nothing writes during the launch, use ordinary cached loads.
//
// Operations (the reference operations each restates are cited where the
// same code serves the launch-per-operation plans):
//   ROP_GEMV    rowops(x)[M][K] * W[K][N] -> epilogue; a work item is C
//               columns x one K split (gemm.hip k_gemv's layout)
//   ROP_ATTN    one key chunk of one (sequence, head) (attention.hip
//               k_attention_split's layout; the QKV epilogue appended k, v);
//               the last chunk of a (sequence, head) to finish rescales the
//               chunks to their common max and sums them, plus the residual
//               (a counter per pair, no grid barrier between the two)
//   ROP_ROWS    materialise rowops(x) for a row or a column chunk of one
// The step state (KV lengths, the ids being fed, the step count) lives in
// every block's LDS: each block finds the greedy ids itself from the vocab
// product's per-tile partials at the start of the next step, so no operation
// reads a KV length or an id from memory.  Every wave of every block reaches
// every barrier; a barrier that waits longer than its spin limit sets
// EB_BARRIER and lets the grid run out.
#pragma once

#include "epilogue.hpp"

namespace mitok {

__host__ __device__ static inline int rcdiv(long a, long b) { return (int)((a + b - 1) / b); }

// ---- step state and access policy -----------------------------------------
static __shared__ int res_kvl[8];       // KV length of each sequence before this step's token
static __shared__ uint32_t res_ids[8];  // the ids fed to this step
static __shared__ int res_cnt;          // ids generated so far (logits-history slot of this step)

struct AccRes {
  template <class T>
  static __device__ __forceinline__ T ld(const T* p) { return ld_dev(p); }
  template <class T>
  static __device__ __forceinline__ void st(T* p, T v) { st_dev(p, v); }
  template <class T>
  static __device__ __forceinline__ T c(const T* p) { return ld_glb(p); }
  static __device__ __forceinline__ int kv(const int*, int m) { return res_kvl[m]; }
  static __device__ __forceinline__ uint32_t id(const uint32_t*, int m) { return res_ids[m]; }
  static __device__ __forceinline__ int cnt(const int*) { return res_cnt; }
};

// ---- polling exchange ---------------------------------------------------------
// In the polling mode (k_resident<.., POLL = true>) no grid barrier separates
// the operations of a step.  Every exchanged value -- activations, split
// partials, the chunk outputs of attention, the cache rows appended this
// step, the argmax partials -- starts the step as the sentinel RES_SENT and
// its consumer re-reads it until it is not, so the data is its own flag: one
// memory round trip where a barrier costs the producers' store
// acknowledgements, a flag round trip and then the data's.  Each operation
// reads only what earlier operations of the step wrote, and no producer ever
// waits for a consumer, so the polls cannot deadlock.  Exchange buffers are
// distinct per operation within a step and alternate between two halves of an
// arena from step to step; after one grid barrier at the start of each step
// (every block has finished the previous one) the blocks fill the previous
// step's half with the sentinel again.  Every poll is bounded: past
// RES_POLL_LIMIT rounds, or once another block has given up, it sets
// EB_BARRIER and returns what it has, so the grid always drains.
constexpr uint32_t RES_POLL_LIMIT = 1u << 20;
static __shared__ uint32_t* res_err;  // the launch's error word (for the polls)

__device__ __forceinline__ unsigned long long ld_bits(const double* p) {
  return __hip_atomic_load((MITOK_GLOBAL unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool poll_give_up(uint32_t spin) {
  if (spin >= RES_POLL_LIMIT) {
    atomicOr(res_err, (uint32_t)EB_BARRIER);
    return true;
  }
  return (spin & 63u) == 63u && (ld_dev(res_err) & EB_BARRIER);
}
// v[j] <- *p[j] for need[j], each re-read until it is not the sentinel; every
// load is issued before the first check
template <int N>
__device__ __forceinline__ void poll2(const double2* const (&p)[N], const bool (&need)[N], double2 (&v)[N]) {
  unsigned long long x[N], y[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    x[j] = need[j] ? ld_bits(&p[j]->x) : 0ull;
    y[j] = need[j] ? ld_bits(&p[j]->y) : 0ull;
  }
  for (uint32_t spin = 0;; ++spin) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok &= x[j] != RES_SENT && y[j] != RES_SENT;
    if (ok || poll_give_up(spin)) break;
#pragma unroll
    for (int j = 0; j < N; ++j) {
      if (x[j] == RES_SENT) x[j] = ld_bits(&p[j]->x);
      if (y[j] == RES_SENT) y[j] = ld_bits(&p[j]->y);
    }
  }
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = make_double2(__longlong_as_double((long long)x[j]), __longlong_as_double((long long)y[j]));
}
__device__ __forceinline__ double2 poll2_one(const double2* p) {
  const double2* a[1] = {p};
  const bool n[1] = {true};
  double2 v[1];
  poll2<1>(a, n, v);
  return v[0];
}
template <int N>
__device__ __forceinline__ void poll_f64(const double* const (&p)[N], const bool (&need)[N], double (&v)[N]) {
  unsigned long long x[N];
#pragma unroll
  for (int j = 0; j < N; ++j) x[j] = need[j] ? ld_bits(p[j]) : 0ull;
  for (uint32_t spin = 0;; ++spin) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok &= x[j] != RES_SENT;
    if (ok || poll_give_up(spin)) break;
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (x[j] == RES_SENT) x[j] = ld_bits(p[j]);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = __longlong_as_double((long long)x[j]);
}
template <int N>
__device__ __forceinline__ void poll_i32(const int* const (&p)[N], const bool (&need)[N], int (&v)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = need[j] ? ld_dev(p[j]) : 0;
  for (uint32_t spin = 0;; ++spin) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok &= v[j] != -1;
    if (ok || poll_give_up(spin)) break;
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (v[j] == -1) v[j] = ld_dev(p[j]);
  }
}

// The prologue of a product in the polling exchange, block-wide: the block's
// input rows m < M, columns [ka, ka + RL) -- an embedding gather, or rows or
// the sum of split partials, polled until written -- then bias, the finite
// check and GELU as ro_base, into LDS; with a LayerNorm (ka = 0, RL = K),
// ro_ln on them.  The same operations in the same order as ro_build, so both
// exchanges give the same bits.  Sources ro_build has and this does not
// (RoPE, a residual, an attention combine) are refused on the host.  Ends
// with a barrier.

// RES_POLL_LOADS loads per thread in flight each round: NPP partial slots (the
// partial count rounded up to a power of two) of RES_POLL_LOADS / NPP elements
constexpr int RES_POLL_LOADS = 16;
template <int NPP>
__device__ __forceinline__ void rows_poll_src(const RowOps& r, int M, int K, int ka, int RL, int tot, int np,
                                              double2* buf) {
  constexpr int E = RES_POLL_LOADS / NPP;
  for (int i0 = threadIdx.x; i0 < tot; i0 += 256 * E) {
    double2 v[E];
    int mm[E], kk[E];
    bool ok[E];
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const int i = i0 + 256 * u;
      mm[u] = i / RL;
      kk[u] = ka + (i - mm[u] * RL);
      ok[u] = i < tot && mm[u] < M && kk[u] < K;
    }
    if (r.table) {
#pragma unroll
      for (int u = 0; u < E; ++u) {
        v[u] = make_double2(0.0, 0.0);
        if (ok[u]) {
          const uint32_t id = res_ids[mm[u]];
          if (!(id == 1u || id >= (uint32_t)r.vocab)) v[u] = ld_glb(r.table + (long)id * K + kk[u]);  // PAD -> 0
        }
      }
    } else {
      const double2* pp[E * NPP];
      bool need[E * NPP];
      double2 t[E * NPP];
#pragma unroll
      for (int u = 0; u < E; ++u)
#pragma unroll
        for (int q = 0; q < NPP; ++q) {
          need[u * NPP + q] = ok[u] && q < np;
          pp[u * NPP + q] = r.x + (long)(ok[u] ? mm[u] : 0) * r.ldx + (ok[u] ? kk[u] : 0) + (long)q * r.part_stride;
        }
      poll2<E * NPP>(pp, need, t);
#pragma unroll
      for (int u = 0; u < E; ++u) {
        v[u] = t[u * NPP];
#pragma unroll
        for (int q = 1; q < NPP; ++q)
          if (q < np) v[u] = cadd(v[u], t[u * NPP + q]);
      }
    }
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const int i = i0 + 256 * u;
      if (i >= tot) continue;
      double2 x = make_double2(0.0, 0.0);
      if (ok[u]) {
        x = v[u];
        if (r.bias) x = cadd(x, ld_glb(r.bias + kk[u]));
        if (r.finite_check && !(isfinite(x.x) && isfinite(x.y))) atomicOr(r.err, (uint32_t)EB_FFN_NONFINITE);
        if (r.gelu) {
          if (r.row_mask && ld_glb(r.row_mask + mm[u]) == 0u) {
            x = make_double2(0.0, 0.0);
          } else {
            bool nan = false;
            x = gelu_nc(x, &nan);
            if (nan) atomicOr(r.err, (uint32_t)EB_GELU_NAN);
          }
        }
      }
      buf[i] = x;
    }
  }
}

template <int MR>
__device__ __forceinline__ void res_rows_poll(const RowOps& r, int M, int K, int ka, int RL, int n0, int n1,
                                              double2* buf, double2* st_mean, double2* st_sd) {
  // the LayerNorm's gamma and beta of this thread's first columns are
  // requested with the polled rows, not after the statistics
  double2 gpre[LN_PRE], bpre[LN_PRE];
#pragma unroll
  for (int j = 0; j < LN_PRE; ++j) {
    const int k = n0 + (int)threadIdx.x + 256 * j;
    const bool ok = r.ln && k < n1;
    gpre[j] = ok ? ld_glb(r.gamma + k) : make_double2(0.0, 0.0);
    bpre[j] = ok ? ld_glb(r.beta + k) : make_double2(0.0, 0.0);
  }
  const int tot = MR * RL;
  const int np = r.npart > 1 ? r.npart : 1;
  if (r.table || np == 1) rows_poll_src<1>(r, M, K, ka, RL, tot, 1, buf);
  else if (np == 2) rows_poll_src<2>(r, M, K, ka, RL, tot, np, buf);
  else if (np <= 4) rows_poll_src<4>(r, M, K, ka, RL, tot, np, buf);
  else rows_poll_src<8>(r, M, K, ka, RL, tot, np, buf);
  __syncthreads();
  if (r.ln) ro_ln<MR, AccRes>(r, M, K, RL, n0, n1, buf, st_mean, st_sd, gpre, bpre);
}

// ---- grid barrier ----------------------------------------------------------
constexpr uint32_t RES_SPIN_LIMIT = 1u << 22;  // ~several seconds of polling

// `pf` runs in waves 1-3 while wave 0 signals and polls: the weight loads it
// issues stay in flight through the barrier.  Wave 0 alone polls (a wave's
// loads complete in order, so a poll would wait for them).
template <class F>
__device__ __forceinline__ void grid_barrier(uint32_t* flags, uint32_t epoch, uint32_t* err, F&& pf) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's coherent stores are acknowledged
  __syncthreads();
  if (threadIdx.x >= 64) pf();
  if (threadIdx.x == 0) st_dev(&flags[blockIdx.x], epoch);
  if (threadIdx.x < 64 && (ld_dev(err) & EB_BARRIER) == 0) {
    const int lane = threadIdx.x, nb = gridDim.x;
    for (uint32_t spin = 0;; ++spin) {
      bool ok = true;
      for (int b0 = 0; b0 < nb; b0 += 256) {  // four flags per lane in flight per round
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int b = b0 + lane + 64 * j;
          v[j] = b < nb ? ld_dev(&flags[b]) : epoch;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) ok &= (int)(v[j] - epoch) >= 0;
      }
      if (__all(ok)) break;
      if (spin >= RES_SPIN_LIMIT) {
        if (lane == 0) atomicOr(err, (uint32_t)EB_BARRIER);
        break;
      }
      if ((spin & 255u) == 255u && (ld_dev(err) & EB_BARRIER)) break;  // another block gave up: run out
    }
  }
  __syncthreads();
}

// ---- ROP_GEMV --------------------------------------------------------------
// Two layouts.  Streaming (waves == 4): lane (r, c) = (lane / C, lane % C) of
// wave w reads rows k0 + r + u*RPW of column n; 16 weight loads per lane are
// in flight before the prologue and the loop keeps 8-16 in flight (outputs
// wider than the grid, e.g. the vocab product).  Prefetched (waves == 3): an
// item is at most RES_NPF loads per lane of waves 1-3, issued during the
// previous operation's barrier (gemv_weights), so the weights are in
// registers when the inputs become visible; wave 0 polls the barrier and owns
// the epilogue.
constexpr int RES_NPF = 24;

// acc[m] += x[m][row u] * w[u - u0] over rows u0 .. u0 + NU - 1 of this lane
// (row u at xw[m * RL + u * RPW] in LDS); rows at or past nu count zero.  A
// group of G rows has all its activations requested from LDS before its first
// product and no branch per row, so the LDS latency is paid once per group.
// ZW: the weights of rows past nu are zero and the activation a clamped row
// reads is this lane's own first row (zero past K), so those rows add exact
// zeros with no select.
// The weights of these rows are w[WO .. WO + NU - 1] (a compile-time offset:
// the array stays in registers).
template <int MR, int NU, int G, bool ZW = false, int WO = 0, int NW>
__device__ __forceinline__ void fma_rows(double2 (&acc)[MR], const double2* xw, int RL, int RPW, int u0, int nu,
                                         const double2 (&w)[NW]) {
  static_assert(NU % G == 0 && WO + NU <= NW, "row groups");
#pragma unroll
  for (int g0 = 0; g0 < NU; g0 += G) {
    double2 xv[MR][G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int u = u0 + g0 + j;
      const int iu = u < nu ? u : 0;
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m][j] = xw[m * RL + iu * RPW];
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (ZW) {
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xv[m][j], w[WO + g0 + j]));
      } else {
        const bool ok = u0 + g0 + j < nu;
        const double2 wv = ok ? w[WO + g0 + j] : make_double2(0.0, 0.0);
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(ok ? xv[m][j] : make_double2(0.0, 0.0), wv));
      }
    }
  }
}

// what a weight load past a lane's rows reads: every lane issues every load,
// so no load sits under a branch and each wait counts only the loads it needs
__device__ const double2 res_zero2 = {0.0, 0.0};

template <int C>
__device__ __forceinline__ void gemv_weights(const ROp& op, int item, double2 (&w)[RES_NPF]) {
  constexpr int RPW = 64 / C;
  const int lane = threadIdx.x & 63, cwv = (threadIdx.x >> 6) - 1;
  const int r = lane / C, c = lane - (lane / C) * C;
  const int bx = item % op.ncb, by = item / op.ncb;
  const int k0 = by * 3 * op.kw + cwv * op.kw;
  const int n = bx * C + c;
  const int kmax = max(0, min(op.kw, op.K - k0));
  const int nu = (n < op.N && kmax > r) ? (kmax - r + RPW - 1) / RPW : 0;
  const double2* wp = op.W + (long)(k0 + r) * op.ldw + n;
  const long wstep = (long)RPW * op.ldw;
#pragma unroll
  for (int u = 0; u < RES_NPF; ++u) w[u] = ld_stream(u < nu ? wp + u * wstep : &res_zero2);
}

// this block's item of a prefetched product (item = blockIdx.x)
__device__ __forceinline__ void prefetch_weights(const ROp& nx, double2 (&w)[RES_NPF]) {
  switch (nx.C) {
    case 8: gemv_weights<8>(nx, blockIdx.x, w); break;
    case 16: gemv_weights<16>(nx, blockIdx.x, w); break;
    case 32: gemv_weights<32>(nx, blockIdx.x, w); break;
    default: gemv_weights<64>(nx, blockIdx.x, w); break;
  }
}

// A product's epilogue for its column block, one output per lane of wave 0
// rather than MR per column owner (a GELU is a chain of transcendentals: two
// or more in one lane take that many times as long).  acc: the owners' sums;
// re: the owners' Re values back (for the fused argmax).  red is free again.
template <int MR, int C>
__device__ __forceinline__ void epi_spread(const Epi& ep, int M, int N, int bx, int n, bool col_ok, bool owner,
                                           const double2 (&acc)[MR], double2* red, double (&re)[MR]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if constexpr (MR == 1) {
    if (owner && col_ok) re[0] = apply_epi<AccRes>(ep, M, N, 0, n, acc[0]);
  } else {
    __shared__ double epi_re[MR * C];
    if (owner)
#pragma unroll
      for (int m = 0; m < MR; ++m) red[m * C + lane] = acc[m];
    __builtin_amdgcn_wave_barrier();
    if (wave == 0)
      for (int i = lane; i < MR * C; i += 64) {
        const int m = i / C, cc = i - (i / C) * C, nn = bx * C + cc;
        if (m < M && nn < N) epi_re[i] = apply_epi<AccRes>(ep, M, N, m, nn, red[i]);
      }
    __builtin_amdgcn_wave_barrier();
    if (owner)
#pragma unroll
      for (int m = 0; m < MR; ++m) re[m] = epi_re[m * C + lane];
  }
}

template <int MR, int C, bool POLL>
__device__ __forceinline__ void r_gemv3(const ROp& op, int item, double2* lds2, double2* red, double2* st_mean,
                                        double2* st_sd, double2 (&w)[RES_NPF], bool have) {
  constexpr int RPW = 64 / C;
  const RowOps& ro = op.ro;
  const int M = op.M, N = op.N, K = op.K, kw = op.kw;
  const int bx = item % op.ncb, by = item / op.ncb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane / C, c = lane - (lane / C) * C;
  const int KB = 3 * kw;
  const int kb0 = by * KB;
  const int n = bx * C + c;
  const bool col_ok = n < N;
  const int ka = ro.ln ? 0 : kb0, RL = ro.ln ? K : KB;
  if constexpr (!POLL) {  // polling: the caller requested the weights and built the rows
    if (!have && wave >= 1) gemv_weights<C>(op, item, w);
    RoLds L;
    L.wts = (double*)(lds2 + MR * RL);
    L.lsum = L.wts + (ro.att.po ? (size_t)M * ro.att.H * ro.att.nsplit : 0);
    L.m0 = 0;
    ro_prepare<AccRes>(ro, M, L);
    ro_build<MR, AccRes>(ro, M, K, ka, RL, kb0, min(K, kb0 + KB), lds2, L, st_mean, st_sd);
  }
  if (bx == 0 && by == 0 && tid < M) ro_check<AccRes>(ro, tid);
  const double2* xs = lds2 + (kb0 - ka);
  if (ro.save && bx == 0)
    for (int i = tid; i < MR * KB; i += 256) {
      const int m = i / KB, k = kb0 + (i - m * KB);
      if (m < M && k < K) st_dev(ro.save + (long)m * ro.ldsave + k, xs[m * RL + (k - kb0)]);
    }
  double2 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = make_double2(0.0, 0.0);
  if (wave >= 1 && col_ok) {
    const int k0 = kb0 + (wave - 1) * kw;
    const int kmax = max(0, min(kw, K - k0));
    const int nu = kmax > r ? (kmax - r + RPW - 1) / RPW : 0;
    const double2* xw = xs + (wave - 1) * kw + r;
    if constexpr (MR == 1) {
      fma_rows<MR, RES_NPF, RES_NPF, true>(acc, xw, RL, RPW, 0, nu, w);  // gemv_weights zero-fills rows past nu
    } else {  // more rows: one row of weights at a time keeps the registers in bounds
#pragma unroll
      for (int u = 0; u < RES_NPF; ++u)
        if (u < nu)
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * RL + u * RPW], w[u]));
    }
  }

#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m].x = col_sum<C>(acc[m].x);
    acc[m].y = col_sum<C>(acc[m].y);
  }
  if (wave > 0 && lane < C)
#pragma unroll
    for (int m = 0; m < MR; ++m) red[((wave - 1) * MR + m) * C + lane] = acc[m];
  __syncthreads();
  const bool owner = wave == 0 && lane < C;
  if (owner)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      acc[m] = cadd(cadd(red[(0 * MR + m) * C + lane], red[(1 * MR + m) * C + lane]), red[(2 * MR + m) * C + lane]);
  const Epi& ep = op.ep;
  if (ep.mode == EPI_PART) {
    if (owner && col_ok)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) st_dev(ep.out + ((long)by * M + m) * N + n, acc[m]);
  } else {
    double re[MR];
    epi_spread<MR, C>(ep, M, N, bx, n, col_ok, owner, acc, red, re);
    const Argmax& am = op.am;
    if (am.part_v && wave == 0)
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
            st_dev(am.part_v + (long)m * op.ncb + bx, bv);
            // the polling exchange reads -1 as "not written": "no value" is -2 there
            st_dev(am.part_i + (long)m * op.ncb + bx, (POLL && bi < 0) ? -2 : bi);
          }
        }
  }
  __syncthreads();
}

// w[WO .. WO + 7] <- rows un .. un + 7 of this lane's column (zero past nu)
template <int WO, int NW>
__device__ __forceinline__ void stream_rows(double2 (&w)[NW], const double2* wp, long wstep, int un, int nu) {
#pragma unroll
  for (int u = 0; u < 8; ++u) w[WO + u] = ld_stream(un + u < nu ? wp + (un + u) * wstep : &res_zero2);
}

// prev: this block's previous item of the operation (-1: none); when it
// built the same rows (a LayerNorm's whole rows, or the same K split) they
// are still in LDS and are not built again.
// The weights a product's item starts with, for the polling exchange: a
// 3-wave product's RES_NPF rows of waves 1-3 (as gemv_weights), or a 4-wave
// product's first 16 rows of every wave.  One code path for both layouts
// (two sibling paths storing to the same registers defeat their promotion).
template <int C>
__device__ __forceinline__ void gemv_issue(const ROp& op, int item, double2 (&w)[RES_NPF], bool w3) {
  constexpr int RPW = 64 / C;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cw = w3 ? wave - 1 : wave;
  const int r = lane / C, c = lane - (lane / C) * C;
  const int bx = item % op.ncb, by = item / op.ncb;
  const int k0 = by * op.waves * op.kw + cw * op.kw;
  const int n = bx * C + c;
  const int kmax = max(0, min(op.kw, op.K - k0));
  const int nu = (n < op.N && kmax > r) ? (kmax - r + RPW - 1) / RPW : 0;
  const double2* wp = op.W + (long)(k0 + r) * op.ldw + n;
  const long wstep = (long)RPW * op.ldw;
#pragma unroll
  for (int u = 0; u < RES_NPF; ++u)
    if (u < 16 || w3) w[u] = ld_stream(u < nu ? wp + u * wstep : &res_zero2);
}

// POLL: wf[0 .. 15] holds the first 16 weight rows and the rows are built
// (the caller)
template <int MR, int C, bool POLL>
__device__ __forceinline__ void r_gemv4(const ROp& op, int item, int prev, double2* lds2, double2* red, double2* st_mean,
                                        double2* st_sd, double2 (&wf)[RES_NPF]) {
  constexpr int RPW = 64 / C;
  const RowOps& ro = op.ro;
  const int M = op.M, N = op.N, K = op.K, kw = op.kw;
  const int bx = item % op.ncb, by = item / op.ncb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane / C, c = lane - (lane / C) * C;
  const int KB = 4 * kw;
  const int kb0 = by * KB;
  const int n = bx * C + c;
  const bool col_ok = n < N;
  const int k0 = kb0 + wave * kw;
  const int kmax = max(0, min(kw, K - k0));
  const int nu = kmax > r ? (kmax - r + RPW - 1) / RPW : 0;
  const double2* wp = op.W + (long)(k0 + r) * op.ldw + n;
  const long wstep = (long)RPW * op.ldw;
  const int ka = ro.ln ? 0 : kb0, RL = ro.ln ? K : KB;
  [[maybe_unused]] RoLds L;
  L.wts = (double*)(lds2 + MR * RL);
  L.lsum = L.wts + (ro.att.po ? (size_t)M * ro.att.H * ro.att.nsplit : 0);
  L.m0 = 0;

  // two buffers of 8 rows per lane keep 16 weight loads in flight (a third
  // spills this kernel's registers); rows past nu load as zero
  double2 w0[8], w1[8];
  if constexpr (POLL) {
#pragma unroll
    for (int u = 0; u < 8; ++u) w0[u] = wf[u], w1[u] = wf[8 + u];
  } else {
    stream_rows<0>(w0, wp, wstep, col_ok ? 0 : nu, nu);
    stream_rows<0>(w1, wp, wstep, col_ok ? 8 : nu, nu);
    const bool built = prev >= 0 && (ro.ln || prev / op.ncb == by);
    if (!built) {
      ro_prepare<AccRes>(ro, M, L);
      ro_build<MR, AccRes>(ro, M, K, ka, RL, kb0, min(K, kb0 + KB), lds2, L, st_mean, st_sd);
    }
  }
  if (bx == 0 && by == 0 && tid < M) ro_check<AccRes>(ro, tid);
  const double2* xs = lds2 + (kb0 - ka);
  if (ro.save && bx == 0)
    for (int i = tid; i < MR * KB; i += 256) {
      const int m = i / KB, k = kb0 + (i - m * KB);
      if (m < M && k < K) st_dev(ro.save + (long)m * ro.ldsave + k, xs[m * RL + (k - kb0)]);
    }

  double2 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = make_double2(0.0, 0.0);
  if (col_ok) {
    const double2* xw = xs + wave * kw + r;  // row u of this lane: xw[m * RL + u * RPW]
    for (int u0 = 0; u0 < nu; u0 += 16) {
      if constexpr (MR == 1) {
        fma_rows<MR, 8, 8, true>(acc, xw, RL, RPW, u0, nu, w0);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u0 + u < nu)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * RL + (u0 + u) * RPW], w0[u]));
      }
      stream_rows<0>(w0, wp, wstep, u0 + 16, nu);
      if constexpr (MR == 1) {
        fma_rows<MR, 8, 8, true>(acc, xw, RL, RPW, u0 + 8, nu, w1);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u0 + 8 + u < nu)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m] = cadd(acc[m], cmul(xw[m * RL + (u0 + 8 + u) * RPW], w1[u]));
      }
      stream_rows<0>(w1, wp, wstep, u0 + 24, nu);
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m].x = col_sum<C>(acc[m].x);
    acc[m].y = col_sum<C>(acc[m].y);
  }
  if (wave > 0 && lane < C)
#pragma unroll
    for (int m = 0; m < MR; ++m) red[((wave - 1) * MR + m) * C + lane] = acc[m];
  __syncthreads();
  const bool owner = wave == 0 && lane < C;
  if (owner)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      acc[m] = cadd(cadd(cadd(acc[m], red[(0 * MR + m) * C + lane]), red[(1 * MR + m) * C + lane]),
                    red[(2 * MR + m) * C + lane]);
  const Epi& ep = op.ep;
  if (ep.mode == EPI_PART) {
    if (owner && col_ok)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) st_dev(ep.out + ((long)by * M + m) * N + n, acc[m]);
  } else {
    double re[MR];
    epi_spread<MR, C>(ep, M, N, bx, n, col_ok, owner, acc, red, re);
    const Argmax& am = op.am;
    if (am.part_v && wave == 0)
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
            st_dev(am.part_v + (long)m * op.ncb + bx, bv);
            // the polling exchange reads -1 as "not written": "no value" is -2 there
            st_dev(am.part_i + (long)m * op.ncb + bx, (POLL && bi < 0) ? -2 : bi);
          }
        }
  }
  __syncthreads();  // LDS (rows, red) is reused by the next item
}

// ---- attention combine (run by the last chunk of a pair) ----------------------
// Item (b, h): out = Re(sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M) + resid)
// over the ns chunks of the sequence (the split form of the softmax-weighted
// sum, masked_attention_head.rs:201-208, then add_matrix_3d_c, utils/matrix.rs:
// 600-613).  Thread (g, e) takes chunks g, g + G, ...; every load of the item
// is requested before the first is used.
template <bool POLL>
__device__ __forceinline__ void r_combine(const ROp& op, int item) {
  constexpr int UPT = 16;  // chunks per thread kept in flight (ns <= 256, G >= 1)
  __shared__ double cw_s[256];
  __shared__ double2 part_s[256];
  __shared__ double red_s[8];
  const Attn& a = op.a;
  const AttnSplit& o = op.o;
  const int dh = a.dh, H = a.H;
  const int b = item / H, h = item - b * H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = res_kvl[b] + 1;
  const int ns = (T + o.CH - 1) / o.CH;
  const long base = ((long)b * H + h) * o.nsplit;
  const int G = 256 / dh;
  const int e = tid % dh, g = tid / dh;
  const bool act = g < G;
  double2 po[UPT];
  double pm, pl, rres;
  const long col = (long)h * dh + e;
  if constexpr (POLL) {  // the chunk outputs and the residual, polled together
    const double2* pp[UPT + 1];
    bool need[UPT + 1];
    double2 t[UPT + 1];
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int sidx = g + u * G;
      need[u] = act && sidx < ns;
      pp[u] = o.po + (base + (need[u] ? sidx : 0)) * dh + e;
    }
    need[UPT] = g == 0 && op.ro.resid;
    pp[UPT] = need[UPT] ? op.ro.resid + (long)b * op.ro.ldr + col : o.po;
    const double* pq[2] = {o.pm + base + (tid < ns ? tid : 0), o.pl + base + (tid < ns ? tid : 0)};
    const bool nq[2] = {tid < ns, tid < ns};
    double q2[2];
    poll2<UPT + 1>(pp, need, t);
    poll_f64<2>(pq, nq, q2);
#pragma unroll
    for (int u = 0; u < UPT; ++u) po[u] = need[u] ? t[u] : make_double2(0.0, 0.0);
    rres = need[UPT] ? t[UPT].x : 0.0;
    pm = tid < ns ? q2[0] : -INFINITY;
    pl = tid < ns ? q2[1] : 0.0;
  } else {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int sidx = g + u * G;
      po[u] = (act && sidx < ns) ? ld_dev(o.po + (base + sidx) * dh + e) : make_double2(0.0, 0.0);
    }
    pm = tid < ns ? ld_dev(o.pm + base + tid) : -INFINITY;
    pl = tid < ns ? ld_dev(o.pl + base + tid) : 0.0;
    rres = (g == 0 && op.ro.resid) ? ld_dev(op.ro.resid + (long)b * op.ro.ldr + col).x : 0.0;
  }
  // common max and chunk weights
  double mx = wave_max(pm);
  if (lane == 0) red_s[wave] = mx;
  __syncthreads();
  mx = fmax(fmax(red_s[0], red_s[1]), fmax(red_s[2], red_s[3]));
  const double w = tid < ns ? exp(pm - mx) : 0.0;
  cw_s[tid] = w;
  double l = wave_sum(pl * w);
  __syncthreads();  // red_s reuse, cw_s complete
  if (lane == 0) red_s[4 + wave] = l;
  double2 acc = make_double2(0.0, 0.0);
#pragma unroll
  for (int u = 0; u < UPT; ++u) {
    const int sidx = g + u * G;
    if (act && sidx < ns) {
      const double ww = cw_s[sidx];
      acc.x += po[u].x * ww;
      acc.y += po[u].y * ww;
    }
  }
  for (int sidx = g + UPT * G; act && sidx < ns; sidx += G) {  // beyond UPT chunks per thread
    const double2 v = POLL ? poll2_one(o.po + (base + sidx) * dh + e) : ld_dev(o.po + (base + sidx) * dh + e);
    const double ww = cw_s[sidx];
    acc.x += v.x * ww;
    acc.y += v.y * ww;
  }
  part_s[tid] = acc;
  __syncthreads();
  if (tid < dh) {
    const double lsum = (red_s[4] + red_s[5]) + (red_s[6] + red_s[7]);
    double2 sum = part_s[tid];
    for (int gg = 1; gg < G; ++gg) sum = cadd(sum, part_s[gg * dh + tid]);
    st_dev(op.out + (long)b * op.ldo + col, make_double2(sum.x / lsum + rres, 0.0));
  }
  __syncthreads();
}

// ---- ROP_ATTN --------------------------------------------------------------
// One chunk of CH <= 32 keys of sequence b, head h (masked_attention_head.rs:
// 184-208 with the cache, bias_pos row 0, no causal mask): scores, the
// chunk's max m and sum l of exp(s - m), and o = sum exp(s - m) v.  The new
// token's k and v were appended by the QKV epilogue of this step.  Keys,
// values, bias and q are all requested before the first is used.
template <int DH, bool POLL>
__device__ __forceinline__ void r_attn(const ROp& op, int item) {
  constexpr int MAXC = 32;
  __shared__ double sc[MAXC];
  __shared__ double2 pv[256];
  __shared__ double2 qs[256];
  __shared__ double stat[2];
  const Attn& a = op.a;
  const AttnSplit& o = op.o;
  const int dh = DH > 0 ? DH : a.dh;
  if constexpr (POLL) {
    // items past the chunks: the combine of (sequence, head) item - chunks,
    // polling the chunks' outputs (every chunk item precedes every combine
    // item in a block's order, so no block waits on its own later work)
    const int nchunk = o.nsplit * a.H * op.M;
    if (item >= nchunk) {
      r_combine<true>(op, item - nchunk);
      return;
    }
  }
  const int split = item % o.nsplit, h = (item / o.nsplit) % a.H, b = item / (o.nsplit * a.H);
  // polling, one item per block: the last split's block combines (b, h); its
  // chunk is empty unless the keys reach it, so it polls the other chunks at once
  const bool comb_here = POLL && !op.comb_items && split == o.nsplit - 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = res_kvl[b] + 1;
  const int CH = o.CH;
  const int c0 = split * CH;
  if (c0 >= T) {  // uniform over the block
    if (comb_here) r_combine<true>(op, b * a.H + h);
    return;
  }
  const int nc = min(CH, T - c0);
  const long bh = (long)b * a.H + h;
  const double2* K = a.kc + bh * a.ctx * dh;
  const double2* V = a.vc + bh * a.ctx * dh;
  const double* bias0 = a.bias_re + (long)h * a.mc * a.mc;
  constexpr int LPK = 16;
  const int sub = lane & (LPK - 1), kq = lane / LPK;
  constexpr int NP = MAXC / 16;
  constexpr int EPL = DH > 0 ? (DH + LPK - 1) / LPK : 1;
  const int G = 256 / dh;
  const int e = tid % dh, g = tid / dh;
  constexpr int VG = 256 / (DH > 0 ? DH : 256);
  constexpr int VU = DH > 0 ? (MAXC + VG - 1) / VG : 1;
  double2 kv[NP][EPL];
  double bj[NP];
  double2 vv[VU];
  if (DH > 0 && POLL) {
    // keys, values (the new token's appended this step) and q, polled together
    constexpr int NK = NP * EPL, NALL = NP * EPL + VU + 1;
    const double2* pp[NALL];
    bool need[NALL];
    double2 t[NALL];
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int j = pass * 16 + wave * 4 + kq;
      const double2* kr = K + (long)(c0 + (j < nc ? j : 0)) * dh;
#pragma unroll
      for (int tt = 0; tt < EPL; ++tt) {
        const int ee = sub + tt * LPK;
        need[pass * EPL + tt] = j < nc && ee < dh;
        pp[pass * EPL + tt] = kr + (ee < dh ? ee : 0);
      }
      bj[pass] = (j < nc && sub == 0) ? ld_glb(bias0 + c0 + j) : 0.0;
    }
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int j = g + u * G;
      need[NK + u] = g < G && j < nc;
      pp[NK + u] = V + (long)(c0 + (need[NK + u] ? j : 0)) * dh + e;
    }
    need[NALL - 1] = tid < dh;
    pp[NALL - 1] = op.q + (long)b * op.ldq + (long)h * dh + (tid < dh ? tid : 0);
    poll2<NALL>(pp, need, t);
#pragma unroll
    for (int pass = 0; pass < NP; ++pass)
#pragma unroll
      for (int tt = 0; tt < EPL; ++tt) kv[pass][tt] = need[pass * EPL + tt] ? t[pass * EPL + tt] : make_double2(0.0, 0.0);
#pragma unroll
    for (int u = 0; u < VU; ++u) vv[u] = need[NK + u] ? t[NK + u] : make_double2(0.0, 0.0);
    if (tid < dh) qs[tid] = t[NALL - 1];
  } else if (DH > 0) {
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int j = pass * 16 + wave * 4 + kq;
      const double2* kr = K + (long)(c0 + j) * dh;
#pragma unroll
      for (int t = 0; t < EPL; ++t) {
        const int ee = sub + t * LPK;
        kv[pass][t] = (j < nc && ee < dh) ? ld_dev(kr + ee) : make_double2(0.0, 0.0);
      }
      bj[pass] = (j < nc && sub == 0) ? ld_glb(bias0 + c0 + j) : 0.0;
    }
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int j = g + u * G;
      vv[u] = (g < G && j < nc) ? ld_dev(V + (long)(c0 + j) * dh + e) : make_double2(0.0, 0.0);
    }
  }
  if (!(DH > 0 && POLL))
    for (int ee = tid; ee < dh; ee += 256) {
      const double2* qp = op.q + (long)b * op.ldq + (long)h * dh + ee;
      qs[ee] = POLL ? poll2_one(qp) : ld_dev(qp);
    }
  __syncthreads();
  if (DH > 0) {
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int j = pass * 16 + wave * 4 + kq;
      double acc = 0.0;
#pragma unroll
      for (int t = 0; t < EPL; ++t) {
        const int ee = sub + t * LPK;
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
        const double2* kr = K + (long)(c0 + j) * dh;
        for (int ee = sub; ee < dh; ee += LPK) {
          const double2 k2 = POLL ? poll2_one(kr + ee) : ld_dev(kr + ee), qv = qs[ee];
          acc += qv.x * k2.x - qv.y * k2.y;
        }
      }
      acc = row16_sum(acc);  // the 16 lanes of key j
      if (j < nc && sub == 0) sc[j] = acc * a.scale + ld_glb(bias0 + c0 + j);
    }
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
  double2 acc = make_double2(0.0, 0.0);
  if (DH > 0) {
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
      const double2 v = POLL ? poll2_one(V + (long)(c0 + j) * dh + e) : ld_dev(V + (long)(c0 + j) * dh + e);
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
    st_dev((double2*)o.po + pidx * dh + tid, s);
  }
  if (tid == 0) {
    st_dev((double*)o.pm + pidx, stat[0]);
    st_dev((double*)o.pl + pidx, stat[1]);
  }
  __syncthreads();  // LDS reuse by the next item
  // barrier exchange: the last of the ceil(T / CH) chunks of (b, h) combines
  // them (one grid barrier per layer fewer than a separate combine operation)
  if (!POLL && op.cnt && arrive_last(op.cnt + bh, (uint32_t)((T + CH - 1) / CH))) r_combine<POLL>(op, (int)bh);
  if (comb_here) r_combine<true>(op, (int)bh);
}

// ---- ROP_ROWS --------------------------------------------------------------
__device__ __forceinline__ void r_rows(const ROp& op, int item, double2* lds2, double2* st_mean, double2* st_sd) {
  const RowOps& ro = op.ro;
  const int K = op.K;
  const int nch = ro.ln ? 1 : rcdiv(K, op.cw);
  const int m = item / nch, ch = item - m * nch;
  const int k0 = ro.ln ? 0 : ch * op.cw, k1 = ro.ln ? K : min(K, k0 + op.cw);
  const int RL = k1 - k0;
  RoLds L;
  L.wts = (double*)(lds2 + RL);
  L.lsum = L.wts + (ro.att.po ? (size_t)ro.att.H * ro.att.nsplit : 0);
  L.m0 = m;
  ro_prepare<AccRes>(ro, 1, L);
  ro_build<1, AccRes>(ro, 1, K, k0, RL, k0, k1, lds2, L, st_mean, st_sd);
  if (ch == 0 && threadIdx.x == 0) ro_check<AccRes>(ro, m);
  for (int k = k0 + threadIdx.x; k < k1; k += 256) {
    const double2 v = lds2[k - k0];
    st_dev(op.out + (long)m * op.ldo + k, v);
    if (ro.save) st_dev(ro.save + (long)m * ro.ldsave + k, v);
  }
  __syncthreads();
}

// ---- greedy ids of the previous step (sampling_methods.rs:5-18) -------------
// Every block reduces the vocab product's per-tile (max, last index) partials
// of each row (ties to the larger index) and advances its step state; block 0
// writes ids, history, counts and KV lengths back for the host.
template <bool POLL>
__device__ __forceinline__ void step_argmax(const RStep& st, bool write, int prev_parity) {
  constexpr int U = 16;
  const double* part_v = (POLL && prev_parity) ? st.part_v1 : st.part_v;
  const int* part_i = (POLL && prev_parity) ? st.part_i1 : st.part_i;
  __shared__ double sv[4][8];
  __shared__ int si[4][8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = st.B, tiles = st.tiles, tot = B * tiles;
  double bv[8];
  int bi[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) bv[m] = -INFINITY, bi[m] = -1;
  for (int i0 = 0; i0 < tot; i0 += 256 * U) {
    double v[U];
    int ix[U];
    if constexpr (POLL) {
      const double* pv[U];
      const int* pi[U];
      bool need[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + tid + 256 * u;
        need[u] = i < tot;
        pv[u] = part_v + (need[u] ? i : 0);
        pi[u] = part_i + (need[u] ? i : 0);
      }
      poll_f64<U>(pv, need, v);
      poll_i32<U>(pi, need, ix);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (!need[u]) v[u] = -INFINITY, ix[u] = -1;
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + tid + 256 * u;
        v[u] = i < tot ? ld_dev(part_v + i) : -INFINITY;
        ix[u] = i < tot ? ld_dev(part_i + i) : -1;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + tid + 256 * u;
      const int row = i < tot ? i / tiles : 8;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        if (row == m) argmax_combine(bv[m], bi[m], v[u], ix[u]);
    }
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m >= B) break;
    wave_argmax(bv[m], bi[m]);
    if (lane == 0) sv[wave][m] = bv[m], si[wave][m] = bi[m];
  }
  __syncthreads();
  if (tid < B) {
    const int m = tid;
    double v = sv[0][m];
    int id = si[0][m];
    for (int w = 1; w < 4; ++w) argmax_combine(v, id, sv[w][m], si[w][m]);
    if (id < 0) {  // every logit was NaN (the reference panics)
      atomicOr(st.err, (uint32_t)EB_ARGMAX_NAN);
      id = 0;
    }
    const int t = res_cnt;
    res_ids[m] = (uint32_t)id;
    res_kvl[m] += 1;
    if (write) {
      st_dev(st.ids + m, (uint32_t)id);
      st_dev(st.hist + (long)m * st.hist_stride + t, (uint32_t)id);
      st_dev(st.hist_cnt + m, t + 1);
      st_dev(st.kv_len + m, res_kvl[m]);
    }
  }
  __syncthreads();
  if (tid == 0) res_cnt += 1;
  __syncthreads();
}

// ---- the resident kernel -----------------------------------------------------
template <int MR, bool POLL>
__device__ __forceinline__ void run_gemv(const ROp& op, int it, int prev, double2* lds2, double2* red, double2* st_mean,
                                         double2* st_sd, double2 (&w)[RES_NPF], bool have) {
  if constexpr (POLL) {
    // the weights are requested first, then the rows are polled and built
    // (here, not per column width: one copy of the prologue in the kernel)
    const int wave = threadIdx.x >> 6;
    const bool w3 = op.waves == 3;
    // (no product prefetches into a 4-wave one: w is free there)
    if (!(w3 && (have || wave == 0))) switch (op.C) {
        case 8: gemv_issue<8>(op, it, w, w3); break;
        case 16: gemv_issue<16>(op, it, w, w3); break;
        case 32: gemv_issue<32>(op, it, w, w3); break;
        default: gemv_issue<64>(op, it, w, w3); break;
      }
    const RowOps& ro = op.ro;
    const int by = it / op.ncb, KB = op.waves * op.kw, kb0 = by * KB;
    const int ka = ro.ln ? 0 : kb0, RL = ro.ln ? op.K : KB;
    // a block's earlier item of the product with the same rows left them in LDS
    const bool built = !w3 && prev >= 0 && (ro.ln || prev / op.ncb == by);
    if (!built) res_rows_poll<MR>(ro, op.M, op.K, ka, RL, kb0, min(op.K, kb0 + KB), lds2, st_mean, st_sd);
  }
  if (op.waves == 3) {
    switch (op.C) {
      case 8: r_gemv3<MR, 8, POLL>(op, it, lds2, red, st_mean, st_sd, w, have); break;
      case 16: r_gemv3<MR, 16, POLL>(op, it, lds2, red, st_mean, st_sd, w, have); break;
      case 32: r_gemv3<MR, 32, POLL>(op, it, lds2, red, st_mean, st_sd, w, have); break;
      default: r_gemv3<MR, 64, POLL>(op, it, lds2, red, st_mean, st_sd, w, have); break;
    }
    return;
  }
  switch (op.C) {
    case 8: r_gemv4<MR, 8, POLL>(op, it, prev, lds2, red, st_mean, st_sd, w); break;
    case 16: r_gemv4<MR, 16, POLL>(op, it, prev, lds2, red, st_mean, st_sd, w); break;
    case 32: r_gemv4<MR, 32, POLL>(op, it, prev, lds2, red, st_mean, st_sd, w); break;
    default: r_gemv4<MR, 64, POLL>(op, it, prev, lds2, red, st_mean, st_sd, w); break;
  }
}

// POLL: the polling exchange (no barrier between operations; ops holds the
// even steps' program, then the odd steps', nops each)
template <int MR, int DH, bool POLL = false>
__global__ __launch_bounds__(256) void k_resident(const ROp* __restrict__ ops, int nops, int nsteps, RStep step,
                                                  uint32_t* flags, uint32_t epoch0, uint32_t* err,
                                                  uint64_t* stamps) {
  extern __shared__ double2 lds2[];
  __shared__ double2 red[3 * MR * 64];
  __shared__ double2 st_mean[MR], st_sd[MR];
  if (stamps && blockIdx.x == 0 && threadIdx.x == 0) stamps[(long)nsteps * nops] = wall_clock64();
  if (threadIdx.x < step.B) {
    res_kvl[threadIdx.x] = ld_dev(step.kv_len + threadIdx.x);
    res_ids[threadIdx.x] = ld_dev(step.ids + threadIdx.x);
  }
  if (threadIdx.x == 0) res_cnt = ld_dev(step.hist_cnt), res_err = err;
  __syncthreads();
  double2 wpf[RES_NPF];  // the next product's weights (waves 1-3)
  bool have = false;
  uint32_t epoch = epoch0;
  for (int s = 0; s < nsteps; ++s) {
    const ROp* sops = POLL ? ops + (long)(s & 1) * nops : ops;
    if (s > 0) {
      step_argmax<POLL>(step, blockIdx.x == 0, (s - 1) & 1);
      if constexpr (POLL) {
        // every block is past the previous step: its half of the arena becomes
        // the sentinel again, for the step after this one
        grid_barrier(flags, ++epoch, err, []() {});
        double* half = step.arena + ((s - 1) & 1) * step.arena_half;
        const long per = (step.arena_half + gridDim.x - 1) / gridDim.x;
        const long lo = (long)blockIdx.x * per, hi = min(step.arena_half, lo + per);
        for (long k = lo + threadIdx.x; k < hi; k += 256) st_dev(half + k, __longlong_as_double((long long)RES_SENT));
      }
    }
    for (int i = 0; i < nops; ++i) {
      const ROp& op = sops[i];
      // the next operation (the next step's first after the last); a
      // prefetched product has at most one item per block
      const bool last = s + 1 == nsteps && i + 1 == nops;
      const ROp& nx = i + 1 < nops ? sops[i + 1] : (POLL ? ops + (long)((s + 1) & 1) * nops : ops)[0];
      const bool pf = !last && nx.kind == ROP_GEMV && nx.waves == 3 && (int)blockIdx.x < nx.items;
      bool early = false;
      if constexpr (POLL) {
        // a block whose attention item has no keys (at most a combine, which
        // waits for the other chunks anyway) requests the next product's
        // weights now: a late request would hold up its next poll
        if (pf && op.kind == ROP_ATTN && !op.comb_items) {
          const int it = blockIdx.x;
          bool empty = it >= op.items;
          if (!empty) {
            const int b = it / (op.o.nsplit * op.a.H);
            empty = (it % op.o.nsplit) * op.o.CH >= res_kvl[b] + 1;
          }
          if (empty) {
            if (threadIdx.x >= 64) prefetch_weights(nx, wpf);
            early = true;
          }
        }
      }
      for (int it = blockIdx.x; it < op.items; it += gridDim.x) {
        switch (op.kind) {
          case ROP_GEMV:
            run_gemv<MR, POLL>(op, it, it == (int)blockIdx.x ? -1 : it - (int)gridDim.x, lds2, red, st_mean, st_sd,
                               wpf, have && it == (int)blockIdx.x);
            break;
          case ROP_ATTN: r_attn<DH, POLL>(op, it); break;
          default: r_rows(op, it, lds2, st_mean, st_sd); break;
        }
      }
      if constexpr (POLL) {
        // no barrier: waves 1-3 request the next product's weights now
        if (pf && !early && threadIdx.x >= 64) prefetch_weights(nx, wpf);
      } else {
        // its weights are requested during the barrier: requested earlier,
        // they delay this operation's own stores and so the barrier
        grid_barrier(flags, ++epoch, err, [&]() {
          if (pf) prefetch_weights(nx, wpf);
        });
      }
      have = pf;
      if (stamps && blockIdx.x == 0 && threadIdx.x == 0) stamps[(long)s * nops + i] = wall_clock64();
    }
  }
  if (blockIdx.x == 0) step_argmax<POLL>(step, true, (nsteps - 1) & 1);
}

}  // namespace mitok
