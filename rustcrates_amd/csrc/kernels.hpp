// kernels.hpp — launch wrappers of the gfx950 kernels (gemm.hip, attention.hip,
// kernels.hip).
//
// Every wrapper enqueues on `st` and never synchronises or allocates, so the
// decode step built from them can be captured into a HIP graph.  Kernels that
// split work across blocks either leave partials for the next launch to sum,
// or finish in the block that arrives last at a per-tile counter (Sync, at
// most 8 arrivals per counter); counters return to zero before the kernel
// ends, so launches on one stream can share them.
#pragma once

#include "common.hpp"

namespace mitok {

// ---- scratch shared by the launches of one stream ----
struct Sync {
  uint32_t* counters = nullptr;  // zero-initialised, SYNC_COUNTERS entries
  void* ws = nullptr;            // split partials
  size_t ws_bytes = 0;
};
constexpr int SYNC_COUNTERS = 1 << 16;

// ---- split decode-attention partials, combined by the consumer's prologue ----
// chunk s of (row m, head h): max m_s, sum l_s of exp(score - m_s), o_s[dh]
struct AttnSplit {
  const double* pm = nullptr;  // [M][H][nsplit]
  const double* pl = nullptr;
  const double2* po = nullptr;  // [M][H][nsplit][dh]
  int H = 0, dh = 0, nsplit = 0, CH = 0;
  const int* kv_len = nullptr;  // keys of row m: kv_len[m] + 1
};

// ---- the row transform a GEMV applies to its input rows (prologue) ----
// source (rows | sum of split partials | embedding gather | attention combine)
//   -> + bias -> finite check -> GELU -> RoPE -> residual Re(x + r) -> LayerNorm
struct RowOps {
  const double2* x = nullptr;  // [M][ldx] rows, or partial p at x + p * part_stride
  long ldx = 0;
  int npart = 0;  // > 1: x[m][k] = sum over p < npart of the partials, in order
  long part_stride = 0;
  const double2* table = nullptr;  // [vocab][K] embedding table gathered by ids (PAD id 1 -> 0)
  const uint32_t* ids = nullptr;
  int vocab = 0;
  AttnSplit att;                     // att.po != null: the attention combine is the source
  const double2* bias = nullptr;     // + bias[k] (utils/matrix.rs:615-625)
  int finite_check = 0;              // flag non-finite values (FFN output, transformer_network.rs:408)
  int gelu = 0;                      // gelu_complex, rows with mask 0 -> 0 (activation.rs:195-212,268-284)
  const uint32_t* row_mask = nullptr;
  const double2* rope_cs = nullptr;  // [rope_max][K/2] (cos, sin); position of row m = rope_pos[m] (+ rope_off[m])
  const int* rope_pos = nullptr;
  const int* rope_off = nullptr;  // per-row position offsets, or null
  int rope_max = 0;
  const double2* resid = nullptr;  // x = Re(x + resid) + 0i  (add_matrix_3d_c, utils/matrix.rs:600-613)
  long ldr = 0;
  int ln = 0;  // NormalNormLayer over the K elements of each row (norm_layer.rs:64-130)
  double eps = 0.0;
  const double2* gamma = nullptr;
  const double2* beta = nullptr;
  double2* save = nullptr;  // optional copy of the transformed rows [M][ldsave]
  long ldsave = 0;
  uint32_t* err = nullptr;
  bool plain() const {
    return x && npart <= 1 && !table && !att.po && !bias && !finite_check && !gelu && !rope_cs && !resid && !ln &&
           !save;
  }
};

// ---- GEMM epilogue: what happens to C[m][n] after the complex dot product ----
enum EpiMode : int {
  EPI_STORE = 0,  // out[m][n] = v (+bias); optional non-finite check (FFN output)
  EPI_GELU = 1,   // out[m][n] = mask[m] ? gelu(v + bias) : 0 (layer.rs:132-166)
  EPI_RE = 2,     // out_re[m][n] = Re(v + bias) (logits, data_converter.rs:244-256)
  EPI_QKV = 3,    // columns [q | k | v] of all heads: q -> out, k/v -> KV cache
  EPI_PART = 4,   // split partial p of C to out + p * M * N (ld N); the consumer sums them (M <= 64)
};

struct Epi {
  int mode = EPI_STORE;
  const double2* bias = nullptr;  // [N]
  double2* out = nullptr;         // STORE / GELU / QKV(q part)
  double* out_re = nullptr;       // RE
  long ldo = 0;
  double* hist_re = nullptr;       // RE: also hist_re[hist_cnt[0]][m][n] (logits history, ld N)
  const int* hist_cnt = nullptr;
  const uint32_t* row_mask = nullptr;  // GELU: rows with mask 0 become 0
  int check_finite = 0;
  uint32_t* err = nullptr;
  // EPI_QKV: row m = b * S + s
  int d = 0, dh = 0, heads = 0, S = 1;
  double2* kc = nullptr;  // [B][heads][ctx][dh]
  double2* vc = nullptr;
  int ctx = 0;
  const int* kv_base = nullptr;  // [B] cache position of row s = 0 (null: 0)
  const int* kv_row = nullptr;   // [B] only this row is appended (null: every row)
};

// ---- greedy_decoding fused into an EPI_RE GEMM (src/utils/sampling_methods.rs:5-18) ----
// Per-tile (max, last index) partials, then the block that finishes last
// reduces them per row: ids[m], optional history append and KV advance.
struct Argmax {
  double* part_v = nullptr;  // [M][tiles]
  int* part_i = nullptr;
  uint32_t* ids = nullptr;
  uint32_t* hist = nullptr;
  int hist_stride = 0;
  int* hist_cnt = nullptr;
  int* kv_len = nullptr;
  int advance_kv = 0;
  uint32_t* err = nullptr;
};

// GEMM C[M][N] = rowops(A)[M][K] * W[K][N] (complex, row-major), then the epilogue
// and the optional fused argmax.  M <= 8 runs the bandwidth GEMV (any RowOps);
// larger M the MFMA-tiled kernel (plain rows only).  gemm_ws_bytes() is the split
// workspace it needs; argmax_part_elems() the size of Argmax::part_v/part_i.
size_t gemm_ws_bytes(int M, int N, int K);
size_t argmax_part_elems(int M, int N);
int gemm(hipStream_t st, int M, int N, int K, const RowOps& ro, const double2* W, long ldw, const Epi& ep,
         const Argmax* am, const Sync& sy);
// EPI_PART products (M <= 64, except outputs wide enough for the 64-column
// MFMA variant): the number of partials gemm() writes (0: not available)
int gemm_parts(int M, int N, int K);
constexpr int GEMM_PART_MAX_M = 64;
// The prologue alone: out[m][k] = rowops(x)[m][k]  (materialises a pending row transform)
void rowops_apply(hipStream_t st, int M, int K, const RowOps& ro, double2* out, long ldo);

// ---- the output head's training step (train.hip) ----
struct TrainStep {
  int first = 0;      // the first update: clipped gradient descent (linear_layer.rs:159-174)
  double lr = 0.0;    // the layer's learning rate
  double batch = 1;   // sequences in the batch (the descent divides by it)
  int time_step = 0;  // AdamW's bias-correction step (at least 1)
};
// G[r][c] (complex, im 0) = tgt[r] < 0 ? 0 : (P[r][c] - [c == tgt[r]]) / norm[r / S]
void softmax_grad(hipStream_t st, const double* P, int rows, int V, const int* tgt, const double* norm, int S,
                  double2* G);
// cross_entropy_loss_batch of P [B][S][V] for targets [B][T] (tlen[b] each):
// part [B] the sequences' losses, out [2] the batch loss (re, im); T <= CE_MAX_T
constexpr int CE_MAX_T = 8192;
void cross_entropy(hipStream_t st, const double* P, int B, int S, int V, const uint32_t* tgt, const uint32_t* tlen,
                   int T, double* part, double* out);
// G = mask[r] ? dH * conj(GELU'(Z)) : 0 (layer.rs:181-192, derivative.rs:48-84); mask may be null (all rows)
void gelu_backward(hipStream_t st, const double2* dH, const double2* Z, const uint32_t* mask, long rows, int F,
                   double2* G);
// out [C][R] = conj(in)^T for in [R][C]
void conj_transpose(hipStream_t st, const double2* in, long R, long C, double2* out);
// db [V] = sum_b sum_s G[b][s][:] (per-sequence sums in row order, then in sequence order); ws [B][V]
void bias_grad(hipStream_t st, const double2* G, int B, int S, int V, double2* ws, double2* db);
// W [n], b [V] updated in place from dW, db (moments mW, vW, mb, vb)
void linear_update(hipStream_t st, double2* W, const double2* dW, double2* mW, double2* vW, long n, double2* b,
                   const double2* db, double2* mb, double2* vb, int V, const TrainStep& ts);
// the Norm's backward per row of x (or Re(x + resid) + 0i); dx real rows, pg = dout * x_hat
void norm_backward(hipStream_t st, const double2* x, const double2* resid, long rows, int n, double eps,
                   const double2* gamma, const double2* beta, const double2* dout, double2* dx, double2* pg);
// out[j] = mult * (sum over sequences b of the row sum of X[b][:][j]), as bias_grad; ws [B][n]
void colsum(hipStream_t st, const double2* X, int B, int S, int n, double mult, double2* ws, double2* out);
// attention weights A and dl_da [B][H][S][S] of a stateless pass from the packed [q | k | v] rows and the
// gradient G [B*S][d] of the heads' output
void attn_probs_grad(hipStream_t st, const double2* qkv, const double* bias_re, int mc, const uint32_t* mask,
                     const double2* G, int B, int S, int H, int dh, double c, double* A, double* dA);
// the gradient of the packed [q | k | v] rows: dQ = c dA conj(K), dK = c dA^T conj(Q), dV = A^T G
void attn_dqkv(hipStream_t st, const double2* qkv, const double* A, const double* dA, const double2* G, int B, int S,
               int H, int dh, double c, double2* dqkv);
// Re(bias_pos)[h][:S][:S] updated from dA summed over the batch (zero moments each call)
void attn_bias_update(hipStream_t st, double* bias_re, int mc, const double* dA, int B, int H, int S,
                      const TrainStep& ts);
// w [n] updated in place (weight: AdamW's EPSILON floor on v_hat's norm)
void param_update(hipStream_t st, double2* w, const double2* g, double2* m, double2* v, long n, bool weight,
                  const TrainStep& ts);
// RoPE's backward on rows [rows][d] of sequences of S rows (cs: the forward's table)
void rope_backward(hipStream_t st, const double2* G, long rows, int S, int d, const double2* cs, double2* out);
// the wavelet layer's backward: out [B][Sin][d] from G [B][S2][d] through a tap table [Sin][4]
void dwt_backward(hipStream_t st, const double2* G, int B, int S2, int Sin, int d, const int* src, const double* w,
                  double2* out);
// the embedding rows of n_ids distinct ids, each with occurrences occ[start[u] .. start[u+1]) (rows of G)
void embedding_update(hipStream_t st, double2* table, int d, const uint32_t* ids, int n_ids, const int* start,
                      const int* occ, const double2* G, double lr, double bs, uint32_t* err);

// ---- attention ----
struct Attn {
  const double2* q = nullptr;  // [B*S][ldq]; head h at column h*dh
  long ldq = 0;
  const double2* kc = nullptr;  // [B][H][ctx][dh]
  const double2* vc = nullptr;
  int ctx = 0;
  const int* kv_len = nullptr;  // [B]: keys = kv_len[b] + T_add (null: T_const)
  int T_add = 0, T_const = 0;
  int T_max = 0;                // upper bound on keys (sizing)
  const double* bias_re = nullptr;  // [H][mc][mc] Re(bias_pos)
  int mc = 0;
  const uint32_t* row_mask = nullptr;  // [B*S]
  double2* out = nullptr;              // [B*S][ldo], head h at column h*dh
  long ldo = 0;
  int B = 0, S = 0, H = 0, dh = 0;
  double scale = 1.0;
  double2* kc_w = nullptr;  // writable cache (attention_decode_split appends the new token)
  double2* vc_w = nullptr;
  uint32_t* err = nullptr;
};
// One query row per block (the general reference case, any T).
void attention_rows(hipStream_t st, const Attn& a);
// Prefill (T == S, no KV length): tiled MFMA kernel for head dims 16, 32, 64,
// 128; returns false (nothing launched) for other shapes.
bool attention_prefill(hipStream_t st, const Attn& a);
// Decode (S == 1): key chunks in parallel; the chunk partials (AttnSplit) are
// combined by a RowOps prologue (rowops_apply or a GEMV).  q is the sum of
// npart partials (row b at q + b * ldq, partial stride part_stride); with
// `append` the partials are [q | k | v] of the new token, whose k and v the
// kernel appends to the cache (kc_w, vc_w).
// MFMA-tiled GEMM (gemm_mfma.hip) for M > 64: block tile GBM x GBN, K step
// GBK; grid (N tiles, M tiles, K splits of kchunk).  ERR_ARG for EPI_PART.
constexpr int GBM = 64, GBN = 64, GBK = 16;
int launch_zgemm_mfma(hipStream_t st, dim3 grid, const double2* A, long lda, const double2* W, long ldw, int M, int N,
                      int K, int kchunk, const Epi& ep, const Argmax& am, double2* ws, uint32_t* cnt);

AttnSplit attention_split_plan(const Attn& a);
size_t attention_split_ws_bytes(int B, int H, int dh, int T_max);
int attention_decode_split(hipStream_t st, const Attn& a, const double2* q, long ldq, int npart, long part_stride,
                           bool append, const AttnSplit& out);

// ---- resident decode loop (resident.hip) ----
// One cooperative launch runs `nsteps` decode steps; each step is the program
// ops[0..nops), with a grid barrier after every operation.  Block b takes work
// items b, b + grid, ... of each operation.  Every block keeps the step state
// (KV lengths, the ids being fed, the step count) in LDS and finds the greedy
// ids itself from the vocab product's argmax partials at the start of the next
// step; block 0 writes ids, history, counts and KV lengths back.
enum ROpKind : int { ROP_GEMV = 0, ROP_ATTN = 1, ROP_ROWS = 2 };
struct ROp {
  int kind = ROP_GEMV;
  int items = 0;
  int M = 0;  // rows (sequences)
  // GEMV: rowops(ro)[M][K] * W[K][N] -> ep; C columns x (4 kw) rows per item,
  // ncb column blocks; EPI_PART leaves the K splits as partials, other modes
  // need one split.  am.part_v != null: per column-block argmax partials.
  RowOps ro;
  const double2* W = nullptr;
  long ldw = 0;
  int N = 0, K = 0, C = 0, kw = 0, ncb = 0, P = 1, waves = 4;
  Epi ep;
  Argmax am;
  // ATTN: chunks of attention_split_plan (items nsplit x H x B); q of sequence b at q + b * ldq.
  //   The combine out[b][h*dh + e] = Re(chunk combine + ro.resid) of (b, h):
  //   barrier exchange: the last chunk to finish (cnt: counters [B][H]);
  //   polling exchange: the item of (b, h)'s last split, after its chunk if
  //   that has keys (comb_items 0), or items nsplit x H x B + b * H + h
  //   after all the chunks (comb_items 1: more items than blocks)
  Attn a;
  AttnSplit o;
  const double2* q = nullptr;
  long ldq = 0;
  uint32_t* cnt = nullptr;
  int comb_items = 0;
  // ROWS: out[m][k] = rowops(ro)[m][k], k < K, in column chunks of cw (whole rows with a LayerNorm)
  double2* out = nullptr;
  long ldo = 0;
  int cw = 0;
};
// the step state and greedy_decoding (sampling_methods.rs:5-18) of the loop
struct RStep {
  int B = 0;
  const double* part_v = nullptr;  // [B][tiles] vocab argmax partials
  const int* part_i = nullptr;
  int tiles = 0;
  uint32_t* ids = nullptr;   // [B] ids fed to the step
  uint32_t* hist = nullptr;  // [B][hist_stride] generated ids
  int hist_stride = 0;
  int* hist_cnt = nullptr;  // [B] ids generated so far (also the logits-history slot)
  int* kv_len = nullptr;    // [B]
  uint32_t* err = nullptr;
  // polling exchange (the ops of even steps, then those of odd steps): the odd
  // steps' argmax partials, and the exchange arena [2][arena_half doubles]
  // whose half of the previous step each step fills with the sentinel
  const double* part_v1 = nullptr;
  const int* part_i1 = nullptr;
  double* arena = nullptr;
  long arena_half = 0;
};
struct ResGemvPlan {
  int mr, C, kw, P, ncb, waves;
};
// narrowest column block with at most `grid` blocks; EPI_PART splits K up to
// the grid (at most 8 ways); waves 3: one item per block whose weights fit the
// prefetch registers of waves 1-3 (kw rows each), else 4 streaming waves
ResGemvPlan resident_gemv_plan(int M, int N, int K, bool part, int grid);
size_t resident_op_lds(const ROp& op);  // dynamic LDS of one operation
// blocks of the launch (one per CU: `cus` compute units, cooperative launch
// supported) if the kernel for (mr, dh) fits with `shm`
int resident_grid(int cus, bool cooperative, int mr, int dh, size_t shm, int* grid, bool poll = false);
// the polling exchange is built for mr rows
bool resident_poll_built(int mr);
// flags: one word per block, epochs below epoch0 + 1 (zeroed at set-up); the
// launch performs resident_barriers(nops, nsteps, poll) barriers.  poll: the
// polling exchange; ops_d then holds 2 * nops operations (the even steps',
// then the odd steps'), and step.arena both halves already filled with the
// sentinel.  stamps (optional, nsteps * nops + 1 words): block 0's wall clock
// (100 MHz) after each operation, then at the start.
int resident_launch(hipStream_t st, const ROp* ops_d, int nops, int nsteps, const RStep& step, int mr, int dh,
                    size_t shm, int grid, uint32_t* flags, uint32_t epoch0, uint32_t* err, uint64_t* stamps,
                    bool poll = false);
// grid barriers a launch performs (the epochs it consumes)
inline uint32_t resident_barriers(int nops, int nsteps, bool poll) {
  return poll ? (uint32_t)(nsteps > 0 ? nsteps - 1 : 0) : (uint32_t)nops * (uint32_t)nsteps;
}
// polling exchange: the sentinel every exchanged value starts a step as
// (all bits set: a NaN no arithmetic produces; as an int, -1), and the rows of
// positions [kv_len[b], kv_len[b] + n) of the caches [B][H][ctx][dh] filled with it
constexpr unsigned long long RES_SENT = 0xFFFFFFFFFFFFFFFFull;
void resident_kv_sentinel(hipStream_t st, double2* kc, double2* vc, int B, int H, int ctx, int dh, const int* kv_len,
                          int n);

// ---- EmbeddingLayer::create_embedding (wavelet_init.hip) ----
constexpr int EW_MAX_SRC = 4096;  // drawn values per token (LDS: two rows of doubles)
// width of a src-wide draw after decompose_in_wavelet_2d_default (0: src not a power of two in [2, EW_MAX_SRC])
int embedding_wavelet_dim(int src);
// table [vocab][dim] <- create_embedding of every token (key: the draw's counter stream);
// kern_d: device room for kern_cap complex values (the CMOR integral, 33 at scale 2)
int embedding_wavelet_init(hipStream_t st, double2* table, int vocab, int dim, int src, uint64_t key,
                           double2* kern_d, size_t kern_cap);

// ---- row kernels ----
void embed(hipStream_t st, const double2* table, int V, int d, const uint32_t* ids, int rows, double2* out,
           uint32_t* err);
// positions per row (pos != null) or per sequence from kv_len (S == 1 decode)
void rope(hipStream_t st, double2* x, int rows, int d, const double2* cs_table, int max_pos, const int* pos,
          const int* kv_len, const int* off, uint32_t* err);
// DiscreteWaveletLayer compression of a prompt pass: [B][S][d] -> [B][S2][d]
// through a tap table [S2][L] (source row or -1, sign) and low-pass filter lo[L]
void dwt_rows(hipStream_t st, const double2* x, int B, int S, int d, const int* src, const double* sgn,
              const double* lo, int L, int S2, double2* out);
void layernorm(hipStream_t st, const double2* x, const double2* before, double2* out, int rows, int d, double eps,
               const double2* gamma, const double2* beta);
void gather_rows(hipStream_t st, const double2* src, int S, int d, const uint32_t* lens, int B, double2* dst);
// argmax per row with last-index ties (greedy_decoding on host-provided logits)
void argmax_rows(hipStream_t st, const double* logits, int rows, int V, uint32_t* ids, uint32_t* err);
void softmax_rows(hipStream_t st, const double2* logits, int rows, int S, int V, const uint32_t* row_mask, int mode,
                  double* out);

// ---- initialisation ----
void fill_seeded(hipStream_t st, double2* dst, int rows, int cols, long ld, uint64_t key, double lim);
void fill_seeded_re(hipStream_t st, double* dst, int rows, int cols, long ld, uint64_t key, double lim);
void fill_const(hipStream_t st, double2* dst, size_t n, double2 v);
void fill_int(hipStream_t st, int* dst, size_t n, int v);
void fill_u32(hipStream_t st, uint32_t* dst, size_t n, uint32_t v);

}  // namespace mitok
