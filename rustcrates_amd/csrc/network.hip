// network.hip — host side of libmitok: the reference's layer/model API over
// device tensors, the forward executor, the greedy token loop and the C ABI
// declared in include/mitok.h.
//
// Reference structure mirrored here (paths relative to src/neural_networks/):
//   NeuralNetwork { layers: Vec<LayerEnum> }   network_types/neural_network_generic.rs:23-31
//   LayerEnum                                  network_components/layer.rs:75-88
//   predict                                    network_types/transformer/transformer_network.rs:315-504
//   predict_token_by_token                     network_types/transformer/transformer_network.rs:165-313
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <memory>
#include <mutex>
#include <string>
#include <map>
#include <vector>

#include "../../include/mitok.h"
#include "kernels.hpp"

namespace mitok {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local char g_err[1024];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(expr)                                                                          \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess) return fail(ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                     \
  } while (0)

#define TRY(expr)          \
  do {                     \
    int rc_ = (expr);      \
    if (rc_) return rc_;   \
  } while (0)

// ---------------------------------------------------------------------------
// device buffers
// ---------------------------------------------------------------------------
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  // grows only; returns 1 in *grew when the address changed
  int reserve(size_t n, bool* grew = nullptr) {
    if (n <= bytes && p) return OK;
    release();
    size_t want = std::max<size_t>(n, 256);
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
      p = nullptr;
      return fail(ERR_NOMEM, "hipMalloc(%zu bytes): %s", want, hipGetErrorString(e));
    }
    bytes = want;
    if (grew) *grew = true;
    return OK;
  }
  template <class T>
  T* as() const {
    return (T*)p;
  }
};

// ---------------------------------------------------------------------------
// layers (LayerEnum variants on the token-loop path)
// ---------------------------------------------------------------------------
enum Kind {
  K_EMBEDDING = 0,
  K_POSENC = 1,
  K_NORM = 2,
  K_SELF_ATTENTION = 3,
  K_FEED_FORWARD = 4,
  K_LINEAR = 5,
  K_SOFTMAX = 6,
  K_WAVELET = 7
};

struct Layer {
  int kind;
  uint32_t d_in = 0, d_out = 0;
  // the layer's learning_rate field (every sublayer's, as update_learning_rate
  // sets them, neural_network_generic.rs:115-186); create_transformer builds
  // its layers at 0.01 (transformer_builder.rs:16)
  double lr = 0.01;
  explicit Layer(int k) : kind(k) {}
  virtual ~Layer() = default;
};

struct EmbeddingLayer : Layer {  // embedding_layer.rs:24-36
  uint32_t vocab = 0;
  DevBuf table;  // [vocab][d]
  EmbeddingLayer() : Layer(K_EMBEDDING) {}
};

struct PositionalEncodingLayer : Layer {  // positional_encoding_layer.rs:15-22
  double base = 1250.0;
  DevBuf cs;  // [positions][d/2] (cos, sin) of the clamped angle
  int positions = 0;
  PositionalEncodingLayer() : Layer(K_POSENC) {}
};

struct NormLayer : Layer {  // norm_layer.rs:17-42
  double eps = 0.0;
  DevBuf gamma, beta;  // [d]
  NormLayer() : Layer(K_NORM) {}
};

struct SelfAttentionLayer : Layer {  // self_attention_layer.rs:16-25 + masked_attention_head.rs:23-61
  uint32_t heads = 0, dh = 0, max_ctx = 0;
  double eps = 0.0;
  DevBuf wqkv;     // [d][3d]: columns [q heads | k heads | v heads], head h at h*dh
  DevBuf bias_re;  // [heads][max_ctx][max_ctx]  Re(bias_pos): only the real part reaches the softmax
  DevBuf gamma, beta;
  DevBuf kc, vc;  // [cache_B][heads][max_ctx][dh]
  // training state: AdamW moments of wqkv and of the Norm's gamma and beta;
  // updates so far of the heads and of the Norm, counted apart because
  // reset_previous_gradient resets the heads' previous gradient but not the
  // Norm's (neural_network_generic.rs:196-205); each one's first update is
  // plain clipped descent
  DevBuf mw, vw, mg, vg, mbt, vbt;
  uint32_t updates = 0, norm_updates = 0;
  SelfAttentionLayer() : Layer(K_SELF_ATTENTION) {}
};

struct FeedForwardLayer : Layer {  // feedforward_layer.rs:14-26, layer.rs:91-112, linear_layer.rs:18-34
  uint32_t hidden = 0;
  DevBuf w1, b1, w2, b2;
  // training state of the Dense (1) and Linear (2) sublayers: AdamW moments
  // and updates so far (each sublayer's first update is plain clipped descent)
  DevBuf mw1, vw1, mb1, vb1, mw2, vw2, mb2, vb2;
  uint32_t updates1 = 0, updates2 = 0;
  FeedForwardLayer() : Layer(K_FEED_FORWARD) {}
};

struct LinearLayer : Layer {  // linear_layer.rs:18-34
  DevBuf w, b;
  // training state (linear_layer.rs:130-175): AdamW moments of the weights and
  // the bias, allocated and zeroed at the first update; updates so far (the
  // first one is plain clipped descent, as when previous_gradient is None)
  DevBuf mw, vw, mb, vb;
  uint32_t updates = 0;
  LinearLayer() : Layer(K_LINEAR) {}
};

struct SoftmaxLayer : Layer {  // softmax_output_layer.rs:15-27
  int mode = 1;
  SoftmaxLayer() : Layer(K_SOFTMAX) {}
};

struct WaveletLayer : Layer {  // DiscreteWaveletLayer, network_types/wavelet_discrete_layer.rs:20-70
  uint32_t wavelet = 1, mode = 2;  // DiscreteWaletetType DB2, WaveletMode SYMMETRIC by default
  int L = 4;                       // filter length
  double lo[4] = {0, 0, 0, 0};     // low-pass filter
  WaveletLayer() : Layer(K_WAVELET) {}
};

// ---------------------------------------------------------------------------
// DiscreteWaveletLayer geometry (host): the reference's dwt_1d padding
// (wavelet_transform/dwt.rs:36-90, 149-293) restated on indices, so the
// device applies it as a tap table
// ---------------------------------------------------------------------------
// Low-pass filters of DB1 and DB2 (dwt_coeffients.rs DB_1, DB_2): 1/sqrt(2)
// twice, and Daubechies' closed form (1+sqrt3, 3+sqrt3, 3-sqrt3, 1-sqrt3) /
// (4 sqrt2), each evaluated in long double and rounded once to double (the
// same doubles as the reference's table).
static bool wavelet_low_pass(uint32_t wavelet, double* lo, int* L) {
  if (wavelet == 0) {
    lo[0] = lo[1] = (double)(1.0L / sqrtl(2.0L));
    *L = 2;
    return true;
  }
  if (wavelet == 1) {
    const long double s3 = sqrtl(3.0L), den = 4.0L * sqrtl(2.0L);
    lo[0] = (double)((1.0L + s3) / den);
    lo[1] = (double)((3.0L + s3) / den);
    lo[2] = (double)((3.0L - s3) / den);
    lo[3] = (double)((1.0L - s3) / den);
    *L = 4;
    return true;
  }
  return false;
}

static bool wavelet_mode_ok(uint32_t mode) { return mode <= 4 || mode == 6; }  // index-expressible paddings

// rows a wavelet layer leaves of S: the low half of dwt_1d's n + L - 2 (+1 if odd) values
static int wavelet_rows(int S, int L) { return (S + L - 2 + (S % 2)) >> 1; }

// Tap table of one prompt-pass compression of S rows: output row j reads rows
// src[j][l] (-1: a padding zero) with signs sgn[j][l], l < L.
struct WaveletTaps {
  int S2 = 0;
  std::vector<int> src;
  std::vector<double> sgn;
};

static WaveletTaps wavelet_taps(int S, int L, uint32_t mode) {
  struct E {
    int idx;
    double sign;
  };
  const int nb = L - 2, len0 = S + nb;
  const int na = (len0 % L != 0) ? L - len0 % L + 2 : L - len0 % L + 1;
  std::vector<E> a;
  a.reserve(S + nb + na);
  for (int i = 0; i < S; ++i) a.push_back({i, 1.0});
  int rtmp = 0;
  for (int i = 0; i < nb; ++i) {  // insert_padding_before
    const int cur = (int)a.size();
    E v = {-1, 1.0};
    switch (mode) {
      case 0: break;
      case 1: v = a[i]; break;
      case 2: v = a[cur % S + i % S]; break;
      case 3: v = a[cur % S + i % S]; v.sign = -v.sign; break;
      case 4:
        if (i > 0) rtmp = (rtmp + 2) % cur;
        if (rtmp == 0) rtmp = 1;
        v = a[rtmp];
        break;
      default: v = {S - 1 - (i % S), 1.0}; break;
    }
    a.insert(a.begin(), v);
  }
  const std::vector<E> orig = a;
  const int olen = (int)orig.size();
  for (int i = 0; i < na; ++i) {  // insert_padding_after
    const int cur = (int)a.size();
    E v = {-1, 1.0};
    switch (mode) {
      case 0: break;
      case 1: v = a[cur - 1]; break;
      case 2: v = a[cur - (cur % olen + i % olen) - 1]; break;
      case 3: v = a[cur - (cur % olen + i % olen) - 1]; v.sign = -v.sign; break;
      case 4: v = orig[olen - ((i + 1) % olen) - 1]; break;
      default: v = orig[i % (olen - nb) + nb]; break;
    }
    a.push_back(v);
  }
  WaveletTaps t;
  t.S2 = wavelet_rows(S, L);
  const int plen = (int)a.size();
  for (int j = 0; j < t.S2; ++j)
    for (int l = 0; l < L; ++l) {
      const E e = a[(2 * j + l) % plen];
      t.src.push_back(e.idx);
      t.sgn.push_back(e.sign);
    }
  return t;
}

enum RunMode { MODE_PREFILL = 0, MODE_CACHED = 1, MODE_STATELESS = 2 };

struct Spec {
  int B = 0, S = 0;
  int mode = MODE_STATELESS;
  bool forward_only = true;
  bool last_row = false;
  uint32_t first = 0, last = 0;      // layer range
  const double2* in = nullptr;       // hidden-state input when first > 0
  const uint32_t* ids = nullptr;     // [B*S] padded ids (first == 0)
  const uint32_t* mask = nullptr;    // [B*S]
  const uint32_t* lens = nullptr;    // [B]
  const int* pos = nullptr;          // [B*S] RoPE positions, or null -> kv_len (S == 1)
  const int* kv_row = nullptr;       // [B] cached append row (S > 1), or null
  double* out_re = nullptr;          // vocab Re-logits
  double* out_prob = nullptr;        // softmax output (not forward_only)
  double2* out_hidden = nullptr;     // result of a hidden-state range
  const Argmax* am = nullptr;        // greedy ids fused into the vocab GEMM (token loop)
  bool compress = false;             // apply the wavelet stages begin_call planned for this call
  double* hist_re = nullptr;         // Re-logits history [step][B][V] at hist_cnt[0] (token loop)
  const int* hist_cnt = nullptr;
  int ctx_bound = 0;                 // keys a decode step of this call can reach (0: the layers' context)
};

struct Timing {
  int cls = 0;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  std::vector<double> pending_bytes;
  std::vector<hipEvent_t> pool;
  std::vector<double> pending_flops;
  double total_ms = 0.0, bytes = 0.0, flops = 0.0;
  uint64_t launches = 0;
};

}  // namespace mitok

struct mitok_network {
  int device = 0;
  int cus = 0;               // compute units (the resident loop runs one block per CU)
  void* scratch = nullptr;   // this device's copy of the no-allocation staging array
  bool cooperative = false;  // cooperative launches supported
  hipStream_t stream = nullptr;
  // NeuralNetwork::learning_rate: the rate backward passes to the Embedding's
  // update (transformer_network.rs:520), changed by decay_learning_rate
  // (neural_network_generic.rs:69-73) and not by update_learning_rate
  double lr = 0.01;
  std::vector<std::unique_ptr<mitok::Layer>> layers;
  // session (KV cache) state
  bool cache_valid = false;
  uint32_t cache_B = 0;
  std::vector<uint32_t> kv_len_h;
  mitok::DevBuf kv_len_d, err_d;
  // workspaces
  mitok::DevBuf act0, act1, qbuf, concat, hbuf, gath, mat0, mat1, logits_c, logits_re, probs, kv_scratch;
  mitok::DevBuf ids_d, mask_d, lens_d, pos_d, kv_row_d, ones_d, dec_ids_d, hist_d, cnt_d, logit_hist_d;
  // split-completion counters (zeroed once, self-resetting), split partials, argmax partials
  mitok::DevBuf sync_cnt, sync_ws, am_v, am_i;
  // fused decode plan: split partials left for the next launch to sum
  mitok::DevBuf dq, df1, dp0, dp1, datt;
  int fused_decode = 1;   // B <= 8 decode steps use the fused GEMV plan
  int tiled_prefill = 1;  // prefill attention runs the tiled MFMA kernel where it applies
  int resident = 1;       // generate's decode loop as one resident launch: 0 never, 1 B == 1, 2 B <= 8
  // resident decode loop: operation table (host copy kept until the next build),
  // one barrier flag per block (zeroed when allocated), the next barrier epoch
  std::vector<mitok::ROp> res_ops_h;
  mitok::DevBuf res_ops, res_flags, res_stamps;
  mitok::DevBuf res_cnt;    // per (layer, sequence, head) attention-chunk counters
  mitok::DevBuf res_arena;  // polling exchange: the exchanged values, two halves
  int res_nops = 0;         // operations per step (res_ops_h holds two programs when polling)
  int res_poll = 1;         // the polling exchange where it is built (else the grid barrier)
  bool res_polled = false;  // the last resident launch polled
  uint32_t res_epoch = 0;
  int res_profile = 0;  // record per-operation times of the next resident launches
  uint32_t res_steps = 0;
  // decode-step graph: generate's step (graph_step 0, ids history of n_new per
  // sequence) or mitok_decode_step's (graph_step 1, one id per sequence)
  hipGraphExec_t graph = nullptr;
  uint32_t graph_B = 0, graph_nnew = 0;
  int graph_step = 0;
  int graph_ctx = 0;  // the decode spec's ctx_bound the graph was captured for
  bool graph_logits = false;
  uint64_t ws_generation = 0, graph_generation = 0;
  int direct_launch = 0;
  double last_t[3] = {0, 0, 0};
  mitok::Timing timing;
  // sum over sequences of the keys the next decode step attends over (the host
  // loop sets it before each timed step): the attention class's algorithmic bytes
  double dec_tsum = 0.0;
  // wavelet compression of the current prompt or stateless call: one stage per
  // DiscreteWaveletLayer in the call's range (tap table, filter, and the
  // compressed mask, lens and row positions on the device); the last stage's
  // mask and lens on the host; rows per sequence after the stages
  struct WaveletStage {
    int S_in = 0, S2 = 0, L = 0;
    int T = 0;                   // target rows passed through after the compressed input rows
    const uint32_t* mask_in = nullptr;  // the padding mask of the stage's input rows
    double lo[4] = {0, 0, 0, 0};
    mitok::DevBuf src, sgn, lo_d, mask, lens, pos;
    mitok::DevBuf gsrc, gw;  // backward's tap table [S_in][4]
  };
  std::vector<std::unique_ptr<WaveletStage>> wstages;
  std::vector<uint32_t> wmask_h, wlens_h;
  int wS = 0;
  // decode-time RoPE offset per sequence after a compressed prompt: prompt
  // length minus its cached rows (positions count the uncompressed prompt)
  mitok::DevBuf pos_off_d;
  bool pos_off = false;
  // the last stateless pass's vocab Linear input rows [head_B * head_S][d]
  // (in act0/act1) and its softmax output (probs), which mitok_backward_head
  // differentiates; any later call clears head_valid
  bool head_valid = false;
  uint32_t train_T = 0;  // target rows of the stateless pass being planned (mitok_predict_targets)
  const double2* head_x = nullptr;
  const uint32_t* head_mask = nullptr;  // the padding mask of those rows
  uint32_t head_B = 0, head_S = 0, head_first = 0;
  // what a stateless pass keeps for backward: each layer's input rows, and
  // the heads' output of each SelfAttention layer (before its residual + Norm)
  std::vector<std::unique_ptr<mitok::DevBuf>> tr_in, tr_cat;
  mitok::DevBuf tr_g, tr_xh, tr_wh, tr_dw, tr_db, tr_ga, tr_gb, tr_tgt, tr_norm;
  mitok::DevBuf tr_z, tr_h, tr_g1, tr_dh, tr_qkv, tr_dqkv, tr_A, tr_dA, tr_pg, tr_eid, tr_est, tr_eocc, tr_bsum;
  mitok::DevBuf ce_buf;  // mitok_cross_entropy_loss: targets, lengths, per-sequence losses, the result
};

namespace mitok {

using Net = mitok_network;

// the RoPE offsets of decode steps after a compressed prompt, or null
static const int* rope_offsets(const Net* n) { return n->pos_off ? n->pos_off_d.as<int>() : nullptr; }

static int set_device(Net* n) {
  HIP_TRY(hipSetDevice(n->device));
  return OK;
}

static void drop_graph(Net* n) {
  if (n->graph) (void)hipGraphExecDestroy(n->graph);
  n->graph = nullptr;
}

static int reserve(Net* n, DevBuf& b, size_t bytes) {
  bool grew = false;
  TRY(b.reserve(bytes, &grew));
  if (grew) {
    n->ws_generation++;
    drop_graph(n);
  }
  return OK;
}

static int upload(Net* n, DevBuf& b, const void* src, size_t bytes) {
  TRY(reserve(n, b, bytes));
  HIP_TRY(hipMemcpyAsync(b.p, src, bytes, hipMemcpyHostToDevice, n->stream));
  return OK;
}

static int check_err_word(Net* n) {
  uint32_t e = 0;
  HIP_TRY(hipMemcpyAsync(&e, n->err_d.p, sizeof e, hipMemcpyDeviceToHost, n->stream));
  HIP_TRY(hipStreamSynchronize(n->stream));
  if (!e) return OK;
  fill_u32(n->stream, n->err_d.as<uint32_t>(), 1, 0);
  HIP_TRY(hipStreamSynchronize(n->stream));
  if (e & EB_BAD_TOKEN) return fail(ERR_ARG, "No token embedding found: token id >= vocab (embedding_layer.rs:305)");
  if (e & EB_GELU_NAN) return fail(ERR_NAN, "NaN detected in tanh(f(z)) (activation.rs:207-209)");
  if (e & EB_FFN_NONFINITE) return fail(ERR_NAN, "output ffn dense: The value is Not Valid (transformer_network.rs:408)");
  if (e & EB_ARGMAX_NAN) return fail(ERR_NAN, "greedy_decoding: NaN in logits (sampling_methods.rs:12)");
  if (e & EB_CTX_OVERFLOW) return fail(ERR_ARG, "context exceeds max_ctx");
  if (e & EB_BARRIER) return fail(ERR_STATE, "resident decode: a grid barrier or an exchange poll timed out");
  if (e & EB_TRAIN_NONFINITE) return fail(ERR_NAN, "gradient in embedding is invalid, contains NaN or infinity values (embedding_layer.rs:242-250)");
  return fail(ERR_STATE, "device error word 0x%x", e);
}

// ---------------------------------------------------------------------------
// timing
// ---------------------------------------------------------------------------
static hipEvent_t take_event(Timing& t) {
  if (!t.pool.empty()) {
    hipEvent_t e = t.pool.back();
    t.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

// Times the first kernel launched inside the scope when `cls` is the enabled
// class (its start and stop stamped by the dispatch, see MITOK_LAUNCH); the
// step class records events around the whole scope instead.
struct TimeScope {
  Net* n;
  bool on, whole;
  hipEvent_t a = nullptr, b = nullptr;
  double bytes, flops;
  TimeScope(Net* net, int cls, double alg_bytes, double alg_flops = 0.0)
      : n(net), on(net->timing.cls == cls), whole(cls == MITOK_TIME_STEP), bytes(alg_bytes), flops(alg_flops) {
    if (!on) return;
    a = take_event(n->timing);
    b = take_event(n->timing);
    if (whole) (void)hipEventRecord(a, n->stream);
    else launch_timing() = {a, b};
  }
  ~TimeScope() {
    if (!on) return;
    LaunchTiming& lt = launch_timing();
    if (whole) {
      (void)hipEventRecord(b, n->stream);
    } else if (lt.start) {  // nothing was launched
      lt = LaunchTiming();
      n->timing.pool.push_back(a);
      n->timing.pool.push_back(b);
      return;
    }
    n->timing.pending.push_back({a, b});
    n->timing.pending_bytes.push_back(bytes);
    n->timing.pending_flops.push_back(flops);
  }
};

static void collect_timing(Net* n) {
  Timing& t = n->timing;
  for (size_t i = 0; i < t.pending.size(); ++i) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, t.pending[i].first, t.pending[i].second) == hipSuccess) {
      t.total_ms += ms;
      t.bytes += t.pending_bytes[i];
      t.flops += t.pending_flops[i];
      t.launches++;
    }
    t.pool.push_back(t.pending[i].first);
    t.pool.push_back(t.pending[i].second);
  }
  t.pending.clear();
  t.pending_bytes.clear();
  t.pending_flops.clear();
}

// algorithmic HBM bytes of C[M][N] = A[M][K] * B[K][N]: B once, A once, C once
static double gemm_bytes(long M, long N, long K, bool re_out) {
  return 16.0 * (double)K * N + 16.0 * (double)M * K + (re_out ? 8.0 : 16.0) * (double)M * N;
}
// real flops of a complex product: 4 multiplies + 4 adds per complex MAC
static double gemm_flops(long M, long N, long K) { return 8.0 * (double)M * N * K; }
// of its real part alone (Re-logits): Re(a b) = ar br - ai bi, 2 + 2 per MAC
static double gemm_flops_re(long M, long N, long K) { return 4.0 * (double)M * N * K; }

// algorithmic HBM bytes of one decode attention launch of a layer (width d,
// H heads): per key of every sequence its K and V rows (16 B per element) and
// the Re(bias_pos) row-0 entry of each head (8 B)
static double attention_decode_bytes(const Net* n, long d, long H) {
  return n->dec_tsum * (2.0 * 16.0 * (double)d + 8.0 * (double)H);
}

// ---------------------------------------------------------------------------
// workspace sizing for one forward shape
// ---------------------------------------------------------------------------
struct Dims {
  uint32_t dmax = 0, dsa = 0, hmax = 0, fmax = 0, vocab = 0, mc_max = 0, dh_max = 0;
};

static Dims net_dims(const Net* n) {
  Dims d;
  for (auto& L : n->layers) {
    d.dmax = std::max({d.dmax, L->d_in, L->d_out});
    if (L->kind == K_SELF_ATTENTION) {
      auto* A = (SelfAttentionLayer*)L.get();
      d.dsa = std::max(d.dsa, A->d_in);
      d.hmax = std::max(d.hmax, A->heads);
      d.mc_max = std::max(d.mc_max, A->max_ctx);
      d.dh_max = std::max(d.dh_max, A->dh);
    }
    if (L->kind == K_FEED_FORWARD) d.fmax = std::max(d.fmax, ((FeedForwardLayer*)L.get())->hidden);
    if (L->kind == K_LINEAR) d.vocab = std::max(d.vocab, L->d_out);
  }
  return d;
}

static bool is_vocab_linear(const Net* n, uint32_t li) {
  return n->layers[li]->kind == K_LINEAR && li + 2 == n->layers.size() && n->layers.back()->kind == K_SOFTMAX;
}

static int prepare(Net* n, const Spec& sp) {
  n->head_valid = false;  // the workspaces that held the last stateless pass's head input are reused
  const Dims dm = net_dims(n);
  const size_t rows = (size_t)sp.B * sp.S;
  const size_t c16 = sizeof(double2);
  TRY(reserve(n, n->act0, rows * dm.dmax * c16));
  TRY(reserve(n, n->act1, rows * dm.dmax * c16));
  TRY(reserve(n, n->qbuf, rows * std::max(1u, dm.dsa) * c16));
  TRY(reserve(n, n->concat, rows * std::max(1u, dm.dsa) * c16));
  TRY(reserve(n, n->hbuf, rows * std::max(1u, dm.fmax) * c16));
  TRY(reserve(n, n->gath, (size_t)sp.B * dm.dmax * c16));
  TRY(reserve(n, n->mat0, rows * dm.dmax * c16));
  TRY(reserve(n, n->mat1, rows * dm.dmax * c16));
  if (sp.mode == MODE_STATELESS) {  // the layer inputs backward reads
    while (n->tr_in.size() < n->layers.size()) n->tr_in.push_back(std::make_unique<DevBuf>());
    while (n->tr_cat.size() < n->layers.size()) n->tr_cat.push_back(std::make_unique<DevBuf>());
    for (uint32_t li = sp.first; li < sp.last; ++li) {
      const Layer* L = n->layers[li].get();
      if (L->kind != K_EMBEDDING && L->kind != K_SOFTMAX) TRY(reserve(n, *n->tr_in[li], rows * L->d_in * c16));
      if (L->kind == K_SELF_ATTENTION) TRY(reserve(n, *n->tr_cat[li], rows * L->d_in * c16));
    }
  }
  size_t ws = 0;
  for (uint32_t li = sp.first; li < sp.last; ++li) {
    Layer* L = n->layers[li].get();
    const int M = (int)rows;
    if (L->kind == K_SELF_ATTENTION) ws = std::max(ws, gemm_ws_bytes(M, 3 * L->d_in, L->d_in));
    if (L->kind == K_FEED_FORWARD) {
      auto* F = (FeedForwardLayer*)L;
      ws = std::max(ws, gemm_ws_bytes(M, F->hidden, F->d_in));
      ws = std::max(ws, gemm_ws_bytes(M, F->d_out, F->hidden));
    }
    if (L->kind == K_LINEAR) {
      const bool vocab = is_vocab_linear(n, li) && sp.first == 0;
      const int Mv = (vocab && sp.last_row) ? sp.B : M;
      ws = std::max(ws, gemm_ws_bytes(Mv, L->d_out, L->d_in));
      if (vocab && !sp.forward_only) {
        TRY(reserve(n, n->logits_c, (size_t)Mv * L->d_out * c16));
        TRY(reserve(n, n->probs, (size_t)Mv * L->d_out * sizeof(double)));
      }
      if (vocab && sp.forward_only) {
        TRY(reserve(n, n->logits_re, (size_t)Mv * L->d_out * sizeof(double)));
        TRY(reserve(n, n->am_v, argmax_part_elems(Mv, L->d_out) * sizeof(double)));
        TRY(reserve(n, n->am_i, argmax_part_elems(Mv, L->d_out) * sizeof(int)));
      }
    }
  }
  if (dm.hmax) {
    if (sp.mode == MODE_CACHED && sp.S == 1)
      TRY(reserve(n, n->datt, attention_split_ws_bytes(sp.B, dm.hmax, dm.dh_max, dm.mc_max)));
    if (sp.mode == MODE_STATELESS) TRY(reserve(n, n->kv_scratch, 2 * rows * dm.dsa * c16));
  }
  TRY(reserve(n, n->sync_ws, ws));
  if (sp.mode == MODE_CACHED && sp.S == 1 && sp.B <= GEMM_PART_MAX_M) {
    const size_t B = sp.B;
    TRY(reserve(n, n->dq, 8 * B * 3 * std::max(1u, dm.dsa) * c16));
    TRY(reserve(n, n->df1, 8 * B * std::max(1u, dm.fmax) * c16));
    TRY(reserve(n, n->dp0, 8 * B * dm.dmax * c16));
    TRY(reserve(n, n->dp1, 8 * B * dm.dmax * c16));
  }
  TRY(reserve(n, n->kv_len_d, (size_t)sp.B * sizeof(int)));
  if (n->pos_off) TRY(reserve(n, n->pos_off_d, (size_t)sp.B * sizeof(int)));
  TRY(reserve(n, n->ones_d, std::max<size_t>(rows, sp.B) * sizeof(uint32_t)));
  TRY(reserve(n, n->dec_ids_d, (size_t)sp.B * sizeof(uint32_t)));
  return OK;
}

static Sync sync_of(Net* n) {
  Sync s;
  s.counters = n->sync_cnt.as<uint32_t>();
  s.ws = n->sync_ws.p;
  s.ws_bytes = n->sync_ws.bytes;
  return s;
}

static RowOps rows_of(const double2* x, long ldx) {
  RowOps r;
  r.x = x;
  r.ldx = ldx;
  return r;
}

// a launch wrapper's refusal (shape beyond the workspace or counters) as an error
static int launch_rc(int rc, const char* what) {
  if (rc) return fail(rc, "%s: launch refused (workspace or shape limit)", what);
  return OK;
}

// RoPE table: (cos, sin) of clamp(pos / base^(2i/d), -1, 1) with the host libm,
// exactly as positional_encoding_layer.rs:188-198 evaluates it.
static int ensure_rope_table(Net* n, PositionalEncodingLayer* P, int positions) {
  if (P->positions >= positions) return OK;
  const uint32_t d = P->d_in, half = d / 2;
  std::vector<double2> cs((size_t)positions * half);
  for (int p = 0; p < positions; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      double theta = (double)p / pow(P->base * 1.0, 2.0 * (double)i / (double)d);
      theta = std::min(1.0, std::max(-1.0, theta));
      cs[(size_t)p * half + i] = make_double2(cos(theta), sin(theta));
    }
  TRY(reserve(n, P->cs, cs.size() * sizeof(double2)));
  HIP_TRY(hipMemcpy(P->cs.p, cs.data(), cs.size() * sizeof(double2), hipMemcpyHostToDevice));
  P->positions = positions;
  return OK;
}

// the chunk partials of decode attention live in n->datt
static AttnSplit split_buffers(Net* n, AttnSplit o, int B, int H) {
  o.pm = n->datt.as<double>();
  o.pl = o.pm + (size_t)B * H * o.nsplit;
  o.po = (const double2*)(o.pl + (size_t)B * H * o.nsplit);
  return o;
}

// ---------------------------------------------------------------------------
// the forward executor: predict's layer walk (transformer_network.rs:335-492)
// ---------------------------------------------------------------------------
static int enqueue_forward(Net* n, const Spec& sp) {
  hipStream_t st = n->stream;
  uint32_t* err = n->err_d.as<uint32_t>();
  const Sync sy = sync_of(n);
  const int B = sp.B;
  int S = sp.S, rows = B * S;  // a wavelet layer of a prompt pass compresses the rows
  const uint32_t* mask = sp.mask;
  const uint32_t* lens = sp.lens;
  const int* pos = sp.pos;
  size_t wi = 0;  // next wavelet stage
  double2* cur = n->act0.as<double2>();
  double2* nxt = n->act1.as<double2>();
  if (sp.in) HIP_TRY(hipMemcpyAsync(cur, sp.in, (size_t)rows * n->layers[sp.first]->d_in * sizeof(double2),
                                   hipMemcpyDeviceToDevice, st));
  for (uint32_t li = sp.first; li < sp.last; ++li) {
    Layer* L = n->layers[li].get();
    if (sp.mode == MODE_STATELESS && L->kind != K_EMBEDDING && L->kind != K_SOFTMAX)  // kept for backward
      HIP_TRY(hipMemcpyAsync(n->tr_in[li]->p, cur, (size_t)rows * L->d_in * sizeof(double2), hipMemcpyDeviceToDevice, st));
    switch (L->kind) {
      case K_EMBEDDING: {
        auto* E = (EmbeddingLayer*)L;
        embed(st, E->table.as<double2>(), E->vocab, E->d_out, sp.ids, rows, cur, err);
        break;
      }
      case K_POSENC: {
        auto* P = (PositionalEncodingLayer*)L;
        rope(st, cur, rows, P->d_in, P->cs.as<double2>(), P->positions, pos, pos ? nullptr : n->kv_len_d.as<int>(),
             pos ? nullptr : rope_offsets(n), err);
        break;
      }
      case K_NORM: {
        auto* N = (NormLayer*)L;
        layernorm(st, cur, nullptr, nxt, rows, N->d_in, N->eps, N->gamma.as<double2>(), N->beta.as<double2>());
        std::swap(cur, nxt);
        break;
      }
      case K_SELF_ATTENTION: {
        auto* A = (SelfAttentionLayer*)L;
        const int d = A->d_in, H = A->heads, dh = A->dh;
        Epi e;
        e.mode = EPI_QKV;
        e.out = n->qbuf.as<double2>();
        e.ldo = d;
        e.d = d;
        e.dh = dh;
        e.heads = H;
        e.S = S;
        e.err = err;
        Attn a;
        a.q = n->qbuf.as<double2>();
        a.ldq = d;
        if (sp.mode == MODE_STATELESS) {
          e.kc = n->kv_scratch.as<double2>();
          e.vc = e.kc + (size_t)rows * d;
          e.ctx = S;
          a.T_const = S;
          a.T_max = S;
        } else {
          e.kc = A->kc.as<double2>();
          e.vc = A->vc.as<double2>();
          e.ctx = A->max_ctx;
          if (sp.mode == MODE_PREFILL) {
            a.T_const = S;
            a.T_max = S;
          } else {
            e.kv_base = n->kv_len_d.as<int>();
            e.kv_row = sp.kv_row;
            a.kv_len = n->kv_len_d.as<int>();
            a.T_add = 1;
            a.T_max = A->max_ctx;
          }
        }
        {
          TimeScope ts(n, S > 1 ? MITOK_TIME_PREFILL_GEMM : MITOK_TIME_LAYER_GEMM, gemm_bytes(rows, 3 * d, d, false),
                       gemm_flops(rows, 3 * d, d));
          TRY(launch_rc(gemm(st, rows, 3 * d, d, rows_of(cur, d), A->wqkv.as<double2>(), 3 * d, e, nullptr, sy), "qkv"));
        }
        a.kc = e.kc;
        a.vc = e.vc;
        a.ctx = e.ctx;
        a.bias_re = A->bias_re.as<double>();
        a.mc = A->max_ctx;
        a.row_mask = mask;
        a.out = n->concat.as<double2>();
        a.ldo = d;
        a.B = B;
        a.S = S;
        a.H = H;
        a.dh = dh;
        a.scale = 1.0 / (1e-8 + sqrt((double)dh));  // scale_attention_scores (masked_attention_head.rs:453-465)
        if (sp.mode == MODE_CACHED && S == 1) {
          // key chunks, then one row transform: chunk combine + residual + Norm (self_attention_layer.rs:101-124)
          AttnSplit o = split_buffers(n, attention_split_plan(a), B, H);
          {
            TimeScope ts(n, MITOK_TIME_ATTENTION, attention_decode_bytes(n, d, H));
            TRY(launch_rc(attention_decode_split(st, a, n->qbuf.as<double2>(), d, 1, 0, false, o), "attention"));
          }
          RowOps r;
          r.err = err;
          r.att = o;
          r.resid = cur;
          r.ldr = d;
          r.ln = 1;
          r.eps = A->eps;
          r.gamma = A->gamma.as<double2>();
          r.beta = A->beta.as<double2>();
          rowops_apply(st, B, d, r, nxt, d);
        } else {
          {
            TimeScope ts(n, MITOK_TIME_ATTENTION, 0.0);
            if (!n->tiled_prefill || !attention_prefill(st, a)) attention_rows(st, a);
          }
          if (sp.mode == MODE_STATELESS)  // the heads' output, kept for backward
            HIP_TRY(hipMemcpyAsync(n->tr_cat[li]->p, n->concat.p, (size_t)rows * d * sizeof(double2),
                                   hipMemcpyDeviceToDevice, st));
          layernorm(st, n->concat.as<double2>(), cur, nxt, rows, d, A->eps, A->gamma.as<double2>(),
                    A->beta.as<double2>());
        }
        std::swap(cur, nxt);
        break;
      }
      case K_FEED_FORWARD: {
        auto* F = (FeedForwardLayer*)L;
        Epi e1;
        e1.mode = EPI_GELU;
        e1.bias = F->b1.as<double2>();
        e1.out = n->hbuf.as<double2>();
        e1.ldo = F->hidden;
        e1.row_mask = mask;
        e1.err = err;
        Epi e2;
        e2.mode = EPI_STORE;
        e2.bias = F->b2.as<double2>();
        e2.out = nxt;
        e2.ldo = F->d_out;
        e2.check_finite = 1;
        e2.err = err;
        {
          TimeScope ts(n, S > 1 ? MITOK_TIME_PREFILL_GEMM : MITOK_TIME_LAYER_GEMM, gemm_bytes(rows, F->hidden, F->d_in, false),
                       gemm_flops(rows, F->hidden, F->d_in));
          TRY(launch_rc(gemm(st, rows, F->hidden, F->d_in, rows_of(cur, F->d_in), F->w1.as<double2>(), F->hidden, e1,
                             nullptr, sy), "ffn1"));
        }
        {
          TimeScope ts(n, S > 1 ? MITOK_TIME_PREFILL_GEMM : MITOK_TIME_LAYER_GEMM, gemm_bytes(rows, F->d_out, F->hidden, false),
                       gemm_flops(rows, F->d_out, F->hidden));
          TRY(launch_rc(gemm(st, rows, F->d_out, F->hidden, rows_of(n->hbuf.as<double2>(), F->hidden),
                             F->w2.as<double2>(), F->d_out, e2, nullptr, sy), "ffn2"));
        }
        std::swap(cur, nxt);
        break;
      }
      case K_LINEAR: {
        auto* Ln = (LinearLayer*)L;
        const bool vocab = is_vocab_linear(n, li) && sp.first == 0;
        if (!vocab) {
          Epi e;
          e.mode = EPI_STORE;
          e.bias = Ln->b.as<double2>();
          e.out = nxt;
          e.ldo = Ln->d_out;
          e.err = err;
          TRY(launch_rc(gemm(st, rows, Ln->d_out, Ln->d_in, rows_of(cur, Ln->d_in), Ln->w.as<double2>(), Ln->d_out, e,
                             nullptr, sy), "linear"));
          std::swap(cur, nxt);
          break;
        }
        const double2* x = cur;
        int M = rows;
        if (sp.last_row) {
          gather_rows(st, cur, S, Ln->d_in, lens, B, n->gath.as<double2>());
          x = n->gath.as<double2>();
          M = B;
        }
        Epi e;
        e.bias = Ln->b.as<double2>();
        e.ldo = Ln->d_out;
        e.err = err;
        if (sp.forward_only) {
          e.mode = EPI_RE;
          e.out_re = sp.out_re;
          e.hist_re = sp.hist_re;
          e.hist_cnt = sp.hist_cnt;
          TimeScope ts(n, MITOK_TIME_VOCAB, gemm_bytes(M, Ln->d_out, Ln->d_in, true), gemm_flops_re(M, Ln->d_out, Ln->d_in));
          TRY(launch_rc(gemm(st, M, Ln->d_out, Ln->d_in, rows_of(x, Ln->d_in), Ln->w.as<double2>(), Ln->d_out, e,
                             sp.am, sy), "vocab"));
        } else {
          e.mode = EPI_STORE;
          e.out = n->logits_c.as<double2>();
          TRY(launch_rc(gemm(st, M, Ln->d_out, Ln->d_in, rows_of(x, Ln->d_in), Ln->w.as<double2>(), Ln->d_out, e,
                             nullptr, sy), "vocab"));
          if (sp.mode == MODE_STATELESS && !sp.last_row) {  // the layer keeps its input for backward
            n->head_valid = true;
            n->head_x = x;
            n->head_first = sp.first;
            n->head_mask = mask;
            n->head_B = (uint32_t)B;
            n->head_S = (uint32_t)S;
          }
          auto* SM = (SoftmaxLayer*)n->layers.back().get();
          softmax_rows(st, n->logits_c.as<double2>(), M, S, Ln->d_out, mask, SM->mode == MITOK_TRAINING ? 0 : 1,
                       sp.out_prob);
        }
        break;
      }
      case K_SOFTMAX: break;  // applied together with the vocab Linear
      case K_WAVELET: {
        // only the call begin_call planned compresses; a cached step's row
        // passes through (wavelet_discrete_layer.rs:102-128)
        if (!sp.compress) break;
        if (wi >= n->wstages.size()) return fail(ERR_STATE, "wavelet stage %zu not planned", wi);
        const auto& W = *n->wstages[wi++];
        dwt_rows(st, cur, B, S, (int)L->d_in, W.src.as<int>(), W.sgn.as<double>(), W.lo_d.as<double>(), W.L, W.S2, nxt);
        std::swap(cur, nxt);
        S = W.S2;
        rows = B * S;
        mask = W.mask.as<uint32_t>();
        lens = W.lens.as<uint32_t>();
        pos = W.pos.as<int>();
        break;
      }
    }
  }
  if (sp.out_hidden && cur != sp.out_hidden) {
    const uint32_t dout = n->layers[sp.last - 1]->d_out;
    HIP_TRY(hipMemcpyAsync(sp.out_hidden, cur, (size_t)rows * dout * sizeof(double2), hipMemcpyDeviceToDevice, st));
  }
  HIP_TRY(hipGetLastError());
  return OK;
}

// ---------------------------------------------------------------------------
// fused decode step for B <= 8 sequences (one row each): the row transforms
// of Embedding / PositionalEncoding / Norm and the residual LayerNorm inside
// SelfAttention are carried as a pending prologue into the next product, so a
// transformer block is 4 launches: QKV (+KV append), attention, FFN Dense
// (+GELU), FFN Linear; the vocab Linear ends the step with the greedy id.
// ---------------------------------------------------------------------------
static bool fused_decode_ok(const Net* n, const Spec& sp) {
  if (!n->fused_decode || sp.mode != MODE_CACHED || sp.S != 1 || sp.B > GEMM_PART_MAX_M || !sp.forward_only)
    return false;
  if (sp.compress) return false;  // a one-row call at time step 0 that a wavelet layer widens
  if (sp.first != 0 || sp.last != n->layers.size() || sp.kv_row || sp.out_hidden) return false;
  if (sp.B <= 8) {
    // the GEMV prologue holds whole input rows of a LayerNorm in LDS
    const size_t mr = sp.B <= 1 ? 1 : sp.B <= 2 ? 2 : sp.B <= 4 ? 4 : 8;
    size_t row = 0;  // widest product input
    for (auto& L : n->layers) row = std::max<size_t>(row, L->d_in);
    if (mr * row * sizeof(double2) > 64 * 1024) return false;
  } else {
    // the MFMA products leave the partials of QKV, FFN Linear and hidden Linears
    for (uint32_t li = 0; li < n->layers.size(); ++li) {
      const Layer* L = n->layers[li].get();
      if (L->kind == K_SELF_ATTENTION && !gemm_parts(sp.B, 3 * L->d_in, L->d_in)) return false;
      if (L->kind == K_FEED_FORWARD) {
        const auto* F = (const FeedForwardLayer*)L;
        if (!gemm_parts(sp.B, F->d_out, F->hidden)) return false;
      }
      if (L->kind == K_LINEAR && !is_vocab_linear(n, li) && !gemm_parts(sp.B, L->d_out, L->d_in)) return false;
    }
  }
  for (auto& L : n->layers)
    if (L->kind == K_SELF_ATTENTION) {
      // the row transform keeps the chunk weights of every head in LDS
      const auto* A = (const SelfAttentionLayer*)L.get();
      Attn a;
      a.B = sp.B;
      a.H = A->heads;
      a.T_max = A->max_ctx;
      const AttnSplit o = attention_split_plan(a);
      if (o.nsplit > 256) return false;
    }
  return true;
}

// Every product of the plan writes split partials (EPI_PART) that the next
// launch sums in its prologue, together with the operations that follow the
// product in the reference (bias, GELU, finite check, residual, LayerNorm),
// so no launch waits on another's blocks.  A transformer block is QKV
// (+ LayerNorm of its input), attention (+ KV append), FFN Dense (+ attention
// combine, residual, LayerNorm) and FFN Linear (+ bias, GELU); the vocab
// Linear and the greedy id end the step.  From 9 to 64 sequences the products
// are MFMA kernels that read plain rows: a pending row transform is first
// materialised (rowops_apply), and FFN Dense finishes its sums in-kernel
// (GELU needs them); QKV and FFN Linear still leave partials for the
// attention and the next row transform.
// From this many sequences plan 1 materialises the rows its GEMV products read
// (the transform before QKV, FFN Dense's GELU output), so every product takes
// plain rows and requests them before its weights (k_gemv's PRE variant).
// Measured on MI355X, decode per step at config 3: with 3 sequences 425 -> 354
// us, with 2 370 -> 332 (the threshold was 4 before the rows-first GEMV)
constexpr int FUSED_PLAIN_MIN_B = 2;
static int enqueue_decode_fused(Net* n, const Spec& sp) {
  hipStream_t st = n->stream;
  uint32_t* err = n->err_d.as<uint32_t>();
  const Sync sy = sync_of(n);
  const int B = sp.B;
  int* kv_len = n->kv_len_d.as<int>();
  RowOps pro;  // pending prologue of the next product
  pro.err = err;
  int width = 0;  // row length the pending prologue produces
  double2* mats[2] = {n->mat0.as<double2>(), n->mat1.as<double2>()};
  int mat_next = 0;
  double2* parts[2] = {n->dp0.as<double2>(), n->dp1.as<double2>()};
  int part_next = 0;
  const bool mat = B > 8;  // the MFMA products read plain rows
  auto materialize = [&]() {
    double2* out = mats[mat_next];
    mat_next ^= 1;
    rowops_apply(st, B, width, pro, out, width);
    RowOps r = rows_of(out, width);
    r.err = err;
    pro = r;
  };
  auto need_plain = [&]() {
    if (mat && !pro.plain()) materialize();
  };
  auto part_rows = [&](double2* buf, int npart, int cols) {
    RowOps r = rows_of(buf, cols);
    r.npart = npart;
    r.part_stride = (long)B * cols;
    r.err = err;
    return r;
  };
  for (uint32_t li = 0; li < n->layers.size(); ++li) {
    Layer* L = n->layers[li].get();
    switch (L->kind) {
      case K_EMBEDDING: {
        auto* E = (EmbeddingLayer*)L;
        pro = RowOps();
        pro.err = err;
        pro.table = E->table.as<double2>();
        pro.ids = sp.ids;
        pro.vocab = (int)E->vocab;
        width = (int)E->d_out;
        break;
      }
      case K_POSENC: {
        auto* P = (PositionalEncodingLayer*)L;
        if (pro.rope_cs || pro.resid || pro.ln) materialize();
        pro.rope_cs = P->cs.as<double2>();
        pro.rope_pos = sp.pos ? sp.pos : kv_len;
        pro.rope_off = sp.pos ? nullptr : rope_offsets(n);
        pro.rope_max = P->positions;
        break;
      }
      case K_NORM: {
        auto* N = (NormLayer*)L;
        if (pro.ln) materialize();
        pro.ln = 1;
        pro.eps = N->eps;
        pro.gamma = N->gamma.as<double2>();
        pro.beta = N->beta.as<double2>();
        break;
      }
      case K_SELF_ATTENTION: {
        auto* A = (SelfAttentionLayer*)L;
        const int d = A->d_in, H = A->heads, dh = A->dh;
        if (pro.resid) materialize();           // its residual source is about to be overwritten
        double2* x1 = n->act0.as<double2>();  // the block input, kept for the residual
        // from FUSED_PLAIN_MIN_B sequences the row transform before QKV (split
        // partials + bias + LayerNorm) is materialised once rather than redone
        // by every QKV block: measured on MI355X before the rows-first GEMV,
        // decode per step 763 -> 708 us at config 3 with 8 sequences, 496 ->
        // 489 with 4, 1943 -> 1911 at config 5 with 4
        if (mat || B >= FUSED_PLAIN_MIN_B) {
          if (!pro.plain()) rowops_apply(st, B, d, pro, x1, d);
          else x1 = const_cast<double2*>(pro.x);  // a materialised row buffer (ld d), not reused before the combine
          pro = rows_of(x1, d);
          pro.err = err;
        } else {
          pro.save = x1;
          pro.ldsave = d;
        }
        const int pq = gemm_parts(B, 3 * d, d);
        Epi e;
        e.mode = EPI_PART;
        e.out = n->dq.as<double2>();
        e.err = err;
        {
          TimeScope ts(n, MITOK_TIME_LAYER_GEMM, gemm_bytes(B, 3 * d, d, false), gemm_flops(B, 3 * d, d));
          TRY(launch_rc(gemm(st, B, 3 * d, d, pro, A->wqkv.as<double2>(), 3 * d, e, nullptr, sy), "qkv"));
        }
        Attn a;
        a.kc = A->kc.as<double2>();
        a.vc = A->vc.as<double2>();
        a.kc_w = A->kc.as<double2>();
        a.vc_w = A->vc.as<double2>();
        a.ctx = A->max_ctx;
        a.kv_len = kv_len;
        a.T_add = 1;
        // the call's reach sizes the chunk split: at config 3 with 32 sequences
        // (128 + 128 keys) 8 chunks, whose combine joins the row transform
        a.T_max = sp.ctx_bound > 0 ? std::min<int>(sp.ctx_bound, (int)A->max_ctx) : (int)A->max_ctx;
        a.bias_re = A->bias_re.as<double>();
        a.mc = A->max_ctx;
        a.B = B;
        a.S = 1;
        a.H = H;
        a.dh = dh;
        a.scale = 1.0 / (1e-8 + sqrt((double)dh));  // masked_attention_head.rs:453-465
        a.err = err;
        const AttnSplit o = split_buffers(n, attention_split_plan(a), B, H);
        {
          TimeScope ts(n, MITOK_TIME_ATTENTION, attention_decode_bytes(n, d, H));
          TRY(launch_rc(attention_decode_split(st, a, n->dq.as<double2>(), 3 * d, pq, (long)B * 3 * d, true, o),
                        "attention"));
        }
        pro = RowOps();  // chunk combine + residual + Norm (self_attention_layer.rs:101-124), once per row
        pro.err = err;
        pro.att = o;
        pro.resid = x1;
        pro.ldr = d;
        pro.ln = 1;
        pro.eps = A->eps;
        pro.gamma = A->gamma.as<double2>();
        pro.beta = A->beta.as<double2>();
        width = d;
        materialize();
        break;
      }
      case K_FEED_FORWARD: {
        auto* F = (FeedForwardLayer*)L;
        RowOps h;
        // Dense: + b1, GELU in the epilogue (layer.rs:132-166).  From
        // FUSED_PLAIN_MIN_B sequences also for the GEMV: in FFN Linear's
        // prologue every column block would evaluate GELU again over its K
        // range (96 times over at config 5).  Measured on MI355X, decode per
        // step 1791 -> 1643 us at config 5 with 4 sequences, 713 -> 707 at
        // config 3 with 8; ids unchanged
        if (mat || B >= FUSED_PLAIN_MIN_B) {
          need_plain();
          Epi e1;
          e1.mode = EPI_GELU;
          e1.bias = F->b1.as<double2>();
          e1.out = n->hbuf.as<double2>();
          e1.ldo = F->hidden;
          e1.row_mask = sp.mask;
          e1.err = err;
          TimeScope ts(n, MITOK_TIME_LAYER_GEMM, gemm_bytes(B, F->hidden, F->d_in, false),
                       gemm_flops(B, F->hidden, F->d_in));
          TRY(launch_rc(gemm(st, B, F->hidden, F->d_in, pro, F->w1.as<double2>(), F->hidden, e1, nullptr, sy), "ffn1"));
          h = rows_of(n->hbuf.as<double2>(), F->hidden);
          h.err = err;
        } else {
          const int p1 = gemm_parts(B, F->hidden, F->d_in);
          Epi e1;
          e1.mode = EPI_PART;
          e1.out = n->df1.as<double2>();
          e1.err = err;
          {
            TimeScope ts(n, MITOK_TIME_LAYER_GEMM, gemm_bytes(B, F->hidden, F->d_in, false),
                         gemm_flops(B, F->hidden, F->d_in));
            TRY(launch_rc(gemm(st, B, F->hidden, F->d_in, pro, F->w1.as<double2>(), F->hidden, e1, nullptr, sy),
                          "ffn1"));
          }
          h = part_rows(n->df1.as<double2>(), p1, F->hidden);  // Dense: + b1, GELU (layer.rs:132-166)
          h.bias = F->b1.as<double2>();
          h.gelu = 1;
          h.row_mask = sp.mask;
        }
        double2* out = parts[part_next];
        part_next ^= 1;
        const int p2 = gemm_parts(B, F->d_out, F->hidden);
        Epi e2;
        e2.mode = EPI_PART;
        e2.out = out;
        e2.err = err;
        {
          TimeScope ts(n, MITOK_TIME_LAYER_GEMM, gemm_bytes(B, F->d_out, F->hidden, false),
                       gemm_flops(B, F->d_out, F->hidden));
          TRY(launch_rc(gemm(st, B, F->d_out, F->hidden, h, F->w2.as<double2>(), F->d_out, e2, nullptr, sy), "ffn2"));
        }
        pro = part_rows(out, p2, F->d_out);  // Linear: + b2; non-finite check (transformer_network.rs:408)
        pro.bias = F->b2.as<double2>();
        pro.finite_check = 1;
        width = (int)F->d_out;
        break;
      }
      case K_LINEAR: {
        auto* Ln = (LinearLayer*)L;
        need_plain();
        if (is_vocab_linear(n, li)) {
          Epi e;
          e.bias = Ln->b.as<double2>();
          e.ldo = Ln->d_out;
          e.err = err;
          e.mode = EPI_RE;
          e.out_re = sp.out_re;
          e.hist_re = sp.hist_re;
          e.hist_cnt = sp.hist_cnt;
          TimeScope ts(n, MITOK_TIME_VOCAB, gemm_bytes(B, Ln->d_out, Ln->d_in, true), gemm_flops_re(B, Ln->d_out, Ln->d_in));
          TRY(launch_rc(gemm(st, B, Ln->d_out, Ln->d_in, pro, Ln->w.as<double2>(), Ln->d_out, e, sp.am, sy), "vocab"));
        } else {
          double2* out = parts[part_next];
          part_next ^= 1;
          const int pl = gemm_parts(B, Ln->d_out, Ln->d_in);
          Epi e;
          e.mode = EPI_PART;
          e.out = out;
          e.err = err;
          TRY(launch_rc(gemm(st, B, Ln->d_out, Ln->d_in, pro, Ln->w.as<double2>(), Ln->d_out, e, nullptr, sy), "linear"));
          pro = part_rows(out, pl, Ln->d_out);
          pro.bias = Ln->b.as<double2>();
          width = (int)Ln->d_out;
        }
        break;
      }
      case K_SOFTMAX: break;
      case K_WAVELET: break;  // a decode step's row passes through (wavelet_discrete_layer.rs:102-128)
    }
  }
  HIP_TRY(hipGetLastError());
  return OK;
}

static int enqueue_step(Net* n, const Spec& sp) {
  return fused_decode_ok(n, sp) ? enqueue_decode_fused(n, sp) : enqueue_forward(n, sp);
}

// ---------------------------------------------------------------------------
// resident decode loop (resident.hip): the decode step of generate for B <= 8
// sequences as a program of operations that one cooperative launch runs for
// every step.  Row transforms are materialised (ROP_ROWS) before a product
// unless they fit its prologue: a LayerNorm of rows that fit LDS, split
// partials + bias, an embedding gather, RoPE.  A transformer block is QKV
// (+ KV append in the epilogue), attention chunks, chunk combine + residual,
// FFN Dense (+ the attention block's LayerNorm in the prologue, GELU in the
// epilogue), FFN Linear (split partials); the vocab product leaves argmax
// partials that every block reduces at the start of the next step.
// ---------------------------------------------------------------------------
constexpr size_t RES_LN_ROWS_BYTES = 64 * 1024;  // LayerNorm prologue rows held in LDS
constexpr size_t RES_MAX_DYN_LDS = 120 * 1024;

static int res_mr(int B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8; }

// measured on MI355X at config 3: the resident loop wins at batch 1; from
// batch 4 the fused launches (graph) are faster
constexpr int RES_AUTO_MAX_B = 1;
// with the polling exchange (config 3, 2 sequences: 349 against 377 us per
// step for plan 1; from 4 sequences plan 1 is faster, 443 against 482)
constexpr int RES_AUTO_MAX_B_POLL = 2;

static bool resident_ok(const Net* n, const Spec& sp) {
  bool rope = false;
  for (auto& L : n->layers) rope = rope || L->kind == K_POSENC;
  const int auto_b = (n->res_poll && !rope) ? RES_AUTO_MAX_B_POLL : RES_AUTO_MAX_B;  // RoPE: the barrier exchange
  const int max_b = n->resident == 2 ? 8 : n->resident == 1 ? auto_b : 0;
  if (sp.mode != MODE_CACHED || sp.S != 1 || sp.B > max_b || !sp.forward_only || !sp.am || sp.compress) return false;
  if (sp.first != 0 || sp.last != n->layers.size() || sp.kv_row || sp.out_hidden) return false;
  for (auto& L : n->layers)
    if (L->kind == K_SELF_ATTENTION) {
      const auto* A = (const SelfAttentionLayer*)L.get();
      Attn a;
      a.B = sp.B;
      a.H = A->heads;
      a.T_max = A->max_ctx;
      a.dh = A->dh;
      const AttnSplit o = attention_split_plan(a);
      if (o.nsplit > 256 || A->dh > 256) return false;
    }
  return true;
}

// The polling exchange's buffers: every value one operation of a step hands
// to another is carved, 256-byte aligned, from one half of the arena.
struct ResArena {
  char* base = nullptr;
  size_t used = 0;  // bytes
  template <class T>
  T* take(size_t count) {
    T* p = (T*)(base + used);
    used += (count * sizeof(T) + 255) & ~(size_t)255;
    return p;
  }
};

struct ResBuilt {
  int dh = 0;       // the head dim the kernel is specialised for (0: generic)
  size_t shm = 0;   // its dynamic LDS
  int tiles = 0;    // the vocab product's argmax partials per row
  double* part_v = nullptr;  // where the vocab product leaves them
  int* part_i = nullptr;
  bool poll_ok = true;  // (with an arena) every operation reads its inputs by polling
};

// Builds the step program into n->res_ops_h.  With an arena, the exchanged
// buffers come from it and poll_ok says whether the program is one the
// polling exchange runs (no materialised rows, no RoPE, at most 8 partials).
static int resident_build(Net* n, const Spec& sp, int grid, ResBuilt* rb, ResArena* ar = nullptr) {
  std::vector<ROp>& ops = n->res_ops_h;
  ops.clear();
  *rb = ResBuilt();
  uint32_t* err = n->err_d.as<uint32_t>();
  const int B = sp.B, mr = res_mr(B);
  int* kv_len = n->kv_len_d.as<int>();
  RowOps pro;
  pro.err = err;
  int width = 0, dh_k = -1;
  double2* mats[2] = {n->mat0.as<double2>(), n->mat1.as<double2>()};
  int mat_next = 0;
  double2* parts[2] = {n->dp0.as<double2>(), n->dp1.as<double2>()};
  int part_next = 0;
  size_t cnt_next = 0;  // chunk counters: distinct per layer
  // the buffers of one exchange: the arena's, else the workspace's
  auto rows_buf = [&](double2* ws, size_t count) { return ar ? ar->take<double2>(count) : ws; };
  auto materialize = [&]() {
    if (ar) rb->poll_ok = false;
    ROp op;
    op.kind = ROP_ROWS;
    op.M = B;
    op.ro = pro;
    op.K = width;
    op.out = rows_buf(mats[mat_next], (size_t)B * width);
    op.ldo = width;
    op.cw = 256;
    op.items = pro.ln ? B : B * ((width + op.cw - 1) / op.cw);
    mat_next ^= 1;
    ops.push_back(op);
    pro = rows_of(op.out, width);
    pro.err = err;
  };
  // a LayerNorm prologue holds whole input rows in LDS
  auto fit_prologue = [&](int K) {
    if (pro.att.po || (pro.ln && (size_t)mr * K * sizeof(double2) > RES_LN_ROWS_BYTES)) materialize();
  };
  auto gemv = [&](const RowOps& ro, const double2* W, int N, int K, const Epi& ep, const Argmax* am) -> ROp& {
    const ResGemvPlan p = resident_gemv_plan(B, N, K, ep.mode == EPI_PART, grid);
    ROp op;
    op.kind = ROP_GEMV;
    op.M = B;
    op.ro = ro;
    op.W = W;
    op.ldw = N;
    op.N = N;
    op.K = K;
    op.C = p.C;
    op.kw = p.kw;
    op.ncb = p.ncb;
    op.P = p.P;
    op.waves = p.waves;
    op.ep = ep;
    if (am) op.am = *am;
    op.items = p.ncb * p.P;
    ops.push_back(op);
    return ops.back();
  };
  auto part_rows = [&](double2* buf, int npart, int cols) {
    RowOps r = rows_of(buf, cols);
    r.npart = npart;
    r.part_stride = (long)B * cols;
    r.err = err;
    return r;
  };
  for (uint32_t li = 0; li < n->layers.size(); ++li) {
    Layer* L = n->layers[li].get();
    switch (L->kind) {
      case K_EMBEDDING: {
        auto* E = (EmbeddingLayer*)L;
        pro = RowOps();
        pro.err = err;
        pro.table = E->table.as<double2>();
        pro.ids = sp.ids;
        pro.vocab = (int)E->vocab;
        width = (int)E->d_out;
        break;
      }
      case K_POSENC: {
        auto* P = (PositionalEncodingLayer*)L;
        if (pro.rope_cs || pro.resid || pro.ln || pro.att.po) materialize();
        if (ar) rb->poll_ok = false;  // RoPE is not in the polled prologue
        pro.rope_cs = P->cs.as<double2>();
        pro.rope_pos = sp.pos ? sp.pos : kv_len;
        pro.rope_off = sp.pos ? nullptr : rope_offsets(n);
        pro.rope_max = P->positions;
        break;
      }
      case K_NORM: {
        auto* N = (NormLayer*)L;
        if (pro.ln || pro.att.po) materialize();
        pro.ln = 1;
        pro.eps = N->eps;
        pro.gamma = N->gamma.as<double2>();
        pro.beta = N->beta.as<double2>();
        break;
      }
      case K_SELF_ATTENTION: {
        auto* A = (SelfAttentionLayer*)L;
        const int d = A->d_in, H = A->heads, dh = A->dh;
        dh_k = (dh_k < 0 || dh_k == dh) ? dh : 0;
        if (pro.resid) materialize();  // its residual source is about to be overwritten
        fit_prologue(d);
        double2* x1 = rows_buf(n->act0.as<double2>(), (size_t)B * d);  // the block input, kept for the residual
        pro.save = x1;
        pro.ldsave = d;
        Epi e;
        e.mode = EPI_QKV;
        e.out = rows_buf(n->qbuf.as<double2>(), (size_t)B * d);
        e.ldo = d;
        e.d = d;
        e.dh = dh;
        e.heads = H;
        e.S = 1;
        e.kc = A->kc.as<double2>();
        e.vc = A->vc.as<double2>();
        e.ctx = A->max_ctx;
        e.kv_base = kv_len;
        e.err = err;
        gemv(pro, A->wqkv.as<double2>(), 3 * d, d, e, nullptr);
        Attn a;
        a.kc = A->kc.as<double2>();
        a.vc = A->vc.as<double2>();
        a.ctx = A->max_ctx;
        a.kv_len = kv_len;
        a.T_add = 1;
        a.T_max = A->max_ctx;
        a.bias_re = A->bias_re.as<double>();
        a.mc = A->max_ctx;
        a.B = B;
        a.S = 1;
        a.H = H;
        a.dh = dh;
        a.scale = 1.0 / (1e-8 + sqrt((double)dh));  // masked_attention_head.rs:453-465
        a.err = err;
        if (sp.ctx_bound > 0 && sp.ctx_bound < (int)A->max_ctx) {
          // the split sized to the call's reach where that gives every chunk a
          // block of its own (config 3, 2 sequences: 347 -> 323 us per step; at
          // 1 sequence, with a block per chunk either way, 255 against 256)
          Attn r = a;
          r.T_max = sp.ctx_bound;
          if ((long)attention_split_plan(a).nsplit * H * B > grid && (long)attention_split_plan(r).nsplit * H * B <= grid)
            a.T_max = sp.ctx_bound;
        }
        ROp at;
        at.kind = ROP_ATTN;
        at.M = B;
        at.a = a;
        at.o = split_buffers(n, attention_split_plan(a), B, H);
        if (ar) {
          const size_t np = (size_t)B * H * at.o.nsplit;
          at.o.pm = ar->take<double>(np);
          at.o.pl = ar->take<double>(np);
          at.o.po = ar->take<double2>(np * dh);
        }
        at.q = e.out;
        at.ldq = d;
        // polling: (b, h)'s last split combines it where every chunk has a
        // block of its own, else the combines are items after the chunks
        at.items = at.o.nsplit * H * B;
        if (ar && at.items > grid) {
          at.comb_items = 1;
          at.items += B * H;
        }
        // chunk combine + residual by the last chunk of each (sequence, head),
        // then the Norm (self_attention_layer.rs:101-124) in the next
        // product's prologue
        if (cnt_next + (size_t)B * H > n->res_cnt.bytes / sizeof(uint32_t)) return fail(ERR_STATE, "chunk counters");
        at.cnt = n->res_cnt.as<uint32_t>() + cnt_next;
        cnt_next += (size_t)B * H;
        at.ro.resid = x1;
        at.ro.ldr = d;
        at.out = rows_buf(mats[mat_next], (size_t)B * d);
        at.ldo = d;
        mat_next ^= 1;
        ops.push_back(at);
        pro = rows_of(at.out, d);
        pro.err = err;
        width = d;
        pro.ln = 1;
        pro.eps = A->eps;
        pro.gamma = A->gamma.as<double2>();
        pro.beta = A->beta.as<double2>();
        break;
      }
      case K_FEED_FORWARD: {
        auto* F = (FeedForwardLayer*)L;
        fit_prologue(F->d_in);
        Epi e1;  // Dense: + b1, GELU, pad rows 0 (layer.rs:132-166)
        e1.mode = EPI_GELU;
        e1.bias = F->b1.as<double2>();
        e1.out = rows_buf(n->hbuf.as<double2>(), (size_t)B * F->hidden);
        e1.ldo = F->hidden;
        e1.row_mask = sp.mask;
        e1.err = err;
        gemv(pro, F->w1.as<double2>(), F->hidden, F->d_in, e1, nullptr);
        const int P2 = resident_gemv_plan(B, F->d_out, F->hidden, true, grid).P;
        double2* out = rows_buf(parts[part_next], (size_t)P2 * B * F->d_out);
        part_next ^= 1;
        Epi e2;
        e2.mode = EPI_PART;
        e2.out = out;
        e2.err = err;
        RowOps h = rows_of(e1.out, F->hidden);
        h.err = err;
        const int p2 = gemv(h, F->w2.as<double2>(), F->d_out, F->hidden, e2, nullptr).P;
        pro = part_rows(out, p2, F->d_out);  // Linear: + b2; non-finite check (transformer_network.rs:408)
        pro.bias = F->b2.as<double2>();
        pro.finite_check = 1;
        width = (int)F->d_out;
        break;
      }
      case K_LINEAR: {
        auto* Ln = (LinearLayer*)L;
        fit_prologue(Ln->d_in);
        if (is_vocab_linear(n, li)) {
          Epi e;
          e.bias = Ln->b.as<double2>();
          e.ldo = Ln->d_out;
          e.err = err;
          e.mode = EPI_RE;
          e.out_re = sp.out_re;
          e.hist_re = sp.hist_re;
          e.hist_cnt = sp.hist_cnt;
          Argmax am = *sp.am;
          const int ncb = resident_gemv_plan(B, Ln->d_out, Ln->d_in, false, grid).ncb;
          if (ar) {
            am.part_v = ar->take<double>((size_t)B * ncb);
            am.part_i = ar->take<int>((size_t)B * ncb);
          } else {
            am.part_v = n->am_v.as<double>();
            am.part_i = n->am_i.as<int>();
            if ((size_t)B * ncb > n->am_v.bytes / sizeof(double)) return fail(ERR_STATE, "argmax partials");
          }
          if (gemv(pro, Ln->w.as<double2>(), Ln->d_out, Ln->d_in, e, &am).ncb != ncb)
            return fail(ERR_STATE, "resident decode: vocab tiles");
          rb->tiles = ncb;
          rb->part_v = am.part_v;
          rb->part_i = am.part_i;
        } else {
          const int PL = resident_gemv_plan(B, Ln->d_out, Ln->d_in, true, grid).P;
          double2* out = rows_buf(parts[part_next], (size_t)PL * B * Ln->d_out);
          part_next ^= 1;
          Epi e;
          e.mode = EPI_PART;
          e.out = out;
          e.err = err;
          const int pl = gemv(pro, Ln->w.as<double2>(), Ln->d_out, Ln->d_in, e, nullptr).P;
          pro = part_rows(out, pl, Ln->d_out);
          pro.bias = Ln->b.as<double2>();
          width = (int)Ln->d_out;
        }
        break;
      }
      case K_SOFTMAX: break;
      case K_WAVELET: break;  // a decode step's row passes through (wavelet_discrete_layer.rs:102-128)
    }
  }
  size_t shm = 0;
  for (const ROp& op : ops) {
    shm = std::max(shm, resident_op_lds(op));
    if (ar && op.kind == ROP_GEMV && (op.ro.npart > 8 || op.ro.att.po || op.ro.rope_cs || op.ro.resid))
      rb->poll_ok = false;
  }
  if (shm > RES_MAX_DYN_LDS) return fail(ERR_ARG, "resident decode: %zu bytes of LDS", shm);
  if (rb->tiles <= 0) return fail(ERR_ARG, "resident decode: no vocab product");
  rb->dh = dh_k < 0 ? 0 : dh_k;
  rb->shm = shm;
  return OK;
}

// nsteps decode steps of generate in one launch (the step is what
// enqueue_decode_step enqueues per launch)
static int run_resident(Net* n, const Spec& sp, uint32_t nsteps) {
  const int grid = n->cus;
  // argmax partials: one per row and column block of the vocab product
  size_t am_elems = 0;
  for (uint32_t li = 0; li < n->layers.size(); ++li)
    if (n->layers[li]->kind == K_LINEAR && is_vocab_linear(n, li))
      am_elems = (size_t)sp.B * resident_gemv_plan(sp.B, n->layers[li]->d_out, n->layers[li]->d_in, false, grid).ncb;
  TRY(reserve(n, n->am_v, am_elems * sizeof(double)));
  TRY(reserve(n, n->am_i, am_elems * sizeof(int)));
  // attention-chunk counters, one set per layer, zeroed before every launch (a
  // launch that ran out on a time-out may leave counts behind)
  size_t bh = 0;
  for (auto& L : n->layers)
    if (L->kind == K_SELF_ATTENTION) bh += (size_t)sp.B * ((const SelfAttentionLayer*)L.get())->heads;
  TRY(reserve(n, n->res_cnt, std::max<size_t>(bh, 1) * sizeof(uint32_t)));
  HIP_TRY(hipMemsetAsync(n->res_cnt.p, 0, n->res_cnt.bytes, n->stream));
  if (n->res_flags.bytes < (size_t)grid * sizeof(uint32_t)) {
    TRY(reserve(n, n->res_flags, (size_t)grid * sizeof(uint32_t)));
    HIP_TRY(hipMemsetAsync(n->res_flags.p, 0, n->res_flags.bytes, n->stream));
    n->res_epoch = 0;
  }
  Argmax am = *sp.am;
  am.part_v = n->am_v.as<double>();
  am.part_i = n->am_i.as<int>();
  Spec s2 = sp;
  s2.am = &am;
  const int mr = res_mr(sp.B);
  // the polling exchange: the program once per half of the arena (even and
  // odd steps), if every operation of it polls its inputs
  bool poll = n->res_poll && resident_poll_built(mr) && nsteps > 0;
  ResBuilt rb, rb1;
  size_t half = 0;
  if (poll) {
    TRY(reserve(n, n->res_arena, std::max<size_t>(n->res_arena.bytes, 1 << 20)));
    for (;;) {
      ResArena ar;
      ar.base = (char*)n->res_arena.p;
      TRY(resident_build(n, s2, grid, &rb, &ar));
      half = ar.used;
      if (!rb.poll_ok || 2 * half <= n->res_arena.bytes) break;
      TRY(reserve(n, n->res_arena, 2 * half));  // grown: carve again from the new base
    }
    poll = rb.poll_ok;
  }
  if (poll) {
    std::vector<ROp> even = n->res_ops_h;
    ResArena ar;
    ar.base = (char*)n->res_arena.p + half;
    TRY(resident_build(n, s2, grid, &rb1, &ar));
    if (ar.used != half || n->res_ops_h.size() != even.size()) return fail(ERR_STATE, "resident decode: arena halves");
    n->res_ops_h.insert(n->res_ops_h.begin(), even.begin(), even.end());
  } else {
    TRY(resident_build(n, s2, grid, &rb));
  }
  const int nops = poll ? (int)n->res_ops_h.size() / 2 : (int)n->res_ops_h.size();
  n->res_nops = nops;
  int g2 = 0;
  TRY(launch_rc(resident_grid(n->cus, n->cooperative, mr, rb.dh, rb.shm, &g2, poll), "resident decode (grid)"));
  if (g2 != grid) return fail(ERR_STATE, "resident decode: grid %d != %d", g2, grid);
  const size_t ob = n->res_ops_h.size() * sizeof(ROp);
  TRY(reserve(n, n->res_ops, ob));
  HIP_TRY(hipMemcpyAsync(n->res_ops.p, n->res_ops_h.data(), ob, hipMemcpyHostToDevice, n->stream));
  uint64_t* stamps = nullptr;
  if (n->res_profile) {
    TRY(reserve(n, n->res_stamps, ((size_t)nops * nsteps + 1) * sizeof(uint64_t)));
    stamps = n->res_stamps.as<uint64_t>();
  }
  n->res_steps = nsteps;
  RStep rst;
  rst.B = sp.B;
  rst.part_v = rb.part_v;
  rst.part_i = rb.part_i;
  rst.tiles = rb.tiles;
  rst.ids = am.ids;
  rst.hist = am.hist;
  rst.hist_stride = am.hist_stride;
  rst.hist_cnt = am.hist_cnt;
  rst.kv_len = am.kv_len;
  rst.err = n->err_d.as<uint32_t>();
  if (poll) {
    rst.part_v1 = rb1.part_v;
    rst.part_i1 = rb1.part_i;
    rst.arena = n->res_arena.as<double>();
    rst.arena_half = (long)(half / sizeof(double));
    // every exchanged value starts as the sentinel: both halves of the arena,
    // and the cache rows this launch appends
    HIP_TRY(hipMemsetAsync(n->res_arena.p, 0xFF, 2 * half, n->stream));
    for (auto& L : n->layers)
      if (L->kind == K_SELF_ATTENTION) {
        auto* A = (SelfAttentionLayer*)L.get();
        resident_kv_sentinel(n->stream, A->kc.as<double2>(), A->vc.as<double2>(), sp.B, A->heads, A->max_ctx, A->dh,
                             n->kv_len_d.as<int>(), (int)nsteps);
        HIP_TRY(hipGetLastError());
      }
  }
  n->res_polled = poll;
  TRY(launch_rc(resident_launch(n->stream, n->res_ops.as<ROp>(), nops, (int)nsteps, rst, mr, rb.dh, rb.shm, grid,
                                n->res_flags.as<uint32_t>(), n->res_epoch, n->err_d.as<uint32_t>(), stamps, poll),
                "resident decode"));
  n->res_epoch += resident_barriers(nops, (int)nsteps, poll);
  return OK;
}

// ---------------------------------------------------------------------------
// session helpers
// ---------------------------------------------------------------------------
static int alloc_caches(Net* n, uint32_t B) {
  for (auto& L : n->layers)
    if (L->kind == K_SELF_ATTENTION) {
      auto* A = (SelfAttentionLayer*)L.get();
      size_t bytes = (size_t)B * A->heads * A->max_ctx * A->dh * sizeof(double2);
      TRY(reserve(n, A->kc, bytes));
      TRY(reserve(n, A->vc, bytes));
    }
  return OK;
}

static uint32_t min_ctx(const Net* n) {
  uint32_t m = UINT32_MAX;
  for (auto& L : n->layers)
    if (L->kind == K_SELF_ATTENTION) m = std::min(m, ((SelfAttentionLayer*)L.get())->max_ctx);
  return m;
}

static int check_stack(const Net* n) {
  if (n->layers.size() < 2 || n->layers[0]->kind != K_EMBEDDING || n->layers.back()->kind != K_SOFTMAX ||
      n->layers[n->layers.size() - 2]->kind != K_LINEAR)
    return fail(ERR_STATE, "network must be Embedding ... Linear, Softmax");
  for (size_t i = 1; i + 2 < n->layers.size(); ++i)
    if (n->layers[i]->kind == K_EMBEDDING || n->layers[i]->kind == K_SOFTMAX)
      return fail(ERR_STATE, "Embedding/Softmax only at the ends of the stack");
  return OK;
}

static int ensure_rope_for(Net* n, uint32_t first, uint32_t last, int positions) {
  for (uint32_t li = first; li < last; ++li)
    if (n->layers[li]->kind == K_POSENC) TRY(ensure_rope_table(n, (PositionalEncodingLayer*)n->layers[li].get(), positions));
  return OK;
}

static int rope_positions_needed(const Net* n) {
  uint32_t m = min_ctx(n);
  return (int)std::max<uint32_t>(m == UINT32_MAX ? 512u : m, 512u);
}

// ---------------------------------------------------------------------------
// staging of mitok_greedy_decoding_noalloc, for callers that cannot allocate
// ---------------------------------------------------------------------------
constexpr size_t NOALLOC_MAX_LOGITS = size_t(1) << 20;  // doubles (8 MiB): 32 rows of a 32000-id vocab
constexpr size_t NOALLOC_MAX_ROWS = 4096;
constexpr size_t NOALLOC_BYTES = NOALLOC_MAX_LOGITS * sizeof(double) + NOALLOC_MAX_ROWS * sizeof(uint32_t);
constexpr int NOALLOC_MAX_DEVICES = 64;

// Every GPU the library runs on holds its own copy for the life of the
// process.  In host code this name is not a device address: kernels and
// copies take the per-device address that noalloc_scratch() resolves.
static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch[NOALLOC_MAX_DEVICES] = {};

// The address of `scratch` on `device`, which must be the current device;
// resolved once per device (at network creation) and kept.
static int noalloc_scratch(int device, void** out) {
  if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail(ERR_ARG, "device %d beyond the staging table", device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(ERR_HIP, "hipGetSymbolAddress returned no address");
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return OK;
}

}  // namespace mitok

using namespace mitok;

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int mitok_version(void) { return 1; }

const char* mitok_last_error(void) { return g_err; }

int mitok_device_count(int* count) {
  if (!count) return fail(ERR_ARG, "null count");
  HIP_TRY(hipGetDeviceCount(count));
  return OK;
}

int mitok_network_create(int device, mitok_network** out) {
  if (!out) return fail(ERR_ARG, "null out");
  *out = nullptr;
  int nd = 0;
  HIP_TRY(hipGetDeviceCount(&nd));
  if (device < 0 || device >= nd) return fail(ERR_ARG, "device %d not present (%d devices)", device, nd);
  auto* n = new (std::nothrow) mitok_network();
  if (!n) return fail(ERR_NOMEM, "out of host memory");
  n->device = device;
  int rc = set_device(n);
  if (!rc) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
      rc = fail(ERR_HIP, "hipGetDeviceProperties failed");
    } else {
      n->cus = prop.multiProcessorCount;
      n->cooperative = prop.cooperativeLaunch != 0;
    }
  }
  if (!rc && hipStreamCreateWithFlags(&n->stream, hipStreamNonBlocking) != hipSuccess)
    rc = fail(ERR_HIP, "hipStreamCreate failed");
  if (!rc) rc = noalloc_scratch(device, &n->scratch);
  if (!rc) rc = n->err_d.reserve(sizeof(uint32_t));
  if (!rc) rc = n->sync_cnt.reserve((size_t)SYNC_COUNTERS * sizeof(uint32_t));
  if (!rc) {
    fill_u32(n->stream, n->err_d.as<uint32_t>(), 1, 0);
    fill_u32(n->stream, n->sync_cnt.as<uint32_t>(), SYNC_COUNTERS, 0);
    if (hipStreamSynchronize(n->stream) != hipSuccess) rc = fail(ERR_HIP, "stream sync failed");
  }
  if (rc) {
    mitok_network_destroy(n);
    return rc;
  }
  *out = n;
  return OK;
}

void mitok_network_destroy(mitok_network* n) {
  if (!n) return;
  (void)hipSetDevice(n->device);
  if (n->stream) (void)hipStreamSynchronize(n->stream);
  drop_graph(n);
  collect_timing(n);
  for (hipEvent_t e : n->timing.pool) (void)hipEventDestroy(e);
  n->layers.clear();
  if (n->stream) (void)hipStreamDestroy(n->stream);
  delete n;
}

int mitok_num_layers(const mitok_network* n) { return n ? (int)n->layers.size() : 0; }

static int upload_c(Net* n, DevBuf& b, const double* src, size_t count, double2 dflt, bool has_default) {
  TRY(reserve(n, b, count * sizeof(double2)));
  if (src) HIP_TRY(hipMemcpy(b.p, src, count * sizeof(double2), hipMemcpyHostToDevice));
  else fill_const(n->stream, b.as<double2>(), count, has_default ? dflt : make_double2(0.0, 0.0));
  HIP_TRY(hipStreamSynchronize(n->stream));
  return OK;
}

static int add_layer(Net* n, Layer* L) {
  n->layers.emplace_back(L);
  n->cache_valid = false;
  drop_graph(n);
  return OK;
}

int mitok_add_embedding(mitok_network* n, uint32_t vocab, uint32_t dim, const double* table) {
  if (!n || !vocab || !dim) return fail(ERR_ARG, "embedding: bad arguments");
  TRY(set_device(n));
  auto* L = new EmbeddingLayer();
  L->vocab = vocab;
  L->d_in = L->d_out = dim;
  add_layer(n, L);
  return upload_c(n, L->table, table, (size_t)vocab * dim, {}, false);
}

int mitok_add_positional_encoding(mitok_network* n, uint32_t dim, double base) {
  if (!n || !dim || dim % 2) return fail(ERR_ARG, "positional encoding: dim must be even (positional_encoding_layer.rs:183)");
  TRY(set_device(n));
  auto* L = new PositionalEncodingLayer();
  L->d_in = L->d_out = dim;
  L->base = base;
  return add_layer(n, L);
}

int mitok_add_norm(mitok_network* n, uint32_t dim, double eps, const double* gamma, const double* beta) {
  if (!n || !dim) return fail(ERR_ARG, "norm: bad arguments");
  if (dim > 1024) return fail(ERR_ARG, "norm: dim %u > 1024 unsupported", dim);
  TRY(set_device(n));
  auto* L = new NormLayer();
  L->d_in = L->d_out = dim;
  L->eps = eps;
  add_layer(n, L);
  TRY(upload_c(n, L->gamma, gamma, dim, make_double2(1.0, 0.0), true));
  return upload_c(n, L->beta, beta, dim, make_double2(0.0, 0.0), true);
}

int mitok_add_self_attention(mitok_network* n, uint32_t heads, uint32_t dim, uint32_t max_ctx, double eps,
                             const double* wq, const double* wk, const double* wv, const double* bias_pos,
                             const double* gamma, const double* beta) {
  if (!n || !heads || !dim || dim % heads || !max_ctx) return fail(ERR_ARG, "self-attention: bad arguments");
  const uint32_t dh = dim / heads;
  if (dh > 256) return fail(ERR_ARG, "self-attention: head dim %u > 256 unsupported", dh);
  if (dim > 1024) return fail(ERR_ARG, "self-attention: dim %u > 1024 unsupported", dim);
  if (max_ctx > 6144) return fail(ERR_ARG, "self-attention: max_ctx %u > 6144 unsupported", max_ctx);
  TRY(set_device(n));
  auto* L = new SelfAttentionLayer();
  L->heads = heads;
  L->d_in = L->d_out = dim;
  L->dh = dh;
  L->max_ctx = max_ctx;
  L->eps = eps;
  add_layer(n, L);
  const size_t d = dim;
  TRY(reserve(n, L->wqkv, d * 3 * d * sizeof(double2)));
  fill_const(n->stream, L->wqkv.as<double2>(), d * 3 * d, make_double2(0.0, 0.0));
  HIP_TRY(hipStreamSynchronize(n->stream));
  const double* srcs[3] = {wq, wk, wv};
  for (int p = 0; p < 3; ++p) {
    if (!srcs[p]) continue;
    // [h][d][dh] -> columns p*d + h*dh of [d][3d]
    std::vector<double2> packed(d * 3 * d);
    HIP_TRY(hipMemcpy(packed.data(), L->wqkv.p, packed.size() * sizeof(double2), hipMemcpyDeviceToHost));
    const double2* s = (const double2*)srcs[p];
    for (uint32_t h = 0; h < heads; ++h)
      for (size_t r = 0; r < d; ++r)
        for (uint32_t e = 0; e < dh; ++e) packed[r * 3 * d + p * d + h * dh + e] = s[((size_t)h * d + r) * dh + e];
    HIP_TRY(hipMemcpy(L->wqkv.p, packed.data(), packed.size() * sizeof(double2), hipMemcpyHostToDevice));
  }
  const size_t bn = (size_t)heads * max_ctx * max_ctx;
  TRY(reserve(n, L->bias_re, bn * sizeof(double)));
  if (bias_pos) {
    std::vector<double> re(bn);
    for (size_t i = 0; i < bn; ++i) re[i] = bias_pos[2 * i];
    HIP_TRY(hipMemcpy(L->bias_re.p, re.data(), bn * sizeof(double), hipMemcpyHostToDevice));
  } else {
    HIP_TRY(hipMemset(L->bias_re.p, 0, bn * sizeof(double)));
  }
  TRY(upload_c(n, L->gamma, gamma, dim, make_double2(1.0, 0.0), true));
  return upload_c(n, L->beta, beta, dim, make_double2(0.0, 0.0), true);
}

int mitok_add_feed_forward(mitok_network* n, uint32_t dim, uint32_t hidden, const double* w1, const double* b1,
                           const double* w2, const double* b2) {
  if (!n || !dim || !hidden) return fail(ERR_ARG, "feed-forward: bad arguments");
  TRY(set_device(n));
  auto* L = new FeedForwardLayer();
  L->d_in = L->d_out = dim;
  L->hidden = hidden;
  add_layer(n, L);
  TRY(upload_c(n, L->w1, w1, (size_t)dim * hidden, {}, false));
  TRY(upload_c(n, L->b1, b1, hidden, make_double2(1.0, 0.0), true));
  TRY(upload_c(n, L->w2, w2, (size_t)hidden * dim, {}, false));
  return upload_c(n, L->b2, b2, dim, make_double2(1.0, 0.0), true);
}

int mitok_add_linear(mitok_network* n, uint32_t in, uint32_t out, const double* w, const double* b) {
  if (!n || !in || !out) return fail(ERR_ARG, "linear: bad arguments");
  TRY(set_device(n));
  auto* L = new LinearLayer();
  L->d_in = in;
  L->d_out = out;
  add_layer(n, L);
  TRY(upload_c(n, L->w, w, (size_t)in * out, {}, false));
  return upload_c(n, L->b, b, out, make_double2(1.0, 0.0), true);
}

int mitok_add_discrete_wavelet(mitok_network* n, uint32_t dim, uint32_t wavelet, uint32_t mode, int is_full_mode) {
  if (!n || !dim) return fail(ERR_ARG, "bad arguments");
  if (is_full_mode) return fail(ERR_ARG, "DiscreteWaveletLayer in full mode (2-D) is not on the device path");
  auto L = std::make_unique<WaveletLayer>();
  if (!wavelet_low_pass(wavelet, L->lo, &L->L))
    return fail(ERR_ARG, "wavelet type %u: only DB1 and DB2 are on the device path", wavelet);
  if (!wavelet_mode_ok(mode)) return fail(ERR_ARG, "wavelet mode %u is not on the device path", mode);
  // one cached length per sequence: every attention layer's cache holds the
  // compressed rows, so compression happens before the first attention layer
  for (auto& P : n->layers)
    if (P->kind == K_SELF_ATTENTION)
      return fail(ERR_ARG, "DiscreteWaveletLayer after a SelfAttentionLayer is not on the device path");
  L->wavelet = wavelet;
  L->mode = mode;
  L->d_in = L->d_out = dim;
  n->pos_off = true;  // decode steps after a compressed prompt shift their RoPE positions
  TRY(set_device(n));
  TRY(reserve(n, n->pos_off_d, 64 * sizeof(int)));
  fill_int(n->stream, n->pos_off_d.as<int>(), 64, 0);
  HIP_TRY(hipStreamSynchronize(n->stream));
  return add_layer(n, L.release());
}

int mitok_seq_out_len(const mitok_network* n, uint32_t first, uint32_t last, uint32_t seq, uint32_t* out) {
  if (!n || !out || first > last || last > n->layers.size()) return fail(ERR_ARG, "bad layer range");
  int S = (int)seq;
  for (uint32_t li = first; li < last; ++li)
    if (n->layers[li]->kind == K_WAVELET) S = wavelet_rows(S, ((const WaveletLayer*)n->layers[li].get())->L);
  *out = (uint32_t)S;
  return OK;
}

int mitok_add_softmax(mitok_network* n, int operation_mode) {
  if (!n) return fail(ERR_ARG, "null network");
  if (operation_mode != MITOK_TRAINING && operation_mode != MITOK_PRODUCTION) return fail(ERR_ARG, "bad operation mode");
  auto* L = new SoftmaxLayer();
  L->mode = operation_mode;
  return add_layer(n, L);
}

int mitok_init_seeded(mitok_network* n, uint64_t seed) {
  if (!n) return fail(ERR_ARG, "null network");
  TRY(set_device(n));
  hipStream_t st = n->stream;
  auto lim = [](uint64_t r, uint64_t c) { return sqrt(6.0 / (double)(r + c)); };
  for (uint32_t li = 0; li < n->layers.size(); ++li) {
    Layer* L = n->layers[li].get();
    switch (L->kind) {
      case K_EMBEDDING: {
        auto* E = (EmbeddingLayer*)L;
        fill_seeded(st, E->table.as<double2>(), E->vocab, E->d_out, E->d_out, stream_key(seed, stream_id(li, 0)),
                    lim(E->vocab, E->d_out));
        break;
      }
      case K_NORM: {
        auto* N = (NormLayer*)L;
        fill_const(st, N->gamma.as<double2>(), N->d_in, make_double2(1.0, 0.0));
        fill_const(st, N->beta.as<double2>(), N->d_in, make_double2(0.0, 0.0));
        break;
      }
      case K_SELF_ATTENTION: {
        auto* A = (SelfAttentionLayer*)L;
        const long d = A->d_in;
        for (uint32_t h = 0; h < A->heads; ++h) {
          for (int p = 0; p < 3; ++p)
            fill_seeded(st, A->wqkv.as<double2>() + p * d + (long)h * A->dh, (int)d, A->dh, 3 * d,
                        stream_key(seed, stream_id(li, 1 + p + 4 * h)), lim(d, A->dh));
          fill_seeded_re(st, A->bias_re.as<double>() + (size_t)h * A->max_ctx * A->max_ctx, A->max_ctx, A->max_ctx,
                         A->max_ctx, stream_key(seed, stream_id(li, 4 + 4 * h)), lim(A->max_ctx, A->max_ctx));
        }
        fill_const(st, A->gamma.as<double2>(), A->d_in, make_double2(1.0, 0.0));
        fill_const(st, A->beta.as<double2>(), A->d_in, make_double2(0.0, 0.0));
        break;
      }
      case K_FEED_FORWARD: {
        auto* F = (FeedForwardLayer*)L;
        fill_seeded(st, F->w1.as<double2>(), F->d_in, F->hidden, F->hidden, stream_key(seed, stream_id(li, 1)),
                    lim(F->d_in, F->hidden));
        fill_seeded(st, F->w2.as<double2>(), F->hidden, F->d_out, F->d_out, stream_key(seed, stream_id(li, 2)),
                    lim(F->hidden, F->d_out));
        fill_const(st, F->b1.as<double2>(), F->hidden, make_double2(1.0, 0.0));
        fill_const(st, F->b2.as<double2>(), F->d_out, make_double2(1.0, 0.0));
        break;
      }
      case K_LINEAR: {
        auto* Ln = (LinearLayer*)L;
        fill_seeded(st, Ln->w.as<double2>(), Ln->d_in, Ln->d_out, Ln->d_out, stream_key(seed, stream_id(li, 1)),
                    lim(Ln->d_in, Ln->d_out));
        fill_const(st, Ln->b.as<double2>(), Ln->d_out, make_double2(1.0, 0.0));
        break;
      }
      default: break;
    }
  }
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(st));
  n->cache_valid = false;
  return OK;
}

int mitok_init_embedding_wavelet(mitok_network* n, uint32_t layer, uint64_t seed, uint32_t src_dim) {
  if (!n) return fail(ERR_ARG, "null network");
  if (layer >= n->layers.size() || n->layers[layer]->kind != K_EMBEDDING)
    return fail(ERR_ARG, "layer %u is not an Embedding", layer);
  auto* E = (EmbeddingLayer*)n->layers[layer].get();
  const int dim = embedding_wavelet_dim((int)src_dim);
  if (dim == 0) return fail(ERR_ARG, "a draw of %u values: a power of two from 2 to %d", src_dim, EW_MAX_SRC);
  if ((uint32_t)dim != E->d_out)
    return fail(ERR_ARG, "a %u-value draw decomposes to %d values, the layer's dim is %u", src_dim, dim, E->d_out);
  TRY(set_device(n));
  DevBuf kern;
  TRY(kern.reserve(64 * sizeof(double2)));
  const int rc = embedding_wavelet_init(n->stream, E->table.as<double2>(), (int)E->vocab, dim, (int)src_dim,
                                        stream_key(seed, stream_id(layer, 0xFFF)), kern.as<double2>(), 64);
  if (rc == ERR_HIP) return fail(ERR_HIP, "embedding wavelet init: %s", hipGetErrorString(hipGetLastError()));
  if (rc) return fail(rc, "embedding wavelet init: the CMOR integral");
  n->cache_valid = false;
  return check_err_word(n);
}

int mitok_get_tensor(mitok_network* n, uint32_t layer, uint32_t slot, double* out, uint64_t count) {
  if (!n || !out || layer >= n->layers.size()) return fail(ERR_ARG, "bad layer index");
  TRY(set_device(n));
  HIP_TRY(hipStreamSynchronize(n->stream));
  Layer* L = n->layers[layer].get();
  auto copy = [&](const DevBuf& b, uint64_t len, size_t elem) -> int {
    if (count != len) return fail(ERR_ARG, "tensor size %llu != %llu", (unsigned long long)count, (unsigned long long)len);
    HIP_TRY(hipMemcpy(out, b.p, len * elem, hipMemcpyDeviceToHost));
    return OK;
  };
  switch (L->kind) {
    case K_EMBEDDING:
      if (slot == 0) return copy(((EmbeddingLayer*)L)->table, (uint64_t)((EmbeddingLayer*)L)->vocab * L->d_out, 16);
      break;
    case K_NORM:
      if (slot == 6) return copy(((NormLayer*)L)->gamma, L->d_in, 16);
      if (slot == 7) return copy(((NormLayer*)L)->beta, L->d_in, 16);
      break;
    case K_SELF_ATTENTION: {
      auto* A = (SelfAttentionLayer*)L;
      if (slot <= 2) {
        const size_t d = A->d_in;
        if (count != (uint64_t)A->heads * d * A->dh) return fail(ERR_ARG, "tensor size mismatch");
        std::vector<double2> packed(d * 3 * d);
        HIP_TRY(hipMemcpy(packed.data(), A->wqkv.p, packed.size() * sizeof(double2), hipMemcpyDeviceToHost));
        double2* o = (double2*)out;
        for (uint32_t h = 0; h < A->heads; ++h)
          for (size_t r = 0; r < d; ++r)
            for (uint32_t e = 0; e < A->dh; ++e) o[((size_t)h * d + r) * A->dh + e] = packed[r * 3 * d + slot * d + h * A->dh + e];
        return OK;
      }
      if (slot == 3) return copy(A->bias_re, (uint64_t)A->heads * A->max_ctx * A->max_ctx, 8);
      if (slot == 6) return copy(A->gamma, A->d_in, 16);
      if (slot == 7) return copy(A->beta, A->d_in, 16);
      break;
    }
    case K_FEED_FORWARD: {
      auto* F = (FeedForwardLayer*)L;
      if (slot == 0) return copy(F->w1, (uint64_t)F->d_in * F->hidden, 16);
      if (slot == 1) return copy(F->w2, (uint64_t)F->hidden * F->d_out, 16);
      if (slot == 4) return copy(F->b1, F->hidden, 16);
      if (slot == 5) return copy(F->b2, F->d_out, 16);
      break;
    }
    case K_LINEAR: {
      auto* Ln = (LinearLayer*)L;
      if (slot == 0) return copy(Ln->w, (uint64_t)Ln->d_in * Ln->d_out, 16);
      if (slot == 4) return copy(Ln->b, Ln->d_out, 16);
      break;
    }
  }
  return fail(ERR_ARG, "layer %u has no tensor in slot %u", layer, slot);
}

int mitok_reset(mitok_network* n) {
  if (!n) return fail(ERR_ARG, "null network");
  n->cache_valid = false;
  n->cache_B = 0;
  n->kv_len_h.clear();
  return OK;
}

static int validate_batch(const uint32_t* lens, uint32_t B, uint32_t S) {
  if (!B || !S) return fail(ERR_ARG, "batch_ids is empty (transformer_network.rs:198-208)");
  for (uint32_t b = 0; b < B; ++b)
    if (!lens[b] || lens[b] > S) return fail(ERR_ARG, "lens[%u]=%u outside [1, %u]", b, lens[b], S);
  return OK;
}

// Host-side part of a predict/forward call: mode, bounds, uploads.
// Host-side part of a predict/forward call: mode, bounds, uploads, and the
// wavelet stages of a prompt or stateless pass.  mask_src: the caller's
// padding mask [B][S] (forward_layers), or null for lens' prefixes.
static int begin_call(Net* n, const uint32_t* lens, uint32_t B, uint32_t S, const uint32_t* ts, bool forward_only,
                      const uint32_t* mask_src, Spec& sp, std::vector<uint32_t>& mask_h) {
  n->head_valid = false;
  sp.B = B;
  sp.S = S;
  sp.forward_only = forward_only;
  const uint32_t mc = min_ctx(n);
  if (forward_only && n->cache_valid) {
    if (B != n->cache_B) return fail(ERR_STATE, "cached batch %u != %u; reset first", n->cache_B, B);
    for (uint32_t b = 0; b < B; ++b)
      if (n->kv_len_h[b] + 1 > mc) return fail(ERR_ARG, "context %u exceeds max context %u", n->kv_len_h[b] + 1, mc);
    sp.mode = MODE_CACHED;
  } else if (forward_only) {
    sp.mode = MODE_PREFILL;
  } else {
    sp.mode = MODE_STATELESS;
  }
  // wavelet layers compress the rows of a stateless pass or one at time step 0
  // (wavelet_discrete_layer.rs:102-128: !forward_only || time_step == 0); a
  // later cached step passes its row through
  std::vector<const WaveletLayer*> wl;
  if (!forward_only || !ts || ts[0] == 0)
    for (uint32_t li = sp.first; li < sp.last; ++li)
      if (n->layers[li]->kind == K_WAVELET) wl.push_back((const WaveletLayer*)n->layers[li].get());
  // a stateless pass with target rows compresses only each sequence's first
  // S - T rows and passes the T targets on (wavelet_discrete_layer.rs:102-134)
  const int T = (!forward_only && !wl.empty()) ? (int)n->train_T : 0;
  if (T) {
    if ((uint32_t)T >= S) return fail(ERR_ARG, "%d target rows need more than %u rows", T, S);
    for (uint32_t b = 0; b < B; ++b)
      if (lens[b] != S || mask_src)
        return fail(ERR_ARG, "target rows need unpadded sequences: separate_input_target "
                             "(wavelet_discrete_layer.rs:233-279) panics on padded ones");
  }
  int S_alloc = (int)S, Sc = (int)S;
  for (const WaveletLayer* W : wl) {
    Sc = T ? wavelet_rows(Sc - T, W->L) + T : wavelet_rows(Sc, W->L);
    if (T && Sc - T < 1) return fail(ERR_ARG, "%d target rows leave no input rows to compress", T);
    S_alloc = std::max(S_alloc, Sc);
  }
  if (mc != UINT32_MAX && (uint32_t)Sc > mc) return fail(ERR_ARG, "sequence %d exceeds max context %u", Sc, mc);
  Spec sz = sp;
  sz.S = S_alloc;
  TRY(prepare(n, sz));
  if (sp.mode == MODE_PREFILL) TRY(alloc_caches(n, B));
  const size_t rows = (size_t)B * S;
  mask_h.assign(rows, 0);
  std::vector<int> pos(rows);
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) {
      mask_h[(size_t)b * S + s] = mask_src ? (mask_src[(size_t)b * S + s] ? 1u : 0u) : (s < lens[b] ? 1u : 0u);
      uint32_t t = ts ? ts[b] : 0;
      pos[(size_t)b * S + s] = (forward_only && t > 0) ? (int)t : (int)s;  // positional_encoding_layer.rs:61-65
    }
  int maxpos = std::max(0, S_alloc - 1);
  for (int p : pos) maxpos = std::max(maxpos, p);
  TRY(ensure_rope_for(n, sp.first, sp.last, std::max(rope_positions_needed(n), maxpos + 1)));
  TRY(upload(n, n->mask_d, mask_h.data(), rows * sizeof(uint32_t)));
  TRY(upload(n, n->lens_d, lens, B * sizeof(uint32_t)));
  TRY(upload(n, n->pos_d, pos.data(), rows * sizeof(int)));
  sp.mask = n->mask_d.as<uint32_t>();
  sp.lens = n->lens_d.as<uint32_t>();
  sp.pos = n->pos_d.as<int>();

  // each stage: tap table, filter, compressed mask (the low half of dwt_1d of
  // the 0/1 mask above 0.99, compress_padding_mask :297-313), the rows left
  // to each sequence (the mask's ones) and row positions 0 .. S2-1
  n->wstages.clear();
  std::vector<std::vector<int>> keep_i;  // host staging kept alive until the synchronisation below
  std::vector<std::vector<double>> keep_d;
  std::vector<std::vector<uint32_t>> keep_u;
  std::vector<uint32_t> m = mask_h, ln(lens, lens + B);
  int Sin = (int)S;
  const uint32_t* mask_prev = n->mask_d.as<uint32_t>();
  for (const WaveletLayer* W : wl) {
    WaveletTaps t = wavelet_taps(Sin - T, W->L, W->mode);
    const int M = t.S2, S2 = M + T, L = W->L;
    for (int j = 0; j < T; ++j) {  // target rows: a copy of input row Sin - T + j (src -2 - row)
      t.src.push_back(-2 - (Sin - T + j));
      t.sgn.push_back(1.0);
      for (int l = 1; l < L; ++l) {
        t.src.push_back(-1);
        t.sgn.push_back(0.0);
      }
    }
    std::vector<uint32_t> m2((size_t)B * S2), ln2(B);
    std::vector<int> p2((size_t)B * S2);
    for (uint32_t b = 0; b < B; ++b) {
      uint32_t ones = 0;
      for (int j = 0; j < S2; ++j) {
        double v = 0.0;
        for (int l = 0; l < L && j < M; ++l) {
          const int sidx = t.src[(size_t)j * L + l];
          const double x = sidx < 0 ? 0.0 : t.sgn[(size_t)j * L + l] * (double)m[(size_t)b * Sin + sidx];
          v = v + x * W->lo[l];
        }
        m2[(size_t)b * S2 + j] = (j >= M || v > 0.99) ? 1u : 0u;  // target rows: mask 1 (:130-134)
        ones += m2[(size_t)b * S2 + j];
        p2[(size_t)b * S2 + j] = j;
      }
      ln2[b] = ones ? ones : 1u;
    }
    auto st = std::make_unique<Net::WaveletStage>();
    st->S_in = Sin;
    st->S2 = S2;
    st->L = L;
    st->T = T;
    st->mask_in = mask_prev;
    for (int l = 0; l < L; ++l) st->lo[l] = W->lo[l];
    keep_i.push_back(t.src);
    keep_d.push_back(t.sgn);
    keep_d.push_back(std::vector<double>(W->lo, W->lo + L));
    TRY(upload(n, st->src, keep_i.back().data(), keep_i.back().size() * sizeof(int)));
    TRY(upload(n, st->sgn, keep_d[keep_d.size() - 2].data(), t.sgn.size() * sizeof(double)));
    TRY(upload(n, st->lo_d, keep_d.back().data(), (size_t)L * sizeof(double)));
    keep_u.push_back(m2);
    TRY(upload(n, st->mask, keep_u.back().data(), m2.size() * sizeof(uint32_t)));
    keep_u.push_back(ln2);
    TRY(upload(n, st->lens, keep_u.back().data(), (size_t)B * sizeof(uint32_t)));
    keep_i.push_back(p2);
    TRY(upload(n, st->pos, keep_i.back().data(), p2.size() * sizeof(int)));
    mask_prev = st->mask.as<uint32_t>();
    n->wstages.push_back(std::move(st));
    m = std::move(m2);
    ln = std::move(ln2);
    Sin = S2;
  }
  n->wS = Sin;
  n->wmask_h = m;
  n->wlens_h = ln;
  sp.compress = !wl.empty();
  if (n->pos_off && sp.mode == MODE_PREFILL) {
    // decode positions count the uncompressed prompt: offset = prompt length - cached rows
    std::vector<int> off(B);
    for (uint32_t b = 0; b < B; ++b) off[b] = (int)lens[b] - (int)ln[b];
    keep_i.push_back(off);
    TRY(upload(n, n->pos_off_d, keep_i.back().data(), (size_t)B * sizeof(int)));
  }
  if (sp.mode == MODE_CACHED) {
    n->dec_tsum = 0.0;
    for (uint32_t b = 0; b < B; ++b) n->dec_tsum += (double)n->kv_len_h[b] + 1;
    std::vector<int> kv(n->kv_len_h.begin(), n->kv_len_h.end());
    TRY(upload(n, n->kv_len_d, kv.data(), B * sizeof(int)));
    if (n->wS > 1) {  // rows per sequence after any compression
      std::vector<int> kr(B);
      for (uint32_t b = 0; b < B; ++b) kr[b] = (int)ln[b] - 1;  // the last token (masked_attention_head.rs:141-153)
      TRY(upload(n, n->kv_row_d, kr.data(), B * sizeof(int)));
      sp.kv_row = n->kv_row_d.as<int>();
    }
    HIP_TRY(hipStreamSynchronize(n->stream));  // kv, kr go out of scope
  }
  HIP_TRY(hipStreamSynchronize(n->stream));  // the host staging vectors above go out of scope
  return OK;
}

// rows each sequence keeps in the cache after a prompt pass (compressed by
// the wavelet stages, if any)
static const uint32_t* cached_lens(const Net* n, const uint32_t* lens) {
  return n->wstages.empty() ? lens : n->wlens_h.data();
}

static void end_call(Net* n, const Spec& sp, const uint32_t* lens) {
  if (sp.mode == MODE_PREFILL) {
    n->cache_valid = true;
    n->cache_B = sp.B;
    const uint32_t* cl = cached_lens(n, lens);
    n->kv_len_h.assign(cl, cl + sp.B);  // the cache keeps each sequence's own rows
  } else if (sp.mode == MODE_CACHED) {
    for (uint32_t b = 0; b < (uint32_t)sp.B; ++b) n->kv_len_h[b] += 1;
  }
}

// out may be null only for a stateless pass of every row (mitok_predict_targets
// without out_probs): the softmax output then stays on the device
static int predict_impl(mitok_network* n, const uint32_t* ids, const uint32_t* lens, uint32_t B, uint32_t S,
                        const uint32_t* time_steps, int forward_only, int last_row_only, double* out,
                        uint32_t* out_mask) {
  if (!n || !ids || !lens || (!out && (forward_only || last_row_only))) return fail(ERR_ARG, "null argument");
  TRY(validate_batch(lens, B, S));
  TRY(check_stack(n));
  TRY(set_device(n));
  Spec sp;
  sp.first = 0;
  sp.last = (uint32_t)n->layers.size();
  sp.last_row = last_row_only && forward_only;
  std::vector<uint32_t> mask_h;
  TRY(begin_call(n, lens, B, S, time_steps, forward_only != 0, nullptr, sp, mask_h));
  const size_t rows = (size_t)B * S;
  const size_t orows = (size_t)B * n->wS;  // output rows (a wavelet layer compresses a prompt pass)
  std::vector<uint32_t> padded(rows);
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) padded[(size_t)b * S + s] = s < lens[b] ? ids[(size_t)b * S + s] : 1u;
  TRY(upload(n, n->ids_d, padded.data(), rows * sizeof(uint32_t)));
  sp.ids = n->ids_d.as<uint32_t>();
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out;
  sp.out_re = n->logits_re.as<double>();
  sp.out_prob = n->probs.as<double>();
  TRY(enqueue_step(n, sp));
  if (forward_only) {
    size_t cnt = (sp.last_row ? (size_t)B : orows) * V;
    HIP_TRY(hipMemcpyAsync(out, sp.out_re, cnt * sizeof(double), hipMemcpyDeviceToHost, n->stream));
    HIP_TRY(hipStreamSynchronize(n->stream));
  } else if (!last_row_only) {  // every row: straight into the caller's buffer
    if (out) HIP_TRY(hipMemcpyAsync(out, sp.out_prob, orows * V * sizeof(double), hipMemcpyDeviceToHost, n->stream));
    HIP_TRY(hipStreamSynchronize(n->stream));
  } else {
    std::vector<double> all(orows * V);
    HIP_TRY(hipMemcpyAsync(all.data(), sp.out_prob, all.size() * sizeof(double), hipMemcpyDeviceToHost, n->stream));
    HIP_TRY(hipStreamSynchronize(n->stream));
    const uint32_t* ol = cached_lens(n, lens);
    for (uint32_t b = 0; b < B; ++b)
      memcpy(out + (size_t)b * V, all.data() + ((size_t)b * n->wS + ol[b] - 1) * V, V * sizeof(double));
  }
  collect_timing(n);
  TRY(check_err_word(n));
  end_call(n, sp, lens);
  if (out_mask) memcpy(out_mask, n->wstages.empty() ? mask_h.data() : n->wmask_h.data(), orows * sizeof(uint32_t));
  return OK;
}

int mitok_predict(mitok_network* n, const uint32_t* ids, const uint32_t* lens, uint32_t B, uint32_t S,
                  const uint32_t* time_steps, int forward_only, int last_row_only, double* out, uint32_t* out_mask) {
  if (!out) return fail(ERR_ARG, "null argument");
  return predict_impl(n, ids, lens, B, S, time_steps, forward_only, last_row_only, out, out_mask);
}

int mitok_predict_targets(mitok_network* n, const uint32_t* ids, const uint32_t* lens, uint32_t B, uint32_t S,
                          uint32_t target_rows, double* out_probs, uint32_t* out_mask) {
  if (!n) return fail(ERR_ARG, "null network");
  n->train_T = target_rows;
  const int rc = predict_impl(n, ids, lens, B, S, nullptr, 0, 0, out_probs, out_mask);
  n->train_T = 0;
  return rc;
}

int mitok_cross_entropy_loss(mitok_network* n, const uint32_t* targets, const uint32_t* tlens, uint32_t B, uint32_t T,
                             double* out_loss) {
  if (!n || !targets || !tlens || !B || !T || !out_loss) return fail(ERR_ARG, "bad arguments");
  if (!n->head_valid) return fail(ERR_STATE, "no stateless (forward_only = 0) predict whose output to score");
  if (B != n->head_B) return fail(ERR_ARG, "batch %u != the forward pass's %u", B, n->head_B);
  if (T > (uint32_t)CE_MAX_T) return fail(ERR_ARG, "%u targets per sequence: at most %d", T, CE_MAX_T);
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out, S = n->head_S;
  // what cross_entropy_loss (transformer_network.rs:674-711) would panic on
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t tl = tlens[b];
    if (tl > T) return fail(ERR_ARG, "target length %u > %u", tl, T);
    if ((uint64_t)tl + 1 > (uint64_t)S) return fail(ERR_ARG, "sequence %u: %u targets need more than %u rows", b, tl, S);
    for (uint32_t t = 0; t < tl; ++t) {
      const uint32_t tc = targets[(size_t)b * T + t];
      if (tc != 1u && tc >= V) return fail(ERR_ARG, "target token %u exceeds vocabulary %u", tc, V);
    }
  }
  TRY(set_device(n));
  const size_t tb = ((size_t)B * T + B) * sizeof(uint32_t), tb8 = (tb + 7) & ~(size_t)7;
  TRY(n->ce_buf.reserve(tb8 + ((size_t)B + 2) * sizeof(double)));  // no graph holds it
  char* base = (char*)n->ce_buf.p;
  uint32_t* tgt_d = (uint32_t*)base;
  uint32_t* tlen_d = tgt_d + (size_t)B * T;
  double* part = (double*)(base + tb8);
  HIP_TRY(hipMemcpyAsync(tgt_d, targets, (size_t)B * T * sizeof(uint32_t), hipMemcpyHostToDevice, n->stream));
  HIP_TRY(hipMemcpyAsync(tlen_d, tlens, (size_t)B * sizeof(uint32_t), hipMemcpyHostToDevice, n->stream));
  cross_entropy(n->stream, n->probs.as<double>(), (int)B, (int)S, (int)V, tgt_d, tlen_d, (int)T, part, part + B);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipMemcpyAsync(out_loss, part + B, 2 * sizeof(double), hipMemcpyDeviceToHost, n->stream));
  HIP_TRY(hipStreamSynchronize(n->stream));
  return OK;
}

// `bytes` of device memory at `p` inside one allocation of the network's
// device: the check that turns a caller's wrong device pointer into an error
// instead of a memory fault.
static int check_device_range(const Net* n, const void* p, size_t bytes, const char* what) {
  hipPointerAttribute_t at;
  if (hipPointerGetAttributes(&at, p) != hipSuccess || at.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    return fail(ERR_ARG, "%s is not device memory", what);
  }
  if (at.device != n->device) return fail(ERR_ARG, "%s is on device %d, the network on %d", what, at.device, n->device);
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return fail(ERR_ARG, "%s: no device allocation holds it", what);
  }
  const size_t off = (size_t)((const char*)p - (const char*)base);
  if (off > size || bytes > size - off)
    return fail(ERR_ARG, "%s: %zu bytes from offset %zu exceed its allocation of %zu", what, bytes, off, size);
  return OK;
}

static int forward_layers_impl(Net* n, uint32_t first, uint32_t last, const double* in, const uint32_t* mask_in,
                               uint32_t B, uint32_t S, const uint32_t* time_steps, int forward_only, double* out,
                               bool on_device) {
  if (!n || !in || !out || first >= last || last > n->layers.size()) return fail(ERR_ARG, "bad layer range");
  if (!B || !S) return fail(ERR_ARG, "empty batch");
  for (uint32_t li = first; li < last; ++li) {
    int k = n->layers[li]->kind;
    if (k == K_EMBEDDING || k == K_SOFTMAX) return fail(ERR_ARG, "layer %u is not a hidden-state layer", li);
  }
  TRY(set_device(n));
  std::vector<uint32_t> lens(B);
  for (uint32_t b = 0; b < B; ++b) {
    uint32_t c = 0;
    for (uint32_t s = 0; s < S; ++s) c += (mask_in ? mask_in[(size_t)b * S + s] : 1) ? 1 : 0;
    lens[b] = c ? c : 1;
  }
  const uint32_t din = n->layers[first]->d_in, dout = n->layers[last - 1]->d_out;
  const size_t rows = (size_t)B * S;
  if (on_device) {
    uint32_t so = 0;
    TRY(mitok_seq_out_len(n, first, last, S, &so));
    TRY(check_device_range(n, in, rows * din * sizeof(double2), "in"));
    TRY(check_device_range(n, out, (size_t)B * so * dout * sizeof(double2), "out"));
  }
  Spec sp;
  sp.first = first;
  sp.last = last;
  std::vector<uint32_t> mask_h;
  TRY(begin_call(n, lens.data(), B, S, time_steps, forward_only != 0, mask_in, sp, mask_h));
  const size_t orows = (size_t)B * n->wS;
  DevBuf xin, xout;
  if (on_device) {
    sp.in = (const double2*)in;
    sp.out_hidden = (double2*)out;
  } else {
    TRY(xin.reserve(rows * din * sizeof(double2)));
    TRY(xout.reserve(orows * dout * sizeof(double2)));
    HIP_TRY(hipMemcpyAsync(xin.p, in, rows * din * sizeof(double2), hipMemcpyHostToDevice, n->stream));
    sp.in = xin.as<double2>();
    sp.out_hidden = xout.as<double2>();
  }
  TRY(enqueue_forward(n, sp));
  if (!on_device)
    HIP_TRY(hipMemcpyAsync(out, xout.p, orows * dout * sizeof(double2), hipMemcpyDeviceToHost, n->stream));
  HIP_TRY(hipStreamSynchronize(n->stream));
  collect_timing(n);
  TRY(check_err_word(n));
  end_call(n, sp, lens.data());
  return OK;
}

int mitok_forward_layers(mitok_network* n, uint32_t first, uint32_t last, const double* in, const uint32_t* mask_in,
                         uint32_t B, uint32_t S, const uint32_t* time_steps, int forward_only, double* out) {
  return forward_layers_impl(n, first, last, in, mask_in, B, S, time_steps, forward_only, out, false);
}

int mitok_forward_layers_device(mitok_network* n, uint32_t first, uint32_t last, const double* d_in,
                                const uint32_t* mask_in, uint32_t B, uint32_t S, const uint32_t* time_steps,
                                int forward_only, double* d_out) {
  return forward_layers_impl(n, first, last, d_in, mask_in, B, S, time_steps, forward_only, d_out, true);
}

// One decode step for every sequence: embed the previous greedy ids, run the
// stack with the cache, vocab Re-logits (+history) and the greedy ids fused
// into the vocab product, which also appends to the id history and advances
// every sequence's KV length.
static int enqueue_decode_step(Net* n, Spec sp, bool want_logits, uint32_t hist_stride) {
  Argmax am;
  am.part_v = n->am_v.as<double>();
  am.part_i = n->am_i.as<int>();
  am.ids = n->dec_ids_d.as<uint32_t>();
  am.hist = n->hist_d.as<uint32_t>();
  am.hist_stride = (int)hist_stride;
  am.hist_cnt = n->cnt_d.as<int>();
  am.kv_len = n->kv_len_d.as<int>();
  am.advance_kv = 1;
  am.err = n->err_d.as<uint32_t>();
  sp.am = &am;
  sp.hist_re = want_logits ? n->logit_hist_d.as<double>() : nullptr;
  sp.hist_cnt = n->cnt_d.as<int>();
  return enqueue_step(n, sp);
}

// The three events of a token-loop call (start, prompt done, decode done),
// destroyed on every return path.
struct CallEvents {
  hipEvent_t e[3] = {nullptr, nullptr, nullptr};
  CallEvents() = default;
  CallEvents(const CallEvents&) = delete;
  CallEvents& operator=(const CallEvents&) = delete;
  ~CallEvents() {
    for (hipEvent_t x : e)
      if (x) (void)hipEventDestroy(x);
  }
  int create() {
    for (hipEvent_t& x : e) HIP_TRY(hipEventCreate(&x));
    return OK;
  }
};

// The decode-step shape of a token-loop call on B sequences.
static Spec decode_spec(Net* n, uint32_t B) {
  Spec dec;
  dec.B = (int)B;
  dec.S = 1;
  dec.mode = MODE_CACHED;
  dec.first = 0;
  dec.last = (uint32_t)n->layers.size();
  return dec;
}

// Decode-step inputs: the ids the previous step left on the device, RoPE
// position = KV length (the fed token's index).
static void bind_decode_inputs(Net* n, Spec& dec) {
  dec.ids = n->dec_ids_d.as<uint32_t>();
  dec.mask = n->ones_d.as<uint32_t>();
  dec.lens = n->ones_d.as<uint32_t>();
  dec.pos = nullptr;
  dec.out_re = n->logits_re.as<double>();
}

// The prompt pass of the token loop (transformer_network.rs:225-248 at t = 0):
// drops the caches, runs every prompt row, and leaves each sequence's first
// greedy id at hist[b * hist_stride] and in dec_ids_d, its Re-logits row at
// logit_hist[0][b] (want_logits), and the KV lengths on the device.  `ctx`
// is the context the later steps will reach (RoPE table size).  The decode
// shape's workspaces are reserved first, so nothing moves once a decode-step
// graph exists.  The host cache state is left valid on success.
static int run_prompt(Net* n, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S,
                      uint32_t hist_stride, uint32_t ctx, bool want_logits) {
  TRY(mitok_reset(n));
  hipStream_t st = n->stream;
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out;
  Spec dec = decode_spec(n, B);
  TRY(prepare(n, dec));
  TRY(reserve(n, n->hist_d, (size_t)B * hist_stride * sizeof(uint32_t)));
  TRY(reserve(n, n->cnt_d, (size_t)B * sizeof(int)));
  if (want_logits) TRY(reserve(n, n->logit_hist_d, (size_t)hist_stride * B * V * sizeof(double)));

  Spec pre;
  pre.first = 0;
  pre.last = (uint32_t)n->layers.size();
  pre.last_row = true;
  std::vector<uint32_t> mask_h;
  TRY(begin_call(n, lens, B, S, nullptr, true, nullptr, pre, mask_h));
  TRY(ensure_rope_for(n, 0, pre.last, (int)std::max<uint32_t>(rope_positions_needed(n), ctx)));
  std::vector<uint32_t> padded((size_t)B * S);
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) padded[(size_t)b * S + s] = s < lens[b] ? prompt[(size_t)b * S + s] : 1u;
  TRY(upload(n, n->ids_d, padded.data(), padded.size() * sizeof(uint32_t)));
  // decode-shape buffers (prepare above may have been superseded by the prefill's larger shape)
  TRY(prepare(n, dec));
  pre.ids = n->ids_d.as<uint32_t>();
  pre.out_re = n->logits_re.as<double>();
  fill_int(st, n->cnt_d.as<int>(), B, 0);
  fill_u32(st, n->ones_d.as<uint32_t>(), B, 1);

  Argmax am0;
  am0.part_v = n->am_v.as<double>();
  am0.part_i = n->am_i.as<int>();
  am0.ids = n->dec_ids_d.as<uint32_t>();
  am0.hist = n->hist_d.as<uint32_t>();
  am0.hist_stride = (int)hist_stride;
  am0.hist_cnt = n->cnt_d.as<int>();
  am0.err = n->err_d.as<uint32_t>();
  pre.am = &am0;
  pre.hist_re = want_logits ? n->logit_hist_d.as<double>() : nullptr;
  pre.hist_cnt = n->cnt_d.as<int>();
  TRY(enqueue_forward(n, pre));
  // KV lengths = the rows each prompt left in the cache (lens_d, or the last
  // wavelet stage's compressed lens; same bits as int)
  const void* kvsrc = n->wstages.empty() ? n->lens_d.p : n->wstages.back()->lens.p;
  HIP_TRY(hipMemcpyAsync(n->kv_len_d.p, kvsrc, B * sizeof(int), hipMemcpyDeviceToDevice, st));
  end_call(n, pre, lens);
  return OK;
}

// (Re)captures the decode-step graph for its key: batch, history length,
// logits history and kind (0: generate's step, 1: mitok_decode_step's step,
// which first zeroes the per-sequence id counters with a fill kernel).  The
// captured graph is destroyed on every return path.
static int ensure_step_graph(Net* n, const Spec& dec, bool want_logits, uint32_t hist_stride, int kind) {
  const uint32_t B = (uint32_t)dec.B;
  if (n->graph && n->graph_B == B && n->graph_nnew == hist_stride && n->graph_logits == want_logits &&
      n->graph_step == kind && n->graph_ctx == dec.ctx_bound && n->graph_generation == n->ws_generation)
    return OK;
  drop_graph(n);
  hipStream_t st = n->stream;
  hipGraph_t g = nullptr;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  if (kind == 1) fill_int(st, n->cnt_d.as<int>(), B, 0);
  const int rc = enqueue_decode_step(n, dec, want_logits, hist_stride);
  const hipError_t ce = hipStreamEndCapture(st, &g);
  int out = rc;
  if (!out && ce != hipSuccess) out = fail(ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ce));
  if (!out) {
    const hipError_t ie = hipGraphInstantiate(&n->graph, g, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
      n->graph = nullptr;
      out = fail(ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ie));
    }
  }
  if (g) (void)hipGraphDestroy(g);
  if (out) return out;
  n->graph_B = B;
  n->graph_ctx = dec.ctx_bound;
  n->graph_nnew = hist_stride;
  n->graph_logits = want_logits;
  n->graph_step = kind;
  n->graph_generation = n->ws_generation;
  return OK;
}

static int generate_impl(Net* n, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S, uint32_t n_new,
                         uint32_t* out_ids, double* out_logits) {
  hipStream_t st = n->stream;
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out;
  const bool want_logits = out_logits != nullptr;
  CallEvents ev;
  TRY(ev.create());
  HIP_TRY(hipEventRecord(ev.e[0], st));
  TRY(run_prompt(n, prompt, lens, B, S, n_new, S + n_new, want_logits));
  HIP_TRY(hipEventRecord(ev.e[1], st));

  // ---- decode steps ----
  Spec dec = decode_spec(n, B);
  bind_decode_inputs(n, dec);
  dec.ctx_bound = (int)(S + n_new);  // every prompt fits S; n_new - 1 tokens follow
  bool used_graph = false, used_resident = false;
  if (n_new > 1 && n->timing.cls == 0) {
    Spec rs = dec;
    Argmax am;
    am.ids = n->dec_ids_d.as<uint32_t>();
    am.hist = n->hist_d.as<uint32_t>();
    am.hist_stride = (int)n_new;
    am.hist_cnt = n->cnt_d.as<int>();
    am.kv_len = n->kv_len_d.as<int>();
    am.advance_kv = 1;
    am.err = n->err_d.as<uint32_t>();
    rs.am = &am;
    rs.hist_re = want_logits ? n->logit_hist_d.as<double>() : nullptr;
    rs.hist_cnt = n->cnt_d.as<int>();
    if (resident_ok(n, rs)) {
      TRY(run_resident(n, rs, n_new - 1));
      used_resident = true;
    }
  }
  if (n_new > 1 && !used_resident) {
    const bool direct = n->direct_launch || n->timing.cls != 0;
    if (!direct) {
      TRY(ensure_step_graph(n, dec, want_logits, n_new, 0));
      for (uint32_t t = 1; t < n_new; ++t) HIP_TRY(hipGraphLaunch(n->graph, st));
      used_graph = true;
    } else {
      for (uint32_t t = 1; t < n_new; ++t) {
        n->dec_tsum = 0.0;
        for (uint32_t b = 0; b < B; ++b) n->dec_tsum += (double)n->kv_len_h[b] + t;
        TimeScope ts(n, MITOK_TIME_STEP, 0.0);
        TRY(enqueue_decode_step(n, dec, want_logits, n_new));
      }
    }
  }
  HIP_TRY(hipEventRecord(ev.e[2], st));
  HIP_TRY(hipMemcpyAsync(out_ids, n->hist_d.p, (size_t)B * n_new * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  if (want_logits)
    HIP_TRY(hipMemcpyAsync(out_logits, n->logit_hist_d.p, (size_t)n_new * B * V * sizeof(double), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  float a = 0.f, b2 = 0.f;
  (void)hipEventElapsedTime(&a, ev.e[0], ev.e[1]);
  (void)hipEventElapsedTime(&b2, ev.e[1], ev.e[2]);
  n->last_t[0] = a;
  n->last_t[1] = b2;
  n->last_t[2] = used_resident ? 2.0 : used_graph ? 1.0 : 0.0;
  collect_timing(n);
  if (used_resident) {
    uint32_t e = 0;
    HIP_TRY(hipMemcpy(&e, n->err_d.p, sizeof e, hipMemcpyDeviceToHost));
    if (e & EB_BARRIER) {  // the flags no longer follow the epochs: start over
      HIP_TRY(hipMemset(n->res_flags.p, 0, n->res_flags.bytes));
      n->res_epoch = 0;
    }
  }
  TRY(check_err_word(n));
  for (uint32_t b = 0; b < B; ++b) n->kv_len_h[b] += n_new - 1;
  return OK;
}

// common argument checks of the token-loop entry points
static int check_loop_args(Net* n, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S, uint32_t ctx_extra,
                           const uint32_t* out_ids) {
  if (!n || !prompt || !lens || !out_ids) return fail(ERR_ARG, "null argument");
  TRY(validate_batch(lens, B, S));
  TRY(check_stack(n));
  TRY(set_device(n));
  const uint32_t mc = min_ctx(n);
  for (uint32_t b = 0; b < B; ++b)
    if (mc != UINT32_MAX && (uint64_t)lens[b] + ctx_extra > mc)
      return fail(ERR_ARG, "prompt %u + %u new tokens exceed max context %u", lens[b], ctx_extra, mc);
  return OK;
}

int mitok_generate(mitok_network* n, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S,
                   uint32_t n_new, uint32_t* out_ids, double* out_logits) {
  TRY(check_loop_args(n, prompt, lens, B, S, n_new ? n_new - 1 : 0, out_ids));
  if (n_new == 0) return OK;
  const int rc = generate_impl(n, prompt, lens, B, S, n_new, out_ids, out_logits);
  if (rc) (void)mitok_reset(n);  // caches and device lengths may be part-way through a step
  return rc;
}

int mitok_prefill(mitok_network* n, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S,
                  uint32_t* out_ids, double* out_logits) {
  TRY(check_loop_args(n, prompt, lens, B, S, 0, out_ids));
  hipStream_t st = n->stream;
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out;
  int rc = run_prompt(n, prompt, lens, B, S, 1, S + 1, out_logits != nullptr);
  if (!rc && hipMemcpyAsync(out_ids, n->hist_d.p, B * sizeof(uint32_t), hipMemcpyDeviceToHost, st) != hipSuccess)
    rc = fail(ERR_HIP, "prefill: id copy failed");
  if (!rc && out_logits &&
      hipMemcpyAsync(out_logits, n->logit_hist_d.p, (size_t)B * V * sizeof(double), hipMemcpyDeviceToHost, st) != hipSuccess)
    rc = fail(ERR_HIP, "prefill: logits copy failed");
  if (!rc && hipStreamSynchronize(st) != hipSuccess) rc = fail(ERR_HIP, "prefill: stream sync failed");
  if (!rc) rc = check_err_word(n);
  if (rc) (void)mitok_reset(n);
  return rc;
}

static int decode_step_impl(Net* n, const uint32_t* ids, uint32_t B, uint32_t* out_ids, double* out_logits) {
  hipStream_t st = n->stream;
  const uint32_t V = n->layers[n->layers.size() - 2]->d_out;
  const bool want_logits = out_logits != nullptr;
  uint32_t kv_max = 0;
  for (uint32_t b = 0; b < B; ++b) kv_max = std::max(kv_max, n->kv_len_h[b]);
  Spec dec = decode_spec(n, B);
  TRY(prepare(n, dec));
  TRY(reserve(n, n->hist_d, (size_t)B * sizeof(uint32_t)));
  TRY(reserve(n, n->cnt_d, (size_t)B * sizeof(int)));
  if (want_logits) TRY(reserve(n, n->logit_hist_d, (size_t)B * V * sizeof(double)));
  TRY(ensure_rope_for(n, 0, dec.last, (int)std::max<uint32_t>(rope_positions_needed(n), kv_max + 1)));
  bind_decode_inputs(n, dec);
  if (ids) {
    // the caller's ids are staged in ids_d (a stream-ordered copy of a host buffer
    // that the call holds until its synchronisation below), then moved into place
    TRY(reserve(n, n->ids_d, (size_t)B * sizeof(uint32_t)));
    HIP_TRY(hipMemcpyAsync(n->ids_d.p, ids, B * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(n->dec_ids_d.p, n->ids_d.p, B * sizeof(uint32_t), hipMemcpyDeviceToDevice, st));
  }
  fill_u32(st, n->ones_d.as<uint32_t>(), B, 1);
  const bool direct = n->direct_launch || n->timing.cls != 0;
  if (!direct) {
    TRY(ensure_step_graph(n, dec, want_logits, 1, 1));
    HIP_TRY(hipGraphLaunch(n->graph, st));
  } else {
    fill_int(st, n->cnt_d.as<int>(), B, 0);
    n->dec_tsum = 0.0;
    for (uint32_t b = 0; b < B; ++b) n->dec_tsum += (double)n->kv_len_h[b] + 1;
    TimeScope ts(n, MITOK_TIME_STEP, 0.0);
    TRY(enqueue_decode_step(n, dec, want_logits, 1));
  }
  HIP_TRY(hipMemcpyAsync(out_ids, n->hist_d.p, B * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  if (want_logits) HIP_TRY(hipMemcpyAsync(out_logits, n->logit_hist_d.p, (size_t)B * V * sizeof(double), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  collect_timing(n);
  TRY(check_err_word(n));
  for (uint32_t b = 0; b < B; ++b) n->kv_len_h[b] += 1;
  return OK;
}

int mitok_decode_step(mitok_network* n, const uint32_t* ids, uint32_t B, uint32_t* out_ids, double* out_logits) {
  if (!n || !out_ids) return fail(ERR_ARG, "null argument");
  if (!n->cache_valid) return fail(ERR_STATE, "decode_step before prefill (no KV cache)");
  if (B != n->cache_B) return fail(ERR_STATE, "cached batch %u != %u; prefill first", n->cache_B, B);
  TRY(set_device(n));
  const uint32_t mc = min_ctx(n);
  for (uint32_t b = 0; b < B; ++b)
    if (mc != UINT32_MAX && n->kv_len_h[b] + 1 > mc)
      return fail(ERR_ARG, "context %u exceeds max context %u", n->kv_len_h[b] + 1, mc);
  if (ids) {
    const uint32_t V0 = ((const EmbeddingLayer*)n->layers[0].get())->vocab;
    for (uint32_t b = 0; b < B; ++b)
      if (ids[b] >= V0) return fail(ERR_ARG, "No token embedding found: token id %u >= vocab %u (embedding_layer.rs:305)", ids[b], V0);
  }
  const int rc = decode_step_impl(n, ids, B, out_ids, out_logits);
  if (rc) (void)mitok_reset(n);
  return rc;
}

// the AdamW moments of a weight (nw) and its bias (nb), allocated and zeroed
// at the first update; nb = 0: a lone array's pair (mw, vw) only
static int ensure_moments(hipStream_t st, size_t nw, size_t nb, DevBuf& mw, DevBuf& vw, DevBuf& mb, DevBuf& vb) {
  if (mw.p) return OK;
  TRY(mw.reserve(nw * sizeof(double2)));
  TRY(vw.reserve(nw * sizeof(double2)));
  fill_const(st, mw.as<double2>(), nw, make_double2(0.0, 0.0));
  fill_const(st, vw.as<double2>(), nw, make_double2(0.0, 0.0));
  if (!nb) return OK;
  TRY(mb.reserve(nb * sizeof(double2)));
  TRY(vb.reserve(nb * sizeof(double2)));
  fill_const(st, mb.as<double2>(), nb, make_double2(0.0, 0.0));
  fill_const(st, vb.as<double2>(), nb, make_double2(0.0, 0.0));
  return OK;
}

// backward (transformer_network.rs:506-636) on the device: the reverse walk
// from the Softmax through `n_layers` layers below it, each layer's backward
// on the inputs the last stateless pass kept, and with update_params each
// layer's update_parameters where the reference calls it (Linear,
// FeedForward, SelfAttention with its Norm, Embedding; a standalone Norm and
// RoPE have no update in the walk).
// own_rates: each layer updates at its own learning rate and the Embedding at
// the network's, as backward does (transformer_network.rs:506-636); else every
// update uses learning_rate.
static int backward_impl(Net* n, const uint32_t* targets, const uint32_t* tlens, uint32_t B, uint32_t T,
                         uint32_t n_layers, int update_params, double learning_rate, uint32_t time_step,
                         double* out_grad_input, bool own_rates = false) {
  if (!n || !targets || !tlens || !B || !T) return fail(ERR_ARG, "bad arguments");
  if (!n->head_valid) return fail(ERR_STATE, "no stateless (forward_only = 0) predict to differentiate");
  if (B != n->head_B) return fail(ERR_ARG, "batch %u != the forward pass's %u", B, n->head_B);
  const uint32_t li_top = (uint32_t)n->layers.size() - 2;
  if (!is_vocab_linear(n, li_top)) return fail(ERR_STATE, "the stack does not end in Linear, Softmax");
  const uint32_t reach = li_top + 1 - n->head_first;  // layers of the forward pass below the Softmax
  if (n_layers < 1 || n_layers > reach)
    return fail(ERR_ARG, "%u layers: from 1 (the vocab Linear) to %u (every layer of the forward pass)", n_layers, reach);
  const uint32_t stop = li_top + 1 - n_layers;
  auto* Ln = (LinearLayer*)n->layers[li_top].get();
  const int S = (int)n->head_S, d = (int)Ln->d_in, V = (int)Ln->d_out;
  const long rows = (long)B * S;
  // rows per sequence of each walked layer's input: a wavelet layer's are its
  // stage's S_in (the stages of the forward pass, in layer order)
  std::vector<int> S_in_at(li_top + 1, S);
  std::vector<Net::WaveletStage*> stage_at(li_top + 1, nullptr);
  {
    size_t si = 0;
    for (uint32_t li = n->head_first; li < li_top; ++li)
      if (n->layers[li]->kind == K_WAVELET) {
        if (si >= n->wstages.size()) return fail(ERR_STATE, "layer %u: the forward pass left no wavelet stage", li);
        stage_at[li] = n->wstages[si++].get();
      }
    int Sc = S;
    for (int li = (int)li_top; li >= (int)stop; --li) {
      if (stage_at[li]) Sc = stage_at[li]->S_in;
      S_in_at[li] = Sc;
    }
  }
  long rows_max = rows;
  for (uint32_t li = stop; li <= li_top; ++li) rows_max = std::max(rows_max, (long)B * S_in_at[li]);
  // host staging of the uploads, alive until the synchronisation at the end
  std::vector<std::vector<int>> keep_i;
  std::vector<std::vector<double>> keep_d;
  // what the walk needs, checked and sized before the first launch
  size_t dmax = (size_t)d, fmax = 0, d3max = 0, att = 0, wmax = (size_t)d * V, bmax = (size_t)V;
  size_t ws = std::max(gemm_ws_bytes(d, V, (int)rows), gemm_ws_bytes((int)rows, d, V));
  for (uint32_t li = stop; li < li_top; ++li) {
    const Layer* L = n->layers[li].get();
    const int di = (int)L->d_in, dn = (int)L->d_out;
    const long rows = (long)B * S_in_at[li];
    dmax = std::max({dmax, (size_t)di, (size_t)dn});
    switch (L->kind) {
      case K_WAVELET: {
        const Net::WaveletStage& W = *stage_at[li];
        if (2 * (W.S2 - W.T) - (W.L - 2) < W.S_in - W.T)
          return fail(ERR_STATE, "layer %u: fewer decompressed rows than inputs", li);
        break;
      }
      case K_LINEAR:
        wmax = std::max(wmax, (size_t)di * dn);
        bmax = std::max(bmax, (size_t)dn);
        ws = std::max({ws, gemm_ws_bytes(di, dn, (int)rows), gemm_ws_bytes((int)rows, di, dn)});
        break;
      case K_FEED_FORWARD: {
        const int F = (int)((const FeedForwardLayer*)L)->hidden;
        fmax = std::max(fmax, (size_t)F);
        wmax = std::max(wmax, (size_t)di * F);
        bmax = std::max(bmax, (size_t)F);
        ws = std::max({ws, gemm_ws_bytes((int)rows, F, di), gemm_ws_bytes(F, dn, (int)rows),
                       gemm_ws_bytes((int)rows, F, dn), gemm_ws_bytes(di, F, (int)rows), gemm_ws_bytes((int)rows, di, F)});
        break;
      }
      case K_SELF_ATTENTION: {
        const auto* A = (const SelfAttentionLayer*)L;
        if ((uint32_t)S > A->max_ctx) return fail(ERR_ARG, "layer %u: %d rows exceed max context %u", li, S, A->max_ctx);
        // k_attn_probs_grad holds a query row's weights and Re(dl_ds) in LDS (2 S doubles beside 6 KB)
        if (S > 3072) return fail(ERR_ARG, "layer %u: attention backward of %d rows (at most 3072)", li, S);
        if (A->dh > 256) return fail(ERR_ARG, "layer %u: attention backward of %u-wide heads (at most 256)", li, A->dh);
        d3max = std::max(d3max, (size_t)3 * di);
        att = std::max(att, (size_t)A->heads * S * S);
        wmax = std::max(wmax, (size_t)3 * di * di);
        ws = std::max({ws, gemm_ws_bytes((int)rows, 3 * di, di), gemm_ws_bytes(di, 3 * di, (int)rows),
                       gemm_ws_bytes((int)rows, di, 3 * di)});
        break;
      }
      default: break;
    }
  }
  // SoftmaxLayer::backward (softmax_output_layer.rs:67-145): which row predicts
  // which target, checked in the reference's order (a target id at or past the
  // vocabulary panics there; PAD targets are skipped; the row before the last
  // ends the sequence's targets); the normalizer B * non-PAD targets
  std::vector<int> tgt((size_t)rows, -1);
  std::vector<double> norm(B, 1.0);
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t tl = tlens[b];
    if (tl > T) return fail(ERR_ARG, "target length %u > %u", tl, T);
    if ((uint64_t)tl + 1 > (uint64_t)S) return fail(ERR_ARG, "sequence %u: %u targets need more than %d rows", b, tl, S);
    double unpadded = 0.0;
    for (uint32_t t = 0; t < tl; ++t)
      if (targets[(size_t)b * T + t] != 1u) unpadded += 1.0;
    norm[b] = (double)B * unpadded;
    const int start = S - (int)tl - 1;
    for (uint32_t t = 0; t < tl; ++t) {
      const uint32_t tc = targets[(size_t)b * T + t];
      if (tc >= (uint32_t)V) return fail(ERR_ARG, "target token %u exceeds vocabulary %d", tc, V);
      if (tc == 1u) continue;
      const int s = start + (int)t;
      if (s >= S - 1) break;
      tgt[(size_t)b * S + s] = (int)tc;
    }
  }
  // EmbeddingLayer::update_parameters' order: sequence by sequence, target by
  // target; grouped per id (a repeated id applies its rows in that order)
  const bool embed_upd = update_params && stop == 0 && n->layers[0]->kind == K_EMBEDDING;
  std::vector<uint32_t> eids;
  std::vector<int> estart, eocc;
  if (embed_upd) {
    const uint32_t EV = ((const EmbeddingLayer*)n->layers[0].get())->vocab;
    std::map<uint32_t, std::vector<int>> by_id;
    for (uint32_t b = 0; b < B; ++b)
      for (uint32_t t = 0; t < tlens[b] && (int)t < S_in_at[0]; ++t) {
        const uint32_t id = targets[(size_t)b * T + t];
        if (id >= EV) return fail(ERR_ARG, "No token embedding found: %u (embedding_layer.rs:233)", id);
        by_id[id].push_back((int)(b * (uint32_t)S_in_at[0] + t));
      }
    for (auto& kv : by_id) {
      eids.push_back(kv.first);
      estart.push_back((int)eocc.size());
      eocc.insert(eocc.end(), kv.second.begin(), kv.second.end());
    }
    estart.push_back((int)eocc.size());
  }
  TRY(set_device(n));
  hipStream_t st = n->stream;
  const size_t c16 = sizeof(double2);
  // DiscreteWaveletLayer::backward's tap tables (wavelet_discrete_layer.rs:163-207)
  for (uint32_t li = stop; li < li_top; ++li) {
    if (!stage_at[li]) continue;
    Net::WaveletStage& W = *stage_at[li];
    const int R = W.S_in - W.T, M = W.S2 - W.T, Lf = W.L, lout = 2 * M - (Lf - 2);
    std::vector<int> gs((size_t)W.S_in * 4, -1);
    std::vector<double> gw((size_t)W.S_in * 4, 0.0);
    // decompressed row k (grad_dwt_1d_trend: inverse_dwt_1d of [g | 0] with the low pass reversed)
    auto dec = [&](int k, int& slot, int r) {
      const int i = k / 2;
      const bool even = (k % 2) == 0;
      auto put = [&](int src, double w) {
        gs[(size_t)r * 4 + slot] = src;
        gw[(size_t)r * 4 + slot] = w;
        ++slot;
      };
      if (Lf == 2) {
        put(i, even ? W.lo[0] : W.lo[1]);
      } else {
        put(i, even ? W.lo[2] : W.lo[3]);
        put(i + 1, even ? W.lo[0] : W.lo[1]);
      }
    };
    for (int r = 0; r < R; ++r) {
      int slot = 0;
      dec(r, slot, r);
      if (r == R - 1 && lout == R + 1) dec(R, slot, r);  // align_gradient_rows_complex (:318-346)
    }
    for (int t = 0; t < W.T; ++t) {
      gs[(size_t)(R + t) * 4] = M + t;  // the target rows' gradient passes through
      gw[(size_t)(R + t) * 4] = 1.0;
    }
    keep_i.push_back(std::move(gs));
    keep_d.push_back(std::move(gw));
    TRY(upload(n, W.gsrc, keep_i.back().data(), keep_i.back().size() * sizeof(int)));
    TRY(upload(n, W.gw, keep_d.back().data(), keep_d.back().size() * sizeof(double)));
  }
  // every workspace is sized before the first launch (a reserve that grows frees the old buffer)
  TRY(upload(n, n->tr_tgt, tgt.data(), tgt.size() * sizeof(int)));
  TRY(upload(n, n->tr_norm, norm.data(), norm.size() * sizeof(double)));
  if (embed_upd && !eids.empty()) {
    TRY(upload(n, n->tr_eid, eids.data(), eids.size() * sizeof(uint32_t)));
    TRY(upload(n, n->tr_est, estart.data(), estart.size() * sizeof(int)));
    TRY(upload(n, n->tr_eocc, eocc.data(), eocc.size() * sizeof(int)));
  }
  TRY(reserve(n, n->tr_g, (size_t)rows * V * c16));
  TRY(reserve(n, n->tr_ga, (size_t)rows_max * dmax * c16));
  TRY(reserve(n, n->tr_gb, (size_t)rows_max * dmax * c16));
  TRY(reserve(n, n->tr_xh, (size_t)rows_max * std::max(dmax, fmax) * c16));
  TRY(reserve(n, n->tr_wh, wmax * c16));
  TRY(reserve(n, n->tr_dw, wmax * c16));
  TRY(reserve(n, n->tr_db, std::max(bmax, dmax) * c16));
  TRY(reserve(n, n->tr_dh, (size_t)rows_max * std::max(fmax, dmax) * c16));
  TRY(reserve(n, n->tr_pg, (size_t)rows_max * dmax * c16));
  TRY(reserve(n, n->tr_bsum, (size_t)B * std::max({bmax, dmax, fmax}) * c16));  // per-sequence column sums
  if (fmax) {
    TRY(reserve(n, n->tr_z, (size_t)rows_max * fmax * c16));
    TRY(reserve(n, n->tr_h, (size_t)rows_max * fmax * c16));
    TRY(reserve(n, n->tr_g1, (size_t)rows_max * fmax * c16));
  }
  if (att) {
    TRY(reserve(n, n->tr_qkv, (size_t)rows_max * d3max * c16));
    TRY(reserve(n, n->tr_dqkv, (size_t)rows_max * d3max * c16));
    TRY(reserve(n, n->tr_A, (size_t)B * att * sizeof(double)));
    TRY(reserve(n, n->tr_dA, (size_t)B * att * sizeof(double)));
  }
  TRY(reserve(n, n->sync_ws, ws));
  if (update_params) {  // AdamW moments, zeroed at a layer's first update
    TRY(ensure_moments(st, (size_t)d * V, V, Ln->mw, Ln->vw, Ln->mb, Ln->vb));
    for (uint32_t li = stop; li < li_top; ++li) {
      Layer* L = n->layers[li].get();
      if (L->kind == K_LINEAR) {
        auto* H = (LinearLayer*)L;
        TRY(ensure_moments(st, (size_t)H->d_in * H->d_out, H->d_out, H->mw, H->vw, H->mb, H->vb));
      } else if (L->kind == K_FEED_FORWARD) {
        auto* F = (FeedForwardLayer*)L;
        TRY(ensure_moments(st, (size_t)F->hidden * F->d_out, F->d_out, F->mw2, F->vw2, F->mb2, F->vb2));
        TRY(ensure_moments(st, (size_t)F->d_in * F->hidden, F->hidden, F->mw1, F->vw1, F->mb1, F->vb1));
      } else if (L->kind == K_SELF_ATTENTION) {
        auto* A = (SelfAttentionLayer*)L;
        TRY(ensure_moments(st, (size_t)3 * A->d_in * A->d_in, A->d_in, A->mw, A->vw, A->mg, A->vg));
        TRY(ensure_moments(st, A->d_in, 0, A->mbt, A->vbt, A->mbt, A->vbt));
      }
    }
  }
  const Sync sy = sync_of(n);
  uint32_t* err = n->err_d.as<uint32_t>();
  long rows_c = rows;  // the current layer's rows (a wavelet layer changes them below it)
  int S_c = S;
  const uint32_t* mask_c = n->head_mask;
  double2* xh = n->tr_xh.as<double2>();
  double2* wh = n->tr_wh.as<double2>();
  double2* dW = n->tr_dw.as<double2>();
  double2* db = n->tr_db.as<double2>();
  // LinearLayer::backward, complex arm (linear_layer.rs:96-108), grouped over
  // the sequences: dW = conj(X)^T G, db = column sums, dX = G conj(W)^T
  auto linear_bwd = [&](const double2* X, const double2* G, const double2* W, int din, int dout, double2* dX) -> int {
    conj_transpose(st, X, rows_c, din, xh);
    Epi e;
    e.mode = EPI_STORE;
    e.err = err;
    e.out = dW;
    e.ldo = dout;
    TRY(launch_rc(gemm(st, din, dout, (int)rows_c, rows_of(xh, rows_c), G, dout, e, nullptr, sy), "weight grad"));
    bias_grad(st, G, (int)B, S_c, dout, n->tr_bsum.as<double2>(), db);
    conj_transpose(st, W, din, dout, wh);
    e.out = dX;
    e.ldo = din;
    TRY(launch_rc(gemm(st, (int)rows_c, din, dout, rows_of(G, dout), wh, din, e, nullptr, sy), "input grad"));
    return OK;
  };
  // update_parameters of a weight and its bias from dW, db (linear_layer.rs:130-175)
  auto rate = [&](const Layer* L) { return own_rates ? L->lr : learning_rate; };
  auto linear_upd = [&](DevBuf& W, DevBuf& b, long nw, int nb, DevBuf& mw, DevBuf& vw, DevBuf& mb, DevBuf& vb,
                        uint32_t& updates, int tstep, double lr) {
    TrainStep ts;
    ts.lr = lr;
    ts.batch = (double)B;
    ts.first = updates == 0 ? 1 : 0;
    ts.time_step = tstep;
    linear_update(st, W.as<double2>(), dW, mw.as<double2>(), vw.as<double2>(), nw, b.as<double2>(), db,
                  mb.as<double2>(), vb.as<double2>(), nb, ts);
    updates++;
  };
  double2* G = n->tr_g.as<double2>();
  softmax_grad(st, n->probs.as<double>(), (int)rows, V, n->tr_tgt.as<int>(), n->tr_norm.as<double>(), S, G);
  double2* gcur = n->tr_ga.as<double2>();  // the gradient of the current layer's output, then its input
  double2* gnext = n->tr_gb.as<double2>();
  TRY(linear_bwd(n->head_x, G, Ln->w.as<double2>(), d, V, gcur));
  if (update_params)
    linear_upd(Ln->w, Ln->b, (long)d * V, V, Ln->mw, Ln->vw, Ln->mb, Ln->vb, Ln->updates, (int)time_step, rate(Ln));
  for (int li = (int)li_top - 1; li >= (int)stop; --li) {
    Layer* L = n->layers[li].get();
    const double2* X = n->tr_in[li]->as<double2>();
    const uint32_t* mask = mask_c;
    if (!stage_at[li]) {  // every other layer keeps its rows
      S_c = S_in_at[li];
      rows_c = (long)B * S_c;
    }
    const long rows = rows_c;
    const int S = S_c;
    switch (L->kind) {
      case K_WAVELET: {
        const Net::WaveletStage& W = *stage_at[li];
        dwt_backward(st, gcur, (int)B, W.S2, W.S_in, (int)L->d_in, W.gsrc.as<int>(), W.gw.as<double>(), gnext);
        std::swap(gcur, gnext);
        S_c = W.S_in;  // the layers below see the stage's input rows and mask
        rows_c = (long)B * S_c;
        mask_c = W.mask_in;
        break;
      }
      case K_LINEAR: {
        auto* H = (LinearLayer*)L;
        TRY(linear_bwd(X, gcur, H->w.as<double2>(), H->d_in, H->d_out, gnext));
        if (update_params) linear_upd(H->w, H->b, (long)H->d_in * H->d_out, H->d_out, H->mw, H->vw, H->mb, H->vb, H->updates,
                                      (int)time_step, rate(H));
        std::swap(gcur, gnext);
        break;
      }
      case K_FEED_FORWARD: {
        // FeedForwardLayer::backward (feedforward_layer.rs:140-186): its Linear,
        // then its Dense (GELU) layer (layer.rs:168-210)
        auto* F = (FeedForwardLayer*)L;
        const int Fh = (int)F->hidden, di = (int)F->d_in, dn = (int)F->d_out;
        Epi e;
        e.err = err;
        e.bias = F->b1.as<double2>();
        e.ldo = Fh;
        e.mode = EPI_GELU;  // the Dense output the forward pass gave its Linear: GELU, padded rows 0
        e.row_mask = mask;
        e.out = n->tr_h.as<double2>();
        TRY(launch_rc(gemm(st, (int)rows, Fh, di, rows_of(X, di), F->w1.as<double2>(), Fh, e, nullptr, sy), "ffn1 output"));
        e.mode = EPI_STORE;  // its pre-activation Z = X W1 + b1 (layer.rs:135-144)
        e.row_mask = nullptr;
        e.out = n->tr_z.as<double2>();
        TRY(launch_rc(gemm(st, (int)rows, Fh, di, rows_of(X, di), F->w1.as<double2>(), Fh, e, nullptr, sy),
                      "ffn1 pre-activation"));
        TRY(linear_bwd(n->tr_h.as<double2>(), gcur, F->w2.as<double2>(), Fh, dn, n->tr_dh.as<double2>()));
        // FeedForwardLayer::update_parameters (:219-250): the Linear at the FFN's time step (:86)
        if (update_params) linear_upd(F->w2, F->b2, (long)Fh * dn, dn, F->mw2, F->vw2, F->mb2, F->vb2, F->updates2,
                                      (int)time_step, rate(F));
        gelu_backward(st, n->tr_dh.as<double2>(), n->tr_z.as<double2>(), mask, rows, Fh, n->tr_g1.as<double2>());
        TRY(linear_bwd(X, n->tr_g1.as<double2>(), F->w1.as<double2>(), di, Fh, gnext));
        // the Dense at step 1: Layer::time_step stays 0 after construction (layer.rs:111,285)
        if (update_params) linear_upd(F->w1, F->b1, (long)di * Fh, Fh, F->mw1, F->vw1, F->mb1, F->vb1, F->updates1, 0, rate(F));
        std::swap(gcur, gnext);
        break;
      }
      case K_SELF_ATTENTION: {
        // SelfAttentionLayer::backward (self_attention_layer.rs:135-196): the
        // Norm's backward on Re(heads' output + X), then every head
        // (masked_attention_head.rs:222-345); no residual gradient is added
        auto* A = (SelfAttentionLayer*)L;
        const int da = (int)A->d_in, H = (int)A->heads, dh = (int)A->dh, mc = (int)A->max_ctx;
        const double c = 1.0 / (1e-8 + sqrt((double)dh));
        double2* gn = n->tr_dh.as<double2>();
        norm_backward(st, n->tr_cat[li]->as<double2>(), X, rows, da, A->eps, A->gamma.as<double2>(), A->beta.as<double2>(),
                      gcur, gn, n->tr_pg.as<double2>());
        Epi e;
        e.mode = EPI_STORE;
        e.err = err;
        e.out = n->tr_qkv.as<double2>();
        e.ldo = 3 * da;
        TRY(launch_rc(gemm(st, (int)rows, 3 * da, da, rows_of(X, da), A->wqkv.as<double2>(), 3 * da, e, nullptr, sy),
                      "qkv"));
        attn_probs_grad(st, n->tr_qkv.as<double2>(), A->bias_re.as<double>(), mc, mask, gn, (int)B, S, H, dh, c,
                        n->tr_A.as<double>(), n->tr_dA.as<double>());
        attn_dqkv(st, n->tr_qkv.as<double2>(), n->tr_A.as<double>(), n->tr_dA.as<double>(), gn, (int)B, S, H, dh, c,
                  n->tr_dqkv.as<double2>());
        // the heads' weight gradients grouped over the batch: conj(X)^T [dq | dk | dv]
        conj_transpose(st, X, rows, da, xh);
        e.out = dW;
        e.ldo = 3 * da;
        TRY(launch_rc(gemm(st, da, 3 * da, (int)rows, rows_of(xh, rows), n->tr_dqkv.as<double2>(), 3 * da, e, nullptr, sy),
                      "qkv weight grad"));
        // the heads' input gradients summed: [dq | dk | dv] conj([Wq | Wk | Wv])^T
        conj_transpose(st, A->wqkv.as<double2>(), da, 3 * da, wh);
        e.out = gnext;
        e.ldo = da;
        TRY(launch_rc(gemm(st, (int)rows, da, 3 * da, rows_of(n->tr_dqkv.as<double2>(), 3 * da), wh, da, e, nullptr, sy),
                      "qkv input grad"));
        if (update_params) {  // SelfAttentionLayer::update_parameters (:260-273): the Norm, then the heads
          TrainStep ts;
          ts.lr = rate(A);
          ts.first = A->norm_updates == 0 ? 1 : 0;
          ts.time_step = (int)time_step;
          ts.batch = (double)da;  // norm_layer.rs:269: gamma's length
          colsum(st, n->tr_pg.as<double2>(), (int)B, S, da, (double)da, n->tr_bsum.as<double2>(), db);  // gamma's: n copies per row
          param_update(st, A->gamma.as<double2>(), db, A->mg.as<double2>(), A->vg.as<double2>(), da, false, ts);
          colsum(st, gcur, (int)B, S, da, (double)da, n->tr_bsum.as<double2>(), db);
          param_update(st, A->beta.as<double2>(), db, A->mbt.as<double2>(), A->vbt.as<double2>(), da, false, ts);
          A->norm_updates++;
          ts.first = A->updates == 0 ? 1 : 0;
          ts.batch = (double)B;  // masked_attention_head.rs:352: the sequences
          param_update(st, A->wqkv.as<double2>(), dW, A->mw.as<double2>(), A->vw.as<double2>(), (long)3 * da * da, true, ts);
          attn_bias_update(st, A->bias_re.as<double>(), mc, n->tr_dA.as<double>(), (int)B, H, S, ts);
          A->updates++;
        }
        std::swap(gcur, gnext);
        break;
      }
      case K_NORM: {  // NormalNormLayer::backward; the walk does not update a standalone Norm
        auto* N = (NormLayer*)L;
        norm_backward(st, X, nullptr, rows, N->d_in, N->eps, N->gamma.as<double2>(), N->beta.as<double2>(), gcur, gnext,
                      n->tr_pg.as<double2>());
        std::swap(gcur, gnext);
        break;
      }
      case K_POSENC: {
        auto* P = (PositionalEncodingLayer*)L;
        rope_backward(st, gcur, rows, S, P->d_in, P->cs.as<double2>(), gnext);
        std::swap(gcur, gnext);
        break;
      }
      case K_EMBEDDING: {  // EmbeddingLayer::backward passes the gradient on (embedding_layer.rs:214-221)
        auto* E = (EmbeddingLayer*)L;
        if (embed_upd && !eids.empty())
          embedding_update(st, E->table.as<double2>(), (int)E->d_out, n->tr_eid.as<uint32_t>(), (int)eids.size(),
                           n->tr_est.as<int>(), n->tr_eocc.as<int>(), gcur, own_rates ? n->lr : learning_rate,
                           (double)B * (double)E->vocab,
                           err);
        break;
      }
      default: break;
    }
  }
  if (update_params) drop_graph(n);  // the weights changed under any captured step
  if (out_grad_input) {
    const int dlow = (int)n->layers[stop]->d_in;
    HIP_TRY(hipMemcpyAsync(out_grad_input, gcur, (size_t)rows_c * dlow * c16, hipMemcpyDeviceToHost, st));
  }
  HIP_TRY(hipStreamSynchronize(st));
  return check_err_word(n);
}

int mitok_backward_head(mitok_network* n, const uint32_t* targets, const uint32_t* tlens, uint32_t B, uint32_t T,
                        int update_params, double learning_rate, uint32_t time_step, double* out_grad_input) {
  return backward_impl(n, targets, tlens, B, T, 1, update_params, learning_rate, time_step, out_grad_input);
}

int mitok_backward(mitok_network* n, const uint32_t* targets, const uint32_t* tlens, uint32_t B, uint32_t T,
                   uint32_t n_layers, int update_params, double learning_rate, uint32_t time_step,
                   double* out_grad_input) {
  return backward_impl(n, targets, tlens, B, T, n_layers, update_params, learning_rate, time_step, out_grad_input);
}

int mitok_backward_walk(mitok_network* n, const uint32_t* targets, const uint32_t* tlens, uint32_t B, uint32_t T,
                        int update_params, uint32_t time_step, double* out_grad_input) {
  if (!n) return fail(ERR_ARG, "null network");
  if (!n->head_valid) return fail(ERR_STATE, "no stateless (forward_only = 0) predict to differentiate");
  if (n->layers.size() < 2) return fail(ERR_STATE, "the stack does not end in Linear, Softmax");
  const uint32_t reach = (uint32_t)n->layers.size() - 1 - n->head_first;
  return backward_impl(n, targets, tlens, B, T, reach, update_params, 0.0, time_step, out_grad_input, true);
}

int mitok_set_learning_rate(mitok_network* n, uint32_t layer, double lr) {
  if (!n) return fail(ERR_ARG, "null network");
  if (!(lr >= 0.0) || !std::isfinite(lr)) return fail(ERR_ARG, "learning rate %g", lr);
  if (layer == MITOK_ALL_LAYERS) {
    for (auto& L : n->layers) L->lr = lr;
    return OK;
  }
  if (layer >= n->layers.size()) return fail(ERR_ARG, "layer %u of %zu", layer, n->layers.size());
  n->layers[layer]->lr = lr;
  return OK;
}

int mitok_get_learning_rate(const mitok_network* n, uint32_t layer, double* out) {
  if (!n || !out) return fail(ERR_ARG, "bad arguments");
  if (layer == MITOK_NETWORK_RATE) {
    *out = n->lr;
    return OK;
  }
  if (layer >= n->layers.size()) return fail(ERR_ARG, "layer %u of %zu", layer, n->layers.size());
  *out = n->layers[layer]->lr;
  return OK;
}

int mitok_set_network_learning_rate(mitok_network* n, double lr) {
  if (!n) return fail(ERR_ARG, "null network");
  if (!(lr >= 0.0) || !std::isfinite(lr)) return fail(ERR_ARG, "learning rate %g", lr);
  n->lr = lr;
  return OK;
}

// reset_previous_gradient (neural_network_generic.rs:188-242): the next update
// of every Linear, every FeedForward's Dense and Linear and every attention
// layer's heads is the clipped descent again, which leaves zero moments for
// the AdamW after it (update1 in train.hip clears them).  Norms keep theirs;
// the Embedding's update never reads a previous gradient.
int mitok_reset_previous_gradient(mitok_network* n) {
  if (!n) return fail(ERR_ARG, "null network");
  for (auto& L : n->layers) switch (L->kind) {
      case K_LINEAR: ((LinearLayer*)L.get())->updates = 0; break;
      case K_FEED_FORWARD: {
        auto* F = (FeedForwardLayer*)L.get();
        F->updates1 = F->updates2 = 0;
        break;
      }
      case K_SELF_ATTENTION: ((SelfAttentionLayer*)L.get())->updates = 0; break;
      default: break;
    }
  return OK;
}

int mitok_greedy_decoding(mitok_network* n, const double* logits, uint32_t rows, uint32_t V, uint32_t* out_ids) {
  if (!n || !logits || !out_ids || !rows || !V) return fail(ERR_ARG, "bad arguments");
  TRY(set_device(n));
  DevBuf lg, ids;
  TRY(lg.reserve((size_t)rows * V * sizeof(double)));
  TRY(ids.reserve((size_t)rows * sizeof(uint32_t)));
  HIP_TRY(hipMemcpyAsync(lg.p, logits, (size_t)rows * V * sizeof(double), hipMemcpyHostToDevice, n->stream));
  argmax_rows(n->stream, lg.as<double>(), rows, V, ids.as<uint32_t>(), n->err_d.as<uint32_t>());
  HIP_TRY(hipMemcpyAsync(out_ids, ids.p, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, n->stream));
  HIP_TRY(hipStreamSynchronize(n->stream));
  return check_err_word(n);
}

int mitok_greedy_decoding_device(mitok_network* n, const double* d_logits, uint32_t rows, uint32_t V,
                                 uint32_t* d_out_ids) {
  if (!n || !d_logits || !d_out_ids || !rows || !V) return fail(ERR_ARG, "bad arguments");
  TRY(set_device(n));
  TRY(check_device_range(n, d_logits, (size_t)rows * V * sizeof(double), "logits"));
  TRY(check_device_range(n, d_out_ids, (size_t)rows * sizeof(uint32_t), "out_ids"));
  argmax_rows(n->stream, d_logits, rows, V, d_out_ids, n->err_d.as<uint32_t>());
  HIP_TRY(hipStreamSynchronize(n->stream));
  return check_err_word(n);
}

int mitok_greedy_decoding_noalloc(mitok_network* n, const double* logits, uint32_t rows, uint32_t V, uint32_t* out_ids) {
  if (!n || !logits || !out_ids || !rows || !V) return fail(ERR_ARG, "bad arguments");
  if (rows > NOALLOC_MAX_ROWS || (uint64_t)rows * V > NOALLOC_MAX_LOGITS)
    return fail(ERR_ARG, "%u x %u logits exceed the no-allocation staging (%zu logits, %zu rows)", rows, V,
                NOALLOC_MAX_LOGITS, NOALLOC_MAX_ROWS);
  if (!n->scratch) return fail(ERR_STATE, "no staging address for device %d", n->device);
  TRY(set_device(n));
  double* lg = (double*)n->scratch;
  uint32_t* ids = (uint32_t*)((unsigned char*)n->scratch + NOALLOC_MAX_LOGITS * sizeof(double));
  HIP_TRY(hipMemcpyAsync(lg, logits, (size_t)rows * V * sizeof(double), hipMemcpyHostToDevice, n->stream));
  argmax_rows(n->stream, lg, rows, V, ids, n->err_d.as<uint32_t>());
  HIP_TRY(hipMemcpyAsync(out_ids, ids, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, n->stream));
  HIP_TRY(hipStreamSynchronize(n->stream));
  return check_err_word(n);
}

int mitok_last_timings(mitok_network* n, double* t3) {
  if (!n || !t3) return fail(ERR_ARG, "null argument");
  memcpy(t3, n->last_t, sizeof n->last_t);
  return OK;
}

int mitok_timing_enable(mitok_network* n, int cls) {
  if (!n) return fail(ERR_ARG, "null network");
  collect_timing(n);
  n->timing.cls = cls;
  n->timing.total_ms = 0.0;
  n->timing.bytes = 0.0;
  n->timing.flops = 0.0;
  n->timing.launches = 0;
  return OK;
}

int mitok_timing_read(mitok_network* n, double* total_ms, uint64_t* launches, double* alg_bytes, double* alg_flops) {
  if (!n) return fail(ERR_ARG, "null network");
  collect_timing(n);
  if (total_ms) *total_ms = n->timing.total_ms;
  if (launches) *launches = n->timing.launches;
  if (alg_bytes) *alg_bytes = n->timing.bytes;
  if (alg_flops) *alg_flops = n->timing.flops;
  return OK;
}

int mitok_device_synchronize(int device) {
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(hipDeviceSynchronize());
  return OK;
}

int mitok_set_graph_mode(mitok_network* n, int direct_launch) {
  if (!n) return fail(ERR_ARG, "null network");
  n->direct_launch = direct_launch;
  return OK;
}

int mitok_resident_profile(mitok_network* n, int enable, int max_ops, int* nops, int* kinds, double* us) {
  if (!n) return fail(ERR_ARG, "null network");
  n->res_profile = enable;
  if (!nops) return OK;
  *nops = 0;
  const int no = n->res_nops;
  if (!n->res_stamps.p || !n->res_steps || !no) return OK;
  const size_t cnt = (size_t)no * n->res_steps + 1;
  if (n->res_stamps.bytes < cnt * sizeof(uint64_t)) return OK;
  std::vector<uint64_t> st(cnt);
  HIP_TRY(hipMemcpy(st.data(), n->res_stamps.p, cnt * sizeof(uint64_t), hipMemcpyDeviceToHost));
  const int m = std::min(no, max_ops);
  for (int i = 0; i < m; ++i) {
    double t = 0.0;
    for (uint32_t s2 = 0; s2 < n->res_steps; ++s2) {
      const size_t k = (size_t)s2 * no + i;
      const uint64_t prev = k == 0 ? st[cnt - 1] : st[k - 1];
      t += (double)(st[k] - prev) * 0.01;  // 100 MHz clock -> us
    }
    if (kinds) kinds[i] = n->res_ops_h[i].kind;
    if (us) us[i] = t / n->res_steps;
  }
  *nops = m;
  return OK;
}

int mitok_resident_exchange(mitok_network* n, int mode, int* polled) {
  if (!n) return fail(ERR_ARG, "null network");
  if (mode < -1 || mode > 1) return fail(ERR_ARG, "resident exchange %d (-1 to 1)", mode);
  if (mode >= 0) n->res_poll = mode;
  if (polled) *polled = n->res_polled ? 1 : 0;
  return OK;
}

int mitok_set_decode_plan(mitok_network* n, int plan) {
  if (!n) return fail(ERR_ARG, "null network");
  if (plan < 0 || plan > 3) return fail(ERR_ARG, "decode plan %d (0 to 3)", plan);
  n->resident = plan == 3 ? 2 : plan == 2 ? 1 : 0;
  n->fused_decode = plan >= 1 ? 1 : 0;
  n->tiled_prefill = plan >= 1 ? 1 : 0;
  drop_graph(n);
  return OK;
}

}  // extern "C"
