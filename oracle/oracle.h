/*
 * oracle.h — CPU restatement of the rustCrates transformer token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path in
 * rustcrates_amd/: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path never links or calls it.
 *
 * Every function restates the Rust source it cites (paths relative to the
 * reference crate root, src/neural_networks/...).  Arithmetic follows the Rust
 * expression order exactly and is compiled with -ffp-contract=off (Rust never
 * fuses a*b+c), against glibc libm (what Rust's f64 methods call on Linux).
 *
 * Complex<f64> is num-complex 0.4.6: #[repr(C)] {re, im}, 16 bytes.
 */
#ifndef RUSTCRATES_ORACLE_H
#define RUSTCRATES_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct { double re, im; } oc64;

/* Layer kinds, in the order of LayerEnum (network_components/layer.rs:75-88)
 * restricted to the variants on the token-loop path. */
enum {
  ORC_EMBEDDING = 0,
  ORC_POSITIONAL_ENCODING = 1,
  ORC_NORM = 2,
  ORC_SELF_ATTENTION = 3,
  ORC_FEED_FORWARD = 4,
  ORC_LINEAR = 5,
  ORC_SOFTMAX = 6,
  ORC_DISCRETE_WAVELET = 7
};

/* OperationMode (network_types/neural_network_generic.rs:17-20) */
enum { ORC_TRAINING = 0, ORC_PRODUCTION = 1 };

/* status codes (match include/mitok.h) */
enum { ORC_OK = 0, ORC_ERR_ARG = 1, ORC_ERR_STATE = 3, ORC_ERR_NAN = 4, ORC_ERR_NOMEM = 5 };

typedef struct orc_net orc_net;

const char* orc_last_error(void);

/* ---- num-complex 0.4.6 scalar ops (exported for pinning tests) ---- */
oc64 orc_cmul(oc64 a, oc64 b);
oc64 orc_cdiv(oc64 a, oc64 b);
oc64 orc_csqrt(oc64 z);
oc64 orc_ctanh(oc64 z);
oc64 orc_gelu(oc64 z, int* nan_flag);

/* ---- L1 numeric kernels ---- */
/* multiply_complex (utils/matrix.rs:16-65): C[m][n] = A[m][k] * B[k][n], row-major */
void orc_zgemm(uint32_t m, uint32_t n, uint32_t k, const oc64* A, const oc64* B, oc64* C);
/* NormalNormLayer::normalize (norm_layer.rs:64-82) on one row; out is Re + 0i */
void orc_layernorm_row(const oc64* x, uint32_t d, double eps, const oc64* gamma, const oc64* beta, oc64* out);
/* softmax_row_real (utils/activation.rs:431-439) */
void orc_softmax_row_real(const oc64* x, uint32_t n, double* out);
/* greedy_decoding row argmax (utils/sampling_methods.rs:5-18); -1 on NaN */
int64_t orc_greedy_row(const double* row, uint32_t n);
/* apply_rotary_positional_encoding (positional_encoding_layer.rs:181-209) */
void orc_rope_row(const oc64* x, uint32_t d, double base, uint64_t position, oc64* out);

/* ---- seeded synthetic data (counter generator shared with the HIP path) ---- */
uint64_t orc_draw(uint64_t seed, uint64_t stream, uint64_t index);
double orc_uniform(uint64_t seed, uint64_t stream, uint64_t index, double lim);
void orc_gen_prompts(uint64_t seed, uint32_t batch, uint32_t max_len, const uint32_t* lens, uint32_t vocab, uint32_t* ids);
void orc_gen_normal(uint64_t seed, uint64_t n, oc64* out);

/* ---- network (NeuralNetwork, network_types/neural_network_generic.rs:23-31) ---- */
orc_net* orc_net_create(void);
void orc_net_destroy(orc_net* net);
int orc_num_layers(const orc_net* net);
/* Tensors may be NULL and filled later by orc_init_seeded. Layouts are the
 * reference's: row-major [in][out], per-head [h][d][dh], bias_pos [h][max_ctx][max_ctx]. */
int orc_add_embedding(orc_net* net, uint32_t vocab, uint32_t dim, const oc64* table);
int orc_add_positional_encoding(orc_net* net, uint32_t dim, double base);
int orc_add_norm(orc_net* net, uint32_t dim, double eps, const oc64* gamma, const oc64* beta);
int orc_add_self_attention(orc_net* net, uint32_t heads, uint32_t dim, uint32_t max_ctx, double eps,
                           const oc64* wq, const oc64* wk, const oc64* wv, const oc64* bias_pos,
                           const oc64* gamma, const oc64* beta);
int orc_add_feed_forward(orc_net* net, uint32_t dim, uint32_t hidden, const oc64* w1, const oc64* b1,
                         const oc64* w2, const oc64* b2);
int orc_add_linear(orc_net* net, uint32_t in, uint32_t out, const oc64* w, const oc64* b);
int orc_add_softmax(orc_net* net, int operation_mode);
/* DiscreteWaveletLayer (network_types/wavelet_discrete_layer.rs:46-161), partial
 * mode: at the prompt pass (time_step 0) or a stateless pass it replaces the
 * rows by the low-pass half of dwt_1d along the sequence of every feature and
 * the padding mask by its thresholded low-pass half; at cached steps it
 * passes the row through.  dim: features per row.  wavelet: DiscreteWaletetType index (0 DB1, 1 DB2);
 * mode: WaveletMode index (0 ZERO, 1 CONSTANT, 2 SYMMETRIC, 3 ANTISYMMETRIC,
 * 4 REFLECT, 6 PERIODIC); is_full_mode must be 0. */
int orc_add_discrete_wavelet(orc_net* net, uint32_t dim, uint32_t wavelet, uint32_t mode, int is_full_mode);
/* dwt_1d (wavelet_transform/dwt.rs:36-90) of n reals: out (at least n + 4
 * doubles) = [low half | high half], *out_len its length. */
int orc_dwt_1d(const double* x, uint32_t n, uint32_t wavelet, uint32_t mode, double* out, uint32_t* out_len);
/* rows per sequence after every wavelet layer of a prompt pass of S rows */
uint32_t orc_seq_out_len(const orc_net* net, uint32_t S);
int orc_init_seeded(orc_net* net, uint64_t seed);
/* reads back a weight tensor (slot: 0 table/w/w1/wq, 1 wk/w2, 2 wv, 3 bias_pos, 4 b/b1, 5 b2, 6 gamma, 7 beta) */
int orc_get_tensor(const orc_net* net, uint32_t layer, uint32_t slot, oc64* out, uint64_t n);
int orc_reset(orc_net* net);
void orc_set_threads(int n);
/* zgemm summation order: 0 k ascending (default); 1 k descending; 2 eight
 * contiguous k chunks summed separately, then combined (noise-floor measurement) */
void orc_set_gemm_order(int order);

/* predict (transformer_network.rs:315-504).  ids [B][S] right-padded (entries
 * at or beyond lens[b] are replaced by PAD=1).  time_steps [B] or NULL.
 * out_rows 0: out [B][S][V];  out_rows 1: out [B][V] (row lens[b]-1). */
int orc_predict(orc_net* net, const uint32_t* ids, const uint32_t* lens, uint32_t B, uint32_t S,
                const uint32_t* time_steps, int forward_only, int out_rows, double* out, uint32_t* out_mask);
/* Layers [first, last) over hidden states in [B][S][d_in] -> out [B][S][d_out]. */
int orc_forward_layers(orc_net* net, uint32_t first, uint32_t last, const oc64* in, const uint32_t* mask,
                       uint32_t B, uint32_t S, const uint32_t* time_steps, int forward_only, oc64* out);
/* Greedy token loop (predict_token_by_token, transformer_network.rs:165-313) on ids:
 * out_ids [B][n_new]; out_logits [n_new][B][V] Re-logits of the row each token came from (or NULL). */
int orc_generate(orc_net* net, const uint32_t* prompt, const uint32_t* lens, uint32_t B, uint32_t S,
                 uint32_t n_new, uint32_t* out_ids, double* out_logits);

/* ---- the output head's training step (transformer_network.rs:506-636 for
 * the Softmax and the vocab Linear) ---- */
/* SoftmaxLayer::backward (softmax_output_layer.rs:67-145): P [B][S][V] the
 * TRAINING softmax output, targets [B][T] (tlens[b] of them used); G [B][S][V]
 * (real; the reference stores it as Complex with im 0). */
int orc_softmax_backward(const double* P, uint32_t B, uint32_t S, uint32_t V, const uint32_t* targets,
                         const uint32_t* tlens, uint32_t T, double* G);
/* cross_entropy_loss_batch (transformer_network.rs:662-711) of P [B][S][V]; out[2] = (re, im) */
int orc_cross_entropy_loss_batch(const double* P, uint32_t B, uint32_t S, uint32_t V, const uint32_t* targets,
                                 const uint32_t* tlens, uint32_t T, double* out);
/* LinearLayer::backward (linear_layer.rs:77-128), complex arm, grouped over
 * the batch (gradient_struct.rs:360-436): X [B][S][d] the layer's input,
 * G [B][S][V], W [d][V]; dW [d][V] = sum_b conj(X_b)^T G_b, db [V] =
 * sum_b sum_s G_b[s], dX [B][S][d] = G_b conj(W)^T. */
int orc_linear_backward(const oc64* X, const double* G, const oc64* W, uint32_t B, uint32_t S, uint32_t d,
                        uint32_t V, oc64* dW, oc64* db, oc64* dX);
/* the same with a complex gradient G [B][S][V] (a layer below the head) */
int orc_linear_backward_c(const oc64* X, const oc64* G, const oc64* W, uint32_t B, uint32_t S, uint32_t d,
                          uint32_t V, oc64* dW, oc64* db, oc64* dX);
/* gelu_derivative_complex (utils/derivative.rs:48-84) */
oc64 orc_gelu_derivative(oc64 z);
/* Layer::backward of the Dense (GELU) layer (layer.rs:168-210): X [B][S][d]
 * its input, Z [B][S][F] its pre-activation X W + b, prev [B][S][F] the
 * gradient of its output, mask [B][S]; dW [d][F], db [F], dX [B][S][d]. */
int orc_dense_backward(const oc64* X, const oc64* Z, const oc64* prev, const uint32_t* mask, const oc64* W,
                       uint32_t B, uint32_t S, uint32_t d, uint32_t F, oc64* dW, oc64* db, oc64* dX);
/* LinearLayer::update_parameters (linear_layer.rs:130-175) for `batch`
 * sequences: first != 0 is the first update (no previous gradient): each
 * element's clipped gradient (clip_gradients, utils/matrix.rs:703-717), if
 * finite, descends by lr * g / batch.  Otherwise AdamW (utils/adam_w.rs:9-103)
 * from the moments mW, vW, mb, vb at time_step.  The moments are updated in
 * place. */
int orc_linear_update(oc64* W, oc64* b, uint32_t d, uint32_t V, const oc64* dW, const oc64* db, uint32_t batch,
                      oc64* mW, oc64* vW, oc64* mb, oc64* vb, int first, double lr, uint32_t time_step);

/* the rest of the reverse walk (transformer_network.rs:506-636) */
int orc_norm_backward(const oc64* x, uint64_t rows, uint32_t n, double eps, const oc64* gamma, const oc64* beta,
                      const oc64* dout, oc64* dx, oc64* dgamma, oc64* dbeta);
int orc_attention_heads_backward(const oc64* X, uint32_t B, uint32_t S, const uint32_t* mask, uint32_t H, uint32_t d,
                                 uint32_t mc, const oc64* wq, const oc64* wk, const oc64* wv, const oc64* bias_pos,
                                 const oc64* Gc, oc64* dX, oc64* dwq, oc64* dwk, oc64* dwv, oc64* dbias);
int orc_self_attention_backward(const oc64* X, uint32_t B, uint32_t S, const uint32_t* mask, uint32_t H, uint32_t d,
                                uint32_t mc, double eps, const oc64* wq, const oc64* wk, const oc64* wv,
                                const oc64* bias_pos, const oc64* gamma, const oc64* beta, const oc64* G, oc64* dX,
                                oc64* dwq, oc64* dwk, oc64* dwv, oc64* dbias, oc64* dgamma, oc64* dbeta);
int orc_rope_backward(const oc64* G, uint32_t B, uint32_t S, uint32_t d, double base, oc64* out);
int orc_embedding_update(oc64* table, uint32_t V, uint32_t d, const oc64* G, uint32_t B, uint32_t S,
                         const uint32_t* targets, const uint32_t* tlens, uint32_t T, double lr);
int orc_param_update(oc64* w, const oc64* g, oc64* m, oc64* v, uint64_t n, int first, double lr, double batch,
                     uint32_t time_step, int weight);
/* target rows T at the end of every sequence of later stateless passes (the
 * DiscreteWavelet layer compresses only the S - T input rows) */
void orc_set_target_rows(orc_net* net, uint32_t T);
int orc_dwt_backward(const oc64* G, uint32_t B, uint32_t S2, uint32_t S_in, uint32_t T, uint32_t wavelet, uint32_t d,
                     oc64* out);

/* ---- EmbeddingLayer::create_embedding (embedding_layer.rs:65-77) ---- */
/* dwt_2d_full (wavelet_transform/dwt.rs:20-34) of a rows x cols real matrix:
 * dwt_1d of every row, then of every column of the result.  out holds at
 * least (rows + 4) x (cols + 4) doubles; *out_rows, *out_cols its shape. */
int orc_dwt_2d_full(const double* x, uint32_t rows, uint32_t cols, uint32_t wavelet, uint32_t mode, double* out,
                    uint32_t* out_rows, uint32_t* out_cols);
/* get_wavelet_complex (wavelet_transform/cwt_complex.rs:195-211) with the CMOR
 * wavelet (cwt_type_resolver.rs:114-123; wavefun_complex at 2^10 points on
 * its range -8..8, cwt_complex.rs:268-289) at one scale: the n complex
 * coefficients of a real row of n. */
int orc_cwt_cmor(const double* x, uint32_t n, double scale, double fb, double fc, oc64* out);
/* create_embedding for tokens 0..vocab-1 with the project's seeded draw in
 * place of rand::rng(): src_dim values uniform in [-0.4, 0.5) (index
 * token * src_dim + k of the counter stream `stream`), then
 * decompose_in_wavelet_2d_default (network_types/wavelet_network.rs:42-135)
 * and its first scale's row.  table: vocab x *dim complex. */
int orc_embedding_wavelet(uint64_t seed, uint64_t stream, uint32_t vocab, uint32_t src_dim, oc64* table,
                          uint32_t* dim);
/* EmbeddingLayer::new (embedding_layer.rs:40-62) for an Embedding layer:
 * create_embedding for every token id, the draw on counter stream
 * (layer << 12) | 0xFFF; the decomposed width must be the layer's dim. */
int orc_init_embedding_wavelet(orc_net* net, uint32_t layer, uint64_t seed, uint32_t src_dim);

#ifdef __cplusplus
}
#endif
#endif
