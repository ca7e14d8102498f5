/*
 * mitok.h — C ABI of the MI355X token loop for the rustCrates transformer.
 *
 * The reference crate (src/neural_networks/..., Rust, CPU-only) has no
 * foreign-function boundary on this path except the OpenBLAS `zgemm_` it
 * calls (utils/matrix.rs:13-15).  This header is the boundary a Rust FFI crate
 * binds instead: each entry point names the Rust item it replaces.  The Rust
 * declarations of this header are bindings/rust/mitok-sys/src/lib.rs.
 *
 * Conventions
 *  - Complex<f64> (num-complex 0.4.6, #[repr(C)] {re, im}) crosses the ABI as
 *    two interleaved doubles; a [rows][cols] complex matrix is rows*cols*2
 *    doubles, row-major, exactly Vec<Vec<Complex<f64>>> flattened.
 *  - Weight layouts are the reference's: Linear/Dense weights [in][out]
 *    (linear_layer.rs:38, layer.rs:268), attention heads [heads][dim][head_dim]
 *    (masked_attention_head.rs:64-75), bias_pos [heads][max_ctx][max_ctx].
 *  - A NULL tensor leaves the device tensor zeroed (fill it with
 *    mitok_init_seeded); NULL gamma/beta/biases take the reference's initial
 *    values (gamma 1, beta 0: norm_layer.rs:45-50; biases 1+0i: layer.rs:269,
 *    linear_layer.rs:39).
 *  - Every call returns 0 or a MITOK_ERR_* code and never aborts; the message
 *    is in mitok_last_error() (thread-local).  Where the reference panics
 *    (NaN in GELU, non-finite FFN output, unknown token id, NaN logits), the
 *    call returns MITOK_ERR_NAN / MITOK_ERR_ARG instead.
 *  - A network is used by one thread at a time (the reference takes
 *    &mut NeuralNetwork); calls are synchronous on return.
 */
#ifndef MITOK_H
#define MITOK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MITOK_OK 0
#define MITOK_ERR_ARG 1
#define MITOK_ERR_HIP 2
#define MITOK_ERR_STATE 3
#define MITOK_ERR_NAN 4
#define MITOK_ERR_NOMEM 5

/* OperationMode (network_types/neural_network_generic.rs:17-20) */
#define MITOK_TRAINING 0
#define MITOK_PRODUCTION 1

/* mitok_set_learning_rate: every layer; mitok_get_learning_rate: the
 * network's own rate (NeuralNetwork::learning_rate) */
#define MITOK_ALL_LAYERS 0xFFFFFFFFu
#define MITOK_NETWORK_RATE 0xFFFFFFFFu

/* kernel classes for mitok_timing_enable */
#define MITOK_TIME_VOCAB 1       /* the vocab Linear (the Linear before Softmax) */
#define MITOK_TIME_LAYER_GEMM 2  /* Q/K/V and FFN projections of one-row (decode) calls */
#define MITOK_TIME_ATTENTION 3   /* attention kernels */
#define MITOK_TIME_STEP 4        /* one whole decode step (one token for every sequence) */
#define MITOK_TIME_PREFILL_GEMM 5 /* Q/K/V and FFN projections of calls with several rows per sequence */

typedef struct mitok_network mitok_network; /* NeuralNetwork (neural_network_generic.rs:23-31) */

int mitok_version(void);
const char* mitok_last_error(void);
int mitok_device_count(int* count);

/* create(...) (neural_network_generic.rs:76-88): an empty layer list on `device`. */
int mitok_network_create(int device, mitok_network** out);
void mitok_network_destroy(mitok_network* net);
int mitok_num_layers(const mitok_network* net);

/* ---- LayerEnum variants, appended in order (network_components/layer.rs:75-88) ---- */
/* EmbeddingLayer (embedding_layer.rs:24-36, forward :158-211); table [vocab][dim] */
int mitok_add_embedding(mitok_network* net, uint32_t vocab, uint32_t dim, const double* table);
/* PositionalEncodingLayer (positional_encoding_layer.rs:15-32, forward :35-99) */
int mitok_add_positional_encoding(mitok_network* net, uint32_t dim, double base);
/* NormalNormLayer (norm_layer.rs:17-62, forward :84-130) */
int mitok_add_norm(mitok_network* net, uint32_t dim, double eps, const double* gamma, const double* beta);
/* SelfAttentionLayer of `heads` MaskedAttentionHeads plus its NormalNormLayer
 * (self_attention_layer.rs:29-50, forward :55-133; masked_attention_head.rs:64-106,
 * forward :122-220).  max_ctx sizes bias_pos (the reference fixes it at 512,
 * transformer_network.rs:32) and the KV cache. */
int mitok_add_self_attention(mitok_network* net, uint32_t heads, uint32_t dim, uint32_t max_ctx, double eps,
                             const double* wq, const double* wk, const double* wv, const double* bias_pos,
                             const double* gamma, const double* beta);
/* FeedForwardLayer = Dense(GELU) -> Linear (feedforward_layer.rs:30-48, forward :56-138) */
int mitok_add_feed_forward(mitok_network* net, uint32_t dim, uint32_t hidden, const double* w1, const double* b1,
                           const double* w2, const double* b2);
/* LinearLayer (linear_layer.rs:37-54, forward :55-75); w [in][out] */
int mitok_add_linear(mitok_network* net, uint32_t in, uint32_t out, const double* w, const double* b);
/* SoftmaxLayer (softmax_output_layer.rs:30-65) */
int mitok_add_softmax(mitok_network* net, int operation_mode);
/* DiscreteWaveletLayer (network_types/wavelet_discrete_layer.rs:46-161), partial
 * mode, over rows of `dim` features.  At a prompt pass (and a stateless one)
 * it replaces each sequence's S rows by the low half of dwt_1d along the
 * sequence of every feature (wavelet_transform/dwt.rs:36-90), and the padding
 * mask by its thresholded low half (:297-313); later layers and the KV cache
 * see S' = mitok_seq_out_len rows.  A cached step's row passes through, and
 * its RoPE position still counts the uncompressed prompt (time_step,
 * transformer_network.rs:300-304).  wavelet: DiscreteWaletetType index (0 DB1,
 * 1 DB2); mode: WaveletMode index (0 ZERO, 1 CONSTANT, 2 SYMMETRIC,
 * 3 ANTISYMMETRIC, 4 REFLECT, 6 PERIODIC); is_full_mode must be 0.  Others
 * are MITOK_ERR_ARG. */
int mitok_add_discrete_wavelet(mitok_network* net, uint32_t dim, uint32_t wavelet, uint32_t mode, int is_full_mode);
/* Rows per sequence that layers [first, last) leave of a prompt pass of `seq`
 * rows (the wavelet layers compress them): the row count of mitok_predict's
 * and mitok_forward_layers' outputs. */
int mitok_seq_out_len(const mitok_network* net, uint32_t first, uint32_t last, uint32_t seq, uint32_t* out);

/* Seeded Xavier-uniform weights (initialize_weights_complex, utils/weights_initializer.rs:73-89),
 * computed on the device from a counter generator: the CPU checker holds the same values. */
int mitok_init_seeded(mitok_network* net, uint64_t seed);
/* EmbeddingLayer::new's embeddings (embedding_layer.rs:40-77) for the
 * Embedding at `layer`: for every token id, create_embedding draws src_dim
 * values uniform in [-0.4, 0.5) (here the counter generator on stream
 * (layer << 12) | 0xFFF, index id * src_dim + k, where the reference draws
 * from the unseeded rand::rng()), decomposes them with
 * decompose_in_wavelet_2d_default (network_types/wavelet_network.rs:42-135:
 * 5 levels of DB1/SYMMETRIC dwt_2d_full keeping the LL quadrant, then the
 * CMOR CWT at scales 2, 8, 16, 32) and keeps the first scale's row.  src_dim:
 * a power of two up to 4096 (512 in create_transformer) whose decomposed
 * width is the layer's dim (16 for 512). */
int mitok_init_embedding_wavelet(mitok_network* net, uint32_t layer, uint64_t seed, uint32_t src_dim);
/* Reads a weight tensor back (slots as in oracle/oracle.h; slot 3 = Re(bias_pos), n doubles). */
int mitok_get_tensor(mitok_network* net, uint32_t layer, uint32_t slot, double* out, uint64_t n);
/* Drops every KV cache (k_cache = v_cache = None, masked_attention_head.rs:54-57). */
int mitok_reset(mitok_network* net);

/* predict (transformer_network.rs:315-504).  ids [batch][seq], right-padded:
 * entries at or beyond lens[b] become PAD=1 (embedding_layer.rs:112-155).
 * time_steps [batch] or NULL: RoPE position when forward_only && > 0.
 * forward_only: KV-cache semantics (masked_attention_head.rs:135-178) and
 *   out = Re(logits) (convert_c_to_f64_3d); otherwise stateless and out = the
 *   SoftmaxLayer output for its OperationMode.
 * last_row_only: out is [batch][vocab] from each sequence's last row, else
 *   [batch][seq'][vocab] with seq' = mitok_seq_out_len (seq without wavelet layers).
 * out_padding_mask [batch][seq'] or NULL (the mask the last layer saw). */
int mitok_predict(mitok_network* net, const uint32_t* ids, const uint32_t* lens, uint32_t batch, uint32_t seq,
                  const uint32_t* time_steps, int forward_only, int last_row_only, double* out,
                  uint32_t* out_padding_mask);
/* The training pass of train (transformer_network.rs:73-79): mitok_predict with
 * forward_only = 0 when each sequence's last target_rows ids are its targets
 * (LayerInput's target_batch_ids).  Only the DiscreteWavelet layer reads them:
 * it compresses each sequence's first seq - target_rows rows and passes the
 * target rows on (wavelet_discrete_layer.rs:102-134, separate_input_target
 * :233-279), so seq' = mitok_seq_out_len(seq - target_rows) + target_rows per
 * wavelet layer.  With a wavelet layer and target_rows > 0 every sequence
 * must be unpadded (lens[b] == seq; the reference panics otherwise).
 * out_probs [batch][seq'][vocab] or NULL: the softmax output then stays on the
 * device, where mitok_cross_entropy_loss and mitok_backward read it. */
int mitok_predict_targets(mitok_network* net, const uint32_t* ids, const uint32_t* lens, uint32_t batch, uint32_t seq,
                          uint32_t target_rows, double* out_probs, uint32_t* out_padding_mask);
/* cross_entropy_loss_batch (transformer_network.rs:662-711), which train
 * (:81) computes on predict's softmax output, computed on the device from the
 * output the last stateless predict left there, so the [batch][seq'][vocab]
 * probabilities need not cross PCIe.  targets [batch][max_t] (target_lens[b]
 * used of each row, max_t <= 8192), the same arrays mitok_backward takes.
 * out_loss[2] = the complex loss (re, im): per sequence the mean of
 * -ln(p + 1e-15) over its non-PAD targets (p at row seq' - len - 1 + t),
 * then the mean over the batch.  MITOK_ERR_ARG where the reference would
 * panic (a target id >= vocab, fewer than len + 1 rows); the forward pass
 * stays valid for mitok_backward. */
int mitok_cross_entropy_loss(mitok_network* net, const uint32_t* targets, const uint32_t* target_lens, uint32_t batch,
                             uint32_t max_t, double* out_loss);

/* Layers [first, last) on hidden states: in [batch][seq][dim_in] complex,
 * out [batch][seq][dim_out] complex; padding_mask [batch][seq] or NULL (all 1).
 * This is each layer's forward(&LayerInput) -> LayerOutput chained. */
int mitok_forward_layers(mitok_network* net, uint32_t first, uint32_t last, const double* in,
                         const uint32_t* padding_mask, uint32_t batch, uint32_t seq, const uint32_t* time_steps,
                         int forward_only, double* out);
/* mitok_forward_layers on device buffers (the per-layer drop-in for a caller
 * whose hidden states stay on the GPU): d_in and d_out are device memory of the
 * network's GPU (hipMalloc), d_out [batch][seq'][dim_out] with
 * seq' = mitok_seq_out_len.  padding_mask and time_steps stay host arrays.  A
 * pointer that is not device memory of that GPU, or an allocation too small
 * for the shape, is MITOK_ERR_ARG. */
int mitok_forward_layers_device(mitok_network* net, uint32_t first, uint32_t last, const double* d_in,
                                const uint32_t* padding_mask, uint32_t batch, uint32_t seq,
                                const uint32_t* time_steps, int forward_only, double* d_out);

/* Greedy token loop on ids (predict_token_by_token, transformer_network.rs:165-313,
 * without the text tokenizer): resets the caches, runs the prompt, then feeds
 * each greedy id back for n_new tokens in total.  Sequence b of a batch is an
 * independent batch-1 run.  Only token ids cross PCIe per step.
 * out_ids [batch][n_new]; out_logits [n_new][batch][vocab] or NULL. */
int mitok_generate(mitok_network* net, const uint32_t* prompt, const uint32_t* lens, uint32_t batch, uint32_t seq,
                   uint32_t n_new, uint32_t* out_ids, double* out_logits);

/* The token loop one step at a time, for a host loop that inspects every id
 * (predict_token_by_token, transformer_network.rs:225-304: the prompt at t = 0,
 * then one fed token per step, the "<eos>" check and the print per token on the
 * host).  Only ids cross PCIe: 4 B per sequence per step.
 * mitok_prefill: resets the caches (k_cache = None) and runs the prompt
 *   (ids [batch][seq] right-padded as for mitok_predict); out_ids [batch] = the
 *   greedy id of each sequence's last prompt row; out_logits [batch][vocab]
 *   Re-logits of that row, or NULL.
 * mitok_decode_step: feeds ids [batch] (NULL: the ids the previous prefill or
 *   step returned, already on the device) at position = each sequence's KV
 *   length, appends to the caches; out_ids [batch] = the next greedy ids;
 *   out_logits [batch][vocab] or NULL.  batch must equal the prefill's.
 * On error the caches are dropped (prefill again). */
int mitok_prefill(mitok_network* net, const uint32_t* prompt, const uint32_t* lens, uint32_t batch, uint32_t seq,
                  uint32_t* out_ids, double* out_logits);
int mitok_decode_step(mitok_network* net, const uint32_t* ids, uint32_t batch, uint32_t* out_ids, double* out_logits);

/* The output head's training step: backward (transformer_network.rs:506-636)
 * through the Softmax and the vocab Linear of the last stateless predict
 * (forward_only = 0; any other call in between is MITOK_ERR_STATE).
 * SoftmaxLayer::backward (softmax_output_layer.rs:67-145): targets [batch][T],
 * tlens[b] of them used; the cross-entropy gradient of the softmax output
 * rows that predict them.  LinearLayer::backward (linear_layer.rs:77-128):
 * dW = conj(X)^T G, db = column sums, and out_grad_input [batch][seq'][d_in]
 * (complex) = G conj(W)^T, or NULL.  update_params: LinearLayer::
 * update_parameters (linear_layer.rs:130-175) at learning_rate: the layer's
 * first update descends by the clipped gradient / batch, later ones run
 * AdamW (utils/adam_w.rs:9-103) at time_step.  The weights stay on the
 * device (mitok_get_tensor reads them).  The layers below the vocab Linear
 * are not differentiated. */
int mitok_backward_head(mitok_network* net, const uint32_t* targets, const uint32_t* tlens, uint32_t batch, uint32_t T,
                        int update_params, double learning_rate, uint32_t time_step, double* out_grad_input);
/* The same reverse walk (transformer_network.rs:506-636) through n_layers
 * layers below the Softmax: 1 = the vocab Linear (mitok_backward_head), up to
 * every layer the stateless predict ran.  Each layer's backward and, with
 * update_params, its update_parameters where the walk calls it:
 *  - Linear: as above, at time_step;
 *  - FeedForward (feedforward_layer.rs:140-186, 219-250): its Linear at
 *    time_step, then its Dense with the GELU derivative of
 *    utils/derivative.rs:48-84 at step 1 (Layer::time_step is never set,
 *    layer.rs:111,285);
 *  - SelfAttention (self_attention_layer.rs:135-196, 260-273): its Norm's
 *    backward (norm_layer.rs:132-209), then every head
 *    (masked_attention_head.rs:222-345); updates the Norm's gamma and beta,
 *    wq / wk / wv and Re(bias_pos) on the pass's S x S slice;
 *  - Norm (backward only), PositionalEncoding (positional_encoding_layer.rs:
 *    101-144);
 *  - Embedding: passes the gradient on; with update_params
 *    EmbeddingLayer::update_parameters (embedding_layer.rs:223-264) moves and
 *    renormalizes the table rows of the target ids.
 *  - DiscreteWavelet (wavelet_discrete_layer.rs:163-207): the gradient of
 *    the compressed rows through decompress_partial (grad_dwt_1d_trend) and
 *    align_gradient_rows_complex, the target rows' gradient passed through.
 * out_grad_input: the gradient of the lowest walked layer's input
 * [batch][rows of that layer's input][its d_in], or NULL. */
int mitok_backward(mitok_network* net, const uint32_t* targets, const uint32_t* tlens, uint32_t batch, uint32_t T,
                   uint32_t n_layers, int update_params, double learning_rate, uint32_t time_step,
                   double* out_grad_input);

/* backward(transformer_network, target_ids, update_params) as train calls it
 * (transformer_network.rs:129, 506-636): the whole reverse walk over every
 * layer the last stateless predict ran, each layer updated at its own
 * learning rate (mitok_set_learning_rate) and the Embedding at the network's
 * (transformer_network.rs:520, mitok_set_network_learning_rate); otherwise as
 * mitok_backward. */
int mitok_backward_walk(mitok_network* net, const uint32_t* targets, const uint32_t* tlens, uint32_t batch, uint32_t T,
                        int update_params, uint32_t time_step, double* out_grad_input);

/* Learning rates (neural_network_generic.rs:57-73, 115-186).  Every layer
 * starts at 0.01 (create_transformer's rate, transformer_builder.rs:16), the
 * network too.  mitok_set_learning_rate(net, MITOK_ALL_LAYERS, lr) is
 * update_learning_rate (what update_step_lr_scheduler calls); with a layer
 * index it sets that layer's field (a SelfAttention's heads and Norm, a
 * FeedForward's Dense and Linear together).  mitok_set_network_learning_rate
 * sets NeuralNetwork::learning_rate, which decay_learning_rate halves and the
 * Embedding's update reads; mitok_get_learning_rate(net, MITOK_NETWORK_RATE)
 * reads it back. */
int mitok_set_learning_rate(mitok_network* net, uint32_t layer, double learning_rate);
int mitok_get_learning_rate(const mitok_network* net, uint32_t layer, double* out);
int mitok_set_network_learning_rate(mitok_network* net, double learning_rate);
/* reset_previous_gradient (neural_network_generic.rs:188-242), which train
 * calls when the loss keeps rising (transformer_network.rs:147-151): the next
 * update of every Linear, FeedForward sublayer and attention head is the
 * clipped descent again, and the AdamW after it starts from zero moments.  An
 * attention layer's Norm keeps its moments, as in the reference. */
int mitok_reset_previous_gradient(mitok_network* net);

/* greedy_decoding (src/utils/sampling_methods.rs:5-18) on the device for host
 * logits [rows][vocab]: last index among equal maxima; NaN -> MITOK_ERR_NAN. */
int mitok_greedy_decoding(mitok_network* net, const double* logits, uint32_t rows, uint32_t vocab, uint32_t* out_ids);
/* greedy_decoding on device buffers: d_logits [rows][vocab] f64 and d_out_ids
 * [rows] are device memory of the network's GPU, checked as for
 * mitok_forward_layers_device. */
int mitok_greedy_decoding_device(mitok_network* net, const double* d_logits, uint32_t rows, uint32_t vocab,
                                 uint32_t* d_out_ids);

/* mitok_greedy_decoding without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  It copies the host logits
 * in and synchronises the network's stream before it returns, so it must not
 * be called while that stream is being captured into a graph, and it is not
 * recorded into a capture on another stream.  The logits and ids are staged in a
 * fixed per-GPU array of the library (8 MiB + 16 KiB, held by every GPU the
 * library runs on until the process ends): rows * vocab <= 1048576 and
 * rows <= 4096, else MITOK_ERR_ARG.  All calls on one GPU share that array, so
 * calls that overlap on one GPU (two networks on one device used from two
 * threads) race; calls through one network are serialised by its stream. */
int mitok_greedy_decoding_noalloc(mitok_network* net, const double* logits, uint32_t rows, uint32_t vocab,
                                  uint32_t* out_ids);

/* ---- measurement (no reference counterpart: the reference prints wall
 * clock only, transformer_network.rs:307-310) ---- */
/* Wall time of the last mitok_generate on the device stream, in ms:
 * t[0] prefill (prompt forward + first id), t[1] all decode steps, t[2] how
 * the decode steps ran: 0 direct launches, 1 a replayed HIP graph, 2 the
 * resident loop. */
int mitok_last_timings(mitok_network* net, double* t3);
/* HIP-event timing of one kernel class during the following calls (0 disables;
 * decode steps then run without graph replay so each launch is bracketed). */
int mitok_timing_enable(mitok_network* net, int kernel_class);
/* Accumulated since enable: total ms, launches, and the algorithmic HBM bytes
 * and real flops of those launches (any pointer may be NULL). */
int mitok_timing_read(mitok_network* net, double* total_ms, uint64_t* launches, double* alg_bytes, double* alg_flops);
/* hipDeviceSynchronize on `device` (bench brackets its timed region with it). */
int mitok_device_synchronize(int device);
/* 0 = replay decode steps as HIP graphs (default), 1 = launch kernels directly. */
int mitok_set_graph_mode(mitok_network* net, int direct_launch);
/* 3 = generate's decode loop for up to 8 sequences runs as one resident
 *     cooperative launch (one block per CU; how its blocks exchange values:
 *     mitok_resident_exchange);
 * 2 = the resident loop for 1 and 2 sequences (1 if the polling exchange is
 *     off or a RoPE layer rules it out), plan 1 above (default);
 * 1 = decode steps of up to 64 sequences run the fused plan (up to 8: GEMV
 *     products with the row transforms in their prologues; 9 to 64: skinny
 *     MFMA products after a row-transform launch), replayed as a graph;
 * 0 = one launch per reference operation and one query row per attention block.
 * Plans 1 to 3 run prefill attention on the tiled kernel.
 * No counterpart in the reference (a scheduling choice; results agree to the
 * parity tolerance). */
int mitok_set_decode_plan(mitok_network* net, int plan);
/* Per-operation profile of the resident decode loop (plan 2).  enable = 1:
 * later launches record block 0's clock after every grid barrier.  Then, if
 * nops is not NULL, reports the last launch's operations (at most max_ops):
 * kinds[i] (0 product, 1 attention chunks with their combine, 2 row transform) and
 * us[i], the microseconds from the previous barrier to the one after op i,
 * averaged over the steps.  No counterpart in the reference (instrumentation). */
int mitok_resident_profile(mitok_network* net, int enable, int max_ops, int* nops, int* kinds, double* us);
/* How the blocks of the resident decode loop hand values to each other.
 * mode 1 (default): polling -- every exchanged value starts a step as a
 * sentinel and its reader re-reads it until written, one grid barrier per
 * step -- where the program allows it (no RoPE); mode 0: a grid barrier
 * after every operation.  mode -1 leaves it unchanged.  *polled (if not
 * NULL): whether the last resident launch polled.  No counterpart in the
 * reference (a scheduling choice; the arithmetic is the same either way). */
int mitok_resident_exchange(mitok_network* net, int mode, int* polled);

#ifdef __cplusplus
}
#endif
#endif
