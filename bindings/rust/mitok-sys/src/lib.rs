//! FFI declarations of `include/mitok.h` and a safe owning handle.
//!
//! The transformer crate's token loop (`predict_token_by_token`,
//! `network_types/transformer/transformer_network.rs:165-313`) and its forward
//! pass (`predict`, `:315-504`) call into this crate when a network has been
//! uploaded to a GPU.  `Complex<f64>` is `#[repr(C)] {re, im}` in num-complex
//! 0.4.6, so a `[rows][cols]` complex matrix flattened row-major is the
//! `*const c_double` of `rows * cols * 2` doubles the ABI takes.
//!
//! Every entry point returns `MITOK_OK` or a `MITOK_ERR_*` code; the message is
//! in `mitok_last_error()` (thread-local).  Where the reference panics (NaN in
//! GELU, a non-finite FFN output, an unknown token id, NaN logits), the call
//! returns an error instead; `Network` turns it into `Err(MitokError)`.

use num_complex::Complex;
use std::ffi::CStr;
use std::os::raw::{c_char, c_double, c_int};

pub mod transformer;

pub const MITOK_OK: c_int = 0;
pub const MITOK_ERR_ARG: c_int = 1;
pub const MITOK_ERR_HIP: c_int = 2;
pub const MITOK_ERR_STATE: c_int = 3;
pub const MITOK_ERR_NAN: c_int = 4;
pub const MITOK_ERR_NOMEM: c_int = 5;

/// OperationMode (network_types/neural_network_generic.rs:17-20)
pub const MITOK_TRAINING: c_int = 0;
pub const MITOK_PRODUCTION: c_int = 1;

/// mitok_set_learning_rate's "every layer" and mitok_get_learning_rate's
/// "the network's own rate"
pub const MITOK_ALL_LAYERS: u32 = 0xFFFF_FFFF;
pub const MITOK_NETWORK_RATE: u32 = 0xFFFF_FFFF;

pub const MITOK_TIME_VOCAB: c_int = 1;
pub const MITOK_TIME_LAYER_GEMM: c_int = 2;
pub const MITOK_TIME_ATTENTION: c_int = 3;
pub const MITOK_TIME_STEP: c_int = 4;
pub const MITOK_TIME_PREFILL_GEMM: c_int = 5;

/// Opaque device network (`NeuralNetwork`, neural_network_generic.rs:23-31).
#[repr(C)]
pub struct MitokNetwork {
    _p: [u8; 0],
}

extern "C" {
    pub fn mitok_version() -> c_int;
    pub fn mitok_last_error() -> *const c_char;
    pub fn mitok_device_count(count: *mut c_int) -> c_int;

    pub fn mitok_network_create(device: c_int, out: *mut *mut MitokNetwork) -> c_int;
    pub fn mitok_network_destroy(net: *mut MitokNetwork);
    pub fn mitok_num_layers(net: *const MitokNetwork) -> c_int;

    // LayerEnum variants, appended in network order (network_components/layer.rs:75-88)
    pub fn mitok_add_embedding(net: *mut MitokNetwork, vocab: u32, dim: u32, table: *const c_double) -> c_int;
    pub fn mitok_add_positional_encoding(net: *mut MitokNetwork, dim: u32, base: c_double) -> c_int;
    pub fn mitok_add_norm(net: *mut MitokNetwork, dim: u32, eps: c_double, gamma: *const c_double,
                          beta: *const c_double) -> c_int;
    pub fn mitok_add_self_attention(net: *mut MitokNetwork, heads: u32, dim: u32, max_ctx: u32, eps: c_double,
                                    wq: *const c_double, wk: *const c_double, wv: *const c_double,
                                    bias_pos: *const c_double, gamma: *const c_double,
                                    beta: *const c_double) -> c_int;
    pub fn mitok_add_feed_forward(net: *mut MitokNetwork, dim: u32, hidden: u32, w1: *const c_double,
                                  b1: *const c_double, w2: *const c_double, b2: *const c_double) -> c_int;
    pub fn mitok_add_linear(net: *mut MitokNetwork, inp: u32, out: u32, w: *const c_double,
                            b: *const c_double) -> c_int;
    pub fn mitok_add_softmax(net: *mut MitokNetwork, operation_mode: c_int) -> c_int;
    pub fn mitok_add_discrete_wavelet(net: *mut MitokNetwork, dim: u32, wavelet: u32, mode: u32,
                                      is_full_mode: c_int) -> c_int;
    pub fn mitok_seq_out_len(net: *const MitokNetwork, first: u32, last: u32, seq: u32, out: *mut u32) -> c_int;

    pub fn mitok_init_seeded(net: *mut MitokNetwork, seed: u64) -> c_int;
    pub fn mitok_init_embedding_wavelet(net: *mut MitokNetwork, layer: u32, seed: u64, src_dim: u32) -> c_int;
    pub fn mitok_get_tensor(net: *mut MitokNetwork, layer: u32, slot: u32, out: *mut c_double, n: u64) -> c_int;
    pub fn mitok_reset(net: *mut MitokNetwork) -> c_int;

    pub fn mitok_predict(net: *mut MitokNetwork, ids: *const u32, lens: *const u32, batch: u32, seq: u32,
                         time_steps: *const u32, forward_only: c_int, last_row_only: c_int, out: *mut c_double,
                         out_padding_mask: *mut u32) -> c_int;
    pub fn mitok_predict_targets(net: *mut MitokNetwork, ids: *const u32, lens: *const u32, batch: u32, seq: u32,
                                 target_rows: u32, out_probs: *mut c_double, out_padding_mask: *mut u32) -> c_int;
    pub fn mitok_cross_entropy_loss(net: *mut MitokNetwork, targets: *const u32, target_lens: *const u32, batch: u32,
                                    max_t: u32, out_loss: *mut c_double) -> c_int;
    pub fn mitok_forward_layers(net: *mut MitokNetwork, first: u32, last: u32, inp: *const c_double,
                                padding_mask: *const u32, batch: u32, seq: u32, time_steps: *const u32,
                                forward_only: c_int, out: *mut c_double) -> c_int;
    pub fn mitok_forward_layers_device(net: *mut MitokNetwork, first: u32, last: u32, d_in: *const c_double,
                                       padding_mask: *const u32, batch: u32, seq: u32, time_steps: *const u32,
                                       forward_only: c_int, d_out: *mut c_double) -> c_int;
    pub fn mitok_generate(net: *mut MitokNetwork, prompt: *const u32, lens: *const u32, batch: u32, seq: u32,
                          n_new: u32, out_ids: *mut u32, out_logits: *mut c_double) -> c_int;
    pub fn mitok_prefill(net: *mut MitokNetwork, prompt: *const u32, lens: *const u32, batch: u32, seq: u32,
                         out_ids: *mut u32, out_logits: *mut c_double) -> c_int;
    pub fn mitok_decode_step(net: *mut MitokNetwork, ids: *const u32, batch: u32, out_ids: *mut u32,
                             out_logits: *mut c_double) -> c_int;
    pub fn mitok_backward_head(net: *mut MitokNetwork, targets: *const u32, tlens: *const u32, batch: u32, t: u32,
                               update_params: c_int, learning_rate: c_double, time_step: u32,
                               out_grad_input: *mut c_double) -> c_int;
    pub fn mitok_backward(net: *mut MitokNetwork, targets: *const u32, tlens: *const u32, batch: u32, t: u32,
                          n_layers: u32, update_params: c_int, learning_rate: c_double, time_step: u32,
                          out_grad_input: *mut c_double) -> c_int;
    pub fn mitok_backward_walk(net: *mut MitokNetwork, targets: *const u32, tlens: *const u32, batch: u32, t: u32,
                               update_params: c_int, time_step: u32, out_grad_input: *mut c_double) -> c_int;
    pub fn mitok_set_learning_rate(net: *mut MitokNetwork, layer: u32, learning_rate: c_double) -> c_int;
    pub fn mitok_get_learning_rate(net: *const MitokNetwork, layer: u32, out: *mut c_double) -> c_int;
    pub fn mitok_set_network_learning_rate(net: *mut MitokNetwork, learning_rate: c_double) -> c_int;
    pub fn mitok_reset_previous_gradient(net: *mut MitokNetwork) -> c_int;
    pub fn mitok_greedy_decoding(net: *mut MitokNetwork, logits: *const c_double, rows: u32, vocab: u32,
                                 out_ids: *mut u32) -> c_int;
    pub fn mitok_greedy_decoding_device(net: *mut MitokNetwork, d_logits: *const c_double, rows: u32, vocab: u32,
                                        d_out_ids: *mut u32) -> c_int;
    // No counterpart in the reference: greedy_decoding for callers that cannot
    // allocate device memory.  Stages in a fixed per-GPU array (8 MiB + 16 KiB):
    // rows * vocab <= 1048576 and rows <= 4096; overlapping calls on one GPU race.
    pub fn mitok_greedy_decoding_noalloc(net: *mut MitokNetwork, logits: *const c_double, rows: u32, vocab: u32,
                                         out_ids: *mut u32) -> c_int;

    // measurement and scheduling (no counterpart in the reference)
    pub fn mitok_last_timings(net: *mut MitokNetwork, t3: *mut c_double) -> c_int;
    pub fn mitok_timing_enable(net: *mut MitokNetwork, kernel_class: c_int) -> c_int;
    pub fn mitok_timing_read(net: *mut MitokNetwork, total_ms: *mut c_double, launches: *mut u64,
                             alg_bytes: *mut c_double, alg_flops: *mut c_double) -> c_int;
    pub fn mitok_device_synchronize(device: c_int) -> c_int;
    pub fn mitok_set_graph_mode(net: *mut MitokNetwork, direct_launch: c_int) -> c_int;
    pub fn mitok_set_decode_plan(net: *mut MitokNetwork, plan: c_int) -> c_int;
    pub fn mitok_resident_profile(net: *mut MitokNetwork, enable: c_int, max_ops: c_int, nops: *mut c_int,
                                  kinds: *mut c_int, us: *mut c_double) -> c_int;
    pub fn mitok_resident_exchange(net: *mut MitokNetwork, mode: c_int, polled: *mut c_int) -> c_int;
}

/// A non-zero status and the library's message for it.
#[derive(Debug, Clone)]
pub struct MitokError {
    pub code: c_int,
    pub message: String,
}

impl std::fmt::Display for MitokError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "mitok error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for MitokError {}

fn check(rc: c_int) -> Result<(), MitokError> {
    if rc == MITOK_OK {
        return Ok(());
    }
    let message = unsafe {
        let p = mitok_last_error();
        if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
    };
    Err(MitokError { code: rc, message })
}

fn flat(m: &[Vec<Complex<f64>>]) -> Vec<Complex<f64>> {
    m.iter().flat_map(|r| r.iter().copied()).collect()
}

/// Owns one device network; dropped with `mitok_network_destroy`.
pub struct Network {
    raw: *mut MitokNetwork,
    vocab: u32,
}

// One thread at a time (the reference takes &mut NeuralNetwork); moving the
// handle between threads is fine.
unsafe impl Send for Network {}

impl Drop for Network {
    fn drop(&mut self) {
        unsafe { mitok_network_destroy(self.raw) }
    }
}

impl Network {
    pub fn new(device: i32) -> Result<Self, MitokError> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { mitok_network_create(device, &mut raw) })?;
        Ok(Network { raw, vocab: 0 })
    }

    pub fn raw(&self) -> *mut MitokNetwork {
        self.raw
    }

    pub fn vocab(&self) -> u32 {
        self.vocab
    }

    /// EmbeddingLayer: `table` [vocab][dim] (embedding_layer.rs:24-36).
    pub fn add_embedding(&mut self, table: &[Vec<Complex<f64>>]) -> Result<(), MitokError> {
        let (v, d) = (table.len() as u32, table.first().map_or(0, |r| r.len()) as u32);
        let t = flat(table);
        check(unsafe { mitok_add_embedding(self.raw, v, d, t.as_ptr() as *const c_double) })
    }

    pub fn add_positional_encoding(&mut self, dim: u32, base: f64) -> Result<(), MitokError> {
        check(unsafe { mitok_add_positional_encoding(self.raw, dim, base) })
    }

    pub fn add_norm(&mut self, dim: u32, eps: f64, gamma: &[Complex<f64>], beta: &[Complex<f64>])
                    -> Result<(), MitokError> {
        check(unsafe {
            mitok_add_norm(self.raw, dim, eps, gamma.as_ptr() as *const c_double, beta.as_ptr() as *const c_double)
        })
    }

    /// SelfAttentionLayer: per head `[d][dh]` projections stacked to
    /// `[heads][d][dh]`, `bias_pos` [heads][max_ctx][max_ctx] (complex), and the
    /// layer's NormalNormLayer gamma/beta.
    #[allow(clippy::too_many_arguments)]
    pub fn add_self_attention(&mut self, heads: u32, dim: u32, max_ctx: u32, eps: f64,
                              wq: &[Complex<f64>], wk: &[Complex<f64>], wv: &[Complex<f64>],
                              bias_pos: &[Complex<f64>], gamma: &[Complex<f64>], beta: &[Complex<f64>])
                              -> Result<(), MitokError> {
        check(unsafe {
            mitok_add_self_attention(self.raw, heads, dim, max_ctx, eps, wq.as_ptr() as *const c_double,
                                     wk.as_ptr() as *const c_double, wv.as_ptr() as *const c_double,
                                     bias_pos.as_ptr() as *const c_double, gamma.as_ptr() as *const c_double,
                                     beta.as_ptr() as *const c_double)
        })
    }

    pub fn add_feed_forward(&mut self, w1: &[Vec<Complex<f64>>], b1: &[Complex<f64>], w2: &[Vec<Complex<f64>>],
                            b2: &[Complex<f64>]) -> Result<(), MitokError> {
        let (d, f) = (w1.len() as u32, b1.len() as u32);
        let (a, b) = (flat(w1), flat(w2));
        check(unsafe {
            mitok_add_feed_forward(self.raw, d, f, a.as_ptr() as *const c_double, b1.as_ptr() as *const c_double,
                                   b.as_ptr() as *const c_double, b2.as_ptr() as *const c_double)
        })
    }

    pub fn add_linear(&mut self, w: &[Vec<Complex<f64>>], b: &[Complex<f64>]) -> Result<(), MitokError> {
        let (i, o) = (w.len() as u32, b.len() as u32);
        let m = flat(w);
        check(unsafe { mitok_add_linear(self.raw, i, o, m.as_ptr() as *const c_double, b.as_ptr() as *const c_double) })?;
        self.vocab = o;
        Ok(())
    }

    pub fn add_softmax(&mut self, operation_mode: c_int) -> Result<(), MitokError> {
        check(unsafe { mitok_add_softmax(self.raw, operation_mode) })
    }

    /// DiscreteWaveletLayer in partial mode (wavelet_discrete_layer.rs:46-161).
    pub fn add_discrete_wavelet(&mut self, dim: u32, wavelet: u32, mode: u32) -> Result<(), MitokError> {
        check(unsafe { mitok_add_discrete_wavelet(self.raw, dim, wavelet, mode, 0) })
    }

    pub fn reset(&mut self) -> Result<(), MitokError> {
        check(unsafe { mitok_reset(self.raw) })
    }

    fn out_rows(&self, seq: u32) -> Result<u32, MitokError> {
        let mut s = 0u32;
        let n = unsafe { mitok_num_layers(self.raw) } as u32;
        check(unsafe { mitok_seq_out_len(self.raw, 0, n, seq, &mut s) })?;
        Ok(s)
    }

    /// The entries of the layer list (LayerEnum order).
    pub fn num_layers(&self) -> u32 {
        let n = unsafe { mitok_num_layers(self.raw) };
        n.max(0) as u32
    }

    /// predict_targets with the softmax output left on the device, where
    /// cross_entropy_loss and backward read it: only the ids cross PCIe.
    pub fn forward_targets(&mut self, batch_ids: &[Vec<u32>], target_rows: u32) -> Result<(), MitokError> {
        let b = batch_ids.len() as u32;
        let s = batch_ids.iter().map(|r| r.len()).max().unwrap_or(0) as u32;
        let lens: Vec<u32> = batch_ids.iter().map(|r| r.len() as u32).collect();
        let mut ids = vec![1u32; (b * s) as usize];
        for (i, r) in batch_ids.iter().enumerate() {
            ids[i * s as usize..i * s as usize + r.len()].copy_from_slice(r);
        }
        check(unsafe {
            mitok_predict_targets(self.raw, ids.as_ptr(), lens.as_ptr(), b, s, target_rows, std::ptr::null_mut(),
                                  std::ptr::null_mut())
        })
    }

    /// `predict` on right-padded ids: Re-logits [batch][seq'][vocab] when
    /// `forward_only` (the KV caches advance), else the softmax output; and the
    /// padding mask [batch][seq'].
    pub fn predict(&mut self, batch_ids: &[Vec<u32>], time_step: Option<u32>, forward_only: bool)
                   -> Result<(Vec<Vec<Vec<f64>>>, Vec<Vec<u32>>), MitokError> {
        let b = batch_ids.len() as u32;
        let s = batch_ids.iter().map(|r| r.len()).max().unwrap_or(0) as u32;
        let lens: Vec<u32> = batch_ids.iter().map(|r| r.len() as u32).collect();
        let mut ids = vec![1u32; (b * s) as usize]; // PAD = 1 (embedding_layer.rs:112-155)
        for (i, r) in batch_ids.iter().enumerate() {
            ids[i * s as usize..i * s as usize + r.len()].copy_from_slice(r);
        }
        let ts: Vec<u32> = vec![time_step.unwrap_or(0); b as usize];
        let so = self.out_rows(s)?;
        let v = self.vocab as usize;
        let mut out = vec![0f64; b as usize * so as usize * v];
        let mut mask = vec![0u32; b as usize * so as usize];
        check(unsafe {
            mitok_predict(self.raw, ids.as_ptr(), lens.as_ptr(), b, s,
                          if time_step.is_some() { ts.as_ptr() } else { std::ptr::null() },
                          forward_only as c_int, 0, out.as_mut_ptr(), mask.as_mut_ptr())
        })?;
        let logits = out
            .chunks(so as usize * v)
            .map(|seq| seq.chunks(v).map(|r| r.to_vec()).collect())
            .collect();
        let m = mask.chunks(so as usize).map(|r| r.to_vec()).collect();
        Ok((logits, m))
    }

    /// train's forward pass (transformer_network.rs:73-79): the stateless
    /// predict of unpadded sequences whose last `target_rows` ids are the
    /// targets (a DiscreteWavelet layer passes them on uncompressed).  The
    /// softmax output [batch][seq'][vocab] and the padding mask; seq' assumes at
    /// most one wavelet layer, as create_transformer builds.
    pub fn predict_targets(&mut self, batch_ids: &[Vec<u32>], target_rows: u32)
                           -> Result<(Vec<Vec<Vec<f64>>>, Vec<Vec<u32>>), MitokError> {
        let b = batch_ids.len() as u32;
        let s = batch_ids.iter().map(|r| r.len()).max().unwrap_or(0) as u32;
        let lens: Vec<u32> = batch_ids.iter().map(|r| r.len() as u32).collect();
        let mut ids = vec![1u32; (b * s) as usize];
        for (i, r) in batch_ids.iter().enumerate() {
            ids[i * s as usize..i * s as usize + r.len()].copy_from_slice(r);
        }
        let t = target_rows.min(s);
        let inner = self.out_rows(s - t)?;
        let so = if inner != s - t { inner + t } else { s };
        let v = self.vocab as usize;
        let mut out = vec![0f64; b as usize * so as usize * v];
        let mut mask = vec![0u32; b as usize * so as usize];
        check(unsafe {
            mitok_predict_targets(self.raw, ids.as_ptr(), lens.as_ptr(), b, s, target_rows, out.as_mut_ptr(),
                                  mask.as_mut_ptr())
        })?;
        let probs = out
            .chunks(so as usize * v)
            .map(|seq| seq.chunks(v).map(|r| r.to_vec()).collect())
            .collect();
        let m = mask.chunks(so as usize).map(|r| r.to_vec()).collect();
        Ok((probs, m))
    }

    /// cross_entropy_loss_batch (transformer_network.rs:662-711) of the softmax
    /// output the last predict_targets left on the device: train's loss
    /// (:81) without the probabilities crossing PCIe.
    pub fn cross_entropy_loss(&mut self, targets: &[Vec<u32>]) -> Result<Complex<f64>, MitokError> {
        let b = targets.len() as u32;
        let t = targets.iter().map(|r| r.len()).max().unwrap_or(0).max(1) as u32;
        let tlens: Vec<u32> = targets.iter().map(|r| r.len() as u32).collect();
        let mut flat = vec![1u32; (b * t) as usize];
        for (i, r) in targets.iter().enumerate() {
            flat[i * t as usize..i * t as usize + r.len()].copy_from_slice(r);
        }
        let mut out = [0f64; 2];
        check(unsafe { mitok_cross_entropy_loss(self.raw, flat.as_ptr(), tlens.as_ptr(), b, t, out.as_mut_ptr()) })?;
        Ok(Complex::new(out[0], out[1]))
    }

    /// backward (transformer_network.rs:506-636) over `n_layers` layers below
    /// the Softmax (num_layers - 1: all of them, the embedding update
    /// included), with update_parameters when `update`; time_step is train's
    /// epoch.  The targets are train's target ids, one Vec per sequence.
    pub fn backward(&mut self, targets: &[Vec<u32>], n_layers: u32, update: bool, learning_rate: f64,
                    time_step: u32) -> Result<(), MitokError> {
        let b = targets.len() as u32;
        let t = targets.iter().map(|r| r.len()).max().unwrap_or(0).max(1) as u32;
        let tlens: Vec<u32> = targets.iter().map(|r| r.len() as u32).collect();
        let mut flat = vec![1u32; (b * t) as usize];
        for (i, r) in targets.iter().enumerate() {
            flat[i * t as usize..i * t as usize + r.len()].copy_from_slice(r);
        }
        check(unsafe {
            mitok_backward(self.raw, flat.as_ptr(), tlens.as_ptr(), b, t, n_layers, update as c_int, learning_rate,
                           time_step, std::ptr::null_mut())
        })
    }

    /// backward(transformer_network, target_ids, update_params) as train calls
    /// it (transformer_network.rs:129): every layer, each at its own learning
    /// rate and the Embedding at the network's.
    pub fn backward_walk(&mut self, targets: &[Vec<u32>], update: bool, time_step: u32) -> Result<(), MitokError> {
        let b = targets.len() as u32;
        let t = targets.iter().map(|r| r.len()).max().unwrap_or(0).max(1) as u32;
        let tlens: Vec<u32> = targets.iter().map(|r| r.len() as u32).collect();
        let mut flat = vec![1u32; (b * t) as usize];
        for (i, r) in targets.iter().enumerate() {
            flat[i * t as usize..i * t as usize + r.len()].copy_from_slice(r);
        }
        check(unsafe {
            mitok_backward_walk(self.raw, flat.as_ptr(), tlens.as_ptr(), b, t, update as c_int, time_step,
                                std::ptr::null_mut())
        })
    }

    /// update_learning_rate (neural_network_generic.rs:115-186): every layer.
    pub fn update_learning_rate(&mut self, learning_rate: f64) -> Result<(), MitokError> {
        check(unsafe { mitok_set_learning_rate(self.raw, MITOK_ALL_LAYERS, learning_rate) })
    }

    /// One layer's learning_rate field.
    pub fn set_layer_learning_rate(&mut self, layer: u32, learning_rate: f64) -> Result<(), MitokError> {
        check(unsafe { mitok_set_learning_rate(self.raw, layer, learning_rate) })
    }

    /// NeuralNetwork::learning_rate (the Embedding's update rate).
    pub fn learning_rate(&self) -> Result<f64, MitokError> {
        let mut out = 0.0;
        check(unsafe { mitok_get_learning_rate(self.raw, MITOK_NETWORK_RATE, &mut out) })?;
        Ok(out)
    }

    pub fn set_learning_rate(&mut self, learning_rate: f64) -> Result<(), MitokError> {
        check(unsafe { mitok_set_network_learning_rate(self.raw, learning_rate) })
    }

    /// reset_previous_gradient (neural_network_generic.rs:188-242).
    pub fn reset_previous_gradient(&mut self) -> Result<(), MitokError> {
        check(unsafe { mitok_reset_previous_gradient(self.raw) })
    }

    /// update_step_lr_scheduler (neural_network_generic.rs:57-67): every layer
    /// at learning_rate * gamma^(epoch / step_size), the network's rate kept.
    pub fn update_step_lr_scheduler(&mut self, epoch: usize, step_size: usize, gamma: f64) -> Result<(), MitokError> {
        let factor = (epoch / step_size) as f64;
        let lr = self.learning_rate()? * gamma.powf(factor);
        self.update_learning_rate(lr)
    }

    /// decay_learning_rate (neural_network_generic.rs:69-73): the network's
    /// rate times the factor, then every layer at it.
    pub fn decay_learning_rate(&mut self, decay_factor: f64) -> Result<(), MitokError> {
        let lr = self.learning_rate()? * decay_factor;
        self.set_learning_rate(lr)?;
        self.update_learning_rate(lr)
    }

    /// The token loop on ids: `n_new` greedy ids per sequence.
    pub fn generate(&mut self, prompt: &[u32], n_new: u32) -> Result<Vec<u32>, MitokError> {
        let mut out = vec![0u32; n_new as usize];
        let lens = [prompt.len() as u32];
        check(unsafe {
            mitok_generate(self.raw, prompt.as_ptr(), lens.as_ptr(), 1, prompt.len() as u32, n_new,
                           out.as_mut_ptr(), std::ptr::null_mut())
        })?;
        Ok(out)
    }

    /// Prompt pass of one sequence (the caches are reset first): the greedy id
    /// of its last row and, if asked for, that row's Re-logits.
    pub fn prefill(&mut self, prompt: &[u32], logits: Option<&mut Vec<f64>>) -> Result<u32, MitokError> {
        let mut id = 0u32;
        let lens = [prompt.len() as u32];
        let lp = match logits {
            Some(l) => {
                l.resize(self.vocab as usize, 0.0);
                l.as_mut_ptr()
            }
            None => std::ptr::null_mut(),
        };
        check(unsafe { mitok_prefill(self.raw, prompt.as_ptr(), lens.as_ptr(), 1, prompt.len() as u32, &mut id, lp) })?;
        Ok(id)
    }

    /// One decode step of one sequence; `id` None feeds the id the previous
    /// call returned, which is already on the device.
    pub fn decode_step(&mut self, id: Option<u32>, logits: Option<&mut Vec<f64>>) -> Result<u32, MitokError> {
        let mut next = 0u32;
        let inp = id.map(|x| [x]);
        let ip = inp.as_ref().map_or(std::ptr::null(), |a| a.as_ptr());
        let lp = match logits {
            Some(l) => {
                l.resize(self.vocab as usize, 0.0);
                l.as_mut_ptr()
            }
            None => std::ptr::null_mut(),
        };
        check(unsafe { mitok_decode_step(self.raw, ip, 1, &mut next, lp) })?;
        Ok(next)
    }
}
