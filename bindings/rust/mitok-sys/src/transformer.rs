//! The device-backed text loop: `predict_token_by_token`
//! (network_types/transformer/transformer_network.rs:165-313) with every
//! forward pass on the GPU.
//!
//! The crate's own function keeps its signature and, when the network holds a
//! device handle, returns `predict_token_by_token_device(handle, input_batch,
//! &tokenizer)`.  What the loop does around the forward passes:
//!   - each input gets the "<bos> " prefix (network_components/input.rs:70-72);
//!   - sequence 0 is tokenized with special tokens and cut to its last
//!     MAX_CONTEXT_WINDOW_SIZE ids (:32, 208-218);
//!   - step 0 runs every prompt row and keeps the [S][V] Re-logits; each later
//!     step feeds the last greedy id at time_step = its position (:225-248,
//!     300-304) and keeps its [1][V] Re-logits (:257);
//!   - the greedy id is the last index among equal maxima of the last row
//!     (sampling_methods.rs:5-18), decoded on its own with special tokens kept;
//!   - "<eos>" ends the loop without being appended (:285-288), any other token
//!     is appended to sequence 0's text (:291), and 21 appended tokens end it
//!     (:293-297).

use crate::{MitokError, Network};
use num_complex::Complex;

pub const MAX_CONTEXT_WINDOW_SIZE: usize = 512;
pub const MAX_NEW_TOKENS: usize = 21;

/// The two tokenizer calls the loop makes (the crate's GPT-NeoX `Tokenizer`,
/// utils/tokenizer.rs:9-50).
pub trait TextTokenizer {
    /// `encode(text, add_special_tokens = true)` ids.
    fn encode_ids(&self, text: &str) -> Vec<u32>;
    /// `decode(&[id], skip_special_tokens = false)`.
    fn decode_id(&self, id: u32) -> String;
}

/// sampling_methods.rs:5-18: `max_by(partial_cmp)` keeps the last of equal
/// maxima; a NaN is an error where the reference's `unwrap()` panics.
pub fn greedy_id(row: &[f64]) -> Result<u32, MitokError> {
    let mut best = 0usize;
    for (i, &x) in row.iter().enumerate() {
        if x.is_nan() {
            return Err(MitokError { code: crate::MITOK_ERR_NAN, message: "greedy_decoding: NaN in logits".into() });
        }
        if x >= row[best] {
            best = i;
        }
    }
    Ok(best as u32)
}

pub fn predict_token_by_token_device<T: TextTokenizer>(net: &mut Network, input_batch: &[String], tokenizer: &T)
                                                      -> Result<(Vec<Vec<Vec<f64>>>, Vec<String>), MitokError> {
    let mut texts: Vec<String> = input_batch.iter().map(|t| format!("<bos> {}", t)).collect();
    let mut predictions: Vec<Vec<Vec<f64>>> = Vec::new();
    if texts.is_empty() {
        return Ok((predictions, texts));
    }
    let all = tokenizer.encode_ids(&texts[0]);
    let ids = all[all.len().saturating_sub(MAX_CONTEXT_WINDOW_SIZE)..].to_vec();
    if ids.is_empty() {
        return Ok((predictions, texts));
    }
    net.reset()?;
    let (mut out, _) = net.predict(&[ids.clone()], None, true)?;
    predictions.push(out.swap_remove(0));
    let mut pos = ids.len() as u32;
    for count in 0..MAX_NEW_TOKENS {
        let last = predictions.last().and_then(|p| p.last()).expect("one row per step");
        let next = greedy_id(last)?;
        let token = tokenizer.decode_id(next);
        if token == "<eos>" {
            break;
        }
        texts[0].push_str(&token);
        if count + 1 == MAX_NEW_TOKENS {
            break;
        }
        let (mut out, _) = net.predict(&[vec![next]], Some(pos), true)?;
        predictions.push(out.swap_remove(0));
        pos += 1;
    }
    Ok((predictions, texts))
}

/// Ids only (no per-step logits): the prompt pass, then one decode step per
/// token with the fed id staying on the device; 4 bytes per step cross PCIe.
/// `eos` is the id whose text is "<eos>" (50279 in the GPT-NeoX vocabulary the
/// crate extends, utils/tokenizer.rs:51-75).
pub fn generate_ids_device(net: &mut Network, prompt: &[u32], eos: u32) -> Result<Vec<u32>, MitokError> {
    let mut out = Vec::with_capacity(MAX_NEW_TOKENS);
    let mut id = net.prefill(prompt, None)?;
    while id != eos {
        out.push(id);
        if out.len() == MAX_NEW_TOKENS {
            break;
        }
        id = net.decode_step(None, None)?;
    }
    Ok(out)
}

/// One batch of `train` (transformer_network.rs:73-104) on the device: the
/// TRAINING predict of the concatenated input + target ids (the last
/// `target_ids[b].len()` ids of each row; a DiscreteWavelet layer passes them
/// on uncompressed and needs unpadded rows, as the reference does), its loss
/// (cross_entropy_loss_batch, :81), then backward over every layer with
/// update_parameters at time_step = epoch (:100).  Returns the loss.  The
/// epoch loop, the loss bookkeeping, the learning-rate schedule and the sled
/// checkpoints of `train` stay on the host around it.
pub fn train_batch_device(net: &mut Network, batch_ids: &[Vec<u32>], target_ids: &[Vec<u32>], epoch: u32)
                          -> Result<Complex<f64>, MitokError> {
    let t = target_ids.iter().map(|r| r.len()).max().unwrap_or(0) as u32;
    net.forward_targets(batch_ids, t)?;
    let loss = net.cross_entropy_loss(target_ids)?;
    net.backward_walk(target_ids, true, epoch)?;
    Ok(loss)
}

/// What `train` decides at the end of an epoch (transformer_network.rs:
/// 112-162), kept apart from the device so it reads like the reference.
#[derive(Default)]
pub struct EpochBook {
    pub previous_last_losses: Vec<f64>,
    pub total_loss_exp_ma: f64,
    pub epoch_processed: usize,
}

pub const LOSS_THRESHOLD: f64 = 0.004;
pub const LOSS_EMA_ALPHA: f64 = 0.2;

impl EpochBook {
    /// The exponential moving average (:116-120) and the rising-loss test
    /// (:127-154): true when the learning rate is to be halved and the
    /// previous gradients dropped.
    pub fn end_epoch(&mut self, epoch: usize, total_loss: Complex<f64>) -> bool {
        if self.total_loss_exp_ma == 0.0 && epoch == 0 {
            self.total_loss_exp_ma = total_loss.re;
        }
        self.total_loss_exp_ma = LOSS_EMA_ALPHA * total_loss.re + (1.0 - LOSS_EMA_ALPHA) * self.total_loss_exp_ma;
        if self.previous_last_losses.len() <= 4 {
            self.previous_last_losses.push(total_loss.re);
        }
        let len = self.previous_last_losses.len();
        self.previous_last_losses[epoch % len] = total_loss.re;
        if len >= 4 {
            let end_ind = epoch % len;
            if end_ind >= 4 {
                let start_ind = end_ind - 4;
                let mut rising = 0;
                for i in start_ind..end_ind - 1 {
                    if self.previous_last_losses[i] < self.previous_last_losses[i + 1] {
                        rising += 1;
                    }
                }
                if rising > 2 && self.epoch_processed != epoch {
                    self.epoch_processed = epoch;
                    return true;
                }
            }
        }
        false
    }
}

/// `train` (transformer_network.rs:35-163) on the device, over batches of
/// (input + target ids, target ids) already tokenized and windowed: per batch
/// the TRAINING predict, its loss, backward with every update at time_step =
/// epoch and update_step_lr_scheduler(epoch, 100, 0.9); per epoch the loss
/// bookkeeping, decay_learning_rate(0.5) with reset_previous_gradient when the
/// loss keeps rising, and the stop at a total loss of norm 0.004.  The sled
/// checkpoints and the progress prints are the caller's.  Returns each
/// epoch's total loss.
pub fn train_device(net: &mut Network, batches: &[(Vec<Vec<u32>>, Vec<Vec<u32>>)], num_epochs: usize)
                    -> Result<Vec<Complex<f64>>, MitokError> {
    let mut book = EpochBook::default();
    let mut totals = Vec::new();
    for epoch in 0..num_epochs {
        let mut total_loss = Complex::new(0.0, 0.0);
        for (batch_ids, target_ids) in batches {
            total_loss += train_batch_device(net, batch_ids, target_ids, epoch as u32)?;
            net.update_step_lr_scheduler(epoch, 100, 0.9)?;
        }
        totals.push(total_loss);
        if book.end_epoch(epoch, total_loss) {
            net.decay_learning_rate(0.5)?;
            net.reset_previous_gradient()?;
        }
        if total_loss.norm() <= LOSS_THRESHOLD {
            break;
        }
    }
    Ok(totals)
}
