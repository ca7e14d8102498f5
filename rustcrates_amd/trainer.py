"""The host side of `train` (network_types/transformer/transformer_network.rs:
35-163) around the device calls: the epoch and batch loops, the step
learning-rate schedule, the loss bookkeeping and its rising-loss response.

Per batch, on the device: the TRAINING predict of the concatenated input +
target ids (`Network.predict(..., target_rows=T, want_output=False)`), its
loss (`cross_entropy_loss`, transformer_network.rs:81), backward over every
layer with every update at time_step = epoch (`backward_walk`, :100), then
update_step_lr_scheduler(epoch, 100, 0.9) (:111).  Per epoch, on the host:
the exponential moving average of the loss (:116-120), decay_learning_rate(0.5)
with reset_previous_gradient when the loss rose three times in a row (:127-154),
and the stop at a total loss of norm 0.004 (:156-160).  Tokenization and the
sliding context windows (:50-71) happen before; the sled checkpoints and the
progress prints (:84-109, :113-114, :122-125) are the caller's.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

LOSS_THRESHOLD = 0.004  # transformer_network.rs:37
LOSS_EMA_ALPHA = 0.2  # :41
LR_STEP_SIZE, LR_GAMMA = 100, 0.9  # :111
LR_DECAY = 0.5  # :149


@dataclass
class EpochBook:
    """What `train` carries from epoch to epoch (:37-43)."""

    previous_last_losses: list = field(default_factory=list)
    total_loss_exp_ma: float = 0.0
    epoch_processed: int = 0

    def end_epoch(self, epoch: int, total_loss: complex) -> bool:
        """The moving average and the rising-loss test of :116-154; True when
        the learning rate is to be halved and the previous gradients dropped.
        The indices are the reference's: the list grows to five entries, entry
        epoch % len is overwritten, and only an epoch with epoch % len == 4
        compares entries 0..3."""
        re = float(np.real(total_loss))
        if self.total_loss_exp_ma == 0.0 and epoch == 0:
            self.total_loss_exp_ma = re
        self.total_loss_exp_ma = LOSS_EMA_ALPHA * re + (1.0 - LOSS_EMA_ALPHA) * self.total_loss_exp_ma
        if len(self.previous_last_losses) <= 4:
            self.previous_last_losses.append(re)
        n = len(self.previous_last_losses)
        self.previous_last_losses[epoch % n] = re
        if n >= 4:
            end_ind = epoch % n
            if end_ind >= 4:
                start_ind = end_ind - 4
                pl = self.previous_last_losses
                rising = sum(1 for i in range(start_ind, end_ind - 1) if pl[i] < pl[i + 1])
                if rising > 2 and self.epoch_processed != epoch:
                    self.epoch_processed = epoch
                    return True
        return False


def update_step_lr_scheduler(net, epoch: int, step_size: int = LR_STEP_SIZE, gamma: float = LR_GAMMA) -> None:
    """neural_network_generic.rs:57-67: every layer at the network's rate
    times gamma^(epoch / step_size) (integer division); the network's own rate
    is kept."""
    net.set_learning_rate(net.learning_rate() * gamma ** float(epoch // step_size))


def decay_learning_rate(net, decay_factor: float = LR_DECAY) -> None:
    """neural_network_generic.rs:69-73: the network's rate times the factor,
    then every layer at it."""
    lr = net.learning_rate() * decay_factor
    net.set_network_learning_rate(lr)
    net.set_learning_rate(lr)


def train_batch(net, batch_ids, target_ids, tlens, epoch: int) -> complex:
    """One batch of train (:73-104) on the device: batch_ids [B][S] holds each
    sequence's input ids followed by its T target ids (the last T columns);
    target_ids [B][T], tlens the targets used per sequence.  Returns the loss."""
    T = np.asarray(target_ids).shape[1]
    net.predict(batch_ids, forward_only=False, target_rows=T, want_output=False)
    loss = net.cross_entropy_loss(target_ids, tlens)
    net.backward_walk(target_ids, tlens, update=True, time_step=epoch)
    return loss


def train(net, batches, num_epochs: int, on_epoch=None) -> list:
    """train (:35-163) over `batches` of (batch_ids, target_ids, tlens) for at
    most num_epochs epochs; returns each epoch's total loss.  on_epoch(epoch,
    total_loss, book), if given, runs after each epoch's bookkeeping (where
    the reference saves its sled checkpoint and prints)."""
    book = EpochBook()
    totals = []
    for epoch in range(num_epochs):
        total = 0j
        for batch_ids, target_ids, tlens in batches:
            total += train_batch(net, batch_ids, target_ids, tlens, epoch)
            update_step_lr_scheduler(net, epoch)
        totals.append(total)
        if book.end_epoch(epoch, total):
            decay_learning_rate(net)
            net.reset_previous_gradient()
        if on_epoch is not None:
            on_epoch(epoch, total, book)
        if abs(total) <= LOSS_THRESHOLD:
            break
    return totals
