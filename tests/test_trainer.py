"""The host side of train (transformer_network.rs:35-163) in
rustcrates_amd/trainer.py, on the CPU with a stand-in network that records the
device calls: the order of the calls per batch, time_step = epoch, the step
schedule of the learning rates, the rising-loss test with the reference's
index arithmetic, and the stop at the loss threshold.  The device side of each
call is checked against the oracle in tests/test_gpu_train.py."""
from __future__ import annotations

import numpy as np

from rustcrates_amd import trainer


class RecordingNet:
    """The Network calls train makes; losses come from a list per epoch."""

    def __init__(self, losses, n_layers=4, lr=0.01):
        self.losses = list(losses)
        self.calls = []
        self.net_lr = lr
        self.layer_lr = [lr] * n_layers

    def predict(self, ids, forward_only=True, target_rows=0, want_output=True):
        assert not forward_only and target_rows > 0 and not want_output
        self.calls.append(("predict", np.asarray(ids).shape, target_rows))
        return None, None

    def cross_entropy_loss(self, targets, tlens=None):
        self.calls.append(("loss",))
        return complex(self.losses.pop(0))

    def backward_walk(self, targets, tlens=None, update=True, time_step=1, want_grad_input=False):
        self.calls.append(("backward", time_step, update))

    def learning_rate(self, layer=None):
        return self.net_lr if layer is None else self.layer_lr[layer]

    def set_learning_rate(self, lr, layer=None):
        self.calls.append(("rates", lr))
        if layer is None:
            self.layer_lr = [lr] * len(self.layer_lr)
        else:
            self.layer_lr[layer] = lr

    def set_network_learning_rate(self, lr):
        self.calls.append(("net_rate", lr))
        self.net_lr = lr

    def reset_previous_gradient(self):
        self.calls.append(("reset",))


def _batch(B=2, S=6, T=2):
    ids = np.arange(B * S, dtype=np.uint32).reshape(B, S) + 2
    return ids, np.ascontiguousarray(ids[:, S - T:]), [T] * B


def test_batch_calls_in_train_order_with_epoch_time_step():
    net = RecordingNet([3.0, 2.5, 2.0, 1.0])
    totals = trainer.train(net, [_batch(), _batch()], 2)
    assert totals == [5.5 + 0j, 3.0 + 0j]
    kinds = [c[0] for c in net.calls]
    assert kinds == ["predict", "loss", "backward", "rates"] * 4
    assert [c[1] for c in net.calls if c[0] == "backward"] == [0, 0, 1, 1]
    assert all(c[2] for c in net.calls if c[0] == "backward")


def test_step_schedule_multiplies_the_network_rate_per_hundred_epochs():
    """update_step_lr_scheduler(epoch, 100, 0.9): the layers get the network's
    rate times 0.9^(epoch div 100), the network's rate stays."""
    net = RecordingNet([], lr=0.01)
    for epoch, want in ((0, 0.01), (99, 0.01), (100, 0.009), (250, 0.01 * 0.81)):
        trainer.update_step_lr_scheduler(net, epoch)
        assert abs(net.layer_lr[0] - want) < 1e-16 and net.net_lr == 0.01


def test_rising_loss_halves_the_rate_and_resets_at_the_reference_epochs():
    """The list grows to five losses and entry epoch % 5 is overwritten; only
    an epoch with epoch % 5 == 4 compares entries 0..3, so rising losses at
    epochs 0..3 trigger at epoch 4 and epochs 5..8 at epoch 9."""
    per_epoch = [1.0, 2.0, 3.0, 4.0, 0.5, 1.0, 2.0, 3.0, 4.0, 0.5, 0.4]
    net = RecordingNet(per_epoch)
    trainer.train(net, [_batch()], len(per_epoch))
    resets = [i for i, c in enumerate(net.calls) if c[0] == "reset"]
    assert len(resets) == 2
    # each reset follows the 5th and the 10th epoch's batch (4 calls per
    # batch) and the decay's two calls
    assert resets[0] == 5 * 4 + 2 and resets[1] == resets[0] + 1 + 5 * 4 + 2
    assert abs(net.net_lr - 0.0025) < 1e-18  # halved twice
    # decay_learning_rate set the layers to the halved rate before the reset
    assert net.calls[resets[0] - 1] == ("rates", 0.005) and net.calls[resets[0] - 2] == ("net_rate", 0.005)


def test_falling_or_mixed_losses_never_reset():
    net = RecordingNet([5.0, 4.0, 3.0, 2.0, 1.0, 1.5, 1.2, 1.3, 1.1, 1.4])
    trainer.train(net, [_batch()], 10)
    assert not any(c[0] == "reset" for c in net.calls)


def test_epoch_book_quirks():
    """The rising count compares entries start..end-1 only (three pairs), and
    one epoch never triggers twice; the moving average starts at the first
    epoch's loss."""
    b = trainer.EpochBook()
    for e, loss in enumerate([1.0, 2.0, 3.0, 3.0]):
        assert not b.end_epoch(e, loss)
    assert not b.end_epoch(4, 9.0)  # 1 < 2 < 3 but 3 == 3: two rises
    assert b.previous_last_losses == [1.0, 2.0, 3.0, 3.0, 9.0]
    b2 = trainer.EpochBook()
    b2.end_epoch(0, 2.0)
    assert abs(b2.total_loss_exp_ma - 2.0) < 1e-15
    b2.end_epoch(1, 1.0)
    assert abs(b2.total_loss_exp_ma - (0.2 * 1.0 + 0.8 * 2.0)) < 1e-15


def test_loss_threshold_stops_training():
    net = RecordingNet([1.0, 0.003, 7.0])
    totals = trainer.train(net, [_batch()], 3)
    assert len(totals) == 2 and len(net.losses) == 1
