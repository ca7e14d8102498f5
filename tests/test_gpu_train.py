"""GPU parity of the output head's training step (transformer_network.rs:
506-636 for the Softmax, the vocab Linear and the FeedForward below it):
mitok_backward_head / mitok_backward after a TRAINING-mode stateless predict,
against the CPU checker's softmax_backward / linear_backward(_c) /
dense_backward / linear_update on the same inputs.

Two steps: the first update is the reference's clipped gradient descent, the
second its AdamW (linear_layer.rs:130-175).  Bar: within 1e-11 of the
largest element (the GPU products sum in a different order)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
import rustcrates_amd as ra
from rustcrates_amd import seeded

pytestmark = pytest.mark.gpu

TOL = 1e-11


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def head_net(net, table, W, b):
    V, d = table.shape
    net.add_embedding(V, d, table)
    net.add_linear(d, W.shape[1], W, b)
    net.add_softmax(ra.TRAINING)
    return net


@pytest.mark.parametrize("V,d,lens,T", [(40, 8, [7, 5], 3), (4000, 64, [24, 17, 24, 9], 6), (300, 16, [3] * 12, 2)])
def test_head_training_steps_match_checker(V, d, lens, T):
    rng = np.random.default_rng(V + d)
    table = rng.standard_normal((V, d)) + 1j * rng.standard_normal((V, d))
    W0 = 0.2 * (rng.standard_normal((d, V)) + 1j * rng.standard_normal((d, V)))
    b0 = 0.1 * (rng.standard_normal(V) + 1j * rng.standard_normal(V))
    B, S = len(lens), max(lens)
    ids = seeded.prompts(70 + V, lens, V)
    targets = rng.integers(0, V, size=(B, T)).astype(np.uint32)
    targets[0, 0] = 1  # a PAD target is skipped
    tlens = [min(T, S - 1)] * B
    g = head_net(ra.Network(0), table, W0, b0)
    state = [np.zeros((d, V), np.complex128), np.zeros((d, V), np.complex128),
             np.zeros(V, np.complex128), np.zeros(V, np.complex128)]
    W, b = W0, b0
    lr = 0.01
    for step in (1, 2):
        o = head_net(oracle.Network(), table, W, b)
        Pg, mg = g.predict(ids, lens=lens, forward_only=False)
        Po, mo = o.predict(ids, lens=lens, forward_only=False)
        # the Linear's input: embedding rows, PAD (id 1 and the padding) zero
        X = np.zeros((B, S, d), np.complex128)
        for bb in range(B):
            for s in range(lens[bb]):
                if ids[bb, s] != 1:
                    X[bb, s] = table[ids[bb, s]]
        G = oracle.softmax_backward(Po, targets, tlens)
        dW, db, dX = oracle.linear_backward(X, G, W)
        W, b = oracle.linear_update(W, b, dW, db, B, state, step == 1, lr, step)
        dXg = g.backward_head(targets, tlens, update=True, learning_rate=lr, time_step=step)
        Wg = g.get_tensor(1, 0, d * V).reshape(d, V)
        bg = g.get_tensor(1, 4, V)
        errs = (close(Pg, Po), close(dXg, dX), close(Wg, W), close(bg, b))
        log(f"head V={V} d={d} B={B} step {step}: P {errs[0]:.1e}, dX {errs[1]:.1e}, W {errs[2]:.1e}, b {errs[3]:.1e}")
        assert np.array_equal(mg, mo)
        assert max(errs) < TOL
        o.close()
    g.close()


def test_backward_head_errors():
    rng = np.random.default_rng(3)
    V, d = 30, 4
    table = rng.standard_normal((V, d)) + 0j
    W0 = rng.standard_normal((d, V)) + 0j
    g = head_net(ra.Network(0), table, W0, np.zeros(V, np.complex128))
    ids = seeded.prompts(5, [6, 6], V)
    with pytest.raises(ra.MitokError, match="no stateless"):
        g.backward_head(np.zeros((2, 2), np.uint32), want_grad_input=False)
    g.predict(ids, forward_only=True)  # a cached pass is not differentiated
    with pytest.raises(ra.MitokError, match="no stateless"):
        g.backward_head(np.zeros((2, 2), np.uint32), want_grad_input=False)
    g.reset()
    g.predict(ids, forward_only=False)
    with pytest.raises(ra.MitokError, match="exceeds vocabulary"):
        g.backward_head(np.full((2, 2), V, np.uint32))
    with pytest.raises(ra.MitokError, match="need more than"):
        g.backward_head(np.zeros((2, 6), np.uint32))
    # the network still differentiates after refused calls, without updating
    dx = g.backward_head(np.zeros((2, 2), np.uint32), update=False)
    assert dx.shape == (2, 6, d) and np.isfinite(dx).all()
    assert np.array_equal(g.get_tensor(1, 0, d * V).reshape(d, V), W0)
    g.close()


def ffn_net(net, table, W1, b1, W2, b2, Wv, bv):
    V, d = table.shape
    net.add_embedding(V, d, table)
    net.add_feed_forward(d, W1.shape[1], W1, b1, W2, b2)
    net.add_linear(d, V, Wv, bv)
    net.add_softmax(ra.TRAINING)
    return net


@pytest.mark.parametrize("V,d,F,lens,T", [(50, 8, 16, [6, 4], 3), (2000, 64, 256, [20, 13, 20], 5)])
def test_ffn_and_head_training_steps_match_checker(V, d, F, lens, T):
    """mitok_backward through the vocab Linear and the FeedForward below it
    (two layers), with updates: the Linear's at time_step, the FeedForward's
    Linear at time_step and its Dense at step 1 (Layer::time_step stays 0)."""
    rng = np.random.default_rng(V + F)
    c = lambda *shape: rng.standard_normal(shape) + 1j * rng.standard_normal(shape)  # noqa: E731
    table = c(V, d)
    W1, b1, W2, b2 = 0.3 * c(d, F), 0.1 * c(F), 0.3 * c(F, d), 0.1 * c(d)
    Wv, bv = 0.2 * c(d, V), 0.1 * c(V)
    B, S = len(lens), max(lens)
    ids = seeded.prompts(90 + V, lens, V)
    targets = rng.integers(0, V, size=(B, T)).astype(np.uint32)
    tlens = [min(T, S - 1)] * B
    gelu = np.vectorize(lambda z: oracle.gelu(z)[0])
    g = ffn_net(ra.Network(0), table, W1, b1, W2, b2, Wv, bv)
    st = {k: [np.zeros(s, np.complex128), np.zeros(s, np.complex128), np.zeros(s2, np.complex128),
              np.zeros(s2, np.complex128)] for k, s, s2 in (("v", (d, V), V), ("2", (F, d), d), ("1", (d, F), F))}
    lr = 0.01
    for step in (1, 2):
        o = ffn_net(oracle.Network(), table, W1, b1, W2, b2, Wv, bv)
        Pg, mg = g.predict(ids, lens=lens, forward_only=False)
        Po, mo = o.predict(ids, lens=lens, forward_only=False)
        X = np.zeros((B, S, d), np.complex128)
        for bb in range(B):
            for s in range(lens[bb]):
                if ids[bb, s] != 1:
                    X[bb, s] = table[ids[bb, s]]
        Z = np.stack([oracle.zgemm(X[bb], W1) for bb in range(B)]) + b1
        H = gelu(Z) * mo[:, :, None]
        Y = o.forward_layers(1, 2, X, mask=mo, forward_only=False)
        G = oracle.softmax_backward(Po, targets, tlens)
        dWv, dbv, dY = oracle.linear_backward(Y, G, Wv)
        Wv, bv = oracle.linear_update(Wv, bv, dWv, dbv, B, st["v"], step == 1, lr, step)
        dW2, db2, dH = oracle.linear_backward_c(H, dY, W2)
        dW1, db1, dX = oracle.dense_backward(X, Z, dH, mo, W1)
        W2, b2 = oracle.linear_update(W2, b2, dW2, db2, B, st["2"], step == 1, lr, step)
        W1, b1 = oracle.linear_update(W1, b1, dW1, db1, B, st["1"], step == 1, lr, 0)
        dXg = g.backward(targets, tlens, layers=2, update=True, learning_rate=lr, time_step=step)
        got = {"W1": g.get_tensor(1, 0, d * F).reshape(d, F), "b1": g.get_tensor(1, 4, F),
               "W2": g.get_tensor(1, 1, F * d).reshape(F, d), "b2": g.get_tensor(1, 5, d),
               "Wv": g.get_tensor(2, 0, d * V).reshape(d, V), "bv": g.get_tensor(2, 4, V)}
        want = {"W1": W1, "b1": b1, "W2": W2, "b2": b2, "Wv": Wv, "bv": bv}
        errs = {k: close(got[k], want[k]) for k in got}
        errs["P"], errs["dX"] = close(Pg, Po), close(dXg, dX)
        log(f"ffn+head V={V} d={d} F={F} step {step}: " + ", ".join(f"{k} {v:.1e}" for k, v in errs.items()))
        assert np.array_equal(mg, mo)
        assert max(errs.values()) < TOL
        o.close()
    g.close()


def test_backward_two_layers_needs_a_feedforward_below():
    rng = np.random.default_rng(4)
    V, d = 30, 4
    g = head_net(ra.Network(0), rng.standard_normal((V, d)) + 0j, rng.standard_normal((d, V)) + 0j,
                 np.zeros(V, np.complex128))
    g.predict(seeded.prompts(6, [5, 5], V), forward_only=False)
    with pytest.raises(ra.MitokError, match="no FeedForward"):
        g.backward(np.zeros((2, 2), np.uint32), layers=2)
    with pytest.raises(ra.MitokError, match="layers"):
        g.backward(np.zeros((2, 2), np.uint32), layers=3)
    g.close()
