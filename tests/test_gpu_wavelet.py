"""GPU parity of the DiscreteWaveletLayer (network_types/wavelet_discrete_layer.rs:
46-161) and of create_transformer's default stack (transformer_builder.rs:10-72:
Embedding(50280, 16) -> DiscreteWavelet(DB2, SYMMETRIC) -> Norm -> RoPE ->
2 x [SelfAttention -> FeedForward] -> Linear -> Softmax) against the CPU oracle.

The prompt pass compresses each sequence's rows to the low half of dwt_1d
along the sequence, the cache keeps the compressed rows, and decode steps
pass their row through with RoPE positions counting the uncompressed prompt.

Bar: ids bit-exact; Re-logits within REL_TOL (conftest.max_rel_err).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
import rustcrates_amd as ra
from conftest import REL_TOL, max_rel_err
from rustcrates_amd import configs, seeded

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("wavelet,mode", [(1, 2), (0, 1), (1, 3), (1, 0), (1, 4), (1, 6)])
def test_wavelet_layer_forward_matches_oracle(wavelet, mode):
    """The layer alone on hidden states, ragged masks, every supported padding mode."""
    rng = np.random.default_rng(40 + mode)
    x = rng.standard_normal((3, 11, 8)) + 1j * rng.standard_normal((3, 11, 8))
    mask = np.array([[1] * 11, [1] * 7 + [0] * 4, [1] * 2 + [0] * 9], np.uint32)
    g, o = ra.Network(0), oracle.Network()
    for net in (g, o):
        net.add_discrete_wavelet(8, wavelet, mode)
    yg = g.forward_layers(0, 1, x, mask=mask, forward_only=False)
    yo = o.forward_layers(0, 1, x, mask=mask, forward_only=False)
    assert yg.shape == yo.shape == (3, oracle.dwt_rows(11, wavelet), 8)
    np.testing.assert_allclose(yg, yo, rtol=1e-14, atol=1e-15)
    g.close()


def test_wavelet_inside_a_block_stack_all_rows_and_masks():
    """Embedding -> wavelet -> Norm -> SelfAttention -> FeedForward -> Linear:
    every compressed row's Re-logits, the compressed padding mask, and the
    TRAINING softmax arm on it."""
    d, V = 16, 300

    def build(net, mode):
        net.add_embedding(V, d)
        net.add_discrete_wavelet(d, 1, 2)
        net.add_norm(d, 1e-5)
        net.add_self_attention(4, d, 64, 1e-12)
        net.add_feed_forward(d, 32)
        net.add_linear(d, V)
        net.add_softmax(mode)
        net.init_seeded(11)
        return net

    lens = [21, 14, 9]
    ids = seeded.prompts(12, lens, V)
    for mode, fwd in ((ra.PRODUCTION, True), (ra.TRAINING, False)):
        g, o = build(ra.Network(0), mode), build(oracle.Network(), mode)
        lg, mg = g.predict(ids, lens=lens, forward_only=fwd)
        lo, mo = o.predict(ids, lens=lens, forward_only=fwd)
        log(f"wavelet stack mode {mode}: rows {lg.shape[1]}, masks equal {np.array_equal(mg, mo)}, "
            f"{max_rel_err(lg, lo):.2e}")
        assert lg.shape == lo.shape == (3, oracle.dwt_rows(21, 1), V)
        assert np.array_equal(mg, mo)
        assert max_rel_err(lg, lo) < REL_TOL
        g.close()


@pytest.mark.parametrize("lens", [[10], [37], [1], [24, 9, 30]])
def test_reference_default_stack_generate(lens):
    """create_transformer's stack at its own sizes (vocab 50280, width 16,
    max_ctx 512) on every decode plan: the compressed prompt in the cache,
    decode rows passed through at uncompressed RoPE positions."""
    g = configs.build_reference_default(ra.Network(0), seed=3)
    o = configs.build_reference_default(oracle.Network(), seed=3)
    prompt = seeded.prompts(20 + len(lens), lens, configs.REFERENCE_VOCAB)
    n_new = 12
    io, lo = o.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    for plan in (3, 1, 0):
        g.set_decode_plan(plan)
        ig, lg = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
        log(f"default stack lens {lens} plan {plan} ({g.last_timings()['decode_loop']}): ids {ig[0].tolist()[:6]}.., "
            f"equal {np.array_equal(ig, io)}, logits {max_rel_err(lg, lo):.2e}")
        assert np.array_equal(ig, io), f"plan {plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan {plan}"
    # the per-step boundary gives the same ids
    g.set_decode_plan(1)
    first = g.prefill(prompt, lens=lens)
    steps = [first] + [g.decode_step() for _ in range(n_new - 1)]
    assert np.array_equal(np.stack(steps, axis=1), io)
    g.close()


def test_wavelet_after_attention_is_refused():
    """Every attention layer's cache holds the rows of one cached length per
    sequence, so a wavelet layer may only precede the attention layers."""
    g = ra.Network(0)
    g.add_embedding(40, 8)
    g.add_self_attention(2, 8, 16, 1e-12)
    with pytest.raises(ra.MitokError, match="after a SelfAttentionLayer"):
        g.add_discrete_wavelet(8, 1, 2)
    g.close()


@pytest.mark.parametrize("vocab,src", [(300, 512), (50280, 512), (40, 1024), (40, 64), (40, 16)])
def test_wavelet_embedding_init_matches_oracle(vocab, src):
    """EmbeddingLayer::new's tables (create_embedding, embedding_layer.rs:
    40-77) on the device against the checker: the seeded draw, five levels of
    DB1/SYMMETRIC dwt_2d_full keeping LL, the CMOR CWT at scale 2.  The
    device forms each value with the reference's multiplies and adds in its
    order, no fused multiply-add, and the wavelet's integral from the same
    host libm as the checker, so the tables are equal bit for bit."""
    dim = {512: 16, 1024: 32, 64: 16, 16: 16}[src]
    g, o = ra.Network(0), oracle.Network()
    for net in (g, o):
        net.add_embedding(vocab, dim)
        net.add_linear(dim, 4)
        net.init_seeded(7)
        net.init_embedding_wavelet(0, 7, src)
    tg = g.get_tensor(0, 0, vocab * dim).reshape(vocab, dim)
    to = o.get_tensor(0, 0, vocab * dim).reshape(vocab, dim)
    diff = int(np.sum(tg != to))
    log(f"wavelet embedding vocab {vocab} src {src}: {diff} values differ, max |diff| {np.max(np.abs(tg - to)):.1e}")
    assert diff == 0
    with pytest.raises(ra.MitokError, match="power of two"):
        g.init_embedding_wavelet(0, 7, 48)
    with pytest.raises(ra.MitokError, match="decomposes"):
        g.init_embedding_wavelet(0, 7, 2048 if dim == 16 else 512)  # decomposes to 64 or 16 values
    g.close()
    o.close()
