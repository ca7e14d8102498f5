"""GPU parity of the decode-step plans against the CPU oracle: the resident
loop (one cooperative launch for every decode step, plan 3), the fused GEMV
plan (row transforms in the product prologues, split-K and greedy argmax
finished in-kernel, plan 1) and the one-launch-per-operation plan (plan 0).

Bar: ids bit-exact, Re-logits within REL_TOL (conftest.max_rel_err).
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


SMALL = configs.ModelConfig("small", layers=2, d=32, heads=4, ffn=64, vocab=211, max_ctx=64, seed=9)
MID = configs.ModelConfig("mid", layers=2, d=64, heads=4, ffn=128, vocab=1000, max_ctx=96, seed=21)
PLANS = (3, 1, 0)


def _generate_both_plans(cfg, lens, n_new, prompt_seed):
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    prompt = seeded.prompts(prompt_seed, lens, cfg.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    out = {}
    for plan in PLANS:
        g.set_decode_plan(plan)
        out[plan] = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
        want = "resident" if plan == 3 and len(lens) <= 8 else None
        if want:
            assert g.last_timings()["decode_loop"] == want
    return out, (io, lo)


@pytest.mark.parametrize("lens", [[12], [9, 30], [5, 17, 3], [20, 11, 8, 25, 2], [7] * 8])
def test_decode_plans_match_oracle(lens):
    log(f"decode plans, lens {lens}")
    out, (io, lo) = _generate_both_plans(MID, lens, 16, len(lens))
    for plan, (ig, lg) in out.items():
        assert np.array_equal(ig, io), f"plan={plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan={plan}"


def test_decode_batch_above_gemv_limit_uses_mfma_with_fused_argmax():
    lens = [10 + (3 * b) % 17 for b in range(12)]
    log("decode B=12 (MFMA + fused argmax)")
    out, (io, lo) = _generate_both_plans(MID, lens, 10, 77)
    for plan in (3, 1):
        ig, lg = out[plan]
        assert np.array_equal(ig, io), f"plan={plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan={plan}"


# FFN 1024 wide enough that FFN Dense takes the row-tile MFMA product with no K
# split (GELU in the block); QKV and FFN Linear leave 2 and 8 partials; 20 and
# 40 sequences end in a partial row tile
WIDE = configs.ModelConfig("wide", layers=2, d=128, heads=4, ffn=1024, vocab=2000, max_ctx=64, seed=5)


@pytest.mark.parametrize("B", [20, 40])
def test_decode_row_tile_products(B):
    lens = [4 + (7 * b) % 23 for b in range(B)]
    log(f"decode B={B} (row-tile MFMA products)")
    out, (io, lo) = _generate_both_plans(WIDE, lens, 8, 100 + B)
    for plan in (1, 0):
        ig, lg = out[plan]
        assert np.array_equal(ig, io), f"plan={plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan={plan}"


def test_fused_decode_rope_model():
    cfg = configs.ModelConfig("rope", layers=2, d=64, heads=4, ffn=128, vocab=500, max_ctx=96, seed=12, rope=True)
    log("fused decode with RoPE")
    out, (io, lo) = _generate_both_plans(cfg, [20, 6], 24, 3)
    for plan, (ig, lg) in out.items():
        assert np.array_equal(ig, io), f"plan={plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan={plan}"


def _odd_stack(net, cfg):
    """Embedding, Norm, Norm, SA, SA, Linear(d->d), FFN, Norm, Linear(vocab), Softmax:
    every pending-prologue case of the fused plan (two norms, attention after
    attention, a hidden Linear, a trailing Norm)."""
    d = cfg.d
    net.add_embedding(cfg.vocab, d)
    net.add_norm(d, 1e-5)
    net.add_norm(d, 1e-5)
    net.add_self_attention(cfg.heads, d, cfg.max_ctx, 1e-12)
    net.add_self_attention(cfg.heads, d, cfg.max_ctx, 1e-12)
    net.add_linear(d, d)
    net.add_feed_forward(d, cfg.ffn)
    net.add_norm(d, 1e-5)
    net.add_linear(d, cfg.vocab)
    net.add_softmax(ra.PRODUCTION)
    net.init_seeded(cfg.seed)
    return net


def test_fused_decode_odd_layer_stack():
    cfg = SMALL
    g, o = _odd_stack(ra.Network(0), cfg), _odd_stack(oracle.Network(), cfg)
    lens = [9, 4, 13]
    prompt = seeded.prompts(31, lens, cfg.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=12, want_logits=True)
    for plan in PLANS:
        g.set_decode_plan(plan)
        ig, lg = g.generate(prompt, lens=lens, n_new=12, want_logits=True)
        assert np.array_equal(ig, io), f"plan={plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan={plan}"


def test_cached_predict_single_row_uses_fused_plan():
    """predict with forward_only on a filled cache, one row per sequence, twice in a row."""
    g = configs.build_network(ra.Network(0), MID)
    o = configs.build_network(oracle.Network(), MID)
    ids = seeded.prompts(41, [14, 14], MID.vocab)
    for net in (g, o):
        net.reset()
    a_g, _ = g.predict(ids[:, :12], forward_only=True)
    a_o, _ = o.predict(ids[:, :12], forward_only=True)
    assert max_rel_err(a_g, a_o) < REL_TOL
    for t in (12, 13):
        b_g, _ = g.predict(ids[:, t:t + 1], time_steps=[t, t], forward_only=True)
        b_o, _ = o.predict(ids[:, t:t + 1], time_steps=[t, t], forward_only=True)
        assert max_rel_err(b_g, b_o) < REL_TOL


def test_resident_loop_repeats_bit_identically():
    """Every partial is summed in a fixed order, so repeated resident launches
    (their barrier epochs carried over from call to call) are bit-identical."""
    g = configs.build_network(ra.Network(0), MID)
    g.set_decode_plan(3)
    prompt = seeded.prompts(6, [13, 3, 40], MID.vocab)
    runs = [g.generate(prompt, n_new=25, lens=[13, 3, 40], want_logits=True) for _ in range(4)]
    assert g.last_timings()["decode_loop"] == "resident"
    for ids, lg in runs[1:]:
        assert np.array_equal(ids, runs[0][0])
        assert np.array_equal(lg, runs[0][1])


def test_default_plan_runs_resident_up_to_two_sequences():
    """The default plan: the resident loop with the polling exchange for 1 and
    2 sequences, the fused graph from 3; with the barrier exchange asked for,
    the resident loop for 1 sequence only."""
    g = configs.build_network(ra.Network(0), MID)
    for lens, want in (([17], "resident"), ([17, 9], "resident"), ([17, 9, 4], "graph")):
        prompt = seeded.prompts(8, lens, MID.vocab)
        g.generate(prompt, lens=lens, n_new=8)
        assert g.last_timings()["decode_loop"] == want, lens
    g.resident_exchange(0)
    prompt = seeded.prompts(8, [17, 9], MID.vocab)
    g.generate(prompt, lens=[17, 9], n_new=8)
    assert g.last_timings()["decode_loop"] == "graph"
    g.close()


def test_graph_replay_fused_plan_is_deterministic():
    """Split-K partials are summed in split order, so replays are bit-identical."""
    g = configs.build_network(ra.Network(0), MID)
    g.set_decode_plan(1)
    prompt = seeded.prompts(5, [11, 29], MID.vocab)
    runs = [g.generate(prompt, n_new=20, lens=[11, 29], want_logits=True) for _ in range(3)]
    g.set_graph_mode(True)
    runs.append(g.generate(prompt, n_new=20, lens=[11, 29], want_logits=True))
    for ids, lg in runs[1:]:
        assert np.array_equal(ids, runs[0][0])
        assert np.array_equal(lg, runs[0][1])
