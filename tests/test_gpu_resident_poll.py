"""GPU parity of the resident decode loop's two exchanges.

The resident loop runs every decode step of generate in one cooperative
launch.  Its blocks hand values to each other either through a grid barrier
after every operation, or by polling: every exchanged value starts a step as
a sentinel and its reader re-reads it until written (one grid barrier per
step, two halves of an exchange arena alternating between steps).  Both must
give the oracle's ids bit-exact and its logits within REL_TOL; the polled
loop must really have polled (mitok_resident_exchange reports it), and a
program it does not run (RoPE in a product prologue) must fall back to the
barrier exchange with the same results.  Both exchanges perform the same
operations in the same order, so their logits agree bit for bit.
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


# config-3 layer shape (d 512, 8 heads of 64, FFN 2048) with two layers, a
# smaller vocab and context, so the oracle finishes in seconds
C3S = configs.ModelConfig("c3s", layers=2, d=512, heads=8, ffn=2048, vocab=4000, max_ctx=192, seed=2)
# head dim 16: the generic attention path of the kernel
SMALL = configs.ModelConfig("small", layers=2, d=64, heads=4, ffn=128, vocab=1000, max_ctx=160, seed=21)
# a long context: more attention chunks than blocks, so the combines are
# items of their own after the chunks
LONG = configs.ModelConfig("long", layers=2, d=128, heads=8, ffn=256, vocab=1000, max_ctx=2048, seed=33)
# RoPE after the embedding: a prologue the polled loop does not run
ROPE = configs.ModelConfig("rope", layers=2, d=64, heads=4, ffn=128, vocab=1000, max_ctx=96, seed=5, rope=True)


def _run(g, prompt, n_new, mode):
    g.set_decode_plan(2)
    g.resident_exchange(mode)
    ids, lg = g.generate(prompt, n_new=n_new, want_logits=True)
    loop = g.last_timings()["decode_loop"]
    return ids, lg, loop, g.resident_exchange(-1)


@pytest.mark.parametrize("cfg,plen,n_new", [(C3S, 40, 20), (C3S, 150, 33), (SMALL, 12, 64), (SMALL, 90, 7),
                                            (LONG, 300, 12), (LONG, 1990, 9)])
def test_polled_and_barrier_loops_match_oracle(cfg, plen, n_new):
    """Batch 1: both exchanges against the oracle, at even and odd step
    counts (the last step's argmax partials in either half of the arena),
    with many attention chunks (prompts near the context) and with more
    chunks than blocks."""
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    prompt = seeded.prompts(80 + plen, [plen], cfg.vocab)
    io, lo = o.generate(prompt, n_new=n_new, want_logits=True)
    try:
        out = {}
        for mode in (1, 0):
            ids, lg, loop, polled = _run(g, prompt, n_new, mode)
            err = max_rel_err(lg, lo)
            log(f"{cfg.name} prompt {plen} n_new {n_new} exchange {mode}: loop {loop}, polled {polled}, "
                f"ids {np.array_equal(ids, io)}, logits {err:.2e}")
            assert loop == "resident"
            assert polled == (mode == 1)
            assert np.array_equal(ids, io), f"exchange {mode}"
            assert err < REL_TOL, f"exchange {mode}"
            out[mode] = lg
        assert np.array_equal(out[1], out[0])
    finally:
        g.close()
        o.close()


@pytest.mark.parametrize("cfg,lens,n_new", [(C3S, [40, 23], 15), (C3S, [150, 7, 64, 33], 12),
                                            (SMALL, [12, 30, 5, 17, 9, 26, 40, 3], 20), (LONG, [300, 120], 8)])
def test_polled_and_barrier_loops_match_oracle_batched(cfg, lens, n_new):
    """2-8 sequences of different lengths (plan 3): both exchanges against the
    oracle, ids bit-exact and logits within REL_TOL, and equal to each other
    bit for bit."""
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    prompt = seeded.prompts(500 + len(lens), lens, cfg.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    try:
        out = {}
        for mode in (1, 0):
            g.set_decode_plan(3)
            g.resident_exchange(mode)
            ids, lg = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
            loop, polled = g.last_timings()["decode_loop"], g.resident_exchange(-1)
            err = max_rel_err(lg, lo)
            log(f"{cfg.name} B={len(lens)} exchange {mode}: loop {loop}, polled {polled}, ids {np.array_equal(ids, io)}, "
                f"logits {err:.2e}")
            assert loop == "resident"
            assert polled == (mode == 1)
            assert np.array_equal(ids, io), f"exchange {mode}"
            assert err < REL_TOL, f"exchange {mode}"
            out[mode] = lg
        assert np.array_equal(out[1], out[0])
    finally:
        g.close()
        o.close()


def test_polled_loop_repeats_on_one_network():
    """Three polled generates in a row on one network (the arena, barrier
    epochs and chunk counters carried between launches), with step counts of
    both parities, each against the oracle."""
    g = configs.build_network(ra.Network(0), C3S)
    o = configs.build_network(oracle.Network(), C3S)
    try:
        for k, (plen, n_new) in enumerate([(30, 9), (61, 16), (17, 25)]):
            prompt = seeded.prompts(300 + k, [plen], C3S.vocab)
            io, lo = o.generate(prompt, n_new=n_new, want_logits=True)
            ids, lg, loop, polled = _run(g, prompt, n_new, 1)
            err = max_rel_err(lg, lo)
            log(f"repeat {k}: prompt {plen} n_new {n_new}: polled {polled}, ids {np.array_equal(ids, io)}, "
                f"logits {err:.2e}")
            assert loop == "resident" and polled
            assert np.array_equal(ids, io)
            assert err < REL_TOL
    finally:
        g.close()
        o.close()


def test_rope_program_falls_back_to_barrier_exchange():
    """With RoPE in a prologue the loop runs the barrier exchange even when
    polling is asked for, and still matches the oracle."""
    g = configs.build_network(ra.Network(0), ROPE)
    o = configs.build_network(oracle.Network(), ROPE)
    prompt = seeded.prompts(9, [14], ROPE.vocab)
    io, lo = o.generate(prompt, n_new=12, want_logits=True)
    try:
        ids, lg, loop, polled = _run(g, prompt, 12, 1)
        err = max_rel_err(lg, lo)
        log(f"rope: loop {loop}, polled {polled}, ids {np.array_equal(ids, io)}, logits {err:.2e}")
        assert loop == "resident" and not polled
        assert np.array_equal(ids, io)
        assert err < REL_TOL
    finally:
        g.close()
        o.close()
