"""GPU parity of prefill attention (T == S keys, causal mask, bias_pos, pad rows).

Head dims 16, 32, 64 and 128 run the tiled MFMA kernel; 24 runs the one-row
kernel.  Each case is checked against the CPU oracle and against the one-row
kernel (set_decode_plan(False)) on the same network, for the cache-filling
prefill (forward_only) and the stateless forward.  Sequence lengths cross the
16-row, 32-key and block boundaries and include ragged batches (pad rows).

Bar: ids bit-exact; Re-logits within REL_TOL of the oracle, or, where the
model's complex LayerNorms amplify rounding past that (long prompts, d = 128),
within NOISE_FACTOR x the oracle's own spread over valid zgemm summation
orders; the same bound between the two kernels.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
import rustcrates_amd as ra
from conftest import NOISE_FACTOR, REL_TOL, max_rel_err, oracle_floor_of
from rustcrates_amd import configs, seeded

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _cfg(dh, heads, max_ctx=320):
    d = dh * heads
    # one layer: each complex LayerNorm amplifies incoming rounding, and the
    # attention kernel is what these cases exercise
    return configs.ModelConfig(f"pf{dh}", layers=1, d=d, heads=heads, ffn=2 * d, vocab=300, max_ctx=max_ctx,
                               seed=dh)


@pytest.mark.parametrize("dh,heads,lens", [
    (16, 4, [1]),
    (16, 4, [37, 5, 128, 129]),
    (32, 2, [255, 16, 33]),
    (64, 2, [300, 31]),
    (64, 8, [130, 17, 64]),
    (128, 2, [140, 7]),
    (24, 2, [50, 9]),
])
def test_prefill_attention_matches_oracle_and_row_kernel(dh, heads, lens):
    cfg = _cfg(dh, heads)
    log(f"prefill dh={dh} heads={heads} lens={lens}")
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    ids = seeded.prompts(dh + len(lens), lens, cfg.vocab)
    for forward_only in (True, False):
        for net in (g, o):
            net.reset()
        lo, mo = o.predict(ids, lens, forward_only=forward_only)

        def rerun():
            o.reset()
            return o.predict(ids, lens, forward_only=forward_only)[0]

        tol = max(REL_TOL, NOISE_FACTOR * oracle_floor_of(rerun, lo)[0])
        got = {}
        for tiled in (True, False):
            g.set_decode_plan(tiled)
            g.reset()
            got[tiled], mg = g.predict(ids, lens, forward_only=forward_only)
            if forward_only:
                assert np.array_equal(mg, mo)
        g.set_decode_plan(True)
        e_t, e_r = max_rel_err(got[True], lo), max_rel_err(got[False], lo)
        log(f"  forward_only={forward_only}: tiled {e_t:.3e}, rows {e_r:.3e}, "
            f"tiled vs rows {max_rel_err(got[True], got[False]):.3e}, tol {tol:.3e}")
        assert e_t < tol
        assert e_r < tol
        assert max_rel_err(got[True], got[False]) < tol


def test_prefill_then_decode_long_prompt():
    """A 250-token prompt through the tiled prefill, then 12 decode steps reading
    the cache it filled (two layers)."""
    cfg = configs.ModelConfig("pfdec", layers=2, d=128, heads=2, ffn=256, vocab=300, max_ctx=272, seed=5)
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    lens = [250, 101]
    prompt = seeded.prompts(17, lens, cfg.vocab)
    log(f"prefill+decode lens={lens}")
    ig, lg = g.generate(prompt, lens=lens, n_new=12, want_logits=True)
    io, lo = o.generate(prompt, lens=lens, n_new=12, want_logits=True)
    floor = oracle_floor_of(lambda: o.generate(prompt, lens=lens, n_new=12, want_logits=True)[1], lo)[0]
    tol = max(REL_TOL, NOISE_FACTOR * floor)
    log(f"  ids match {np.array_equal(ig, io)}, err {max_rel_err(lg, lo):.3e}, tol {tol:.3e}")
    assert np.array_equal(ig, io)
    assert max_rel_err(lg, lo) < tol
