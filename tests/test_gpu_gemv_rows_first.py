"""GPU parity of the 2-8-sequence GEMV whose plain input rows are requested
before its weights (plan 1): the layer products of config 3's shape (K 512
and 2048, up to 8 x 512 staged row elements per block, the most the staging
registers take) and of config 5's (K 768 per block, 24 weight rows per lane:
16 requested before the rows land and 8 after), with 2 to 8 sequences (plan 1
materialises its products' rows from 2), partial row groups included (3, 6
and 7 sequences in 4- and 8-row blocks).

Bar: ids bit-exact against the oracle, Re-logits within REL_TOL.
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

# config 3's layer shape with two layers and a small vocab
C3W = configs.ModelConfig("c3w", layers=2, d=512, heads=8, ffn=2048, vocab=3000, max_ctx=96, seed=41)
# config 5's layer shape, one layer
C5W = configs.ModelConfig("c5w", layers=1, d=768, heads=12, ffn=3072, vocab=3000, max_ctx=64, seed=43)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("cfg,B", [(C3W, 2), (C3W, 3), (C3W, 4), (C3W, 6), (C3W, 7), (C3W, 8), (C5W, 4), (C5W, 5)])
def test_rows_first_gemv_matches_oracle(cfg, B):
    lens = [5 + (11 * b) % 29 for b in range(B)]
    g = configs.build_network(ra.Network(0), cfg)
    o = configs.build_network(oracle.Network(), cfg)
    prompt = seeded.prompts(900 + B, lens, cfg.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=12, want_logits=True)
    try:
        g.set_decode_plan(1)
        ig, lg = g.generate(prompt, lens=lens, n_new=12, want_logits=True)
        err = max_rel_err(lg, lo)
        log(f"{cfg.name} B={B}: loop {g.last_timings()['decode_loop']}, ids {np.array_equal(ig, io)}, logits {err:.2e}")
        assert np.array_equal(ig, io)
        assert err < REL_TOL
    finally:
        g.close()
        o.close()
