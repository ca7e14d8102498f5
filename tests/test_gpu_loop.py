"""GPU parity of the token-loop entry points beyond mitok_generate with
logits: the logits-free generate that bench.py times, the per-step
mitok_prefill / mitok_decode_step boundary, PAD (id 1) fed back by greedy
decoding, and the error paths of the per-step calls.

Bar: ids bit-exact against the CPU oracle; Re-logits within REL_TOL; the
per-step path and generate on the same plan bit-identical (same kernels, same
summation order).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
import rustcrates_amd as ra
from conftest import NOISE_FACTOR, REL_TOL, build_explicit, max_rel_err, oracle_noise_floor, seeded_tensors
from rustcrates_amd import configs, seeded

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# config-3 layer shape (d 512, 8 heads, FFN 2048) with two layers and a
# smaller vocab and context, so the oracle finishes in seconds
C3S = configs.ModelConfig("c3s", layers=2, d=512, heads=8, ffn=2048, vocab=4000, max_ctx=192, seed=2)


@pytest.fixture(scope="module")
def c3s_nets():
    g = configs.build_network(ra.Network(0), C3S)
    o = configs.build_network(oracle.Network(), C3S)
    yield g, o
    g.close()
    o.close()


@pytest.mark.parametrize("lens", [[40], [33, 17], [24 + (5 * b) % 29 for b in range(32)]])
def test_logits_free_generate_matches_logits_run_and_oracle(c3s_nets, lens):
    """generate(want_logits=False) is what bench.py times: its own captured
    graph and resident build (no logits history).  Its ids must equal the
    logits run's on every plan, and sequence 0 the oracle's."""
    g, o = c3s_nets
    B, n_new = len(lens), 20
    prompt = seeded.prompts(60 + B, lens, C3S.vocab)
    io = o.generate(prompt[:1, :lens[0]], n_new=n_new)
    for plan in (3, 1, 0):
        g.set_decode_plan(plan)
        ids_l, _ = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
        ids = g.generate(prompt, lens=lens, n_new=n_new)
        loop = g.last_timings()["decode_loop"]
        log(f"logits-free generate B={B} plan {plan} ({loop}): equal {np.array_equal(ids, ids_l)}, "
            f"seq 0 vs oracle {np.array_equal(ids[:1], io)}")
        if plan == 3 and B <= 8:
            assert loop == "resident"
        assert np.array_equal(ids, ids_l), f"plan {plan}"
        assert np.array_equal(ids[:1], io), f"plan {plan}"


def test_pad_id_fed_back_by_greedy_decoding():
    """A vocab bias on id 1 makes PAD the greedy id at some steps, so the loop
    feeds PAD (embedded as the zero vector, embedding_layer.rs:183-184) back
    and later leaves it again; a PAD also sits mid-prompt.  Every plan matches
    the oracle."""
    cfg = configs.ModelConfig("pad", layers=2, d=64, heads=4, ffn=128, vocab=500, max_ctx=96, seed=13)
    t = seeded_tensors(cfg)
    t[-1]["b"] = t[-1]["b"].copy()
    t[-1]["b"][1] += 5.0
    g, o = build_explicit(ra.Network(0), cfg, t), build_explicit(oracle.Network(), cfg, t)
    lens = [10, 7]
    prompt = seeded.prompts(3, lens, cfg.vocab)
    prompt[0, 4] = 1
    io, lo = o.generate(prompt, lens=lens, n_new=24, want_logits=True)
    fed_back = [any(io[b, k] == 1 and io[b, k + 1] != 1 for k in range(23)) for b in range(2)]
    assert any(fed_back), io  # PAD is generated, fed back, and followed by another id
    for plan in (3, 1, 0):
        g.set_decode_plan(plan)
        ig, lg = g.generate(prompt, lens=lens, n_new=24, want_logits=True)
        log(f"PAD feedback plan {plan}: ids {np.array_equal(ig, io)}, logits {max_rel_err(lg, lo):.2e}")
        assert np.array_equal(ig, io), f"plan {plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan {plan}"
    g.close()


MID = configs.ModelConfig("mid", layers=2, d=64, heads=4, ffn=128, vocab=1000, max_ctx=96, seed=21)


@pytest.mark.parametrize("lens", [[15], [9, 30, 4], [6 + (7 * b) % 19 for b in range(20)]])
def test_prefill_and_decode_steps_equal_generate(lens):
    """mitok_prefill + mitok_decode_step (ids fed back on the device) give the
    same ids and the bit-identical logits as generate on the same plan, and
    match the oracle."""
    g = configs.build_network(ra.Network(0), MID)
    o = configs.build_network(oracle.Network(), MID)
    B, n_new = len(lens), 12
    prompt = seeded.prompts(70 + B, lens, MID.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    g.set_decode_plan(1)
    ig, lg = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    ids, lgs = [], []
    first, l0 = g.prefill(prompt, lens=lens, want_logits=True)
    ids.append(first)
    lgs.append(l0)
    for _ in range(n_new - 1):
        nxt, ln = g.decode_step(want_logits=True)
        ids.append(nxt)
        lgs.append(ln)
    steps, steps_lg = np.stack(ids, axis=1), np.stack(lgs)
    # the batched products sum in another order than the oracle; at the edge of
    # the bar the oracle's own valid orders set it (conftest.oracle_noise_floor)
    floor = oracle_noise_floor(o, prompt, lens, n_new, lo)[0]
    tol = max(REL_TOL, NOISE_FACTOR * floor)
    log(f"per-step B={B}: equals generate {np.array_equal(steps, ig)}, logits identical "
        f"{np.array_equal(steps_lg, lg)}, vs oracle {max_rel_err(steps_lg, lo):.2e} (tol {tol:.2e})")
    assert np.array_equal(steps, ig)
    assert np.array_equal(steps_lg, lg)
    assert np.array_equal(steps, io)
    assert max_rel_err(steps_lg, lo) < tol
    # logits-free steps give the same ids
    first2 = g.prefill(prompt, lens=lens)
    seq = [first2] + [g.decode_step() for _ in range(n_new - 1)]
    assert np.array_equal(np.stack(seq, axis=1), io)
    g.close()


def test_decode_step_with_caller_ids_matches_cached_predict():
    """decode_step(ids) feeds the caller's ids (teacher forcing), as the
    oracle's cached predict does with one row per sequence."""
    g = configs.build_network(ra.Network(0), MID)
    o = configs.build_network(oracle.Network(), MID)
    lens = [11, 11]
    prompt = seeded.prompts(81, [14, 14], MID.vocab)
    g.prefill(prompt[:, :11], lens=lens)
    o.reset()
    o.predict(prompt[:, :11], forward_only=True)
    for t in (11, 12, 13):
        got_ids, got = g.decode_step(prompt[:, t], want_logits=True)
        want, _ = o.predict(prompt[:, t:t + 1], time_steps=[t, t], forward_only=True)
        log(f"teacher-forced step {t}: {max_rel_err(got, want[:, 0]):.2e}")
        assert max_rel_err(got, want[:, 0]) < REL_TOL
        assert np.array_equal(got_ids, [oracle.greedy_row(want[b, 0]) for b in range(2)])
    g.close()


def test_decode_step_errors_leave_network_usable():
    g = configs.build_network(ra.Network(0), MID)
    with pytest.raises(ra.MitokError, match="ERR_STATE"):
        g.decode_step(batch=1)  # no prefill yet
    prompt = seeded.prompts(90, [8, 8], MID.vocab)
    g.prefill(prompt)
    with pytest.raises(ra.MitokError, match="ERR_STATE"):
        g.decode_step(np.array([3], np.uint32))  # batch 1 against a prefill of 2
    g.prefill(prompt)
    with pytest.raises(ra.MitokError, match="ERR_ARG"):
        g.decode_step(np.array([3, MID.vocab], np.uint32))  # id beyond the vocab
    # a prompt that leaves no room: max_ctx 96 keys
    full = seeded.prompts(91, [96], MID.vocab)
    g.prefill(full)
    with pytest.raises(ra.MitokError, match="ERR_ARG"):
        g.decode_step()
    with pytest.raises(ra.MitokError, match="ERR_ARG"):
        g.generate(seeded.prompts(92, [90], MID.vocab), n_new=8)  # 90 + 7 > 96
    # still usable after every error
    p = seeded.prompts(93, [12], MID.vocab)
    a = g.generate(p, n_new=6)
    o = configs.build_network(oracle.Network(), MID)
    assert np.array_equal(a, o.generate(p, n_new=6))
    g.close()


def test_generate_to_max_context_exactly():
    """prompt + n_new - 1 == max_ctx: the last step attends over every cache
    row (the boundary of the KV cache), on every plan."""
    lens = [60, 33]
    n_new = 96 - 60 + 1
    g = configs.build_network(ra.Network(0), MID)
    o = configs.build_network(oracle.Network(), MID)
    prompt = seeded.prompts(94, lens, MID.vocab)
    io, lo = o.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
    for plan in (3, 1, 0):
        g.set_decode_plan(plan)
        ig, lg = g.generate(prompt, lens=lens, n_new=n_new, want_logits=True)
        assert np.array_equal(ig, io), f"plan {plan}"
        assert max_rel_err(lg, lo) < REL_TOL, f"plan {plan}"
    g.close()


def test_imported_reference_model_file_runs_on_gpu():
    """The committed model file in the reference's layout (bincode
    NeuralNetwork + sled embedding pairs, tests/golden/make_model_fixture.py)
    imported onto the HIP network: ids equal the stored checker ids, logits
    within REL_TOL, on every decode plan."""
    import os

    from conftest import ROOT
    from rustcrates_amd import model_io

    gold = os.path.join(ROOT, "tests", "golden")
    m = model_io.read_network(os.path.join(gold, "tiny_model.bincode"))
    pairs = model_io.read_embedding_pairs(open(os.path.join(gold, "tiny_embeddings.pairs"), "rb").read())
    exp = np.load(os.path.join(gold, "tiny_expected.npz"))
    g = model_io.to_device(m, ra.Network(0), pairs)
    for plan in (3, 1, 0):
        g.set_decode_plan(plan)
        ig, lg = g.generate(exp["prompt"], n_new=exp["ids"].shape[1], want_logits=True)
        log(f"imported model plan {plan}: ids {ig[0].tolist()}, logits {max_rel_err(lg, exp['logits']):.2e}")
        assert np.array_equal(ig, exp["ids"]), f"plan {plan}"
        assert max_rel_err(lg, exp["logits"]) < REL_TOL, f"plan {plan}"
    g.close()


def test_import_of_a_config3_shaped_file_equals_the_seeded_network():
    """A config-3-shaped model written in the reference's file layout and read
    back uploads the same tensors: the imported and the seeded HIP networks
    give bit-identical ids and logits."""
    from rustcrates_amd import model_io

    cfg = configs.ModelConfig("c3f", layers=2, d=512, heads=8, ffn=2048, vocab=3000, max_ctx=160, seed=4)
    t = seeded_tensors(cfg)
    blob = model_io.write_network(model_io.from_tensors(cfg, t))
    table = t[0]["table"].reshape(cfg.vocab, cfg.d)
    pairs = model_io.read_embedding_pairs(model_io.write_embedding_pairs({i: table[i] for i in range(cfg.vocab)}))
    a = model_io.to_device(model_io.read_network(blob), ra.Network(0), pairs)
    b = configs.build_network(ra.Network(0), cfg)
    prompt = seeded.prompts(15, [40, 23], cfg.vocab)
    ia, la = a.generate(prompt, lens=[40, 23], n_new=10, want_logits=True)
    ib, lb = b.generate(prompt, lens=[40, 23], n_new=10, want_logits=True)
    log(f"c3-shaped import: {len(blob) / 1e6:.1f} MB file, ids equal {np.array_equal(ia, ib)}")
    assert np.array_equal(ia, ib) and np.array_equal(la, lb)
    a.close()
    b.close()
