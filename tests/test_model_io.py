"""Reference model import (rustcrates_amd/model_io.py): the bincode layout of
the NeuralNetwork file and of the sled embedding values, pinned against bytes
assembled field by field from the reference's struct declarations, the
reference's own STORAGE/embedding/embedding_layer.json, and round trips; the
imported model then runs on the CPU checker (here) and the HIP path
(test_gpu_model_io in tests/test_gpu_loop.py) with the seeded model's results.
"""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

import oracle
from conftest import ROOT, build_explicit, seeded_tensors
from rustcrates_amd import configs, model_io

GOLDEN = os.path.join(ROOT, "tests", "golden")


def _u64(v):
    return struct.pack("<Q", v)


def _u32(v):
    return struct.pack("<I", v)


def _f64(v):
    return struct.pack("<d", v)


def _vec_c(vals):
    return _u64(len(vals)) + b"".join(struct.pack("<dd", c.real, c.imag) for c in vals)


def _mat_c(rows):
    return _u64(len(rows)) + b"".join(_vec_c(r) for r in rows)


def test_reference_embedding_layer_file_decodes():
    """The reference's own bincode file (EmbeddingLayer::serialize,
    embedding_layer.rs:271-287): vocab_size 50280, embedding_dim 16 (the
    create_transformer default, transformer_builder.rs:10-72), lr 0.001."""
    data = open(os.path.join(GOLDEN, "reference_embedding_layer.bin"), "rb").read()
    f = model_io.read_embedding_layer_meta(data)
    assert f == {"vocab_size": 50280, "embedding_dim": 16, "learning_rate": 0.001, "time_step": 0}
    # the same fields inside a LayerEnum: variant index 0 (u32) in front
    m = model_io.read_network(_u64(1) + _u32(0) + data + _f64(0.01) + _u64(1) + _u64(2) + _u64(3) + _u64(4) + _u64(5))
    assert m.layers[0].kind == "Embedding" and m.layers[0].f == f
    assert (m.learning_rate, m.number_of_input_neurons, m.minibatch_size) == (0.01, 1, 5)


def _hand_model():
    """A NeuralNetwork assembled byte by byte from the struct declarations:
    Norm, SelfAttention (1 head, with its Norm), FeedForward (Dense GELU ->
    Linear, no norm), Linear, Softmax."""
    g = [1 + 2j, 3 - 1j]
    b = [0.5 + 0j, -0.25 + 1j]
    norm = _u32(5) + _vec_c(g) + _vec_c(b) + _f64(1e-5) + _f64(0.01) + _u64(0)  # norm_layer.rs:17-42
    wq, wk, wv = [[1 + 1j, 2 + 0j], [0 + 3j, -1 + 0j]], [[2 + 0j, 0 + 1j], [1 + 0j, 1 + 1j]], [[0 + 1j, 1 + 0j], [3 + 0j, 2 - 1j]]
    bp = [[0.1 + 0j, 0.2 + 0j], [0.3 + 0j, 0.4 + 0j]]
    head = (_mat_c(wq) + _mat_c(wk) + _mat_c(wv) + _mat_c(bp) + _vec_c([0j, 0j]) * 3 + _u32(3) + _f64(0.01) + _u64(7)
            + _mat_c([]) + _mat_c([]))  # masked_attention_head.rs:23-61
    attn_norm = _u32(5) + _vec_c([1 + 0j, 1 + 0j]) + _vec_c([0j, 0j]) + _f64(1e-12) + _f64(0.01) + _u64(0)
    sa = _u32(6) + _u64(1) + head + _mat_c([]) + b"\x01" + attn_norm + _u64(0)  # self_attention_layer.rs:16-25
    w1, b1 = [[1 + 0j, 0 + 1j, 2 + 0j], [0 + 0j, 1 + 0j, 1 - 1j]], [1 + 0j, 1 + 0j, 1 + 0j]
    w2, b2 = [[1 + 0j, 2 + 0j], [0 + 1j, 0 + 0j], [3 + 0j, 1 + 1j]], [1 + 0j, 0 + 2j]
    dense = _u32(2) + _mat_c(w1) + _vec_c(b1) + _u32(8) + _u32(4) + _f64(0.01) + _u64(0)  # layer.rs:91-112
    lin2 = _u32(7) + _mat_c(w2) + _vec_c(b2) + _f64(0.01) + _u64(0)  # linear_layer.rs:18-34
    ffn = _u32(3) + _u64(2) + dense + lin2 + b"\x00" + _f64(0.01) + _u64(0)  # feedforward_layer.rs:14-26
    wv_ = [[1 + 0j, 2 + 0j, 3 + 0j], [4 + 0j, 5 + 1j, 6 + 0j]]
    vocab = _u32(7) + _mat_c(wv_) + _vec_c([1 + 0j] * 3) + _f64(0.01) + _u64(0)
    smax = _u32(11) + _f64(0.01) + _u32(1)  # softmax_output_layer.rs:15-27, PRODUCTION
    blob = _u64(5) + norm + sa + ffn + vocab + smax + _f64(0.01) + _u64(2) + _u64(3) + _u64(1) + _u64(3) + _u64(1)
    return blob, dict(g=g, b=b, wq=wq, wk=wk, wv=wv, bp=bp, w1=w1, b1=b1, w2=w2, b2=b2, wv_=wv_)


def test_hand_assembled_network_decodes_field_by_field():
    blob, v = _hand_model()
    m = model_io.read_network(blob)
    assert [L.kind for L in m.layers] == ["Norm", "SelfAttention", "FeedForward", "Linear", "Softmax"]
    n = m.layers[0].f
    assert np.array_equal(n["gamma"], v["g"]) and np.array_equal(n["beta"], v["b"]) and n["epsilon"] == 1e-5
    sa = m.layers[1].f
    h = sa["attention_heads"][0]
    for k, want in (("weights_q", "wq"), ("weights_k", "wk"), ("weights_v", "wv"), ("bias_pos", "bp")):
        assert np.array_equal(h[k], np.array(v[want]))
    assert h["layer_type"] == 3 and h["time_step"] == 7
    assert sa["norm_layer"].kind == "Norm" and sa["norm_layer"].f["epsilon"] == 1e-12
    ff = m.layers[2].f
    assert [s.kind for s in ff["layers"]] == ["Dense", "Linear"] and ff["norm_layer"] is None
    assert ff["layers"][0].f["activation_type"] == model_io.GELU
    assert np.array_equal(ff["layers"][0].f["weights"], np.array(v["w1"]))  # [in][out] as stored
    assert np.array_equal(ff["layers"][1].f["bias"], v["b2"])
    assert np.array_equal(m.layers[3].f["weights"], np.array(v["wv_"]))
    assert m.layers[4].f["operation_mode"] == model_io.PRODUCTION
    assert (m.number_of_output_neurons, m.number_of_hidden_neurons) == (3, 3)
    assert model_io.write_network(m) == blob  # the writer restates the same bytes


def test_truncated_and_trailing_bytes_are_errors():
    blob, _ = _hand_model()
    with pytest.raises(model_io.FormatError, match="truncated"):
        model_io.read_network(blob[:-3])
    with pytest.raises(model_io.FormatError, match="trailing"):
        model_io.read_network(blob + b"\x00")
    with pytest.raises(model_io.FormatError, match="variant"):
        model_io.read_network(_u64(1) + _u32(12))


def test_embedding_values_and_pairs():
    """A sled value is bincode Vec<Complex<f64>> (embedding_layer.rs:263-269)."""
    vals = [0.5 - 1j, 2 + 0.25j, -3 + 0j]
    assert np.array_equal(model_io.decode_embedding(_vec_c(vals)), vals)
    assert model_io.encode_embedding(vals) == _vec_c(vals)
    stream = b"".join(_u64(len(str(k))) + str(k).encode() + _u64(len(_vec_c(x))) + _vec_c(x)
                      for k, x in ((0, vals), (2, vals[::-1])))
    pairs = model_io.read_embedding_pairs(stream)
    assert set(pairs) == {0, 2} and np.array_equal(pairs[2], vals[::-1])
    t = model_io.embedding_table(pairs, 3, 3)  # id 1 (PAD) may be absent
    assert np.array_equal(t[1], [0, 0, 0])
    with pytest.raises(model_io.FormatError, match="no embedding"):
        model_io.embedding_table(pairs, 4, 3)


def test_hand_model_runs_on_checker_like_explicit_layers():
    """The decoded model appends exactly the layers the explicit calls would."""
    blob, v = _hand_model()
    m = model_io.read_network(blob)
    table = np.array([[1 + 0j, 0.5 - 0.5j], [0, 0], [2 - 1j, 0.25 + 0j]])
    pairs = {0: table[0], 2: table[2]}
    a = oracle.Network()
    a.add_embedding(3, 2, table)
    b = oracle.Network()
    b.add_embedding(3, 2, table)
    m_no_emb = model_io.Model(m.layers)
    model_io.to_device(m_no_emb, a)
    b.add_norm(2, 1e-5, v["g"], v["b"])
    b.add_self_attention(1, 2, 2, 1e-12, [v["wq"]], [v["wk"]], [v["wv"]], [v["bp"]], [1, 1], [0, 0])
    b.add_feed_forward(2, 3, v["w1"], v["b1"], v["w2"], v["b2"])
    b.add_linear(2, 3, v["wv_"], [1, 1, 1])
    b.add_softmax(1)
    ids = np.array([[0, 2]], np.uint32)
    la, _ = a.predict(ids, forward_only=True)
    lb, _ = b.predict(ids, forward_only=True)
    assert np.array_equal(la, lb)
    assert model_io.embedding_table(pairs, 3, 2)[2][0] == 2 - 1j


def test_seeded_model_round_trip_and_golden_fixture():
    """The committed fixture (tests/golden/make_model_fixture.py) decodes,
    re-encodes to the same bytes, and its model reproduces the stored ids and
    logits on the checker and the seeded stack's results bit for bit."""
    import sys

    sys.path.insert(0, GOLDEN)
    import make_model_fixture as mk

    blob = open(os.path.join(GOLDEN, "tiny_model.bincode"), "rb").read()
    emb = open(os.path.join(GOLDEN, "tiny_embeddings.pairs"), "rb").read()
    exp = np.load(os.path.join(GOLDEN, "tiny_expected.npz"))
    m = model_io.read_network(blob)
    assert model_io.write_network(m) == blob
    pairs = model_io.read_embedding_pairs(emb)
    assert model_io.write_embedding_pairs(pairs) == emb
    o = model_io.to_device(m, oracle.Network(), pairs)
    ids, lg = o.generate(exp["prompt"], n_new=mk.N_NEW, want_logits=True)
    assert np.array_equal(ids, exp["ids"]) and np.array_equal(lg, exp["logits"])
    ref = build_explicit(oracle.Network(), mk.CFG, seeded_tensors(mk.CFG))
    ids2, lg2 = ref.generate(exp["prompt"], n_new=mk.N_NEW, want_logits=True)
    assert np.array_equal(ids, ids2) and np.array_equal(lg, lg2)


def test_unsupported_layers_are_refused():
    cfg = configs.ModelConfig("t", layers=1, d=4, heads=1, ffn=8, vocab=10, max_ctx=8, seed=1)
    m = model_io.from_tensors(cfg, seeded_tensors(cfg))
    m.layers.insert(1, model_io.Layer("RMSNorm", {"gamma": np.ones(4), "epsilon": 1e-8, "learning_rate": 0.0,
                                                  "time_step": 0}))
    blob = model_io.write_network(m)
    m2 = model_io.read_network(blob)
    assert m2.layers[1].kind == "RMSNorm"
    with pytest.raises(NotImplementedError, match="RMSNorm"):
        model_io.to_device(m2, oracle.Network(), {i: np.zeros(4) for i in range(10)})


def test_default_stack_file_with_wavelet_layer_imports():
    """A DiscreteWavelet layer (wavelet_discrete_layer.rs:20-52: time_step,
    wavelet, wavelet_mode, is_full_mode) decodes from hand-assembled bytes and
    imports as the device stack's wavelet layer."""
    blob = (_u64(1) + _u32(9) + _u64(0) + _u32(1) + _u32(2) + b"\x00" + _f64(0.01) + _u64(0) * 5)
    m = model_io.read_network(blob)
    assert m.layers[0].kind == "DiscreteWavelet"
    assert m.layers[0].f == {"time_step": 0, "wavelet": 1, "wavelet_mode": 2, "is_full_mode": False}
    assert model_io.write_network(m) == blob
    cfg = configs.ModelConfig("t", layers=1, d=8, heads=2, ffn=16, vocab=40, max_ctx=24, seed=3)
    full = model_io.from_tensors(cfg, seeded_tensors(cfg))
    full.layers.insert(1, m.layers[0])
    t = seeded_tensors(cfg)[0]["table"].reshape(40, 8)
    a = model_io.to_device(model_io.read_network(model_io.write_network(full)), oracle.Network(),
                           {i: t[i] for i in range(40) if i != 1})
    b = oracle.Network()
    b.add_embedding(40, 8, t)
    b.add_discrete_wavelet(8, 1, 2)
    rest = model_io.Model(full.layers[2:])
    model_io.to_device(rest, b)
    ids = np.array([[3, 9, 27, 5, 11, 2, 30]], np.uint32)
    la, _ = a.predict(ids, forward_only=True)
    lb, _ = b.predict(ids, forward_only=True)
    assert la.shape == (1, oracle.dwt_rows(7, 1), 40) and np.array_equal(la, lb)
