"""The text path of predict_token_by_token (transformer_network.rs:165-313):
"<bos> " prefix, tokenization, context-window cut, per-step outputs ([S][V]
at step 0), per-token decode, "<eos>" stop and the 21-token cap.

Tokenization is pinned by tests/golden/gpt_neox_fixture.json: ids and
strings that the `tokenizers` library produced from the reference's GPT-NeoX
tokenizer file (tests/golden/make_tokenizer_fixture.py), so the loop runs on
the real vocabulary's ids ("<bos>" 50277, "<eos>" 50279, "<|padding|>" 1)
without the tokenizer file at test time.  The loop logic is pinned with a stub
network whose logits are fixed; the GPU test runs the whole path on a model
with the reference's vocabulary size against the CPU checker.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import REL_TOL, ROOT, max_rel_err
from rustcrates_amd import configs, text

FIXTURE = json.load(open(os.path.join(ROOT, "tests", "golden", "gpt_neox_fixture.json"), encoding="utf-8"))
BOS, EOS = FIXTURE["special"]["<bos>"], FIXTURE["special"]["<eos>"]


class _Enc:
    def __init__(self, ids):
        self.ids = list(ids)


class FixtureTokenizer:
    """encode / decode of the reference's tokenizer, answered from the fixture
    (an input the fixture does not hold is a test error, not a guess)."""

    def encode(self, s, add_special_tokens=True):
        assert add_special_tokens and s.startswith(text.BOS_PREFIX), s
        return _Enc(FIXTURE["encodings"][s[len(text.BOS_PREFIX):]]["ids"])

    def decode(self, ids, skip_special_tokens=False):
        assert not skip_special_tokens and len(ids) == 1
        return FIXTURE["decodings"][str(int(ids[0]))]


def test_fixture_pins_the_reference_special_tokens():
    # create_custom_tokenizer added these (utils/tokenizer.rs:51-75); PAD = 1
    # is also the embedding layer's padding id (embedding_layer.rs:112-155)
    assert FIXTURE["special"] == {"<bos>": 50277, "<eos>": 50279, "<sep>": 50278, "<|padding|>": 1,
                                  "<|endoftext|>": 0}
    for t, e in FIXTURE["encodings"].items():
        assert e["ids"][0] == BOS and e["tokens"][0] == "<bos>", t
    assert FIXTURE["decodings"][str(EOS)] == "<eos>"
    in_text = FIXTURE["encodings"]["<eos> inside text and <sep> too"]
    assert in_text["ids"][2] == EOS and in_text["tokens"][1:3] == ["\u0120", "<eos>"]  # in-text special tokens


class _StubNet:
    """predict returns logits whose argmax follows `ids`, one per call, and
    records what it was fed."""

    def __init__(self, ids, V=50280):
        self.ids, self.V = list(ids), V
        self.calls = []

    def reset(self):
        self.calls.append("reset")

    def predict(self, ids, lens=None, time_steps=None, forward_only=True):
        ids = np.asarray(ids)
        self.calls.append((ids.copy(), None if time_steps is None else list(time_steps)))
        k = sum(1 for c in self.calls if c != "reset") - 1
        out = np.zeros((1, ids.shape[1], self.V))
        out[0, -1, self.ids[k]] = 1.0
        return out, np.ones(ids.shape, np.uint32)


def test_text_loop_21_tokens_with_real_vocabulary_ids():
    tok = FixtureTokenizer()
    gen = [int(i) for i in FIXTURE["encodings"]["What is the capital of France?"]["ids"][1:]] * 3
    net = _StubNet(gen)
    preds, texts = text.predict_token_by_token(net, ["What is the capital of France?"], tok)
    prompt = FIXTURE["encodings"]["What is the capital of France?"]["ids"]
    assert net.calls[0] == "reset"
    assert net.calls[1][0].tolist() == [prompt] and net.calls[1][1] is None  # step 0: every prompt row
    assert [c[1] for c in net.calls[2:]] == [[len(prompt) + k] for k in range(20)]  # time_step = position
    assert len(preds) == 21
    assert preds[0].shape == (len(prompt), 50280) and all(p.shape == (1, 50280) for p in preds[1:])
    want = "<bos> What is the capital of France?" + "".join(tok.decode([i]) for i in gen[:21])
    assert texts == [want]


def test_text_loop_stops_at_eos_and_keeps_other_texts():
    tok = FixtureTokenizer()
    a, b = FIXTURE["encodings"]["Hallo, wie geht es dir?"]["ids"][1:3]
    net = _StubNet([a, b, EOS, a])
    preds, texts = text.predict_token_by_token(net, ["Hallo, wie geht es dir?", "Привет, как дела?"], tok)
    assert texts == ["<bos> Hallo, wie geht es dir?" + tok.decode([a]) + tok.decode([b]), "<bos> Привет, как дела?"]
    assert len(preds) == 3  # the "<eos>" step's output is kept: the reference pushes it first (:257)
    assert text.greedy_id(preds[2][-1]) == EOS


def test_greedy_id_ties_and_nan():
    assert text.greedy_id([1.0, 3.0, 3.0, 2.0]) == 2  # last of equal maxima (max_by)
    with pytest.raises(ValueError, match="NaN"):
        text.greedy_id([1.0, np.nan])


def test_text_loop_keeps_the_last_512_ids():
    class LongTok(FixtureTokenizer):
        def encode(self, s, add_special_tokens=True):
            return _Enc([BOS] + [100 + (k % 900) for k in range(700)])

    any_id = FIXTURE["encodings"]["Hallo, wie geht es dir?"]["ids"][1]
    net = _StubNet([any_id] * 30)
    text.predict_token_by_token(net, ["long"], LongTok())
    fed = net.calls[1][0]
    assert fed.shape == (1, 512) and fed[0].tolist() == [100 + (k % 900) for k in range(700)][-512:]
    assert net.calls[2][1] == [512]


MODEL = configs.ModelConfig(**FIXTURE["model"])


@pytest.mark.gpu
def test_text_path_gpu_with_gpt_neox_ids():
    """A model with the reference's vocabulary size (50280) and embedding width
    16 (create_transformer's defaults, transformer_builder.rs:10-72): the GPU
    text path produces the texts the CPU checker produced with the real
    tokenizer (stored in the fixture), and every step's logits match the
    checker's within REL_TOL."""
    import oracle
    import rustcrates_amd as ra

    tok = FixtureTokenizer()
    g = configs.build_network(ra.Network(0), MODEL)
    o = configs.build_network(oracle.Network(), MODEL)
    for loop in FIXTURE["text_loop"]:
        pg, tg = text.predict_token_by_token(g, loop["inputs"], tok)
        po, to = text.predict_token_by_token(o, loop["inputs"], tok)
        print(f"text path: {tg[0]!r}", flush=True)
        assert tg == loop["texts"] and to == loop["texts"]
        assert [text.greedy_id(p[-1]) for p in pg] == loop["generated"]
        assert len(pg) == len(po) and pg[0].shape == po[0].shape
        for a, b in zip(pg, po):
            assert max_rel_err(a, b) < REL_TOL
    g.close()
