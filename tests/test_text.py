"""The text path of predict_token_by_token (transformer_network.rs:165-313):
"<bos> " prefix, tokenization, context-window cut, per-token decode, "<eos>"
stop and the 21-token cap.  The loop logic is pinned with a stub network
whose ids are fixed; the GPU test checks the whole path against the oracle's
network on the same model and tokenizer (texts identical, logits within
REL_TOL).  The tokenizer here is a word-level one built in the test: the
reference's GPT-NeoX file is data of the reference and is not read.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REL_TOL, max_rel_err
from rustcrates_amd import configs, text

V = 300
WORDS = ["[UNK]", "<eos>", "<bos>"] + [f"w{i}" for i in range(3, V)]


def _tokenizer():
    from tokenizers import Tokenizer, models, pre_tokenizers

    tok = Tokenizer(models.WordLevel({w: i for i, w in enumerate(WORDS)}, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    return tok


class _StubNet:
    """generate() returns fixed ids and records the prompt it was given."""

    def __init__(self, ids):
        self.ids = list(ids)
        self.prompt = None

    def generate(self, prompt, lens=None, n_new=1, want_logits=False):
        self.prompt = np.asarray(prompt)
        ids = np.asarray([self.ids[:n_new]], np.uint32)
        logits = np.zeros((n_new, 1, V))
        for k in range(n_new):
            logits[k, 0, ids[0, k]] = 1.0
        return ids, logits


def test_text_loop_appends_21_tokens_without_eos():
    tok = _tokenizer()
    ids = [10 + k for k in range(30)]
    net = _StubNet(ids)
    preds, texts = text.predict_token_by_token(net, ["w5 w6"], tok)
    assert net.prompt.tolist() == [[2, 5, 6]]  # "<bos> w5 w6"
    assert len(preds) == 21
    assert texts == ["<bos> w5 w6" + "".join(f"w{i}" for i in ids[:21])]


def test_text_loop_stops_at_eos_without_appending_it():
    tok = _tokenizer()
    net = _StubNet([7, 8, 9, 1, 11] + [12] * 30)  # id 1 decodes to "<eos>"
    preds, texts = text.predict_token_by_token(net, ["w4"], tok)
    assert texts == ["<bos> w4w7w8w9"]
    assert len(preds) == 4  # the "<eos>" step's output is kept, as the reference pushes it first
    assert int(np.argmax(preds[3])) == 1


def test_text_loop_keeps_the_last_512_ids_and_other_texts():
    tok = _tokenizer()
    long = " ".join(f"w{3 + (k % 290)}" for k in range(700))
    net = _StubNet([20] * 30)
    _, texts = text.predict_token_by_token(net, [long, "w9"], tok)
    want = tok.encode("<bos> " + long).ids[-512:]
    assert net.prompt.shape == (1, 512)
    assert net.prompt[0].tolist() == want
    assert texts[1] == "<bos> w9"


TEXT_MODEL = configs.ModelConfig("text", layers=2, d=32, heads=4, ffn=64, vocab=V, max_ctx=64, seed=3)


@pytest.mark.gpu
def test_text_path_gpu_matches_oracle():
    import oracle
    import rustcrates_amd as ra

    tok = _tokenizer()
    inputs = ["w5 w17 w42 w8"]
    o = configs.build_network(oracle.Network(), TEXT_MODEL)
    g = configs.build_network(ra.Network(0), TEXT_MODEL)
    po, to = text.predict_token_by_token(o, inputs, tok)
    pg, tg = text.predict_token_by_token(g, inputs, tok)
    print(f"text path: {tg[0]!r}", flush=True)
    assert tg == to
    assert len(pg) == len(po)
    assert max_rel_err(np.stack(pg), np.stack(po)) < REL_TOL
