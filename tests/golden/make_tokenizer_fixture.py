"""Writes tests/golden/gpt_neox_fixture.json from the reference's tokenizer
file (src/neural_networks/tokenizers/gtp_neox_tokenizer.json, read with the
`tokenizers` library as utils/tokenizer.rs:9-49 does):

  - encodings: "<bos> " + text (the prefix of extend_input_with_bos,
    network_components/input.rs:70-72) encoded with special tokens added,
    for a set of texts;
  - decodings: each id of those encodings, the special ids, and every id the
    text-path test model generates, decoded alone with special tokens kept
    (detokenize(ids, false));
  - text_loop: the CPU checker's predict_token_by_token on that model
    (texts and generated ids), which the GPU test reproduces.

Only ids and strings are stored, not the tokenizer file.

    python tests/golden/make_tokenizer_fixture.py /path/to/gtp_neox_tokenizer.json
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT]

TEXTS = [
    "Hallo, wie geht es dir?",
    "What is the capital of France?",
    "Привет, как дела?",
    "The price of BTC rose 3.5% to $64,000 on 2024-03-11.",
    "<eos> inside text and <sep> too",
    "  leading spaces, tabs\tand\nnewlines",
    "emoji 🚀 and accents: café, naïve, Zürich",
]
# the model of tests/test_text.py::test_text_path_gpu_with_gpt_neox_ids
MODEL = dict(name="neox16", layers=2, d=16, heads=2, ffn=64, vocab=50280, max_ctx=512, seed=5)
LOOP_INPUTS = [["What is the capital of France?"], ["Hallo, wie geht es dir?"]]


def main(path):
    import oracle
    from rustcrates_amd import configs, text

    tok = text.load_tokenizer(path)
    enc = {}
    for t in TEXTS:
        e = tok.encode(text.BOS_PREFIX + t, add_special_tokens=True)
        enc[t] = {"ids": e.ids, "tokens": e.tokens}
    ids = {i for v in enc.values() for i in v["ids"]} | {0, 1, 50277, 50278, 50279, 50280, 50281}
    cfg = configs.ModelConfig(**MODEL)
    net = configs.build_network(oracle.Network(), cfg)
    loops = []
    for inp in LOOP_INPUTS:
        preds, texts = text.predict_token_by_token(net, inp, tok)
        gen = [text.greedy_id(p[-1]) for p in preds]
        ids |= set(gen)
        e = tok.encode(text.BOS_PREFIX + inp[0], add_special_tokens=True)
        enc.setdefault(inp[0], {"ids": e.ids, "tokens": e.tokens})
        loops.append({"inputs": inp, "texts": texts, "generated": gen})
    dec = {str(i): tok.decode([i], skip_special_tokens=False) for i in sorted(ids)}
    out = {"tokenizer": "gtp_neox_tokenizer.json of the reference (utils/tokenizer.rs:6)",
           "vocab_size_with_added": tok.get_vocab_size(), "special": {s: tok.token_to_id(s) for s in
                                                                      ("<bos>", "<eos>", "<sep>", "<|padding|>", "<|endoftext|>")},
           "encodings": enc, "decodings": dec, "model": MODEL, "text_loop": loops}
    with open(os.path.join(HERE, "gpt_neox_fixture.json"), "w", encoding="utf-8") as fh:
        json.dump(out, fh, ensure_ascii=False, indent=0)
    print(f"{len(enc)} encodings, {len(dec)} decodings; loops {[lp['texts'][0] for lp in loops]}")


if __name__ == "__main__":
    main(sys.argv[1])
