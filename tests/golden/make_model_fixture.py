"""Writes tests/golden/tiny_model.bincode and tiny_embeddings.pairs: a small
transformer in the reference's model-file layout (bincode of NeuralNetwork,
network_types/neural_network_generic.rs:90-113) and its token embeddings as
exported from the sled tree (decimal id -> bincode Vec<Complex<f64>>,
embedding_layer.rs:263-310), plus tiny_expected.npz: the CPU checker's greedy
ids and Re-logits for a fixed prompt on that model.

    python tests/golden/make_model_fixture.py

The weights are the seeded ones of the stack below; the file layout is
rustcrates_amd.model_io's, itself pinned by tests/test_model_io.py against
hand-assembled bytes and the reference's own STORAGE/embedding file.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.dirname(HERE)]

import oracle  # noqa: E402
from conftest import seeded_tensors  # noqa: E402
from rustcrates_amd import configs, model_io  # noqa: E402

CFG = configs.ModelConfig("tiny", layers=2, d=8, heads=2, ffn=16, vocab=50, max_ctx=24, seed=31)
PROMPT = np.array([[5, 17, 3, 1, 42, 9]], np.uint32)  # a PAD (id 1) mid-prompt
N_NEW = 10


def main():
    t = seeded_tensors(CFG)
    model = model_io.from_tensors(CFG, t)
    table = t[0]["table"].reshape(CFG.vocab, CFG.d)
    pairs = {i: table[i] for i in range(CFG.vocab) if i != 1}  # PAD is never stored
    blob = model_io.write_network(model)
    emb = model_io.write_embedding_pairs(pairs)
    o = model_io.to_device(model_io.read_network(blob), oracle.Network(), model_io.read_embedding_pairs(emb))
    ids, logits = o.generate(PROMPT, n_new=N_NEW, want_logits=True)
    with open(os.path.join(HERE, "tiny_model.bincode"), "wb") as fh:
        fh.write(blob)
    with open(os.path.join(HERE, "tiny_embeddings.pairs"), "wb") as fh:
        fh.write(emb)
    np.savez(os.path.join(HERE, "tiny_expected.npz"), prompt=PROMPT, ids=ids, logits=logits)
    print(f"model {len(blob)} B, embeddings {len(emb)} B, ids {ids[0].tolist()}")


if __name__ == "__main__":
    main()
