"""Counter-based generator for synthetic weights, prompts and hidden states.

Value i of a stream is a pure function of (seed, stream, i), so the HIP
library (csrc/seeded.hip), the CPU checker and this module produce identical
numbers in any order.  The reference draws from an unseeded thread RNG
(utils/weights_initializer.rs:73-89); seeding is this project's addition.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
STREAM_PROMPT = 0x7F00000000
STREAM_NORMAL = 0x7E00000000


def mix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def draw(seed: int, stream: int, index: int) -> int:
    return mix64(mix64(mix64(seed) ^ stream) ^ index)


def _mix64_np(z: np.ndarray) -> np.ndarray:
    z = z + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def draw_np(seed: int, stream: int, index: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        key = np.uint64(mix64(mix64(seed) ^ stream))
        return _mix64_np(key ^ index.astype(np.uint64))


def prompts(seed: int, lens, vocab: int, max_len: int | None = None) -> np.ndarray:
    """ids[b][s] uniform in [0, vocab) for s < lens[b], PAD=1 after (embedding_layer.rs:112-155)."""
    lens = [int(x) for x in lens]
    S = int(max_len if max_len is not None else max(lens))
    ids = np.ones((len(lens), S), np.uint32)
    for b, n in enumerate(lens):
        h = draw_np(seed, STREAM_PROMPT + b, np.arange(n, dtype=np.uint64))
        hi = (h >> np.uint64(32)).astype(np.uint64)
        lo = (h & np.uint64(0xFFFFFFFF)).astype(np.uint64)
        # floor(h * vocab / 2^64) computed exactly in 64-bit pieces
        v = np.uint64(vocab)
        ids[b, :n] = ((hi * v + ((lo * v) >> np.uint64(32))) >> np.uint64(32)).astype(np.uint32)
    return ids


def normal(seed: int, shape) -> np.ndarray:
    """Box-Muller pairs: element p gets re, im from draws (2p, 2p+1)."""
    n = int(np.prod(shape))
    idx = np.arange(n, dtype=np.uint64)
    h1 = draw_np(seed, STREAM_NORMAL, 2 * idx)
    h2 = draw_np(seed, STREAM_NORMAL, 2 * idx + np.uint64(1))
    u1 = ((h1 >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0**-53
    u2 = (h2 >> np.uint64(11)).astype(np.float64) * 2.0**-53
    r = np.sqrt(-2.0 * np.log(u1))
    return (r * np.cos(2.0 * np.pi * u2) + 1j * r * np.sin(2.0 * np.pi * u2)).reshape(shape)
