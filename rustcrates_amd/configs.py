"""Model configurations of the benchmark suite and the layer stack they build.

The stack uses only the reference's own layer types, in LayerEnum order
(network_components/layer.rs:75-88), and is shared by the HIP network and the
CPU checker so both hold the same seeded weights:

    Embedding(V, d)
    repeat L times:
        Norm(d, eps=1e-5)              standalone pre-norm, no residual (transformer_network.rs:365-378)
        SelfAttention(h, d, max_ctx)   heads + residual + Norm(eps=1e-12) inside (self_attention_layer.rs:55-133)
        FeedForward(d, F)              Dense(GELU) -> Linear, no residual (feedforward_layer.rs:30-48)
    Linear(d, V)                       vocab projection (linear_layer.rs:55-75)
    Softmax(PRODUCTION)                forward_only => Re(logits) (transformer_network.rs:472-489)
"""
from __future__ import annotations

from dataclasses import dataclass, field

PRODUCTION = 1


@dataclass(frozen=True)
class ModelConfig:
    name: str
    layers: int
    d: int
    heads: int
    ffn: int
    vocab: int
    max_ctx: int = 512  # MAX_CONTEXT_WINDOW_SIZE (transformer_network.rs:32)
    seed: int = 0
    norm_eps: float = 1e-5
    attn_eps: float = 1e-12  # self_attention_layer.rs:38
    rope: bool = False  # PositionalEncoding after Embedding (off: not in the configs)
    rope_base: float = 1250.0  # positional_encoding_layer.rs:10

    @property
    def dh(self) -> int:
        return self.d // self.heads

    def weight_elems(self) -> int:
        """complex weights read once per decode step (Q/K/V, FFN, vocab)."""
        per_layer = 3 * self.d * self.d + 2 * self.d * self.ffn
        return self.layers * per_layer + self.d * self.vocab


@dataclass(frozen=True)
class Workload:
    model: ModelConfig
    batch: int
    prompt_len: int
    n_new: int
    ragged: tuple = field(default=())  # (lo, hi) per-sequence prompt length range, right-padded
    prompt_seed: int = 0


C1 = ModelConfig("c1", layers=2, d=64, heads=4, ffn=256, vocab=4096, seed=0)
C2 = ModelConfig("c2", layers=1, d=512, heads=8, ffn=2048, vocab=32000, seed=1)
C3 = ModelConfig("c3", layers=6, d=512, heads=8, ffn=2048, vocab=32000, seed=2)
C4 = ModelConfig("c4", layers=12, d=768, heads=12, ffn=3072, vocab=32000, seed=3)
C5 = ModelConfig("c5", layers=12, d=768, heads=12, ffn=3072, vocab=32000, seed=3, max_ctx=2048)

MODELS = {m.name: m for m in (C1, C2, C3, C4, C5)}

WORKLOADS = {
    "c1": Workload(C1, batch=1, prompt_len=16, n_new=32),
    "c3b1": Workload(C3, batch=1, prompt_len=128, n_new=128),
    "c3b32": Workload(C3, batch=32, prompt_len=128, n_new=128),
    "c4": Workload(C4, batch=64, prompt_len=256, n_new=256, ragged=(64, 256)),
    "c5": Workload(C5, batch=4, prompt_len=1920, n_new=128),
}


def build_network(net, cfg: ModelConfig, seed: int | None = None, mode: int = PRODUCTION):
    """Appends cfg's layer stack to `net` (HIP Network or the CPU checker) and
    fills every tensor from the seeded counter generator; `mode` is the
    Softmax's (TRAINING for a network that backward differentiates)."""
    net.add_embedding(cfg.vocab, cfg.d)
    if cfg.rope:
        net.add_positional_encoding(cfg.d, cfg.rope_base)
    for _ in range(cfg.layers):
        net.add_norm(cfg.d, cfg.norm_eps)
        net.add_self_attention(cfg.heads, cfg.d, cfg.max_ctx, cfg.attn_eps)
        net.add_feed_forward(cfg.d, cfg.ffn)
    net.add_linear(cfg.d, cfg.vocab)
    net.add_softmax(mode)
    net.init_seeded(cfg.seed if seed is None else seed)
    return net


# create_transformer's default stack (network_types/transformer/transformer_builder.rs:10-72)
REFERENCE_VOCAB = 50280
REFERENCE_DIM = 16  # 512 / 2^DECOMPOSITION_LEVELS (wavelet_network.rs:13)
WAVELET_DB2, WAVELET_MODE_SYMMETRIC = 1, 2  # DiscreteWaveletLayer::new (wavelet_discrete_layer.rs:46-70)


REFERENCE_EMBEDDING_SRC = 512  # embedding_dim_original (transformer_builder.rs:23)


def build_reference_default(net, vocab: int = REFERENCE_VOCAB, seed: int = 0, max_ctx: int = 512,
                            mode: int = PRODUCTION, wavelet_embedding: bool = True):
    """The layer stack create_transformer builds, in its order, with seeded
    weights where the reference draws them unseeded:

        Embedding(V, 16) -> DiscreteWavelet(DB2, SYMMETRIC) -> Norm(16, 1e-8)
        -> PositionalEncoding(16) -> SelfAttention(2 heads) -> FeedForward(16, 512)
        -> SelfAttention(4 heads) -> FeedForward(16, 1024) -> Linear(16, V) -> Softmax

    The embedding table is EmbeddingLayer::new's (create_embedding of a
    512-value draw per token, embedding_layer.rs:40-77), or with
    wavelet_embedding=False Xavier-uniform like the other weights."""
    d = REFERENCE_DIM
    net.add_embedding(vocab, d)
    net.add_discrete_wavelet(d, WAVELET_DB2, WAVELET_MODE_SYMMETRIC)
    net.add_norm(d, 1e-8)
    net.add_positional_encoding(d, 1250.0)
    for i in range(2):
        net.add_self_attention(2 if i == 0 else 4, d, max_ctx, 1e-12)
        net.add_feed_forward(d, 512 if i == 0 else 1024)
    net.add_linear(d, vocab)
    net.add_softmax(mode)
    net.init_seeded(seed)
    if wavelet_embedding:
        net.init_embedding_wavelet(0, seed, REFERENCE_EMBEDDING_SRC)
    return net


def prompt_lengths(w: Workload):
    """Per-sequence prompt lengths: fixed, or uniform in [lo, hi] from the counter generator."""
    if not w.ragged:
        return [w.prompt_len] * w.batch
    lo, hi = w.ragged
    from .seeded import draw

    return [lo + draw(w.prompt_seed, 0x7D00000000, b) % (hi - lo + 1) for b in range(w.batch)]
