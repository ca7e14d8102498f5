"""Reference model import: the bincode `NeuralNetwork` file and the token embeddings.

The reference stores a trained transformer as `bincode::serialize(&NeuralNetwork)`
written verbatim to a file (save_to_sled / get_from_db,
network_types/neural_network_generic.rs:90-113; utils/file.rs:54-72), and each
token's embedding in a sled tree under the decimal id with a bincode
`Vec<Complex<f64>>` value (embedding_layer.rs:267-310; database/sled_db.rs:24-26).

bincode 1.3's `serialize`/`deserialize` use its legacy configuration: little
endian, fixed-width integers (usize as u64), sequence and string lengths as
u64, enum variant indices as u32, `Option` as a u8 tag, `bool` as a u8.
Complex<f64> (num-complex 0.4, feature "serde") serialises as the tuple
(re, im).  `#[serde(skip)]` fields are absent.  The reference's own
STORAGE/embedding/embedding_layer.json (EmbeddingLayer metadata, written by
EmbeddingLayer::serialize, embedding_layer.rs:271-287) decodes under these
rules as (50280, 16, 0.001, 0).

This module reads and writes that layout (`read_network`, `write_network`),
decodes embedding values (`decode_embedding`, `read_embedding_pairs`), and
builds the stack on a HIP `Network` (`to_device`).  The sled storage engine
itself is not reimplemented: its `db` log file is absent from the reference
snapshot and sled's on-disk format belongs to the storage engine, not to the
token loop.  Embeddings come in as the (key, value bytes) pairs a sled tree
iterates to, exported one after another as (u64 key length, key bytes, u64
value length, value bytes): a loop of four writes over `db.iter()` in Rust.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

# LayerEnum variant indices (network_components/layer.rs:75-88, declaration order)
EMBEDDING, POSITIONAL_ENCODING, DENSE, FEED_FORWARD, RMS_NORM, NORM, SELF_ATTENTION, LINEAR, MULTI_LINEAR, \
    DISCRETE_WAVELET, WAVELET, SOFTMAX = range(12)
VARIANTS = ["Embedding", "PositionalEncoding", "Dense", "FeedForward", "RMSNorm", "Norm", "SelfAttention", "Linear",
            "MultiLinear", "DiscreteWavelet", "Wavelet", "Softmax"]
# ActivationType (layer.rs:25-42) and LayerType (layer.rs:55-62) are unit enums
GELU = 8
ATTENTION_LAYER, DENSE_LAYER = 3, 4  # LayerType of the attention heads / the FFN's Dense (layer.rs:55-62)
TRAINING, PRODUCTION = 0, 1  # OperationMode (neural_network_generic.rs:17-20)

_C16 = np.dtype("<c16")


class FormatError(ValueError):
    pass


class _Reader:
    def __init__(self, data: bytes):
        self.b = memoryview(data)
        self.o = 0

    def take(self, n: int) -> memoryview:
        if self.o + n > len(self.b):
            raise FormatError(f"truncated: need {n} bytes at offset {self.o}, have {len(self.b) - self.o}")
        v = self.b[self.o:self.o + n]
        self.o += n
        return v

    def u8(self) -> int:
        return self.take(1)[0]

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def f64(self) -> float:
        return struct.unpack("<d", self.take(8))[0]

    def boolean(self) -> bool:
        v = self.u8()
        if v > 1:
            raise FormatError(f"bool byte {v} at offset {self.o - 1}")
        return bool(v)

    def option_tag(self) -> bool:
        v = self.u8()
        if v > 1:
            raise FormatError(f"Option tag {v} at offset {self.o - 1}")
        return bool(v)

    def vec_c(self) -> np.ndarray:
        """Vec<Complex<f64>>"""
        n = self.u64()
        return np.frombuffer(self.take(16 * n), _C16).copy()

    def vec_f64(self) -> np.ndarray:
        n = self.u64()
        return np.frombuffer(self.take(8 * n), "<f8").copy()

    def mat_c(self):
        """Vec<Vec<Complex<f64>>>: [rows][cols] when every row has one length
        (weights), else a list of rows."""
        rows = self.u64()
        if rows == 0:
            return np.zeros((0, 0), _C16)
        start = self.o
        cols = self.u64()
        self.o = start
        stride = 8 + 16 * cols
        if self.o + rows * stride <= len(self.b):
            blk = np.frombuffer(self.b[self.o:self.o + rows * stride], np.uint8).reshape(rows, stride)
            lens = blk[:, :8].copy().view("<u8").ravel()
            if np.all(lens == cols):
                self.o += rows * stride
                return blk[:, 8:].copy().view(_C16).reshape(rows, cols)
        return [self.vec_c() for _ in range(rows)]  # ragged rows


class _Writer:
    def __init__(self):
        self.parts: list[bytes] = []

    def u8(self, v):
        self.parts.append(struct.pack("<B", v))

    def u32(self, v):
        self.parts.append(struct.pack("<I", v))

    def u64(self, v):
        self.parts.append(struct.pack("<Q", v))

    def f64(self, v):
        self.parts.append(struct.pack("<d", v))

    def vec_c(self, a):
        a = np.ascontiguousarray(a, _C16).ravel()
        self.u64(a.size)
        self.parts.append(a.tobytes())

    def vec_f64(self, a):
        a = np.ascontiguousarray(a, "<f8").ravel()
        self.u64(a.size)
        self.parts.append(a.tobytes())

    def mat_c(self, m):
        if isinstance(m, list):  # ragged rows
            self.u64(len(m))
            for row in m:
                self.vec_c(row)
            return
        m = np.ascontiguousarray(m, _C16)
        rows = m.shape[0]
        self.u64(rows)
        if rows:
            cols = m.shape[1]
            blk = np.empty((rows, 8 + 16 * cols), np.uint8)
            blk[:, :8] = np.frombuffer(struct.pack("<Q", cols), np.uint8)
            blk[:, 8:] = m.view(np.uint8).reshape(rows, 16 * cols)
            self.parts.append(blk.tobytes())

    def bytes(self) -> bytes:
        return b"".join(self.parts)


@dataclass
class Layer:
    """One LayerEnum value: `kind` is its variant name; `f` holds the
    serialised fields under the reference's field names."""
    kind: str
    f: dict = field(default_factory=dict)


@dataclass
class Model:
    """NeuralNetwork (neural_network_generic.rs:23-31)."""
    layers: list
    learning_rate: float = 0.0
    number_of_input_neurons: int = 0
    number_of_output_neurons: int = 0
    number_of_hidden_layers: int = 0
    number_of_hidden_neurons: int = 0
    minibatch_size: int = 0


# ---- per-variant field layouts (serialised fields in declaration order) ----
def _read_head(r: _Reader) -> dict:
    # MaskedAttentionHead (masked_attention_head.rs:23-61)
    h = {"weights_q": r.mat_c(), "weights_k": r.mat_c(), "weights_v": r.mat_c(), "bias_pos": r.mat_c(),
         "bias_q": r.vec_c(), "bias_k": r.vec_c(), "bias_v": r.vec_c(), "layer_type": r.u32(),
         "learning_rate": r.f64(), "time_step": r.u64(), "m1": r.mat_c(), "v1": r.mat_c()}
    return h


def _write_head(w: _Writer, h: dict):
    for k in ("weights_q", "weights_k", "weights_v", "bias_pos"):
        w.mat_c(h[k])
    for k in ("bias_q", "bias_k", "bias_v"):
        w.vec_c(h[k])
    w.u32(h["layer_type"])
    w.f64(h["learning_rate"])
    w.u64(h["time_step"])
    w.mat_c(h["m1"])
    w.mat_c(h["v1"])


def _read_linear(r: _Reader) -> dict:
    # LinearLayer (linear_layer.rs:18-34)
    return {"weights": r.mat_c(), "bias": r.vec_c(), "learning_rate": r.f64(), "time_step": r.u64()}


def _write_linear(w: _Writer, f: dict):
    w.mat_c(f["weights"])
    w.vec_c(f["bias"])
    w.f64(f["learning_rate"])
    w.u64(f["time_step"])


def _read_layer(r: _Reader) -> Layer:
    v = r.u32()
    if v >= len(VARIANTS):
        raise FormatError(f"LayerEnum variant {v} at offset {r.o - 4}")
    kind = VARIANTS[v]
    if v == EMBEDDING:  # embedding_layer.rs:24-36
        f = {"vocab_size": r.u64(), "embedding_dim": r.u64(), "learning_rate": r.f64(), "time_step": r.u64()}
    elif v == POSITIONAL_ENCODING:  # positional_encoding_layer.rs:15-22
        f = {"embedding_dim": r.u64(), "base": r.f64()}
    elif v == DENSE:  # layer.rs:91-112
        f = {"weights": r.mat_c(), "bias": r.vec_c(), "activation_type": r.u32(), "layer_type": r.u32(),
             "learning_rate": r.f64(), "time_step": r.u64()}
    elif v == FEED_FORWARD:  # feedforward_layer.rs:14-26
        layers = [_read_layer(r) for _ in range(r.u64())]
        norm = _read_layer(r) if r.option_tag() else None
        f = {"layers": layers, "norm_layer": norm, "learning_rate": r.f64(), "time_step": r.u64()}
    elif v == RMS_NORM:  # add_rms_norm_layer.rs:13-25
        f = {"gamma": r.vec_c(), "epsilon": r.f64(), "learning_rate": r.f64(), "time_step": r.u64()}
    elif v == NORM:  # norm_layer.rs:17-42
        f = {"gamma": r.vec_c(), "beta": r.vec_c(), "epsilon": r.f64(), "learning_rate": r.f64(),
             "time_step": r.u64()}
    elif v == SELF_ATTENTION:  # self_attention_layer.rs:16-25
        heads = [_read_head(r) for _ in range(r.u64())]
        f = {"attention_heads": heads, "activated_output": r.mat_c()}
        f["norm_layer"] = _read_layer(r) if r.option_tag() else None
        f["time_step"] = r.u64()
    elif v == LINEAR:
        f = _read_linear(r)
    elif v == MULTI_LINEAR:  # multi_linear_layer.rs:12-22
        f = {"layers": [_read_linear(r) for _ in range(r.u64())], "learning_rate": r.f64(), "time_step": r.u64()}
    elif v == DISCRETE_WAVELET:  # wavelet_discrete_layer.rs:20-52
        f = {"time_step": r.u64(), "wavelet": r.u32(), "wavelet_mode": r.u32(), "is_full_mode": r.boolean()}
    elif v == WAVELET:  # wavelet_complex_layer.rs:15-27, CWTComplex (wavelet_transform/cwt_complex.rs:16-24)
        f = {"time_step": r.u64(), "scales": r.vec_f64(), "cw_type": r.u32(), "sampling_period": r.f64(),
             "m": r.f64(), "fb": r.f64(), "fc": r.f64(), "frequencies": r.vec_f64(), "is_full_mode": r.boolean()}
    else:  # SOFTMAX, softmax_output_layer.rs:15-27
        f = {"learning_rate": r.f64(), "operation_mode": r.u32()}
    return Layer(kind, f)


def _write_layer(w: _Writer, L: Layer):
    v = VARIANTS.index(L.kind)
    w.u32(v)
    f = L.f
    if v == EMBEDDING:
        w.u64(f["vocab_size"]), w.u64(f["embedding_dim"]), w.f64(f["learning_rate"]), w.u64(f["time_step"])
    elif v == POSITIONAL_ENCODING:
        w.u64(f["embedding_dim"]), w.f64(f["base"])
    elif v == DENSE:
        w.mat_c(f["weights"]), w.vec_c(f["bias"]), w.u32(f["activation_type"]), w.u32(f["layer_type"])
        w.f64(f["learning_rate"]), w.u64(f["time_step"])
    elif v == FEED_FORWARD:
        w.u64(len(f["layers"]))
        for s in f["layers"]:
            _write_layer(w, s)
        if f["norm_layer"] is None:
            w.u8(0)
        else:
            w.u8(1)
            _write_layer(w, f["norm_layer"])
        w.f64(f["learning_rate"]), w.u64(f["time_step"])
    elif v == RMS_NORM:
        w.vec_c(f["gamma"]), w.f64(f["epsilon"]), w.f64(f["learning_rate"]), w.u64(f["time_step"])
    elif v == NORM:
        w.vec_c(f["gamma"]), w.vec_c(f["beta"]), w.f64(f["epsilon"]), w.f64(f["learning_rate"])
        w.u64(f["time_step"])
    elif v == SELF_ATTENTION:
        w.u64(len(f["attention_heads"]))
        for h in f["attention_heads"]:
            _write_head(w, h)
        w.mat_c(f["activated_output"])
        if f["norm_layer"] is None:
            w.u8(0)
        else:
            w.u8(1)
            _write_layer(w, f["norm_layer"])
        w.u64(f["time_step"])
    elif v == LINEAR:
        _write_linear(w, f)
    elif v == MULTI_LINEAR:
        w.u64(len(f["layers"]))
        for s in f["layers"]:
            _write_linear(w, s)
        w.f64(f["learning_rate"]), w.u64(f["time_step"])
    elif v == DISCRETE_WAVELET:
        w.u64(f["time_step"]), w.u32(f["wavelet"]), w.u32(f["wavelet_mode"]), w.u8(int(f["is_full_mode"]))
    elif v == WAVELET:
        w.u64(f["time_step"]), w.vec_f64(f["scales"]), w.u32(f["cw_type"]), w.f64(f["sampling_period"])
        w.f64(f["m"]), w.f64(f["fb"]), w.f64(f["fc"]), w.vec_f64(f["frequencies"]), w.u8(int(f["is_full_mode"]))
    else:
        w.f64(f["learning_rate"]), w.u32(f["operation_mode"])


def read_network(data) -> Model:
    """Decodes bincode::serialize(&NeuralNetwork) (bytes or a file path)."""
    if isinstance(data, (str, os.PathLike)):
        with open(data, "rb") as fh:
            data = fh.read()
    r = _Reader(bytes(data))
    layers = [_read_layer(r) for _ in range(r.u64())]
    m = Model(layers, r.f64(), r.u64(), r.u64(), r.u64(), r.u64(), r.u64())
    if r.o != len(r.b):
        raise FormatError(f"{len(r.b) - r.o} trailing bytes after NeuralNetwork")
    return m


def write_network(m: Model) -> bytes:
    """bincode::serialize(&NeuralNetwork) of `m` (the bytes save_to_sled writes)."""
    w = _Writer()
    w.u64(len(m.layers))
    for L in m.layers:
        _write_layer(w, L)
    w.f64(m.learning_rate)
    for v in (m.number_of_input_neurons, m.number_of_output_neurons, m.number_of_hidden_layers,
              m.number_of_hidden_neurons, m.minibatch_size):
        w.u64(v)
    return w.bytes()


def read_embedding_layer_meta(data: bytes) -> dict:
    """EmbeddingLayer as EmbeddingLayer::serialize writes it (embedding_layer.rs:271-287)."""
    r = _Reader(bytes(data))
    f = {"vocab_size": r.u64(), "embedding_dim": r.u64(), "learning_rate": r.f64(), "time_step": r.u64()}
    if r.o != len(r.b):
        raise FormatError("trailing bytes after EmbeddingLayer")
    return f


def decode_embedding(value: bytes) -> np.ndarray:
    """One sled value: bincode Vec<Complex<f64>> (update_embedding, embedding_layer.rs:263-269)."""
    r = _Reader(bytes(value))
    v = r.vec_c()
    if r.o != len(r.b):
        raise FormatError("trailing bytes after an embedding value")
    return v


def encode_embedding(vec) -> bytes:
    w = _Writer()
    w.vec_c(vec)
    return w.bytes()


def read_embedding_pairs(data: bytes) -> dict:
    """Embedding pairs exported from the sled tree, one after another as
    (u64 key length, key bytes, u64 value length, value bytes), keys the
    decimal token ids (the export is bincode of Vec<(String, Vec<u8>)>
    without its outer length, so a stream can be appended to)."""
    r = _Reader(bytes(data))
    out = {}
    while r.o < len(r.b):
        key = bytes(r.take(r.u64())).decode("ascii")
        if not key.isdigit():
            raise FormatError(f"embedding key {key!r} is not a decimal token id")
        out[int(key)] = decode_embedding(bytes(r.take(r.u64())))
    return out


def write_embedding_pairs(table: dict) -> bytes:
    w = _Writer()
    for tid in sorted(table):
        k = str(int(tid)).encode()
        v = encode_embedding(table[tid])
        w.u64(len(k)), w.parts.append(k), w.u64(len(v)), w.parts.append(v)
    return w.bytes()


def embedding_table(pairs: dict, vocab: int, dim: int, missing: str = "error") -> np.ndarray:
    """[vocab][dim] table from decoded pairs.  Id 1 (PAD) is never looked up
    (embedding_layer.rs:183-184).  A missing id is an error (the reference
    panics when it meets one, :305); missing="zero" fills zeros instead."""
    t = np.zeros((vocab, dim), np.complex128)
    absent = []
    for tid in range(vocab):
        v = pairs.get(tid)
        if v is None:
            if tid != 1:
                absent.append(tid)
            continue
        if v.shape[0] != dim:
            raise FormatError(f"embedding of id {tid} has {v.shape[0]} values, layer dim {dim}")
        t[tid] = v
    if absent and missing == "error":
        raise FormatError(f"{len(absent)} token ids have no embedding (first {absent[:5]})")
    return t


def _norm_of(layer):
    if layer is None:
        return None
    if layer.kind != "Norm":
        raise NotImplementedError(f"{layer.kind} inside a block is not on the device path (NormalNormLayer only)")
    return layer.f


def to_device(model: Model, net, embeddings: dict | None = None, missing: str = "error"):
    """Appends `model`'s layers to `net` (rustcrates_amd.Network, or the CPU
    checker's Network with the same methods) in LayerEnum order, with every
    weight uploaded as stored.  Returns net."""
    width = 0  # features per row after the layers so far
    for L in model.layers:
        f = L.f
        if L.kind == "Embedding":
            V, d = f["vocab_size"], f["embedding_dim"]
            if embeddings is None:
                raise ValueError("the model has an Embedding layer: pass the embedding pairs")
            net.add_embedding(V, d, embedding_table(embeddings, V, d, missing))
            width = d
        elif L.kind == "DiscreteWavelet":
            net.add_discrete_wavelet(width, f["wavelet"], f["wavelet_mode"], f["is_full_mode"])
        elif L.kind == "PositionalEncoding":
            net.add_positional_encoding(f["embedding_dim"], f["base"])
        elif L.kind == "Norm":
            net.add_norm(f["gamma"].shape[0], f["epsilon"], f["gamma"], f["beta"])
        elif L.kind == "SelfAttention":
            heads = f["attention_heads"]
            H = len(heads)
            d, dh = heads[0]["weights_q"].shape
            mc = heads[0]["bias_pos"].shape[0]
            if heads[0]["bias_pos"].shape != (mc, mc):
                raise FormatError(f"bias_pos {heads[0]['bias_pos'].shape} is not square")
            norm = _norm_of(f["norm_layer"])
            if norm is None:
                raise NotImplementedError("SelfAttention without its NormalNormLayer is not on the device path")
            stack = lambda k: np.stack([h[k] for h in heads])  # noqa: E731  [heads][d][dh]
            net.add_self_attention(H, d, mc, norm["epsilon"], stack("weights_q"), stack("weights_k"),
                                   stack("weights_v"), stack("bias_pos"), norm["gamma"], norm["beta"])
        elif L.kind == "FeedForward":
            subs = f["layers"]
            if [s.kind for s in subs] != ["Dense", "Linear"] or subs[0].f["activation_type"] != GELU:
                raise NotImplementedError("FeedForward other than Dense(GELU) -> Linear is not on the device path")
            if f["norm_layer"] is not None:
                raise NotImplementedError("FeedForward with a norm layer is not on the device path "
                                          "(create_transformer leaves it None, feedforward_layer.rs:44)")
            w1, b1 = subs[0].f["weights"], subs[0].f["bias"]
            w2, b2 = subs[1].f["weights"], subs[1].f["bias"]
            net.add_feed_forward(w1.shape[0], w1.shape[1], w1, b1, w2, b2)
        elif L.kind == "Linear":
            w = f["weights"]
            net.add_linear(w.shape[0], w.shape[1], w, f["bias"])
            width = w.shape[1]
        elif L.kind == "Softmax":
            net.add_softmax(f["operation_mode"])
        else:
            raise NotImplementedError(f"{L.kind} is not on the device path of the token loop")
    return net


def from_tensors(cfg, tensors) -> Model:
    """The Model of configs.build_network's stack with the given tensors (the
    layout of conftest.seeded_tensors): the file create_transformer would have
    written for such a stack, for fixtures and round trips."""
    d, F, V, h, mc = cfg.d, cfg.ffn, cfg.vocab, cfg.heads, cfg.max_ctx
    dh = d // h
    z = lambda *s: np.zeros(s, np.complex128)  # noqa: E731
    layers = [Layer("Embedding", {"vocab_size": V, "embedding_dim": d, "learning_rate": 0.001, "time_step": 0})]
    k = 1
    for _ in range(cfg.layers):
        n = tensors[k]
        layers.append(Layer("Norm", {"gamma": n["gamma"], "beta": n["beta"], "epsilon": cfg.norm_eps,
                                     "learning_rate": 0.001, "time_step": 0}))
        a = tensors[k + 1]
        wq, wk, wv = (np.asarray(a[x]).reshape(h, d, dh) for x in ("wq", "wk", "wv"))
        bp = np.asarray(a["bias_pos"]).reshape(h, mc, mc)
        heads = [{"weights_q": wq[i], "weights_k": wk[i], "weights_v": wv[i], "bias_pos": bp[i],
                  "bias_q": z(dh), "bias_k": z(dh), "bias_v": z(dh), "layer_type": ATTENTION_LAYER, "learning_rate": 0.001,
                  "time_step": 0, "m1": z(0, 0), "v1": z(0, 0)} for i in range(h)]
        norm = Layer("Norm", {"gamma": a["gamma"], "beta": a["beta"], "epsilon": cfg.attn_eps, "learning_rate": 0.001,
                              "time_step": 0})
        layers.append(Layer("SelfAttention", {"attention_heads": heads, "activated_output": z(0, 0),
                                              "norm_layer": norm, "time_step": 0}))
        f = tensors[k + 2]
        dense = Layer("Dense", {"weights": np.asarray(f["w1"]).reshape(d, F), "bias": f["b1"], "activation_type": GELU,
                                "layer_type": DENSE_LAYER, "learning_rate": 0.001, "time_step": 0})
        lin = Layer("Linear", {"weights": np.asarray(f["w2"]).reshape(F, d), "bias": f["b2"], "learning_rate": 0.001,
                               "time_step": 0})
        layers.append(Layer("FeedForward", {"layers": [dense, lin], "norm_layer": None, "learning_rate": 0.001,
                                            "time_step": 0}))
        k += 3
    layers.append(Layer("Linear", {"weights": np.asarray(tensors[k]["w"]).reshape(d, V), "bias": tensors[k]["b"],
                                   "learning_rate": 0.001, "time_step": 0}))
    layers.append(Layer("Softmax", {"learning_rate": 0.001, "operation_mode": PRODUCTION}))
    return Model(layers, 0.001, V, V, cfg.layers, F, 1)
