"""rustcrates_amd — MI355X token loop for the rustCrates complex-valued transformer.

Python handle over libmitok.so (include/mitok.h).  The methods mirror the
reference's model API (src/neural_networks/...):

    Network.add_embedding / add_norm / add_self_attention / ...   LayerEnum variants (layer.rs:75-88)
    Network.predict                                               predict (transformer_network.rs:315-504)
    Network.forward_layers                                        Layer::forward chains
    Network.generate                                              predict_token_by_token on ids (:165-313)

All compute runs in the HIP library; importing this package never falls back
to a CPU path: if libmitok.so is missing or no GPU is present, the calls raise.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import weakref

import numpy as np

from . import configs, seeded  # noqa: F401

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmitok.so")

TRAINING, PRODUCTION = 0, 1
TIME_VOCAB, TIME_LAYER_GEMM, TIME_ATTENTION, TIME_STEP, TIME_PREFILL_GEMM = 1, 2, 3, 4, 5

ERRORS = {1: "ERR_ARG", 2: "ERR_HIP", 3: "ERR_STATE", 4: "ERR_NAN", 5: "ERR_NOMEM"}

# every entry point declared in include/mitok.h: name -> (restype, argtypes)
_P = C.c_void_p
_u32, _u64, _i32, _f64 = C.c_uint32, C.c_uint64, C.c_int, C.c_double
SIGNATURES = {
    "mitok_version": (_i32, []),
    "mitok_last_error": (C.c_char_p, []),
    "mitok_device_count": (_i32, [_P]),
    "mitok_network_create": (_i32, [_i32, _P]),
    "mitok_network_destroy": (None, [_P]),
    "mitok_num_layers": (_i32, [_P]),
    "mitok_add_embedding": (_i32, [_P, _u32, _u32, _P]),
    "mitok_add_positional_encoding": (_i32, [_P, _u32, _f64]),
    "mitok_add_norm": (_i32, [_P, _u32, _f64, _P, _P]),
    "mitok_add_self_attention": (_i32, [_P, _u32, _u32, _u32, _f64, _P, _P, _P, _P, _P, _P]),
    "mitok_add_feed_forward": (_i32, [_P, _u32, _u32, _P, _P, _P, _P]),
    "mitok_add_linear": (_i32, [_P, _u32, _u32, _P, _P]),
    "mitok_add_softmax": (_i32, [_P, _i32]),
    "mitok_add_discrete_wavelet": (_i32, [_P, _u32, _u32, _u32, _i32]),
    "mitok_seq_out_len": (_i32, [_P, _u32, _u32, _u32, _P]),
    "mitok_init_seeded": (_i32, [_P, _u64]),
    "mitok_init_embedding_wavelet": (_i32, [_P, _u32, _u64, _u32]),
    "mitok_get_tensor": (_i32, [_P, _u32, _u32, _P, _u64]),
    "mitok_reset": (_i32, [_P]),
    "mitok_predict": (_i32, [_P, _P, _P, _u32, _u32, _P, _i32, _i32, _P, _P]),
    "mitok_predict_targets": (_i32, [_P, _P, _P, _u32, _u32, _u32, _P, _P]),
    "mitok_cross_entropy_loss": (_i32, [_P, _P, _P, _u32, _u32, _P]),
    "mitok_forward_layers": (_i32, [_P, _u32, _u32, _P, _P, _u32, _u32, _P, _i32, _P]),
    "mitok_generate": (_i32, [_P, _P, _P, _u32, _u32, _u32, _P, _P]),
    "mitok_prefill": (_i32, [_P, _P, _P, _u32, _u32, _P, _P]),
    "mitok_decode_step": (_i32, [_P, _P, _u32, _P, _P]),
    "mitok_greedy_decoding": (_i32, [_P, _P, _u32, _u32, _P]),
    "mitok_backward_head": (_i32, [_P, _P, _P, _u32, _u32, _i32, C.c_double, _u32, _P]),
    "mitok_backward": (_i32, [_P, _P, _P, _u32, _u32, _u32, _i32, C.c_double, _u32, _P]),
    "mitok_backward_walk": (_i32, [_P, _P, _P, _u32, _u32, _i32, _u32, _P]),
    "mitok_set_learning_rate": (_i32, [_P, _u32, C.c_double]),
    "mitok_get_learning_rate": (_i32, [_P, _u32, _P]),
    "mitok_set_network_learning_rate": (_i32, [_P, C.c_double]),
    "mitok_reset_previous_gradient": (_i32, [_P]),
    "mitok_greedy_decoding_device": (_i32, [_P, _P, _u32, _u32, _P]),
    "mitok_forward_layers_device": (_i32, [_P, _u32, _u32, _P, _P, _u32, _u32, _P, _i32, _P]),
    "mitok_greedy_decoding_noalloc": (_i32, [_P, _P, _u32, _u32, _P]),
    "mitok_last_timings": (_i32, [_P, _P]),
    "mitok_timing_enable": (_i32, [_P, _i32]),
    "mitok_timing_read": (_i32, [_P, _P, _P, _P, _P]),
    "mitok_device_synchronize": (_i32, [_i32]),
    "mitok_set_graph_mode": (_i32, [_P, _i32]),
    "mitok_set_decode_plan": (_i32, [_P, _i32]),
    "mitok_resident_exchange": (_i32, [_P, _i32, C.POINTER(_i32)]),
    "mitok_resident_profile": (_i32, [_P, _i32, _i32, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(C.c_double)]),
}


class MitokError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def load_library():
    """Loads libmitok.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m rustcrates_amd.build` first")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(rc: int):
    if rc != 0:
        raise MitokError(rc, load_library().mitok_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _dev(p):
    return C.c_void_p(p.ptr if isinstance(p, DeviceBuffer) else int(p))


class DeviceBuffer:
    """Device memory for the *_device entry points, from the HIP runtime the
    library links (hipMalloc / hipMemcpy / hipFree).  torch in this image
    bundles a HIP runtime of its own, and one process holds the GPU through one
    runtime, so a process using the library takes its device memory here."""

    def __init__(self, nbytes: int, device: int = 0):
        load_library()
        self._hip = C.CDLL("libamdhip64.so.7")  # the copy the library loaded
        self.nbytes, self.device = int(nbytes), device
        self._p = C.c_void_p()
        if self._hip.hipSetDevice(device) != 0 or self._hip.hipMalloc(C.byref(self._p), C.c_size_t(self.nbytes)) != 0:
            raise MitokError(2, f"hipMalloc of {self.nbytes} bytes on device {device} failed")

    @property
    def ptr(self) -> int:
        return self._p.value

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError(f"{a.nbytes} bytes do not fit a {self.nbytes}-byte buffer")
        if self._hip.hipMemcpy(self._p, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) != 0:  # H2D
            raise MitokError(2, "hipMemcpy to the device failed")

    def download(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise ValueError(f"{out.nbytes} bytes exceed a {self.nbytes}-byte buffer")
        if self._hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), self._p, C.c_size_t(out.nbytes), 2) != 0:  # D2H
            raise MitokError(2, "hipMemcpy from the device failed")
        return out

    def free(self):
        if self._p.value:
            self._hip.hipFree(self._p)
            self._p = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


def _c128(a, n=None, what="tensor"):
    """A contiguous complex128 copy of `a` (None stays None); with n, its size
    must be n elements, so the library never reads past a short host buffer."""
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.complex128)
    if n is not None and a.size != n:
        raise ValueError(f"{what}: {a.size} elements, expected {n}")
    return a


def _u32_vec(a, n, what):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    if a.shape != (n,):
        raise ValueError(f"{what}: shape {a.shape}, expected ({n},)")
    return a


# every open network, closed at interpreter exit before the HIP runtime's own
# teardown (atexit handlers run before module globals are cleared)
_live = weakref.WeakSet()


@atexit.register
def _close_all():
    for net in list(_live):
        try:
            net.close()
        except Exception:
            pass


def device_synchronize(device: int = 0) -> None:
    """hipDeviceSynchronize on `device`."""
    _check(load_library().mitok_device_synchronize(device))


def device_count() -> int:
    n = C.c_int(0)
    _check(load_library().mitok_device_count(C.byref(n)))
    return n.value


class Network:
    """NeuralNetwork on one GPU (neural_network_generic.rs:23-31).

    Release it with close() or a `with` block; networks still open at exit are
    closed by an atexit hook, while the HIP runtime is still up."""

    def __init__(self, device: int = 0):
        lib = load_library()
        h = C.c_void_p()
        _check(lib.mitok_network_create(device, C.byref(h)))
        self._h = h
        self._lib = lib
        self.vocab = None
        self.dim = None
        self._in_dims = []  # each layer's input width, for the gradient backward returns
        self._wavelet_filters = []  # filter length of each DiscreteWavelet layer, in order
        self._kinds = []  # each layer's kind
        _live.add(self)

    def close(self):
        if getattr(self, "_h", None):
            self._lib.mitok_network_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_layers(self) -> int:
        return self._lib.mitok_num_layers(self._h)

    # ---- LayerEnum variants ----
    def add_embedding(self, vocab, dim, table=None):
        self.dim = dim
        self._in_dims.append(dim)
        self._kinds.append("embedding")
        _check(self._lib.mitok_add_embedding(self._h, vocab, dim, _ptr(_c128(table, vocab * dim, "table"))))

    def add_positional_encoding(self, dim, base=1250.0):
        self._in_dims.append(dim)
        self._kinds.append("posenc")
        _check(self._lib.mitok_add_positional_encoding(self._h, dim, base))

    def add_norm(self, dim, eps, gamma=None, beta=None):
        self._in_dims.append(dim)
        self._kinds.append("norm")
        _check(self._lib.mitok_add_norm(self._h, dim, eps, _ptr(_c128(gamma, dim, "gamma")),
                                        _ptr(_c128(beta, dim, "beta"))))

    def add_self_attention(self, heads, dim, max_ctx, eps=1e-12, wq=None, wk=None, wv=None, bias_pos=None,
                           gamma=None, beta=None):
        nw = dim * dim  # [heads][dim][dim / heads]
        self._in_dims.append(dim)
        self._kinds.append("attention")
        _check(self._lib.mitok_add_self_attention(self._h, heads, dim, max_ctx, eps, _ptr(_c128(wq, nw, "wq")),
                                                  _ptr(_c128(wk, nw, "wk")), _ptr(_c128(wv, nw, "wv")),
                                                  _ptr(_c128(bias_pos, heads * max_ctx * max_ctx, "bias_pos")),
                                                  _ptr(_c128(gamma, dim, "gamma")), _ptr(_c128(beta, dim, "beta"))))

    def add_feed_forward(self, dim, hidden, w1=None, b1=None, w2=None, b2=None):
        self._in_dims.append(dim)
        self._kinds.append("ffn")
        _check(self._lib.mitok_add_feed_forward(self._h, dim, hidden, _ptr(_c128(w1, dim * hidden, "w1")),
                                                _ptr(_c128(b1, hidden, "b1")), _ptr(_c128(w2, hidden * dim, "w2")),
                                                _ptr(_c128(b2, dim, "b2"))))

    def add_linear(self, d_in, d_out, w=None, b=None):
        self.vocab = d_out
        self._head_in = d_in
        self._in_dims.append(d_in)
        self._kinds.append("linear")
        _check(self._lib.mitok_add_linear(self._h, d_in, d_out, _ptr(_c128(w, d_in * d_out, "w")),
                                          _ptr(_c128(b, d_out, "b"))))

    def add_softmax(self, mode=PRODUCTION):
        self._in_dims.append(getattr(self, "vocab", 0))
        self._kinds.append("softmax")
        _check(self._lib.mitok_add_softmax(self._h, mode))

    def add_discrete_wavelet(self, dim, wavelet=1, mode=2, is_full_mode=False):
        """DiscreteWaveletLayer over rows of `dim` features; defaults DB2 /
        SYMMETRIC (wavelet_discrete_layer.rs:46-70)."""
        self._in_dims.append(dim)
        self._kinds.append("wavelet")
        self._wavelet_filters.append(2 if wavelet == 0 else 4)
        _check(self._lib.mitok_add_discrete_wavelet(self._h, dim, wavelet, mode, int(is_full_mode)))

    def seq_out_len(self, S, first=0, last=None):
        """Rows per sequence that layers [first, last) leave of a prompt pass of S rows."""
        out = C.c_uint32(0)
        _check(self._lib.mitok_seq_out_len(self._h, first, self.num_layers if last is None else last, S,
                                           C.byref(out)))
        return out.value

    def init_seeded(self, seed):
        _check(self._lib.mitok_init_seeded(self._h, seed))

    def init_embedding_wavelet(self, layer=0, seed=0, src_dim=512):
        """EmbeddingLayer::new's create_embedding for every token id
        (embedding_layer.rs:40-77): a seeded uniform draw of src_dim values in
        [-0.4, 0.5) decomposed by decompose_in_wavelet_2d_default."""
        _check(self._lib.mitok_init_embedding_wavelet(self._h, int(layer), int(seed), int(src_dim)))

    def get_tensor(self, layer, slot, n):
        if slot == 3:
            out = np.empty(n, np.float64)
        else:
            out = np.empty(n, np.complex128)
        _check(self._lib.mitok_get_tensor(self._h, layer, slot, _ptr(out), n))
        return out

    def reset(self):
        _check(self._lib.mitok_reset(self._h))

    # ---- forward paths ----
    def predict(self, ids, lens=None, time_steps=None, forward_only=True, last_row_only=False, target_rows=0,
                want_output=True):
        """predict (transformer_network.rs:315-492).  target_rows (a stateless
        pass, forward_only=False): the last T rows of every sequence are the
        targets, which a DiscreteWavelet layer passes on uncompressed
        (wavelet_discrete_layer.rs:102-134; mitok_predict_targets).
        want_output=False (a stateless pass of all rows): the softmax output
        stays on the device for cross_entropy_loss and backward, and the
        first value returned is None."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        B, S = ids.shape
        lens = np.full(B, S, np.uint32) if lens is None else _u32_vec(lens, B, "lens")
        ts = None if time_steps is None else _u32_vec(time_steps, B, "time_steps")
        V = self.vocab
        prompt_pass = not forward_only or ts is None or ts[0] == 0
        T = int(target_rows)
        if T and (forward_only or last_row_only or time_steps is not None):
            raise ValueError("target_rows applies to a stateless pass of all rows only")
        if not want_output and (forward_only or last_row_only or time_steps is not None):
            raise ValueError("want_output=False applies to a stateless pass of all rows only")
        if T:
            So = S
            for w in self._wavelet_filters:
                So = (So - T + w - 2 + ((So - T) % 2)) // 2 + T
        else:
            So = self.seq_out_len(S) if prompt_pass else S
        out = np.empty((B, V) if last_row_only else (B, So, V), np.float64) if want_output else None
        mask = np.empty((B, So), np.uint32)
        self._head_rows = None
        if T or not want_output:
            _check(self._lib.mitok_predict_targets(self._h, _ptr(ids), _ptr(lens), B, S, T, _ptr(out), _ptr(mask)))
        else:
            _check(self._lib.mitok_predict(self._h, _ptr(ids), _ptr(lens), B, S, _ptr(ts), int(forward_only),
                                           int(last_row_only), _ptr(out), _ptr(mask)))
        if not forward_only:
            # what backward differentiates: rows at the head and, below the
            # first wavelet layer, the uncompressed S rows
            first_w = self._kinds.index("wavelet") if "wavelet" in self._kinds else -1
            self._head_rows = (B, So, S if first_w >= 0 else None, first_w)
        return out, mask

    def forward_layers(self, first, last, x, mask=None, time_steps=None, forward_only=True, d_out=None):
        x = _c128(x)
        if x.ndim != 3:
            raise ValueError(f"hidden states: shape {x.shape}, expected (batch, seq, dim)")
        B, S, _ = x.shape
        m = None
        if mask is not None:
            m = np.ascontiguousarray(mask, dtype=np.uint32)
            if m.shape != (B, S):
                raise ValueError(f"padding mask: shape {m.shape}, expected ({B}, {S})")
        ts = None if time_steps is None else _u32_vec(time_steps, B, "time_steps")
        prompt_pass = not forward_only or ts is None or ts[0] == 0
        So = self.seq_out_len(S, first, last) if prompt_pass else S
        out = np.empty((B, So, d_out if d_out else x.shape[2]), np.complex128)
        _check(self._lib.mitok_forward_layers(self._h, first, last, _ptr(x), _ptr(m), B, S, _ptr(ts),
                                              int(forward_only), _ptr(out)))
        return out

    def forward_layers_device(self, first, last, d_in, B, S, d_out, mask=None, time_steps=None, forward_only=True):
        """forward_layers on device memory: `d_in` holds [B][S][d_in] complex,
        `d_out` receives [B][S'][d_out] (DeviceBuffer or a device address).
        The mask and time steps stay host arrays.  Returns S'."""
        m = None
        if mask is not None:
            m = np.ascontiguousarray(mask, dtype=np.uint32)
            if m.shape != (B, S):
                raise ValueError(f"padding mask: shape {m.shape}, expected ({B}, {S})")
        ts = None if time_steps is None else _u32_vec(time_steps, B, "time_steps")
        prompt_pass = not forward_only or ts is None or ts[0] == 0
        _check(self._lib.mitok_forward_layers_device(self._h, first, last, _dev(d_in), _ptr(m), B, S, _ptr(ts),
                                                     int(forward_only), _dev(d_out)))
        return self.seq_out_len(S, first, last) if prompt_pass else S

    def greedy_decoding_device(self, d_logits, rows, vocab, d_ids):
        """greedy_decoding of [rows][vocab] f64 logits in device memory into
        [rows] u32 ids in device memory."""
        _check(self._lib.mitok_greedy_decoding_device(self._h, _dev(d_logits), rows, vocab, _dev(d_ids)))

    def generate(self, prompt, lens=None, n_new=1, want_logits=False):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        B, S = prompt.shape
        lens = np.full(B, S, np.uint32) if lens is None else _u32_vec(lens, B, "lens")
        ids = np.empty((B, n_new), np.uint32)
        logits = np.empty((n_new, B, self.vocab), np.float64) if want_logits else None
        _check(self._lib.mitok_generate(self._h, _ptr(prompt), _ptr(lens), B, S, n_new, _ptr(ids), _ptr(logits)))
        return (ids, logits) if want_logits else ids

    def prefill(self, prompt, lens=None, want_logits=False):
        """The prompt pass of the token loop: returns each sequence's first
        greedy id [B] (and its Re-logits row [B][V])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        B, S = prompt.shape
        lens = np.full(B, S, np.uint32) if lens is None else _u32_vec(lens, B, "lens")
        ids = np.empty(B, np.uint32)
        logits = np.empty((B, self.vocab), np.float64) if want_logits else None
        _check(self._lib.mitok_prefill(self._h, _ptr(prompt), _ptr(lens), B, S, _ptr(ids), _ptr(logits)))
        self._batch = B
        return (ids, logits) if want_logits else ids

    def decode_step(self, ids=None, want_logits=False, batch=None):
        """One decode step: feeds `ids` [B] (None: the ids the previous call
        returned, still on the device) and returns the next greedy ids [B]."""
        B = batch if batch is not None else (len(ids) if ids is not None else getattr(self, "_batch", 0))
        fed = None if ids is None else _u32_vec(ids, B, "ids")
        out = np.empty(B, np.uint32)
        logits = np.empty((B, self.vocab), np.float64) if want_logits else None
        _check(self._lib.mitok_decode_step(self._h, _ptr(fed), B, _ptr(out), _ptr(logits)))
        return (out, logits) if want_logits else out

    def backward_head(self, targets, tlens=None, update=True, learning_rate=0.001, time_step=1, want_grad_input=True):
        """backward through the Softmax and the vocab Linear of the last
        stateless predict (transformer_network.rs:506-636 for those two
        layers); with `update`, the Linear's update_parameters.  Returns the
        gradient with respect to the Linear's input [B][S'][d_in] (complex)."""
        return self.backward(targets, tlens, 1, update, learning_rate, time_step, want_grad_input)

    def backward(self, targets, tlens=None, layers=1, update=True, learning_rate=0.001, time_step=1,
                 want_grad_input=True):
        """The reverse walk of backward (transformer_network.rs:506-636)
        through `layers` layers below the Softmax (1: the vocab Linear only; up
        to every layer of the last stateless predict, the Embedding's update
        included).  Returns the gradient of the lowest differentiated layer's
        input [B][S'][d] (complex)."""
        t = np.ascontiguousarray(targets, dtype=np.uint32)
        if t.ndim != 2:
            raise ValueError(f"targets: shape {t.shape}, expected (batch, T)")
        B, T = t.shape
        tl = np.full(B, T, np.uint32) if tlens is None else _u32_vec(tlens, B, "tlens")
        gx = self._grad_input_buffer(B, int(layers)) if want_grad_input else None
        _check(self._lib.mitok_backward(self._h, _ptr(t), _ptr(tl), B, T, int(layers), int(bool(update)),
                                        float(learning_rate), int(time_step), _ptr(gx)))
        return gx

    def _grad_input_buffer(self, B, layers):
        """[B][rows][d_in] for the input gradient of the lowest of `layers`
        walked layers (below the first wavelet layer: the uncompressed rows)."""
        rows = getattr(self, "_head_rows", None)
        if rows is None or rows[0] != B:
            raise MitokError(3, "no stateless predict of this batch to differentiate")
        lowest = len(self._in_dims) - 1 - layers
        width = self._in_dims[lowest] if 0 <= lowest < len(self._in_dims) else self._head_in
        n_rows = rows[2] if rows[2] is not None and lowest <= rows[3] else rows[1]
        return np.empty((B, n_rows, width), np.complex128)

    def backward_walk(self, targets, tlens=None, update=True, time_step=1, want_grad_input=False):
        """backward(transformer_network, target_ids, update) as train calls it
        (transformer_network.rs:506-636): every layer of the last stateless
        predict, each updated at its own learning rate (set_learning_rate) and
        the Embedding at the network's (set_network_learning_rate)."""
        t = np.ascontiguousarray(targets, dtype=np.uint32)
        if t.ndim != 2:
            raise ValueError(f"targets: shape {t.shape}, expected (batch, T)")
        B, T = t.shape
        tl = np.full(B, T, np.uint32) if tlens is None else _u32_vec(tlens, B, "tlens")
        gx = self._grad_input_buffer(B, self.num_layers - 1) if want_grad_input else None
        _check(self._lib.mitok_backward_walk(self._h, _ptr(t), _ptr(tl), B, T, int(bool(update)), int(time_step),
                                             _ptr(gx)))
        return gx

    ALL_LAYERS = 0xFFFFFFFF
    NETWORK_RATE = 0xFFFFFFFF

    def set_learning_rate(self, learning_rate, layer=None):
        """update_learning_rate (neural_network_generic.rs:115-186) for every
        layer, or one layer's learning_rate field when `layer` is given."""
        _check(self._lib.mitok_set_learning_rate(self._h, self.ALL_LAYERS if layer is None else int(layer),
                                                 float(learning_rate)))

    def learning_rate(self, layer=None):
        """A layer's learning rate, or the network's (layer None)."""
        out = C.c_double()
        _check(self._lib.mitok_get_learning_rate(self._h, self.NETWORK_RATE if layer is None else int(layer),
                                                 C.byref(out)))
        return out.value

    def set_network_learning_rate(self, learning_rate):
        """NeuralNetwork::learning_rate: the Embedding's update rate, halved by
        decay_learning_rate (neural_network_generic.rs:69-73)."""
        _check(self._lib.mitok_set_network_learning_rate(self._h, float(learning_rate)))

    def reset_previous_gradient(self):
        """reset_previous_gradient (neural_network_generic.rs:188-242): the
        next update of every Linear, FeedForward sublayer and attention head
        is the clipped descent; attention Norms keep their moments."""
        _check(self._lib.mitok_reset_previous_gradient(self._h))

    def cross_entropy_loss(self, targets, tlens=None):
        """cross_entropy_loss_batch (transformer_network.rs:662-711) of the
        softmax output the last stateless predict left on the device
        (mitok_cross_entropy_loss); targets as backward takes them."""
        t = np.ascontiguousarray(targets, dtype=np.uint32)
        if t.ndim != 2:
            raise ValueError(f"targets: shape {t.shape}, expected (batch, T)")
        B, T = t.shape
        tl = np.full(B, T, np.uint32) if tlens is None else _u32_vec(tlens, B, "tlens")
        out = np.empty(2, np.float64)
        _check(self._lib.mitok_cross_entropy_loss(self._h, _ptr(t), _ptr(tl), B, T, _ptr(out)))
        return complex(out[0], out[1])

    def greedy_decoding(self, logits):
        logits = np.ascontiguousarray(logits, dtype=np.float64)
        if logits.ndim != 2:
            raise ValueError(f"logits: shape {logits.shape}, expected (rows, vocab)")
        rows, V = logits.shape
        out = np.empty(rows, np.uint32)
        _check(self._lib.mitok_greedy_decoding(self._h, _ptr(logits), rows, V, _ptr(out)))
        return out

    # ---- measurement ----
    def last_timings(self):
        t = np.zeros(3, np.float64)
        _check(self._lib.mitok_last_timings(self._h, _ptr(t)))
        plan = {0.0: "direct", 1.0: "graph", 2.0: "resident"}.get(float(t[2]), "direct")
        return {"prefill_ms": float(t[0]), "decode_ms": float(t[1]), "graph": plan == "graph", "decode_loop": plan}

    def timing_enable(self, kernel_class: int):
        _check(self._lib.mitok_timing_enable(self._h, kernel_class))

    def timing_read(self):
        ms, n, b, f = C.c_double(), C.c_uint64(), C.c_double(), C.c_double()
        _check(self._lib.mitok_timing_read(self._h, C.byref(ms), C.byref(n), C.byref(b), C.byref(f)))
        return {"total_ms": ms.value, "launches": n.value, "alg_bytes": b.value, "alg_flops": f.value}

    def set_graph_mode(self, direct_launch: bool):
        _check(self._lib.mitok_set_graph_mode(self._h, int(direct_launch)))

    def resident_profile(self, enable: bool = True):
        """Enables per-operation timing of the resident decode loop and returns
        the last launch's [(kind, microseconds per step)]."""
        mx = 512
        n = _i32()
        kinds = (_i32 * mx)()
        us = (C.c_double * mx)()
        _check(self._lib.mitok_resident_profile(self._h, int(enable), mx, C.byref(n), kinds, us))
        names = {0: "gemv", 1: "attn", 2: "rows"}
        return [(names.get(kinds[i], "?"), us[i]) for i in range(n.value)]

    def resident_exchange(self, mode: int = -1) -> bool:
        """mode 1: the resident loop's blocks exchange values by polling them
        (one grid barrier per step) where the program allows it (no RoPE);
        0: a grid barrier after every operation; -1: unchanged.  Returns
        whether the last resident launch polled."""
        polled = _i32()
        _check(self._lib.mitok_resident_exchange(self._h, int(mode), C.byref(polled)))
        return bool(polled.value)

    def set_decode_plan(self, plan: int):
        """3: generate's decode loop for up to 8 sequences as one resident
        launch; 2: resident for 1 and 2 sequences (1 without the polling
        exchange), fused above (default); 1 (True):
        fused launches, replayed as a graph; 0 (False): one launch per
        reference operation."""
        _check(self._lib.mitok_set_decode_plan(self._h, int(plan)))
