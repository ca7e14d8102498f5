"""mitok_greedy_decoding_noalloc against mitok_greedy_decoding, through the C
ABI: two calls in a row (the second smaller, so a stale tail of the first
call's staging would show), ties and NaN, and the size limit.

Bar: ids bit-exact (integer results)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import rustcrates_amd as ra

pytestmark = pytest.mark.gpu


def _call(net, name, logits):
    logits = np.ascontiguousarray(logits, dtype=np.float64)
    rows, V = logits.shape
    out = np.full(rows, 0xFFFFFFFF, np.uint32)
    rc = getattr(net._lib, name)(net._h, logits.ctypes.data_as(C.c_void_p), rows, V, out.ctypes.data_as(C.c_void_p))
    return rc, out


def test_noalloc_matches_allocating_entry_point_twice():
    rng = np.random.default_rng(7)
    with ra.Network(0) as net:
        for rows, V in ((32, 32000), (3, 5000)):  # the second call is smaller
            lg = rng.standard_normal((rows, V))
            lg[0, [11, 4000]] = lg[0].max() + 1.0  # a tie: the last index wins (sampling_methods.rs:5-18)
            rc_a, want = _call(net, "mitok_greedy_decoding", lg)
            rc_b, got = _call(net, "mitok_greedy_decoding_noalloc", lg)
            print(f"noalloc {rows}x{V}: rc {rc_a} {rc_b}, equal {np.array_equal(got, want)}", flush=True)
            assert rc_a == 0 and rc_b == 0
            assert np.array_equal(got, want)
            assert np.array_equal(got, lg.shape[1] - 1 - np.argmax(lg[:, ::-1], axis=1))
            assert got[0] == 4000


def test_noalloc_nan_and_size_limit():
    with ra.Network(0) as net:
        lg = np.zeros((2, 100))
        lg[1, 7] = np.nan
        rc, _ = _call(net, "mitok_greedy_decoding_noalloc", lg)
        assert rc == 4  # MITOK_ERR_NAN, as the allocating entry point
        rc, _ = _call(net, "mitok_greedy_decoding_noalloc", np.zeros((33, 32000)))
        assert rc == 1  # beyond the staging: MITOK_ERR_ARG, nothing launched
        assert b"no-allocation" in net._lib.mitok_last_error()
        rc, out = _call(net, "mitok_greedy_decoding_noalloc", np.eye(4))
        assert rc == 0 and out.tolist() == [0, 1, 2, 3]  # usable after both errors
