"""The per-layer drop-in on device buffers: mitok_forward_layers_device and
mitok_greedy_decoding_device take hidden states, logits and ids that stay on
the GPU.  Each must equal its host-buffer twin bit for bit (same kernels), and
a pointer that is not device memory of the network's GPU, or an allocation too
small for the shape, must be refused before any kernel runs.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import rustcrates_amd as ra
from rustcrates_amd import configs

pytestmark = pytest.mark.gpu

ERR_ARG = 1


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


C2S = configs.ModelConfig("c2s", layers=1, d=64, heads=4, ffn=128, vocab=300, max_ctx=48, seed=5)


def test_forward_layers_on_device_buffers_equal_host_buffers():
    g = configs.build_network(ra.Network(0), C2S)
    first, last = 1, g.num_layers - 2  # every hidden-state layer: no Embedding, no vocab Linear + Softmax
    rng = np.random.default_rng(8)
    B, S, d = 3, 20, C2S.d
    x = rng.standard_normal((B, S, d)) + 1j * rng.standard_normal((B, S, d))
    mask = np.ones((B, S), np.uint32)
    mask[1, 14:] = 0
    mask[2, 7:] = 0
    with ra.DeviceBuffer(x.nbytes) as din, ra.DeviceBuffer(x.nbytes) as dout:
        din.upload(x)
        for fwd in (False, True):
            g.reset()
            host = g.forward_layers(first, last, x, mask=mask, forward_only=fwd)
            g.reset()
            so = g.forward_layers_device(first, last, din, B, S, dout, mask=mask, forward_only=fwd)
            got = dout.download((B, so, d), np.complex128)
            log(f"forward_layers_device forward_only={fwd}: rows {so}, equal {np.array_equal(got, host)}")
            assert got.shape == host.shape and np.array_equal(got, host)
    g.close()


def test_greedy_decoding_on_device_buffers_equals_host_buffers():
    g = ra.Network(0)
    rng = np.random.default_rng(9)
    lg = rng.standard_normal((37, 5003))
    lg[5, [17, 4000]] = 50.0  # a tie: the last index wins
    host = g.greedy_decoding(lg)
    with ra.DeviceBuffer(lg.nbytes) as dl, ra.DeviceBuffer(37 * 4) as di:
        dl.upload(lg)
        g.greedy_decoding_device(dl, 37, 5003, di)
        dev = di.download(37, np.uint32)
    log(f"greedy_decoding_device: equal {np.array_equal(dev, host)}, tie -> {dev[5]}")
    assert np.array_equal(dev, host) and dev[5] == 4000
    g.close()


def test_device_entry_points_refuse_host_and_short_buffers():
    g = configs.build_network(ra.Network(0), C2S)
    B, S, d = 2, 40, C2S.d
    x = np.zeros((B, S, d), np.complex128)
    out = np.zeros_like(x)
    with pytest.raises(ra.MitokError, match="not device memory") as e:
        g.forward_layers_device(1, 3, x.ctypes.data, B, S, out.ctypes.data)
    log(f"host pointers: {e.value}")
    assert e.value.code == ERR_ARG
    with ra.DeviceBuffer(x.nbytes) as din, ra.DeviceBuffer(16384) as short:  # 81920 bytes needed
        with pytest.raises(ra.MitokError, match="exceed") as e:
            g.forward_layers_device(1, 3, din, B, S, short)
        log(f"short output: {e.value}")
        assert e.value.code == ERR_ARG
    with ra.DeviceBuffer(1 << 20) as dl, ra.DeviceBuffer(4096) as di:  # 64 x 4096 logits need 2 MiB
        with pytest.raises(ra.MitokError, match="exceed") as e:
            g.greedy_decoding_device(dl, 64, 4096, di)
        log(f"short logits: {e.value}")
        assert e.value.code == ERR_ARG
    # the network still works after the refusals
    with ra.DeviceBuffer(x.nbytes) as din, ra.DeviceBuffer(x.nbytes) as dout:
        din.upload(x)
        assert g.forward_layers_device(1, 3, din, B, S, dout) == S
        assert np.array_equal(dout.download((B, S, d), np.complex128), g.forward_layers(1, 3, x))
    g.close()
