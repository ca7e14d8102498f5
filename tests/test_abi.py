"""The C-ABI library loads and exports every entry point include/mitok.h declares.

CPU-only: loads libmitok.so and resolves symbols; makes no compute call.
"""
import ctypes
import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mitok.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mitok_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ["mitok_network_create", "mitok_predict", "mitok_generate", "mitok_forward_layers",
                 "mitok_greedy_decoding", "mitok_add_self_attention", "mitok_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    import rustcrates_amd

    lib = ctypes.CDLL(rustcrates_amd.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_bindings_cover_the_header():
    import rustcrates_amd

    assert sorted(rustcrates_amd.SIGNATURES) == declared_functions()
    rustcrates_amd.load_library()  # resolves every signature


def test_library_is_gfx950_code():
    import rustcrates_amd

    blob = open(rustcrates_amd.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_bench_refuses_more_than_one_gpu():
    # one GPU per box: --gpus N > 1 exits with a message before touching a device
    import subprocess
    import sys

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
