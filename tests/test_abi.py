"""The C-ABI library loads and exports every entry point include/mitok.h declares.

CPU-only: loads libmitok.so and resolves symbols; makes no compute call.
"""
import ctypes
import os
import re

import pytest

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


# --------------------------------------------------------------------------
# prototypes: header against the ctypes bindings, and a C client of the header
# --------------------------------------------------------------------------
_C_TO_CTYPES = {
    "void": None, "int": ctypes.c_int, "uint32_t": ctypes.c_uint32, "uint64_t": ctypes.c_uint64,
    "double": ctypes.c_double,
}


def declared_prototypes():
    """name -> (return type, [parameter types]) parsed from include/mitok.h."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(mitok_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        ps = [] if params in ("", "void") else [" ".join(p.split()) for p in params.split(",")]
        types = []
        for p in ps:
            p = p.replace("const ", "")
            t = re.sub(r"\s*\b\w+$", "", p) if not p.endswith("*") else p  # drop the parameter name
            types.append(t.replace(" *", "*").strip())
        out[name] = (ret.replace("const ", "").replace(" *", "*").strip(), types)
    return out


def _ctype_of(c_type):
    if c_type == "char*":
        return ctypes.c_char_p
    if c_type.endswith("*"):
        return "ptr"
    return _C_TO_CTYPES[c_type]


def _matches(py, c_type):
    want = _ctype_of(c_type)
    if want == "ptr":  # any pointer binding: void* or a typed POINTER(...)
        return py is ctypes.c_void_p or (isinstance(py, type) and issubclass(py, ctypes._Pointer))
    return py is want


def test_python_signatures_match_header_prototypes():
    import rustcrates_amd

    protos = declared_prototypes()
    assert sorted(protos) == declared_functions()
    for name, (ret, params) in protos.items():
        res, args = rustcrates_amd.SIGNATURES[name]
        assert _matches(res, ret) if ret != "void" else res is None, (name, ret, res)
        assert len(args) == len(params), (name, params, args)
        for i, (a, p) in enumerate(zip(args, params)):
            assert _matches(a, p), (name, i, p, a)


def _build_c_client(tmp_path):
    import shutil
    import subprocess

    import rustcrates_amd

    cc = shutil.which("gcc") or shutil.which("cc")
    exe = str(tmp_path / "abi_client")
    libdir = os.path.dirname(rustcrates_amd.LIB_PATH)
    cmd = [cc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c", "abi_client.c"), "-L", libdir, "-lmitok",
           f"-Wl,-rpath,{libdir}", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_c_client_compiles_and_links_against_header(tmp_path):
    """A C translation unit that includes mitok.h and calls the token-loop
    entry points builds warning-free and links against libmitok.so."""
    import subprocess

    exe = _build_c_client(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "version" in r.stdout, r.stderr


@pytest.mark.gpu
def test_c_client_runs_token_loop(tmp_path):
    """Through the C ABI alone: generate and prefill + decode_step agree on
    every id, and a step before prefill returns MITOK_ERR_STATE."""
    import subprocess

    exe = _build_c_client(tmp_path)
    print("C client: generate vs prefill + decode_step", flush=True)
    r = subprocess.run([exe, "run"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = dict(line.split(":", 1) for line in r.stdout.strip().splitlines())
    assert lines["generate"].split() == lines["steps"].split()
    assert len(lines["generate"].split()) == 9
