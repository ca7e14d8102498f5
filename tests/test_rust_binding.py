"""The Rust FFI crate (bindings/rust/mitok-sys) declares exactly the C ABI of
include/mitok.h: every entry point, with the same parameter and return types,
const-ness included.  No Rust toolchain exists in this image, so this is the
check that the crate a maintainer adds to the reference binds the library as
built."""
from __future__ import annotations

import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mitok.h")
CRATE = os.path.join(ROOT, "bindings", "rust", "mitok-sys")

_SCALARS = {"int": "c_int", "uint32_t": "u32", "uint64_t": "u64", "double": "c_double", "char": "c_char",
            "mitok_network": "MitokNetwork", "void": "()"}


def _c_to_rust(c_type: str) -> str:
    """`const uint32_t*` -> `*const u32`, `mitok_network**` -> `*mut *mut MitokNetwork`."""
    t = " ".join(c_type.split())
    stars = t.count("*")
    t = t.replace("*", "").strip()
    const = t.startswith("const ")
    base = _SCALARS[t.replace("const ", "").strip()]
    if not stars:
        return base
    out = base
    for i in range(stars):
        # the const applies to the pointee, i.e. the innermost pointer
        out = ("*const " if (i == 0 and const) else "*mut ") + out
    return out


def header_prototypes():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(mitok_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        ps = [] if params in ("", "void") else [" ".join(p.split()) for p in params.split(",")]
        types = []
        for p in ps:
            t = p if p.endswith("*") else re.sub(r"\s*\b\w+$", "", p)  # drop the parameter name
            if "*" in p:
                t = p[: p.rindex("*") + 1]
            types.append(_c_to_rust(t))
        out[name] = (_c_to_rust(ret), types)
    return out


def crate_prototypes():
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = src[src.index('extern "C" {'):]
    block = block[: block.index("\n}\n")]
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (mitok_[a-z0-9_]+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block):
        name, params, ret = m.group(1), m.group(2).strip().rstrip(","), (m.group(4) or "()").strip()
        types = [] if not params else [" ".join(p.split(":", 1)[1].split()) for p in params.split(",")]
        out[name] = (ret, types)
    return out


def test_crate_declares_every_header_entry_point_with_its_types():
    h, r = header_prototypes(), crate_prototypes()
    assert len(h) > 30
    assert sorted(h) == sorted(r), (set(h) ^ set(r))
    for name in h:
        assert r[name] == h[name], (name, h[name], r[name])


def test_crate_constants_match_the_header():
    def value(v):  # 5, 0xFFFFFFFFu (C) or 0xFFFF_FFFF (Rust)
        return int(v.rstrip("uU").replace("_", ""), 0)

    text = open(HEADER).read()
    hdr = {k: value(v) for k, v in re.findall(r"#define (MITOK_[A-Z_]+) (0x[0-9A-Fa-f]+[uU]?|\d+)\b", text)}
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    rs = {k: value(v) for k, v in re.findall(r"pub const (MITOK_[A-Z_]+): (?:c_int|u32) = (0x[0-9A-Fa-f_]+|\d+);", src)}
    assert hdr == rs and "MITOK_ALL_LAYERS" in hdr


def test_crate_manifest_links_the_library():
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "mitok"' in toml and 'num-complex = "0.4.6"' in toml  # the reference's num-complex
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=mitok" in build and "MITOK_DIR" in build
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    assert "pub mod transformer;" in lib and os.path.exists(os.path.join(CRATE, "src", "transformer.rs"))
