"""Builds libmitok.so (the HIP C-ABI library) in-tree for gfx950.

    python -m rustcrates_amd.build          # or __graft_entry__.build()

Each .hip source is compiled in parallel by hipcc, then linked into
rustcrates_amd/libmitok.so, which travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmitok.so")
SOURCES = ["kernels.hip", "gemm.hip", "gemm_mfma.hip", "attention.hip", "resident.hip", "resident_k1.hip", "resident_k2.hip",
           "resident_k4.hip", "resident_k8.hip", "train.hip", "wavelet_init.hip", "network.hip"]
ARCH = os.environ.get("MITOK_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep packed-FP32 instructions out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # warnings fail the build: -Wuninitialized and its kin find on the CPU
    # what would otherwise surface as a GPU memory fault
    "-Wall", "-Wno-unused-function", "-Wno-unused-result", "-Werror",
]

# hipcc's host pass does not know the packed-FP32 target feature and says so
# once per translation unit; that line is not a diagnostic of the source
_HOST_FEATURE_NOTE = "'-packed-fp32-ops' is not a recognized feature"


# per-file flags: the prompt-pass GEMM keeps its MFMA accumulators in VGPRs
# (the reason is in gemm_mfma.hip's header)
FILE_FLAGS = {"gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              # the optimizer's arithmetic rounds every multiply and add, as Rust does
              "train.hip": ["-ffp-contract=off"],
              # the wavelet embedding follows the reference's multiply and add order
              "wavelet_init.hip": ["-ffp-contract=off"]}


def source_hash() -> str:
    """SHA-256 (16 hex digits) of every device/host source file in csrc/: counter
    measurements are stamped with it, so a stale one is recognised."""
    import hashlib

    h = hashlib.sha256()
    for name in sorted(os.listdir(SRC)):
        if name.endswith((".hip", ".hpp", ".h")):
            h.update(name.encode())
            with open(os.path.join(SRC, name), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(SRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    rest = [ln for ln in r.stderr.splitlines() if _HOST_FEATURE_NOTE not in ln and ln.strip()]
    if rest:
        print(f"hipcc output for {src}:", *rest, sep="\n", file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
