"""Builds the gfx950 engine library ``instantcua_amd/libicua.so`` with hipcc.

Each ``csrc/*.hip`` translation unit is compiled to an object (in parallel), then linked into
one shared library that exports the C ABI of ``include/icua.h``.

``--trace`` builds ``libicua_trace.so`` instead: the same library with the persistent decode
kernel's stage timeline compiled in (``ICUA_PERSIST_TRACE``), read by ``trace_decode.py``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libicua.so")
TRACE_LIB = os.path.join(HERE, "libicua_trace.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["engine.hip", "gemv.hip", "gemv8.hip", "attention.hip", "misc.hip", "persist.hip", "prefill.hip", "quant.hip", "vision.hip", "tokenizer.cpp"]

# Packed-FP32 instructions are disabled for every device pass (the host pass ignores the
# feature with a warning).
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}",
    f"-I{CSRC}",
]


def _compile(src: str, trace: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + (".trace.o" if trace else ".o"))
    cmd = [HIPCC, *FLAGS, *(["-DICUA_PERSIST_TRACE"] if trace else []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False, trace: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, trace), SOURCES))
    out = TRACE_LIB if trace else LIB
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, trace="--trace" in sys.argv[1:])
    sys.exit(0)
