"""Builds libmimizuku_amd.so in-tree with hipcc for gfx950 (no CMake, no JIT cache).

    python -m mimizuku_amd.build          # or __graft_entry__.build()

Every source under csrc/ is compiled to an object in _build/ (in parallel), then linked into
mimizuku_amd/libmimizuku_amd.so. Packed fp32 VALU forms are disabled for the device code. The command-line tool
cli/mimizuku.cpp (host code over the C ABI) is linked against the library as mimizuku_amd/mimizuku, which finds
the library next to itself.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmimizuku_amd.so")
CLI_SRC = os.path.join(HERE, "cli", "mimizuku.cpp")
CLI_OUT = os.path.join(HERE, "mimizuku")
BUILD = os.path.join(ROOT, "_build")
ARCH = os.environ.get("MZ_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wno-unused-result"]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


# host-only sources with their own instruction-set flags (checked at run time before use)
EXTRA = {"align.cpp": ["-mf16c", "-mavx2"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *FLAGS, *EXTRA.get(os.path.basename(src), []), *lang, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    tmp = CLI_OUT + ".tmp"
    cmd = [HIPCC, "-O2", "-std=c++17", "-Wno-unused-result", CLI_SRC, "-o", tmp, f"-L{HERE}", "-lmimizuku_amd",
           "-Wl,-rpath,$ORIGIN", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building the command-line tool failed:\n{r.stderr}")
    os.replace(tmp, CLI_OUT)
    if verbose:
        print(f"built {OUT} and {CLI_OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build()
