"""Builds libtabicl_attn.so (the C-ABI HIP library) for gfx950 with hipcc, in-tree.

Usage: python build_lib.py [-v]. Objects go to _build/ next to this file; the library is written
next to this file, where tabicl_mi355_native.py loads it from.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libtabicl_attn.so"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in any kernel of this library.
# -amdgpu-mfma-vgpr-form: MFMA results in arch VGPRs; the default AGPR form makes the compiler copy
#  every accumulator between AGPRs and VGPRs around the softmax (measured: ~128 copies per tile).
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form", "-Wall", "-Wno-unused-function",
         "-Wno-unused-command-line-argument"]
SOURCES = ["abi.hip", "icl_fwd.hip", "icl_bwd.hip", "smallhead_fwd.hip", "smallhead_stream.hip", "smallhead_bwd.hip", "keymask.hip",
           "layernorm.hip"]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, flush=True)


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        futs = [ex.submit(_compile, CSRC / s, o, verbose) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
