"""Builds and runs issue_gfx950 (the gfx950 issue-rate microbenchmarks behind the attention kernels'
design limits; not part of libtabicl_attn.so).

Usage: python run.py [build|rates|coissue|step]. `build` only compiles (hipcc, gfx950, the library's
flags) into _build/ next to this file; any other argument (or none: all three groups) runs the binary,
building it first if it is missing. Needs an MI355X to run."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "issue_gfx950.hip"
BIN = HERE / "_build" / "issue_gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build() -> Path:
    BIN.parent.mkdir(exist_ok=True)
    subprocess.run([HIPCC, *FLAGS, str(SRC), "-o", str(BIN)], check=True)
    return BIN


def main() -> int:
    arg = sys.argv[1] if len(sys.argv) > 1 else ""
    if arg == "build":
        print(build())
        return 0
    if not BIN.exists():
        build()
    return subprocess.run([str(BIN), *([arg] if arg else [])]).returncode


if __name__ == "__main__":
    sys.exit(main())
