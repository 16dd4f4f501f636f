"""Build recipe for the CPU oracle (test infrastructure only).

  oracle/liborc_w4a16.so   plain-C restatement of the reference's CPU path
                           (w4a16_oracle.c, bf16_oracle.c, swiglu_oracle.c),
                           gcc, -ffp-contract=off
  oracle/_ref/libref_stage_compare.so
                           the reference's own header-only fp16/bf16 decoders
                           and compare_bf16_stages
                           (include/cudalm/stage_compare.h), compiled from
                           /root/reference in place through ref_shim.cpp.
                           Built only where /root/reference exists; the rest
                           of the reference's W4A16 path needs CUDA headers
                           and nvcc and is not buildable here.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liborc_w4a16.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_LIB = os.path.join(REF_DIR, "libref_stage_compare.so")
REFERENCE = "/root/reference"


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + res.stdout + res.stderr)
        raise RuntimeError(f"oracle build failed: {cmd[0]}")


def build_oracle() -> str:
    tmp = ORACLE_LIB + ".tmp"
    _run(["gcc", "-O2", "-std=c99", "-D_POSIX_C_SOURCE=200809L", "-fPIC", "-shared",
          "-ffp-contract=off", "-fno-fast-math", "-Wall",
          os.path.join(HERE, "w4a16_oracle.c"), os.path.join(HERE, "bf16_oracle.c"),
          os.path.join(HERE, "swiglu_oracle.c"),
          "-o", tmp, "-lm", "-lpthread"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_ref() -> str | None:
    header = os.path.join(REFERENCE, "include", "cudalm", "stage_compare.h")
    if not os.path.exists(header):
        return None
    os.makedirs(REF_DIR, exist_ok=True)
    tmp = REF_LIB + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
          "-I", os.path.join(REFERENCE, "include"),
          os.path.join(HERE, "ref_shim.cpp"), "-o", tmp])
    os.replace(tmp, REF_LIB)
    return REF_LIB


def build() -> None:
    build_oracle()
    build_ref()


if __name__ == "__main__":
    build()
    print(ORACLE_LIB)
