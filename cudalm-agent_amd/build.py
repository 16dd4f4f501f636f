"""Build recipe for the W4A16 engine's shared library (gfx950, in-tree).

    python cudalm-agent_amd/build.py

compiles csrc/*.hip with hipcc into cudalm_w4a16/libcudalm_w4a16.so. The
library is what the tests, the smoke check and bench.py load; they never
build it themselves.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB = os.path.join(PKG_DIR, "cudalm_w4a16", "libcudalm_w4a16.so")
SOURCES = ["w4a16_kernels.hip", "w4a16_chain.hip", "w4a16_gemm.hip", "bf16_gemv_kernels.hip", "w4a16_host.hip",
           "cudalm_v2_reader.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops are kept out of all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel arguments preloaded into SGPRs at dispatch (first 16 dwords)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # explicit fp32 operation sequence: no mul+add contraction
    "-ffp-contract=off",
    "-fno-strict-aliasing",
    "-Wno-unused-command-line-argument",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def _stale(obj: str, src: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + [os.path.join(d, f) for d in (CSRC, os.path.join(REPO, "include"))
                    for f in os.listdir(d) if f.endswith(".h")]
    deps += [os.path.join(REPO, "include", "cudalm", d, f)
             for d in ("", "kernels") if os.path.isdir(os.path.join(REPO, "include", "cudalm", d))
             for f in os.listdir(os.path.join(REPO, "include", "cudalm", d)) if f.endswith(".h")]
    return any(os.path.getmtime(p) > t for p in deps)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every source to an object in parallel (one hipcc per file),
    then link the shared library. incremental: recompile only objects older
    than their source or any header."""
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    objdir = os.path.join(PKG_DIR, "_build")
    os.makedirs(objdir, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        if incremental and not _stale(obj, os.path.join(CSRC, src)):
            continue
        cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(REPO, "include"), "-c",
               os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.stderr.write(out)
            failed.append(src)
    if failed:
        raise RuntimeError("hipcc failed on " + ", ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed linking libcudalm_w4a16.so")
    os.replace(tmp, LIB)
    build_boundary_check(verbose)
    return LIB


CHECK_SRC = os.path.join(REPO, "tests", "cpp", "boundary_check.cpp")
CHECK_BIN = os.path.join(REPO, "tests", "cpp", "boundary_check")


def build_boundary_check(verbose: bool = False) -> str:
    """The reference-side C++ caller used by tests/test_gpu_cpp_boundary.py:
    compiled against include/cudalm/ and linked with the library (rpath to
    the package directory)."""
    rpath = "$ORIGIN/" + os.path.relpath(os.path.dirname(LIB), os.path.dirname(CHECK_BIN))
    cmd = [hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel arguments preloaded into SGPRs at dispatch (first 16 dwords)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
           "-Wno-unused-command-line-argument", "-I", os.path.join(REPO, "include"), CHECK_SRC,
           "-L", os.path.dirname(LIB), "-lcudalm_w4a16", f"-Wl,-rpath,{rpath}", "-o", CHECK_BIN + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building tests/cpp/boundary_check")
    os.replace(CHECK_BIN + ".tmp", CHECK_BIN)
    build_round_check(verbose)
    return CHECK_BIN


ROUND_SRC = os.path.join(REPO, "tests", "cpp", "bf16_round_check.hip")
ROUND_BIN = os.path.join(REPO, "tests", "cpp", "bf16_round_check")


def build_round_check(verbose: bool = False) -> str:
    """tests/test_gpu_bf16_round.py's device program: the library's own
    f32_to_bf16_rne (csrc/hip_common.h, same flags as the library)."""
    cmd = [hipcc(), *[f for f in HIPCC_FLAGS if f != "-fPIC"], "-I", os.path.join(REPO, "include"),
           "-I", CSRC, ROUND_SRC, "-o", ROUND_BIN + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building tests/cpp/bf16_round_check")
    os.replace(ROUND_BIN + ".tmp", ROUND_BIN)
    return ROUND_BIN


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
