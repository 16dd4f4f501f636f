"""Writes tests/golden/w4a16_golden.npz: small seeded W4A16 vectors.

Inputs follow the reference's own fixture recipes (xorshift32 seeds and
input classes of tests/cuda/test_int4_gemv_bf16.cpp:77-88,127-135,181-186
and tests/cuda/test_w4a16_qwen35_optimized.cpp:66-171,456); expected
outputs are the oracle's restatement of ref_gemv_bf16
(tests/cuda/test_int4_gemv_bf16.cpp:54-69). The reference commits no golden
vectors of its own, so these are regression data for the oracle and
portable expected outputs for the GPU tests.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def cases():
    # test_int4_gemv_bf16.cpp:127-135 (small members) with its seed rule
    for N, K in ((3, 128), (16, 1024)):
        yield f"vec_N{N}_K{K}", oracle.fixture_gemv(0x51ED51 + N + K, N, K), (N, K, 1)
    # scalar-fallback fixture, test_int4_gemv_bf16.cpp:181-186
    yield "fallback_N37_K256", oracle.fixture_gemv(777, 37, 256), (37, 256, 1)
    # input classes x reference seeds, edge shapes, B = 3
    for kind in ("random", "zero", "small", "mixed_sign", "boundary"):
        for seed in oracle.REFERENCE_SEEDS:
            for N, K in ((5, 256), (9, 1024)):
                yield (f"{kind}_s{seed:08x}_N{N}_K{K}",
                       oracle.fixture_kind(kind, seed, N, K, 3), (N, K, 3))


def main():
    out = {}
    for name, (W, S, X), (N, K, M) in cases():
        out[name + "__W"] = W
        out[name + "__S"] = S
        out[name + "__X"] = X
        out[name + "__Y"] = oracle.gemv_bf16(W, S, X, N, K, M)
        out[name + "__shape"] = np.array([N, K, M], np.int64)
    path = os.path.join(HERE, "w4a16_golden.npz")
    np.savez_compressed(path, **out)
    print(path, len(out) // 5, "cases", os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
