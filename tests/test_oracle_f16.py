"""Pins the fp16-activation GEMV oracle (orc_gemv_f16, a restatement of
ref_gemv in the reference's tests/cuda/test_int4_gemv.cpp:49-63) and its
fixture (test_int4_gemv.cpp:70-83): numpy brute force in float16/float32
(bit-exact), the fp64 bound, closed forms, and agreement with the bf16
fixture, which draws the same numbers."""
import numpy as np
import pytest


def _numpy_sequential_f16(W, S, X, N, K):
    f32 = np.float32
    xs = X.view(np.float16).astype(np.float32).ravel()
    out = np.empty(N, np.float32)
    for n in range(N):
        acc = f32(0)
        for b in range(K // 2):
            s = S[n, b // 64].view(np.float16).astype(np.float32)
            byte = int(W[n, b])
            lo = (byte & 0xF) - 16 if (byte & 0xF) >= 8 else (byte & 0xF)
            hi = (byte >> 4) - 16 if (byte >> 4) >= 8 else (byte >> 4)
            acc = f32(acc + f32(f32(f32(lo) * s) * xs[2 * b]))
            acc = f32(acc + f32(f32(f32(hi) * s) * xs[2 * b + 1]))
        out[n] = acc
    return out.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("N,K,seed", [(1, 128, 1), (3, 128, 0x1001), (5, 256, 9)])
def test_gemv_f16_bruteforce_bitexact(orc, N, K, seed):
    W, S, X = orc.fixture_gemv_f16(seed, N, K)
    assert np.array_equal(orc.gemv_f16(W, S, X, N, K)[0], _numpy_sequential_f16(W, S, X, N, K))


def test_fixture_f16_matches_bf16_draws(orc):
    N, K = 7, 256
    W1, S1, X1 = orc.fixture_gemv(0x1008, N, K)
    W2, S2, X2 = orc.fixture_gemv_f16(0x1008, N, K)
    assert np.array_equal(W1, W2) and np.array_equal(S1, S2)
    # same n01 draws: fp16 (11-bit) and bf16 (8-bit) roundings of one value
    xf = X2.view(np.float16).astype(np.float64)
    xb = orc.bf16_to_f32(X1).astype(np.float64)
    assert np.all(np.abs(xf - xb) <= orc.bf16_ulp(xb)) and np.abs(xf).max() <= 1.0


@pytest.mark.parametrize("N,K", [(1024, 1024), (64, 2816), (1005, 1024)])
def test_gemv_f16_within_fp64_bound(orc, N, K):
    # test_int4_gemv.cpp:117-130 shapes (subset), seed 0x1000 + 7 i + 1
    W, S, X = orc.fixture_gemv_f16(0x1000 + N, N, K)
    y = orc.gemv_f16(W, S, X, N, K)
    ok, st = orc.check_f16_tolerance(y, W, S, X, N, K, 1, ulps=1.0)
    assert ok, st
    w = orc.dequant(W, S, N, K).astype(np.float64)
    r = w @ X[0].view(np.float16).astype(np.float64)
    assert np.all(np.abs(y[0].view(np.float16).astype(np.float64) - r) <= orc.fp16_ulp(r) + 1e-6)


def test_gemv_f16_closed_forms(orc):
    N, K = 9, 256
    W, S, X = orc.fixture_gemv_f16(5, N, K)
    W0 = W.copy()
    W0[4] = 0
    assert orc.gemv_f16(W0, S, X, N, K)[0, 4] == 0
    k = 131
    Xh = np.zeros_like(X)
    Xh[0, k] = np.float16(1.0).view(np.uint16)
    q = orc.unpack(W, N, K)[:, k].astype(np.float32)
    s = orc.fp16_to_f32(S[:, k // 128])
    assert np.array_equal(orc.gemv_f16(W, S, Xh, N, K)[0], (q * s).astype(np.float16).view(np.uint16))
    yp = orc.gemv_f16(W, S, X, N, K)[0]
    yn = orc.gemv_f16(W, S, X ^ np.uint16(0x8000), N, K)[0]
    nz = (yp & 0x7FFF) != 0
    assert np.array_equal(yn[nz], yp[nz] ^ np.uint16(0x8000))


def test_f16_tolerance_rejects_wrong_answers(orc):
    N, K = 64, 1024
    W, S, X = orc.fixture_gemv_f16(8, N, K)
    y = orc.gemv_f16(W, S, X, N, K)
    S2 = S.copy()
    S2[:, [0, 1]] = S2[:, [1, 0]]
    ok, _ = orc.check_f16_tolerance(orc.gemv_f16(W, S2, X, N, K), W, S, X, N, K, 1)
    assert not ok
    ok, _ = orc.check_f16_tolerance(y + np.uint16(1), W, S, X, N, K, 1)
    assert ok
    y3 = y.copy()
    y3[np.abs(y.view(np.float16).astype(np.float32)) > 1e-2] += np.uint16(4)
    ok, _ = orc.check_f16_tolerance(y3, W, S, X, N, K, 1)
    assert not ok
