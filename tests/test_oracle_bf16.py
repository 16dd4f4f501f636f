"""Pins the bf16 GEMV oracle (oracle/bf16_oracle.c) before it checks the HIP
kernels: the LCG fixture of tests/cuda/test_bf16_gemv.cpp:44-57 against an
independent Python restatement and published known answers, brute-force
numpy fp32 on tiny shapes (bit-exact), numpy fp64 matmul bounds, closed
forms, and the reference's own compare_bf16_stages (oracle/_ref)."""
import numpy as np
import pytest
import torch


def _bf16_bits(f32):
    t = torch.from_numpy(np.ascontiguousarray(f32, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def _lcg_values(seed, n):
    s = seed
    out = np.empty(n, np.float32)
    for e in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[e] = np.float32((s >> 8) * 2.0 ** -23 - 1.0)  # exact in fp32
    return out


def test_lcg_known_answers():
    # Numerical Recipes LCG (a = 1664525, c = 1013904223): from 0 the state
    # runs 1013904223, 1196435762, 3519870697.
    s, seq = 0, []
    for _ in range(3):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        seq.append(s)
    assert seq == [1013904223, 1196435762, 3519870697]


@pytest.mark.parametrize("seed,N,K", [(0, 1, 8), (0x51ed51 + 108, 100, 8), (0xbeef, 3, 37)])
def test_fixture_matches_python_restatement(orc, seed, N, K):
    W, X = orc.bf16_fixture(seed, N, K)
    v = _lcg_values(seed, N * K + K)
    assert np.array_equal(W.ravel(), _bf16_bits(v[:N * K]))
    assert np.array_equal(X.ravel(), _bf16_bits(v[N * K:]))
    f = orc.bf16_to_f32(np.concatenate([W.ravel(), X.ravel()]))
    assert f.min() >= -1.0 and f.max() <= 1.0


def _numpy_sequential(W, X, N, K, M):
    f32 = np.float32
    wf = orc_f32(W)
    xf = orc_f32(X)
    out = np.empty((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            acc = f32(0)
            for k in range(K):
                acc = f32(acc + f32(wf[n, k] * xf[m, k]))
            out[m, n] = acc
    return _bf16_bits(out)


def orc_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("N,K,M", [(1, 1, 1), (3, 3, 1), (5, 17, 2), (4, 64, 3), (2, 200, 1)])
def test_bf16_gemv_bruteforce_bitexact(orc, N, K, M):
    W, x = orc.bf16_fixture(0x77aa77 + 131 * N + K, N, K)
    X = np.ascontiguousarray(np.tile(x, (M, 1)))
    if M > 1:
        X[1:] = _bf16_bits(orc_f32(X[1:]) * np.float32(-0.75))
    assert np.array_equal(orc.bf16_gemv(W, X, N, K, M), _numpy_sequential(W, X, N, K, M))


@pytest.mark.parametrize("N,K", [(100, 1024), (7, 1024), (37, 1000), (64, 4096)])
def test_bf16_gemv_within_fp64_bound(orc, N, K):
    W, X = orc.bf16_fixture(0x51ed51 + N + K, N, K)
    y = orc.bf16_gemv(W, X, N, K)
    ok, st = orc.check_bf16_tolerance(y, W, X, N, K, 1, ulps=1.0)
    assert ok, st
    r = orc_f32(W).astype(np.float64) @ orc_f32(X[0]).astype(np.float64)
    yf = orc_f32(y[0]).astype(np.float64)
    assert np.all(np.abs(yf - r) <= orc.bf16_ulp(r) + 2.0 ** -16 * (np.abs(orc_f32(W)) @ np.abs(orc_f32(X[0]))))


def test_bf16_gemv_closed_forms(orc):
    N, K = 9, 256
    W, X = orc.bf16_fixture(5, N, K)
    # zero weight row -> exact +0 (test_bf16_gemv.cpp: zero row case)
    W0 = W.copy()
    W0[4] = 0
    assert orc.bf16_gemv(W0, X, N, K)[0, 4] == 0
    # one-hot x = 1.0 at k: y = W[:, k] exactly
    k = 131
    Xh = np.zeros_like(X)
    Xh[0, k] = 0x3F80
    assert np.array_equal(orc.bf16_gemv(W, Xh, N, K)[0], W[:, k])
    # sign flip of x negates every nonzero output
    yp = orc.bf16_gemv(W, X, N, K)[0]
    yn = orc.bf16_gemv(W, X ^ np.uint16(0x8000), N, K)[0]
    nz = (yp & 0x7FFF) != 0
    assert np.array_equal(yn[nz], yp[nz] ^ np.uint16(0x8000))
    # batch rows equal single rows; threads do not change bits
    X3 = np.concatenate([X, X ^ np.uint16(0x8000), Xh])
    Y3 = orc.bf16_gemv(W, X3, N, K, 3)
    for b in range(3):
        assert np.array_equal(Y3[b], orc.bf16_gemv(W, X3[b:b + 1].copy(), N, K)[0])
    assert np.array_equal(orc.bf16_gemv(W, X3, N, K, 3, nthreads=4), Y3)


def test_bf16_tolerance_rejects_wrong_answers(orc):
    N, K = 64, 1024
    W, X = orc.bf16_fixture(8, N, K)
    y = orc.bf16_gemv(W, X, N, K)
    # a transposed pair of k (wrong index) must fail
    xf = orc_f32(X[0])
    k = int(np.argmax(np.abs(xf)))
    k2 = int(np.argmin(np.abs(xf)))
    W2 = W.copy()
    W2[:, [k, k2]] = W2[:, [k2, k]]
    ok, st = orc.check_bf16_tolerance(orc.bf16_gemv(W2, X, N, K), W, X, N, K, 1)
    assert not ok and st["n_bad"] >= 1
    # a 1-ulp perturbation passes, 4 ulp fails
    ok, _ = orc.check_bf16_tolerance(y + np.uint16(1), W, X, N, K, 1)
    assert ok
    y3 = y.copy()
    y3[np.abs(orc_f32(y)) > 1e-2] += np.uint16(4)
    ok, _ = orc.check_bf16_tolerance(y3, W, X, N, K, 1)
    assert not ok


def test_bf16_tolerance_implies_reference_comparator(orc):
    # The reference's gate for this kernel is compare_bf16_stages
    # (test_bf16_gemv.cpp:93-103); an output inside our gate passes it too.
    if orc.ref is None:
        pytest.skip("oracle/_ref not built")
    N, K = 512, 1024
    W, X = orc.bf16_fixture(0x51ed51 + N + K, N, K)
    y = orc.bf16_gemv(W, X, N, K)
    ok, _ = orc.check_bf16_tolerance(y, W, X, N, K, 1)
    assert ok
    ok_ref, mx, _ = orc.ref.compare_bf16_stages(y, y)
    assert ok_ref and mx == 0.0
    r, _ = orc.bf16_gemv_f64(W, X, N, K, 1)
    ok_ref, mx, _ = orc.ref.compare_bf16_stages(orc.f32_to_bf16(r.astype(np.float32)), y)
    assert ok_ref, mx
