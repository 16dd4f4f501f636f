"""GPU parity of the fp16-activation twin (cudalm_w4a16_gemv_f16, the
reference's int4_gemv) against the CPU oracle (ref_gemv of
tests/cuda/test_int4_gemv.cpp:49-63), on that test's fixtures, shapes,
zero-group and misaligned cases (test_int4_gemv.cpp:115-290), plus row
parity and layout bit-identity.

Bar: |y - r| <= 2 ulp_fp16(r) + 2^-16 sum|terms| (oracle.check_f16_tolerance)
and the reference's compare_fp16_stages where oracle/_ref is built. On the
reference's own fixtures no output may be more than 2 fp16 ulp from the
fp64 value (the floor term is for cancellation-heavy synthetic inputs)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def up(dev, W, S, X):
    w = torch.from_numpy(np.ascontiguousarray(W)).to(dev)
    s = torch.from_numpy(np.ascontiguousarray(S).view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(np.ascontiguousarray(X).view(np.int16)).to(dev).view(torch.float16)
    return w, s, x


def down(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def check(orc, Y, W, S, X, N, K, M, label, strict=False):
    ok, st = orc.check_f16_tolerance(Y, W, S, X, N, K, M)
    print(f"  {label} N={N} K={K} M={M}: {st}", flush=True)
    assert ok, (label, st)
    if strict:
        assert st["n_over_2ulp"] == 0, (label, st)
    if orc.ref is not None:
        ok, mx, idx = orc.ref.compare_fp16_stages(orc.gemv_f16(W, S, X, N, K, M), Y)
        assert ok, (label, mx, idx)
    return st


SHAPES = [(1024, 1024), (512, 1024), (2816, 1024), (1024, 2816), (1005, 1024), (1, 128)]


@pytest.mark.parametrize("i", range(len(SHAPES)))
def test_reference_shapes(w4, orc, dev, i):
    N, K = SHAPES[i]
    W, S, X = orc.fixture_gemv_f16(0x1000 + 7 * i + 1, N, K)
    w, s, x = up(dev, W, S, X)
    y = torch.empty(N, dtype=torch.float16, device=dev)
    w4.int4_gemv(w, s, x[0], y, N, K)
    Y = down(y).reshape(1, N)
    check(orc, Y, W, S, X, N, K, 1, "int4_gemv", strict=True)
    p = w4.repack(w, s, N, K)
    assert np.array_equal(down(w4.gemv_f16_prepacked(p, x, N, K)).reshape(1, N), Y)


def test_zero_group_exact_zero(w4, orc, dev):
    N, K = 8, 128
    W, S, X = orc.fixture_gemv_f16(0x700, N, K)
    S[:] = 0
    Y = down(w4.gemv_f16(*up(dev, W, S, X), N, K))
    assert not (Y & 0x7FFF).any()


def test_misaligned_bases(w4, orc, dev):
    N, K = 512, 1024
    W, S, X = orc.fixture_gemv_f16(0xABC, N, K)
    w, s, x = up(dev, W, S, X)
    st = torch.cuda.current_stream().cuda_stream
    # x misaligned by 2 halves, W misaligned by 8 bytes
    xb = torch.zeros(K + 8, dtype=torch.float16, device=dev)
    xb[2:2 + K] = x[0]
    wb = torch.zeros(W.size + 16, dtype=torch.uint8, device=dev)
    wb[8:8 + W.size] = w.view(-1)
    y = torch.empty(N, dtype=torch.float16, device=dev)
    lib = w4.lib()
    assert lib.cudalm_w4a16_gemv_f16(wb.data_ptr() + 8, s.data_ptr(), xb.data_ptr() + 4,
                                     y.data_ptr(), N, K, 1, st) == 0
    Ym = down(y).reshape(1, N)
    check(orc, Ym, W, S, X, N, K, 1, "misaligned", strict=True)
    Ya = down(w4.gemv_f16(w, s, x, N, K)).reshape(1, N)
    if orc.ref is not None:
        ok, mx, _ = orc.ref.compare_fp16_stages(Ya, Ym)
        assert ok, mx


@pytest.mark.parametrize("M", [2, 8, 17, 32, 40, 100])
def test_rows_bitidentical_and_layouts(w4, orc, dev, M):
    N, K = 777, 2048
    W, S = orc.synth_w4a16(0xF16 + M, N, K)
    rng = np.random.default_rng(M)
    X = rng.normal(0, 1, (M, K)).astype(np.float16).view(np.uint16)
    w, s, x = up(dev, W, S, X)
    Y = down(w4.gemv_f16(w, s, x, N, K, M)).reshape(M, N)
    check(orc, Y, W, S, X, N, K, M, "batch")
    for b in sorted({0, M // 2, M - 1}):
        y1 = down(w4.gemv_f16(w, s, x[b:b + 1].contiguous(), N, K, 1))
        assert np.array_equal(Y[b], y1.reshape(N)), b
    p = w4.repack(w, s, N, K)
    assert np.array_equal(down(w4.gemv_f16_prepacked(p, x, N, K, M)).reshape(M, N), Y)


def test_overflow_to_infinity(w4, orc, dev):
    # outputs beyond the fp16 range round to infinities of the right sign
    N, K = 16, 256
    W = np.full((N, K // 2), 0x77, np.uint8)  # q = 7 everywhere
    S = np.full((N, K // 128), np.float16(60.0).view(np.uint16), np.uint16)
    X = np.full((1, K), np.float16(1.0).view(np.uint16), np.uint16)
    X[0, :] = np.where(np.arange(K) % 2 == 0, X[0], np.float16(1.0).view(np.uint16))
    Y = down(w4.gemv_f16(*up(dev, W, S, X), N, K))  # 7 * 60 * 256 = 107520 > 65504
    assert np.all(Y == 0x7C00)
    ok, st = orc.check_f16_tolerance(Y.reshape(1, N), W, S, X, N, K, 1)
    assert ok, st
