"""GPU parity tests of the bf16 GEMV (tied LM head) through the C ABI
(include/cudalm_bf16_gemv.h) against the CPU oracle, a restatement of the
reference's ref_gemv_bf16 (tests/cuda/test_bf16_gemv.cpp:62-73), on the
reference's own fixture recipe and shape lists (test_bf16_gemv.cpp:44-57,
112-200) and its batch contract (batch_decode.h:69-79,
tests/cuda/test_qwen35_batch_kernels.cpp:133-165).

Bars:
  * outputs: |y - r| <= 2 ulp_bf16(r) + 2^-16 * sum_k |w x|, r the exact
    (fp64) sum (oracle.check_bf16_tolerance), and the reference's own
    compare_bf16_stages against the oracle where oracle/_ref is built;
  * zero weight row: exact +0;
  * batch row b: bit-identical to the single-row call on x_b, for every
    chunking of M.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def up(dev, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
            for a in arrays]


def down(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run(w4, w, x, N, K, M, variant="auto"):
    y = torch.empty((M, N), dtype=torch.bfloat16, device=w.device)
    w4.bf16_gemv_any(w, x, N, K, M, y=y, variant=variant)
    return down(y).reshape(M, N)


def check(orc, Y, W, X, N, K, M, label, ref_cmp=True):
    ok, st = orc.check_bf16_tolerance(Y, W, X, N, K, M)
    print(f"  {label} N={N} K={K} M={M}: {st}", flush=True)
    assert ok, (label, st)
    if ref_cmp and orc.ref is not None:
        ok, mx, idx = orc.ref.compare_bf16_stages(orc.bf16_gemv(W, X, N, K, M, nthreads=8), Y)
        assert ok, (label, mx, idx)


# test_bf16_gemv.cpp:112-131 (vec4 shapes, including the LM head)
VEC_SHAPES = [(248320, 1024), (1, 1024), (7, 1024), (100, 1024), (1024, 1024), (4096, 1024),
              (100, 8), (100, 16), (100, 64), (100, 512), (3, 8)]
# test_bf16_gemv.cpp:137-152 (listed as K % 8 != 0 cases; 1000 is a
# multiple of 8, so that one takes the stream kernel)
SCALAR_SHAPES = [(5, 1000), (5, 1025), (1, 1), (3, 3), (100, 7), (100, 9)]


@pytest.mark.parametrize("N,K", VEC_SHAPES)
def test_reference_vectorized_shapes(w4, orc, dev, N, K):
    W, X = orc.bf16_fixture(0x51ED51 + N + K, N, K)
    Y = run(w4, *up(dev, W, X), N, K, 1, "stream")
    check(orc, Y, W, X, N, K, 1, "stream")
    assert np.array_equal(run(w4, *up(dev, W, X), N, K, 1), Y)  # auto picks the same kernel


@pytest.mark.parametrize("N,K", SCALAR_SHAPES)
def test_reference_scalar_shapes(w4, orc, dev, N, K):
    W, X = orc.bf16_fixture(0x77AA77 + N * 131 + K, N, K)
    Y = run(w4, *up(dev, W, X), N, K, 1)
    check(orc, Y, W, X, N, K, 1, "auto")
    check(orc, run(w4, *up(dev, W, X), N, K, 1, "scalar"), W, X, N, K, 1, "scalar")
    if K % 8:
        with pytest.raises(ValueError):
            run(w4, *up(dev, W, X), N, K, 1, "stream")


def test_misaligned_bases_take_scalar_path(w4, orc, dev):
    # test_bf16_gemv.cpp:159-200: 2-byte offsets on both bases, and the
    # element-wise result agrees with the aligned stream kernel
    N, K = 37, 1024
    W, X = orc.bf16_fixture(0xBEEF, N, K)
    wbuf = torch.zeros(W.size + 8, dtype=torch.int16, device=dev)
    wbuf[1:1 + W.size] = torch.from_numpy(W.ravel().view(np.int16)).to(dev)
    xbuf = torch.zeros(X.size + 8, dtype=torch.int16, device=dev)
    xbuf[1:1 + X.size] = torch.from_numpy(X.ravel().view(np.int16)).to(dev)
    y = torch.empty(N, dtype=torch.int16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert w4.bf16_gemv_ptr(wbuf.data_ptr() + 2, xbuf.data_ptr() + 2, y.data_ptr(), N, K, 1,
                            w4.BF16_VARIANT_STREAM, st) == w4.EVARIANT
    assert w4.bf16_gemv_ptr(wbuf.data_ptr() + 2, xbuf.data_ptr() + 2, y.data_ptr(), N, K, 1,
                            w4.BF16_VARIANT_AUTO, st) == 0
    Ys = down(y).reshape(1, N)
    check(orc, Ys, W, X, N, K, 1, "misaligned")
    Yv = run(w4, *up(dev, W, X), N, K, 1)
    check(orc, Yv, W, X, N, K, 1, "aligned")
    if orc.ref is not None:
        ok, mx, _ = orc.ref.compare_bf16_stages(Yv, Ys)
        assert ok, mx


@pytest.mark.parametrize("variant", ["stream", "scalar"])
def test_zero_weight_row_exact_zero(w4, orc, dev, variant):
    N, K = 40, 1024
    W, X = orc.bf16_fixture(99, N, K)
    W[[0, 17, 39]] = 0
    for M in (1, 5):
        Xm = np.ascontiguousarray(np.repeat(X, M, axis=0))
        Y = run(w4, *up(dev, W, Xm), N, K, M, variant)
        assert not Y[:, [0, 17, 39]].any()


@pytest.mark.parametrize("M", [2, 3, 8, 16, 17, 32, 33, 64, 100])
def test_batch_rows_bitidentical_to_single(w4, orc, dev, M):
    # batch_bf16_gemv row b == bf16_gemv on x_b (test_qwen35_batch_kernels.cpp:133-165)
    N, K = 1000, 1024
    W, _ = orc.bf16_fixture(0xB0 + M, N, K)
    X = orc.synth_act(0x5EED + M, M, K)
    w, x = up(dev, W, X)
    Y = run(w4, w, x, N, K, M)
    check(orc, Y, W, X, N, K, M, "batch", ref_cmp=False)
    for b in sorted({0, M // 2, M - 1}):
        y1 = run(w4, w, x[b:b + 1].contiguous(), N, K, 1)
        assert np.array_equal(Y[b], y1[0]), b


@pytest.mark.parametrize("N,K,M", [(40, 8200, 3), (33, 65536, 2), (20, 90112, 2), (64, 2560, 40)])
def test_long_rows_and_lds_chunking(w4, orc, dev, N, K, M):
    # rows longer than the LDS holds for 32 activation rows are chunked;
    # beyond one row per chunk the element-wise kernel serves the call
    W, _ = orc.bf16_fixture(K + M, N, K)
    X = orc.synth_act(0xC4 + M, M, K)
    Y = run(w4, *up(dev, W, X), N, K, M)
    check(orc, Y, W, X, N, K, M, "long", ref_cmp=False)
    if K <= 65536:
        y1 = run(w4, *up(dev, W, X[M - 1:M]), N, K, 1)
        assert np.array_equal(Y[M - 1], y1[0])


def test_lm_head_synthetic_batch8(w4, orc, dev):
    # the tied LM head at M = 8 on N(0, 0.02) weights (the benchmark's data)
    N, K, M = 248320, 1024, 8
    W = orc.f32_to_bf16(orc.synth_normal(0xC0DA, 0.02, N * K)).reshape(N, K)
    X = orc.synth_act(0xAC7, M, K)
    Y = run(w4, *up(dev, W, X), N, K, M)
    # every output within the bound, and over these 2M outputs no more beyond
    # 2 ulp than the reference's own CPU loop (ref_gemv_bf16) has
    ok, st, _ = orc.check_bf16_against_reference_loop(Y, W, X, N, K, M,
                                                     max(1, min(16, __import__("os").cpu_count() or 1)))
    print(f"  lm_head M=8: {st}", flush=True)
    assert ok, st


def test_cpp_reference_names(w4, orc, dev):
    N, K, B = 512, 1024, 3
    W, _ = orc.bf16_fixture(3, N, K)
    X = orc.synth_act(0x33, B, K)
    w, x = up(dev, W, X)
    y1 = torch.empty(N, dtype=torch.bfloat16, device=dev)
    w4.bf16_gemv(w, x[1], y1, N, K)
    yb = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
    w4.batch_bf16_gemv(w, x, yb, N, K, B)
    assert np.array_equal(down(yb).reshape(B, N)[1], down(y1))
    assert w4.bf16_gemv_kernel_regs() > 0


def test_non_default_stream(w4, orc, dev):
    N, K, M = 777, 1024, 4
    W, _ = orc.bf16_fixture(4, N, K)
    X = orc.synth_act(0x44, M, K)
    w, x = up(dev, W, X)
    ref = run(w4, w, x, N, K, M)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.bf16_gemv_any(w, x, N, K, M, y=y, stream=st)
    st.synchronize()
    assert np.array_equal(down(y).reshape(M, N), ref)


def test_repack_layout(w4, dev):
    """The tile-major copy (include/cudalm_bf16_gemv.h): slab j of unit u of
    tile t holds, at 16-byte block l, row 16 t + l % 16, k = 256 u + 32 j +
    8 (l / 16) .. + 7; restated here with a numpy reshape."""
    N, K = 48, 512
    rng = np.random.default_rng(0xB1)
    W = rng.integers(0, 1 << 16, size=(N, K), dtype=np.uint16)
    (w,) = up(dev, W)
    P = down(w4.bf16_repack(w, N, K))
    # [t, i, u, j, a, e] -> [t, u, j, a, i, e]
    exp = W.reshape(N // 16, 16, K // 256, 8, 4, 8).transpose(0, 2, 3, 4, 1, 5).reshape(-1)
    assert np.array_equal(P, exp)


@pytest.mark.parametrize("N,K,M", [(16, 256, 1), (4096, 1024, 1), (4096, 1024, 8),
                                   (1024, 2048, 17), (4096, 1024, 32), (512, 1024, 40),
                                   (248320, 1024, 1), (248320, 1024, 8)])
def test_prepacked_equals_row_major(w4, orc, dev, N, K, M):
    """The packed copy gives the row-major call's bits (same kernel, same
    MFMA chain per output) and so the same oracle bound."""
    W = orc.f32_to_bf16(orc.synth_normal(0xB0 + N + K, 0.02, N * K)).reshape(N, K)
    X = orc.synth_act(0xB1 + M, M, K)
    w, x = up(dev, W, X)
    Y = run(w4, w, x, N, K, M)
    p = w4.bf16_repack(w, N, K)
    Yp = down(w4.bf16_gemv_prepacked(p, x, N, K, M)).reshape(M, N)
    assert np.array_equal(Yp, Y), (N, K, M)
    if N * K <= 4096 * 2048:
        check(orc, Yp, W, X, N, K, M, "prepacked", ref_cmp=False)
