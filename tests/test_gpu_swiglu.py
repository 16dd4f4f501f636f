"""GPU tests of the SwiGLU stage: the element-wise silu*mul kernel
(qwen35_silu_mul_bf16, include/cudalm/kernels/qwen35_kernels.h:146-155)
against the CPU oracle, and the fused gate/up + silu*mul launch against the
reference's three-step sequence (src/runtime/qwen35_deltanet.cpp:236-247)
run on this library.

Bars:
  * silu*mul: equal to the oracle's bits except where the device expf and
    the host expf round differently; those outputs differ by at most one
    bf16 ulp and are fewer than 1 in 1000;
  * fused launch: bit-identical to gemv(gate) -> gemv(up) -> silu*mul for
    every M, both weight layouts.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def up(dev, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev) for a in arrays]


def down(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def ulp_diff(a, b):
    """Distance in bf16 steps between same-sign bit patterns (large if signs differ)."""
    a = a.astype(np.int64)
    b = b.astype(np.int64)
    sa, sb = a >> 15, b >> 15
    d = np.abs((a & 0x7FFF) - (b & 0x7FFF))
    return np.where((sa == sb) | ((a & 0x7FFF) == 0) | ((b & 0x7FFF) == 0), d, 1 << 20)


def silu_mul_dev(w4, dev, g, u, offset=0):
    n = g.size
    gb = torch.zeros(n + 16, dtype=torch.int16, device=dev)
    ub = torch.zeros(n + 16, dtype=torch.int16, device=dev)
    yb = torch.zeros(n + 16, dtype=torch.int16, device=dev)
    gb[offset:offset + n] = torch.from_numpy(g.view(np.int16)).to(dev)
    ub[offset:offset + n] = torch.from_numpy(u.view(np.int16)).to(dev)
    ys = yb[offset:offset + n]
    w4.qwen35_silu_mul_bf16(gb[offset:offset + n], ub[offset:offset + n], ys, n)
    out = down(yb)
    assert not out[:offset].any() and not out[offset + n:].any()  # no writes outside [0, n)
    return out[offset:offset + n]


def test_silu_mul_all_bf16_gate_values(w4, orc, dev):
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = g[((g & 0x7F80) != 0x7F80) | ((g & 0x7F) == 0)]  # NaN payloads excluded
    one = np.full(g.size, 0x3F80, np.uint16)  # u = 1: y = silu_bf16(g) exactly
    y = silu_mul_dev(w4, dev, g, one)
    ref = orc.silu_mul_bf16(g, one)
    d = ulp_diff(y, ref)
    print(f"  silu: {int((d != 0).sum())} of {g.size} differ, max {int(d.max())} ulp", flush=True)
    assert d.max() <= 1 and (d != 0).sum() <= g.size // 1000
    rng = np.random.default_rng(11)
    u = orc.f32_to_bf16(rng.normal(0, 1, g.size).astype(np.float32))
    y = silu_mul_dev(w4, dev, g, u)
    d = ulp_diff(y, orc.silu_mul_bf16(g, u))
    assert d.max() <= 1 and (d != 0).sum() <= g.size // 1000


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (8, 0), (13, 1), (3584, 0), (3584, 3),
                                      (100003, 0)])
def test_silu_mul_ragged_and_misaligned(w4, orc, dev, n, offset):
    rng = np.random.default_rng(n)
    g = orc.f32_to_bf16(rng.normal(0, 4, n).astype(np.float32))
    u = orc.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    y = silu_mul_dev(w4, dev, g, u, offset)
    d = ulp_diff(y, orc.silu_mul_bf16(g, u))
    assert d.max() <= 1 and (d != 0).sum() <= max(1, n // 1000)


def three_step(w4, gw, gs, uw, us, x, N, K, M, packed):
    if packed:
        g = w4.gemv_prepacked(gw, x, N, K, M)
        u = w4.gemv_prepacked(uw, x, N, K, M)
    else:
        g = w4.gemv(gw, gs, x, N, K, M)
        u = w4.gemv(uw, us, x, N, K, M)
    y = torch.empty_like(g)
    w4.qwen35_silu_mul_bf16(g, u, y, M * N)
    return down(g), down(u), down(y)


@pytest.mark.parametrize("N,K", [(3584, 1024), (37, 256), (100, 3584), (16, 1024), (1000, 2048),
                                 (5000, 640)])
@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 32, 33, 64, 100])
@pytest.mark.parametrize("packed", [False, True])
def test_fused_swiglu_equals_three_step(w4, orc, dev, N, K, M, packed):
    Wg, Sg = orc.synth_w4a16(0x6A7E + N + K, N, K)
    Wu, Su = orc.synth_w4a16(0x0B0B + N + K, N, K)
    X = orc.synth_act(0x5A + M, M, K)
    gw = torch.from_numpy(Wg).to(dev)
    uw = torch.from_numpy(Wu).to(dev)
    gs, us, x = up(dev, Sg, Su, X)
    gs, us, x = gs.view(torch.float16), us.view(torch.float16), x.view(torch.bfloat16)
    if packed:
        gw, uw = w4.repack(gw, gs, N, K), w4.repack(uw, us, N, K)
    g, u, y3 = three_step(w4, gw, gs, uw, us, x, N, K, M, packed)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.swiglu(gw, None if packed else gs, uw, None if packed else us, x, N, K, M, y=y,
              prepacked=packed)
    yf = down(y).reshape(M, N)
    assert np.array_equal(yf, y3.reshape(M, N))
    # and the epilogue is the oracle's silu*mul of the projections' bits
    d = ulp_diff(yf.ravel(), orc.silu_mul_bf16(g.ravel(), u.ravel()))
    assert d.max() <= 1 and (d != 0).sum() <= max(1, d.size // 1000)


@pytest.mark.parametrize("M", [1, 8, 33])
@pytest.mark.parametrize("packed", [False, True])
def test_fused_swiglu_infinite_activation(w4, orc, dev, M, packed):
    """A row of x with an infinity: the fused launch still equals the
    three-step sequence, whose projections give the reference loop's +-Inf /
    NaN outputs (ref_gemv_bf16, tests/cuda/test_int4_gemv_bf16.cpp:54-69)."""
    N, K = 3584, 1024
    Wg, Sg = orc.synth_w4a16(0x1F6A, N, K)
    Wu, Su = orc.synth_w4a16(0x1F6B, N, K)
    X = orc.synth_act(0x1F6C + M, M, K)
    X[M - 1, 300] = 0x7F80  # +Inf
    gw = torch.from_numpy(Wg).to(dev)
    uw = torch.from_numpy(Wu).to(dev)
    gs, us, x = up(dev, Sg, Su, X)
    gs, us, x = gs.view(torch.float16), us.view(torch.float16), x.view(torch.bfloat16)
    if packed:
        gw, uw = w4.repack(gw, gs, N, K), w4.repack(uw, us, N, K)
    g, u, y3 = three_step(w4, gw, gs, uw, us, x, N, K, M, packed)
    ref_g = orc.gemv_bf16(Wg, Sg, X, N, K, M)
    gi = g.reshape(M, N)[M - 1]
    assert np.array_equal(np.isinf(orc.bf16_to_f32(gi)), np.isinf(orc.bf16_to_f32(ref_g[M - 1])))
    assert np.isinf(orc.bf16_to_f32(gi)).sum() > N // 2
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.swiglu(gw, None if packed else gs, uw, None if packed else us, x, N, K, M, y=y,
              prepacked=packed)
    assert np.array_equal(down(y).reshape(M, N), y3.reshape(M, N))


def test_fused_swiglu_rejects_bad_input(w4, dev):
    x = torch.zeros((1, 1024), dtype=torch.bfloat16, device=dev)
    w = torch.zeros(512 * 512, dtype=torch.uint8, device=dev)
    s = torch.zeros(512 * 8, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):
        w4.swiglu(w, s, w, s, x, 512, 1000, 1)  # K % 128 != 0
    with pytest.raises(ValueError):
        w4.swiglu(w[1:], s, w, s, x, 512, 1024, 1)  # misaligned weight
