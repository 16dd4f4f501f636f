"""Pins the CPU oracle (oracle/w4a16_oracle.c) before it is trusted as the
checker of the HIP kernels. Each check is independent of the oracle's own
code: exhaustive tables, IEEE conversions done by numpy / torch, the
reference's own compiled stage_compare.h (oracle/_ref), closed forms and
brute force on tiny shapes, and the quantization invariants of
tests/cpu/test_weights_crosslang.cpp:58-100 in the reference.
"""
import os

import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- int4 ------

def test_unpack_exhaustive_256(orc):
    # weight_loader.h:106-117: lo = sext4(b & 0xF) (k = 2b), hi = sext4(b >> 4)
    for b in range(256):
        lo, hi = orc.unpack_byte(b)
        exp_lo = (b & 0xF) - 16 if (b & 0xF) >= 8 else (b & 0xF)
        exp_hi = (b >> 4) - 16 if (b >> 4) >= 8 else (b >> 4)
        assert (lo, hi) == (exp_lo, exp_hi), b


def test_pack_unpack_roundtrip_full_domain(orc):
    # tests/cpu/test_weight_file.cpp:212-225
    for lo in range(-8, 8):
        for hi in range(-8, 8):
            assert orc.unpack_byte(orc.pack_byte(lo, hi)) == (lo, hi)


def test_unpack_array_matches_numpy(orc):
    rng = np.random.default_rng(1)
    N, K = 7, 256
    W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    q = orc.unpack(W, N, K)
    lo = (W & 0xF).astype(np.int16)
    hi = (W >> 4).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    exp = np.stack([lo, hi], axis=-1).reshape(N, K)
    assert np.array_equal(q.astype(np.int16), exp)


# ---------------------------------------------------------------- formats ---

def test_fp16_decode_all_patterns_vs_numpy(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ours = orc.fp16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_decode_all_patterns_vs_reference_code(orc):
    # oracle/_ref is the reference's own stage_compare.h fp16_bits_to_f32
    if orc.ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ours = orc.fp16_to_f32(np.arange(65536, dtype=np.uint16)).view(np.uint32)
    for h in range(65536):
        assert orc.ref.fp16_to_f32_bits(h) == ours[h], hex(h)


def _edge_f32_patterns():
    e = [0x00000000, 0x80000000, 0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000, 0x477FE000,
         0x477FF000, 0x477FEFFF, 0x47800000, 0x33800000, 0x33000000, 0x33000001, 0x387FC000,
         0x38800000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x3F808000, 0x3F818000, 0x3F807FFF,
         0x3F808001, 0x7F7F8000, 0x7F7FFFFF]
    return np.array(e, dtype=np.uint32)


def test_f32_to_fp16_rne_vs_numpy(orc):
    rng = np.random.default_rng(2)
    pats = np.concatenate([rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                           _edge_f32_patterns()])
    f = pats.view(np.float32)
    ours = orc.f32_to_fp16(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))


def test_f32_to_bf16_rne_vs_torch(orc):
    rng = np.random.default_rng(3)
    pats = np.concatenate([rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                           _edge_f32_patterns()])
    f = pats.view(np.float32)
    ours = orc.f32_to_bf16(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(orc.bf16_to_f32(ours[nan])))


def test_dequant_all_q_all_finite_scales(orc):
    # w = q * f32(s) (w4a16_quant.py:74-82) is exact in fp32: check all 16 q
    # against numpy float32 products for every finite fp16 scale.
    sbits = np.arange(65536, dtype=np.uint16)
    sf = sbits.view(np.float16).astype(np.float32)
    sbits = sbits[np.isfinite(sf)]
    G = sbits.size // 1  # one scale per group: N rows of K = 128
    W = np.empty((G, 64), np.uint8)
    q = np.arange(-8, 8)
    # 128 elements per group: q pattern repeated 8 times (lo = even k, hi = odd k)
    qq = np.tile(q, 8)
    W[:] = ((qq[1::2] & 0xF) << 4 | (qq[0::2] & 0xF)).astype(np.uint8)
    out = orc.dequant(W, sbits.reshape(G, 1), G, 128)
    exp = qq[None, :].astype(np.float32) * sbits.view(np.float16).astype(np.float32)[:, None]
    assert np.array_equal(out.view(np.uint32), exp.astype(np.float32).view(np.uint32))


# ---------------------------------------------------------------- quantizer --

def _torch_quantize(Wf: np.ndarray):
    """docs/weight_format.md:135-153 restated with torch ops."""
    W = torch.from_numpy(Wf).float()
    N, K = W.shape
    Wg = W.view(N, K // 128, 128)
    amax = Wg.abs().amax(dim=2)
    s32 = amax / 7
    zero = s32 == 0
    safe = torch.where(zero, torch.ones_like(s32), s32)
    q = torch.round(Wg / safe.unsqueeze(2)).clamp(-7, 7)
    q = torch.where(zero.unsqueeze(2), torch.zeros_like(q), q).view(N, K).to(torch.int32)
    lo = q[:, 0::2] & 15
    hi = q[:, 1::2] & 15
    Wp = ((hi << 4) | lo).to(torch.uint8).numpy()
    S = s32.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    return Wp, S


def test_quantizer_matches_torch_restatement(orc):
    Wf = orc.synth_normal(0xC0DA0000, 0.02, 64 * 1024).reshape(64, 1024)
    Wf[3, 128:256] = 0.0  # a zero group
    Wf[5, 0] = 0.5        # an outlier
    Wp, S = orc.quantize(Wf)
    Wp2, S2 = _torch_quantize(Wf)
    assert np.array_equal(Wp, Wp2)
    assert np.array_equal(S, S2)


def test_quantizer_domain_invariants(orc):
    # tests/cpu/test_weights_crosslang.cpp:58-100: nibbles in [-7, 7];
    # scale > 0 => max|q| == 7; scale == 0 => q == 0
    Wf = orc.synth_normal(7, 0.02, 32 * 1024).reshape(32, 1024)
    Wf[0, :128] = 0.0
    Wp, S = orc.quantize(Wf)
    q = orc.unpack(Wp, 32, 1024).reshape(32, 8, 128).astype(np.int32)
    s = orc.fp16_to_f32(S)
    assert q.min() >= -7 and q.max() <= 7
    amax = np.abs(q).max(axis=2)
    assert np.all(amax[s > 0] == 7)
    assert np.all(np.abs(q[s == 0]).max(axis=-1) == 0)
    assert s[0, 0] == 0.0


def test_quantizer_rejects_bad_input(orc):
    with pytest.raises(ValueError):
        orc.quantize(np.zeros((2, 100), np.float32))
    bad = np.zeros((1, 128), np.float32)
    bad[0, 5] = np.inf
    with pytest.raises(ValueError):
        orc.quantize(bad)


# ---------------------------------------------------------------- gemv ------

def _numpy_sequential_acc(W, S, X, N, K):
    """fp32 accumulator, k ascending, lo before hi, each term (q*s)*x."""
    f32 = np.float32
    out = np.empty(N, np.float32)
    xs = (X.astype(np.uint32) << 16).view(np.float32).ravel()
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
    return out


def _numpy_sequential_gemv(W, S, X, N, K):
    """The same, then bf16 RNE."""
    out = _numpy_sequential_acc(W, S, X, N, K)
    return torch.from_numpy(out).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("N,K,seed", [(1, 128, 1), (3, 128, 0x51ed), (5, 256, 9), (2, 384, 77)])
def test_gemv_bruteforce_bitexact(orc, N, K, seed):
    W, S, X = orc.fixture_gemv(seed, N, K)
    y = orc.gemv_bf16(W, S, X, N, K, 1)[0]
    assert np.array_equal(y, _numpy_sequential_gemv(W, S, X, N, K))


@pytest.mark.parametrize("N,K,seed", [(1, 128, 1), (3, 128, 0x51ed), (5, 256, 9), (2, 384, 77)])
def test_gemv_f32acc_bruteforce_bitexact(orc, N, K, seed):
    """The fp32-accumulated reference: the loop's accumulator, bit for bit."""
    W, S, X = orc.fixture_gemv(seed, N, K)
    acc = orc.gemv_f32acc(W, S, X, N, K, 1)[0]
    assert np.array_equal(acc.view(np.uint32), _numpy_sequential_acc(W, S, X, N, K).view(np.uint32))


@pytest.mark.parametrize("N,K,M", [(37, 256, 3), (64, 1024, 1), (16, 3584, 2), (1000, 1024, 4)])
def test_gemv_f32acc_rounds_to_reference(orc, N, K, M):
    """bf16_rne(accumulator) is the reference loop's output at every shape,
    single- and multi-threaded; ulp_vs_fp32_reference of the loop's own
    output is at most 0.5 ulp (one rounding), and a one-ulp shift of every
    output is seen as 0.5 to 1.5 ulp (2.5 where the output crosses a power
    of two: a step above it is two ulps of an accumulator just below it)."""
    W, S, _ = orc.fixture_gemv(N * 7 + K, N, K)
    X = orc.synth_act(N + K + M, M, K)
    acc1 = orc.gemv_f32acc(W, S, X, N, K, M, 1)
    acc8 = orc.gemv_f32acc(W, S, X, N, K, M, 8)
    assert np.array_equal(acc1.view(np.uint32), acc8.view(np.uint32))
    y = orc.gemv_bf16(W, S, X, N, K, M)
    assert np.array_equal(orc.f32_to_bf16(acc1), y)
    st = orc.ulp_vs_fp32_reference(y, acc1)
    assert st["max_ulp_vs_fp32_ref"] <= 0.5 + 1e-9 and st["n_over_2ulp_vs_fp32_ref"] == 0
    # move every nonzero output one bf16 step away from zero: 0.5..1.5 ulp
    nz = (y & 0x7FFF) != 0
    y2 = np.where(nz & ((y & 0x7F80) != 0x7F80), y + 1, y).astype(np.uint16)
    st2 = orc.ulp_vs_fp32_reference(y2, acc1)
    assert 0.5 <= st2["max_ulp_vs_fp32_ref"] <= 2.5 + 1e-9
    assert st2["n_over_2ulp_vs_fp32_ref"] <= nz.sum() // 50


@pytest.mark.parametrize("N,K", [(37, 256), (64, 1024), (16, 3584)])
def test_gemv_within_fp64_bound(orc, N, K):
    W, S, X = orc.fixture_gemv(N * 31 + K, N, K)
    y = orc.gemv_bf16(W, S, X, N, K, 1)
    ok, st = orc.check_tolerance(y, W, S, X, N, K, 1, ulps=1.0)
    assert ok, st
    # against numpy's fp64 matmul of the dequantized weights
    w = orc.dequant(W, S, N, K).astype(np.float64)
    r = w @ orc.bf16_to_f32(X[0]).astype(np.float64)
    yf = orc.bf16_to_f32(y[0]).astype(np.float64)
    assert np.all(np.abs(yf - r) <= orc.bf16_ulp(r) + 1e-6)


def test_gemv_closed_forms(orc):
    N, K = 9, 256
    W, S, X = orc.fixture_gemv(5, N, K)
    # zero row -> exact zero (test_int4_gemv_bf16.cpp:146-176)
    W0 = W.copy()
    W0[4] = 0
    y = orc.gemv_bf16(W0, S, X, N, K)[0]
    assert y[4] == 0
    # one-hot x: y[n] = bf16(q[n,k] * s[n, k/128]) exactly
    k = 131
    Xh = np.zeros_like(X)
    Xh[0, k] = orc.f32_to_bf16(np.array([1.0], np.float32))[0]
    y = orc.gemv_bf16(W, S, Xh, N, K)[0]
    q = orc.unpack(W, N, K)[:, k].astype(np.float32)
    s = orc.fp16_to_f32(S[:, k // 128])
    assert np.array_equal(y, orc.f32_to_bf16(q * s))
    # sign flip of x negates every output bit-exactly
    Xn = X ^ np.uint16(0x8000)
    yp = orc.gemv_bf16(W, S, X, N, K)[0]
    yn = orc.gemv_bf16(W, S, Xn, N, K)[0]
    nz = (yp & 0x7FFF) != 0
    assert np.array_equal(yn[nz], yp[nz] ^ np.uint16(0x8000))
    # doubling x doubles y exactly (power-of-two scaling commutes with rounding)
    X2 = orc.f32_to_bf16(orc.bf16_to_f32(X) * 2)
    y2 = orc.gemv_bf16(W, S, X2, N, K)[0]
    assert np.array_equal(orc.bf16_to_f32(y2), orc.bf16_to_f32(yp) * 2)


def test_gemv_batch_rows_equal_single_rows(orc):
    N, K, B = 33, 512, 3
    W, S, X = orc.fixture_kind("mixed_sign", 0x1234ABCD, N, K, B)
    Y = orc.gemv_bf16(W, S, X, N, K, B)
    for b in range(B):
        assert np.array_equal(Y[b], orc.gemv_bf16(W, S, X[b:b + 1].copy(), N, K, 1)[0])


def test_gemv_multithread_bitidentical(orc):
    N, K = 1000, 1024
    W, S, X = orc.fixture_gemv(11, N, K)
    assert np.array_equal(orc.gemv_bf16(W, S, X, N, K, 1, nthreads=1),
                          orc.gemv_bf16(W, S, X, N, K, 1, nthreads=8))


def test_tolerance_implies_reference_comparator(orc):
    # An output inside our 2-ulp gate must also pass the reference's own
    # compare_bf16_stages (atol = rtol = 1e-2, stage_compare.h:117-137).
    if orc.ref is None:
        pytest.skip("oracle/_ref not built")
    N, K = 512, 1024
    W, S, X = orc.fixture_gemv(3, N, K)
    y = orc.gemv_bf16(W, S, X, N, K)
    ok, _ = orc.check_tolerance(y, W, S, X, N, K, 1)
    assert ok
    r, _ = orc.gemv_f64(W, S, X, N, K, 1)
    rb = orc.f32_to_bf16(r.astype(np.float32))
    ok_ref, mx, _ = orc.ref.compare_bf16_stages(rb, y)
    assert ok_ref, mx


def test_tolerance_rejects_wrong_answers(orc):
    N, K = 64, 1024
    W, S, X = orc.fixture_gemv(8, N, K)
    y = orc.gemv_bf16(W, S, X, N, K)
    # one wrong nibble (off by 8, at the largest |x|) must fail the gate
    xf = orc.bf16_to_f32(X[0])
    b = int(np.argmax(np.abs(xf[0::2])))
    W2 = W.copy()
    W2[10, b] ^= 0x08
    y2 = orc.gemv_bf16(W2, S, X, N, K)
    ok, st = orc.check_tolerance(y2, W, S, X, N, K, 1)
    assert not ok and st["n_bad"] >= 1
    # wrong group scale index fails
    S2 = S.copy()
    S2[:, [0, 1]] = S2[:, [1, 0]]
    ok, _ = orc.check_tolerance(orc.gemv_bf16(W, S2, X, N, K), W, S, X, N, K, 1)
    assert not ok
    # a 3-ulp perturbation fails, a 1-ulp one passes
    ok, _ = orc.check_tolerance(y + np.uint16(1), W, S, X, N, K, 1)
    assert ok
    big = np.abs(orc.bf16_to_f32(y)) > 1e-3
    y3 = y.copy()
    y3[big] += np.uint16(4)
    ok, _ = orc.check_tolerance(y3, W, S, X, N, K, 1)
    assert not ok


# ---------------------------------------------------------------- fixtures --

def test_xorshift32_known_answers(orc):
    # Marsaglia 2003, xorshift32 (13, 17, 5): from seed 1 the first outputs
    # are 270369, 67634689, 2647435461.
    assert list(orc.xorshift32(1, 3)) == [270369, 67634689, 2647435461]
    # seed 0 is replaced by 0x9e3779b9 (test_int4_gemv_bf16.cpp:34)
    assert np.array_equal(orc.xorshift32(0, 5), orc.xorshift32(0x9E3779B9, 5))


def test_fixture_ranges(orc):
    W, S, X = orc.fixture_gemv(0x51ed51, 64, 1024)
    s = orc.fp16_to_f32(S)
    assert s.min() >= 0.00099 and s.max() < 0.0211
    x = orc.bf16_to_f32(X)
    assert x.min() >= -1.0 and x.max() <= 1.0
    for kind in range(5):
        W, S, X = orc.fixture_kind(kind, 0xCAFEBABE, 32, 256, 2)
        q = orc.unpack(W, 32, 256)
        if kind == orc.KIND_ZERO:
            assert not q.any() and not X.any()
        if kind == orc.KIND_SMALL:
            assert q.min() >= 0 and q.max() <= 2
            assert np.abs(orc.bf16_to_f32(X)).max() <= 0.00501
        if kind == orc.KIND_BOUNDARY:
            assert set(np.unique(q)) <= {7, -7, -8, 0, -1}
            assert (S == 0).any()


def test_synthetic_normal_moments(orc):
    x = orc.synth_normal(42, 0.02, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 1e-4
    assert abs(x.std() - 0.02) < 2e-4
    # element i depends only on (seed, i): threads do not change the stream
    y = orc.synth_normal(42, 0.02, 1000)
    assert np.array_equal(x[:1000].astype(np.float32), y)


# ---------------------------------------------------------------- goldens ---

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "w4a16_golden.npz")


def test_golden_vectors_reproduce(orc):
    g = np.load(GOLDEN)
    names = sorted({k.rsplit("__", 1)[0] for k in g.files})
    assert names
    for name in names:
        N, K, M = (int(v) for v in g[name + "__shape"])
        W, S, X, Y = (g[name + "__" + f] for f in ("W", "S", "X", "Y"))
        assert np.array_equal(orc.gemv_bf16(W, S, X, N, K, M), Y), name
