"""Pins the SwiGLU element-wise oracle (oracle/swiglu_oracle.c): SiLU
rounded to bf16 against the fp64 SiLU over every bf16 input, and the
product against the exact fp64 product rounded once
(src/kernels/qwen35_kernels.cu:458-476)."""
import numpy as np
import torch


def _f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _bf16_of_f64(v):
    # round-to-nearest-even of fp64 values to bf16 via an exact two-step
    # (fp64 -> fp32 can double-round, so ties are excluded by the caller)
    return torch.from_numpy(np.asarray(v, np.float64)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_silu_all_bf16_inputs(orc):
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    gf = _f32(g).astype(np.float64)
    finite = np.isfinite(gf)
    with np.errstate(over="ignore", invalid="ignore"):
        exact = gf / (1.0 + np.exp(-gf))
    got = orc.silu_bf16(g)
    want = _bf16_of_f64(exact)
    # distance of the exact value from the nearest bf16 rounding boundary,
    # in units of the bf16 spacing: cases within 2^-12 of a tie may round
    # either way under a correctly implemented fp32 expf
    spacing = orc.bf16_ulp(exact)
    frac = np.abs(exact) / spacing
    near_tie = np.abs(frac - np.floor(frac) - 0.5) < 2.0 ** -12
    # fp32 semantics: for g < -88.72, expf(-g) overflows to +inf and the
    # quotient is -0 (the reference evaluates the same fp32 expression)
    overflow = finite & (gf < -88.72283935546875)
    assert np.all(got[overflow] == 0x8000)
    ok = finite & ~near_tie & np.isfinite(exact) & ~overflow
    assert np.array_equal(got[ok], want[ok])
    assert ok.sum() > 45000  # NaNs and the overflow range are checked separately
    # closed forms: silu(0) = 0, silu(-0) = -0, silu(+inf) = +inf, silu(-inf) = -0 or NaN-free
    assert orc.silu_bf16(np.array([0x0000], np.uint16))[0] == 0x0000
    assert orc.silu_bf16(np.array([0x7F80], np.uint16))[0] == 0x7F80
    # large negative g: silu underflows toward -0
    assert _f32(orc.silu_bf16(np.array([0xC2C8], np.uint16)))[0] <= 0.0  # g = -100


def test_silu_mul_product_rounds_once(orc):
    rng = np.random.default_rng(5)
    g = orc.f32_to_bf16(rng.normal(0, 3, 20000).astype(np.float32))
    u = orc.f32_to_bf16(rng.normal(0, 1, 20000).astype(np.float32))
    y = orc.silu_mul_bf16(g, u)
    s = _f32(orc.silu_bf16(g)).astype(np.float64)
    prod = s * _f32(u).astype(np.float64)  # exact: 8-bit x 8-bit significands
    assert np.array_equal(y, orc.f32_to_bf16(prod.astype(np.float32)))
    # sign symmetry in u and the zero cases
    assert np.array_equal(orc.silu_mul_bf16(g, u ^ np.uint16(0x8000))[y & 0x7FFF != 0],
                          (y ^ np.uint16(0x8000))[y & 0x7FFF != 0])
    assert not (orc.silu_mul_bf16(g, np.zeros_like(u)) & 0x7FFF).any()
