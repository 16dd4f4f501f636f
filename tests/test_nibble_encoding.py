"""Weight-element encodings of the MFMA kernels (w4a16_kernels.hip: decode_nibbles,
ActF16::decode, prepack_dword), checked against the values they must equal.

The file format stores signed int4 q in two's complement, low nibble first
(element 2b in the low nibble of byte b: src/kernels/int4_gemv.cu:38-42), so
element k of a little-endian dword sits at bits 4k. The kernels turn each dword
into 4 pairs (k, k + 4) of 16-bit values equal to c + q/u exactly: bf16
c = 1.5, u = 16 (nibble at mantissa bits 3..6); fp16 c = 1.5, u = 16 (nibble
at mantissa bits 6..9). The bit operations below are the
kernels' shift / mask / xor steps; the expected values come from the int4
definition, so a wrong shift, mask or constant fails here.
"""
import numpy as np
import pytest

# kind -> (mask, xor constant, c, u)
ENC = {"bf16": (0x00780078, 0x3FC03FC0, 1.5, 16.0), "f16": (0x03C003C0, 0x3E003E00, 1.5, 16.0)}


def _rotr(w, s):
    w = np.uint64(w)
    return int(((w >> np.uint64(s)) | (w << np.uint64(32 - s))) & np.uint64(0xFFFFFFFF)) if s else int(w)


def _half_value(h, kind):
    h = np.uint16(h)
    if kind == "bf16":
        return float(np.frombuffer((np.uint32(h) << np.uint32(16)).tobytes(), np.float32)[0])
    return float(np.frombuffer(h.tobytes(), np.float16)[0])


def _decode(w, kind, prepacked):
    mask, xor = ENC[kind][0], ENC[kind][1]
    if prepacked:
        p = ((w << 3) | (w >> 29)) & 0xFFFFFFFF  # prepack_dword
        rot = {"bf16": (0, 4, 8, 12), "f16": (29, 1, 5, 9)}[kind]
        src = [_rotr(p, r) for r in rot]
    elif kind == "bf16":
        src = [(w << 3) & 0xFFFFFFFF, w >> 1, w >> 5, w >> 9]
    else:
        src = [(w << 6) & 0xFFFFFFFF, (w << 2) & 0xFFFFFFFF, w >> 2, w >> 6]
    return [(s & mask) ^ xor for s in src]


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("prepacked", [False, True])
def test_pairs_equal_c_plus_q_over_u(kind, prepacked):
    _, _, c, u = ENC[kind]
    rng = np.random.default_rng(7)
    words = [0, 0xFFFFFFFF, 0x88888888, 0x77777777, 0x76543210, 0xFEDCBA98]
    words += [int(v) for v in rng.integers(0, 2**32, 500, dtype=np.uint64)]
    for w in words:
        q = [((w >> (4 * k)) & 0xF) - 16 * (((w >> (4 * k)) & 0xF) >= 8) for k in range(8)]
        for p, d in enumerate(_decode(w, kind, prepacked)):
            lo, hi = d & 0xFFFF, d >> 16
            assert _half_value(lo, kind) == c + q[p] / u, (hex(w), p)
            assert _half_value(hi, kind) == c + q[p + 4] / u, (hex(w), p)


@pytest.mark.parametrize("kind,neg", [("bf16", 0xBFC0), ("f16", 0xBE00)])
def test_offset_constant_is_minus_c(kind, neg):
    assert _half_value(neg, kind) == -ENC[kind][2]
