"""The 32 x 32 MFMA prefill GEMM (w4a16_gemm.hip), forced with
CUDALM_W4A16_VARIANT_PREFILL32 on census shapes and ragged ones (N not a
multiple of 32 or of 256, M not a multiple of 32, a short last 8-group
unit, K spanning several units, file-layout scale rows not 16 B aligned),
both weight layouts. Outputs must equal the tile kernel's bit for bit (the
per-output operation sequence every kernel shares: each 16 x 16 x 32 MFMA
step equals two 32 x 32 x 16 steps over its k-block halves) and be within
the oracle's bound (the restatement of tests/cuda/test_int4_gemv_bf16.cpp:
54-69). Every row equals the single-row call on it. At K = 1024 the
split kernel runs with wave sets of 8 (3584 x 512, 1000 x 70), 2
(2048 x 129) and 4 (2000 x 500) waves on a 256-CU part."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("N,K,M", [(3584, 1024, 512), (4096, 1024, 512), (1000, 1024, 70),
                                   (16, 1024, 33), (2048, 1024, 129), (1024, 3584, 100),
                                   (1024, 2048, 64), (37, 384, 40), (300, 2176, 97),
                                   (1, 128, 33), (257, 1024, 1), (2000, 1024, 500)])
def test_prefill32_bit_identity(w4, orc, dev, N, K, M):
    W, S = orc.synth_w4a16(0x919E + N + M + K, N, K)
    X = orc.synth_act(0x919F + M, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv(w, s, x, N, K, M, y=y, variant="prefill32")
    yt = torch.empty_like(y)
    w4.gemv(w, s, x, N, K, M, y=yt, variant="tile32")
    p = w4.repack(w, s, N, K)
    yp = torch.empty_like(y)
    w4.gemv_prepacked(p, x, N, K, M, y=yp, variant="prefill32")
    Y = _bits(y).reshape(M, N)
    assert np.array_equal(Y, _bits(yt).reshape(M, N)), ("tile32", N, K, M)
    assert np.array_equal(Y, _bits(yp).reshape(M, N)), ("prepacked", N, K, M)
    ok, st = orc.check_tolerance(Y, W, S, X, N, K, M)
    print(f"  prefill32 N={N} K={K} M={M}: {st}", flush=True)
    assert ok, st
    for b in sorted({0, M // 2, M - 1}):
        y1 = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
        w4.gemv(w, s, x[b:b + 1], N, K, 1, y=y1)
        assert np.array_equal(Y[b], _bits(y1).reshape(N)), b


@pytest.mark.parametrize("N,M", [(3584, 512), (2000, 500), (2048, 129), (1000, 40)])
def test_prefill_scale_base_not_8_aligned(w4, orc, dev, N, M):
    # file-layout scales whose base is 2 bytes past an 8-byte boundary: the
    # K = 1024 split kernel (wave sets of 8, 4 and 2 waves; the last shape
    # takes the unit GEMM) reads them one at a time instead of 8 bytes per
    # row. Same bits as with aligned scales, for the shape's dispatch and the
    # forced 32x32 variant.
    K = 1024
    W, S = orc.synth_w4a16(0x5CA1 + N + M, N, K)
    X = orc.synth_act(0x5CA2 + M, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    buf = torch.empty(N * (K // 128) + 4, dtype=torch.float16, device=dev)
    s_mis = buf[1:1 + N * (K // 128)].view(N, K // 128)
    s_mis.copy_(s)
    assert s_mis.data_ptr() % 8 != 0
    for variant in ("auto", "prefill32"):
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.gemv(w, s, x, N, K, M, y=y, variant=variant)
        ym = torch.empty_like(y)
        w4.gemv(w, s_mis, x, N, K, M, y=ym, variant=variant)
        assert np.array_equal(_bits(y), _bits(ym)), (variant, N, M)
    yt = torch.empty_like(y)
    w4.gemv(w, s, x, N, K, M, y=yt, variant="tile32")
    assert np.array_equal(_bits(ym), _bits(yt)), ("tile32", N, M)
