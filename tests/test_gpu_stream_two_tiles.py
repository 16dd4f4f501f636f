"""The stream kernel with two 16-row activation tiles (17 <= M <= 32, one
projection) on the LM head and census-like shapes: prepacked and file
layout equal the tile kernel bit for bit (the per-output operation sequence
every kernel shares) and are within the oracle's bound; the
fp16-activation twin through the same kernel, both layouts."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 32), (248320, 32), (1024, 32), (4096, 24), (1000, 17)]  # (N, M), K = 1024


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("N,M", SHAPES)
def test_two_tile_stream(w4, orc, dev, N, M):
    K = 1024
    W, S = orc.synth_w4a16(0x5A1 + N + M, N, K)
    X = orc.synth_act(0x5A2 + M, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv_prepacked(w4.repack(w, s, N, K), x, N, K, M, y=y)
    yf = torch.empty_like(y)
    w4.gemv(w, s, x, N, K, M, y=yf)
    yt = torch.empty_like(y)
    w4.gemv(w, s, x, N, K, M, y=yt, variant="tile32")
    torch.cuda.synchronize()
    Y = _bits(y)
    assert np.array_equal(Y, _bits(yt)), ("tile32", N, M)
    assert np.array_equal(Y, _bits(yf)), ("file layout", N, M)
    if N <= 4096:
        ok, st = orc.check_tolerance(Y, W, S, X, N, K, M)
        assert ok, (N, M, st)
        print(f"  two-tile stream N={N} M={M}: max {st['max_ulp']:.3f} ulp", flush=True)


def test_two_tile_stream_f16(w4, orc, dev):
    N, K, M = 4096, 1024, 32
    W, S = orc.synth_w4a16(0x5F16, N, K)
    rng = np.random.default_rng(0x5F16)
    X = rng.normal(0, 1, (M, K)).astype(np.float16).view(np.uint16)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.float16)
    y_file = w4.gemv_f16(w, s, x, N, K, M)
    y_packed = w4.gemv_f16_prepacked(w4.repack(w, s, N, K), x, N, K, M)
    torch.cuda.synchronize()
    Yf = _bits(y_file).reshape(M, N)
    Yp = _bits(y_packed).reshape(M, N)
    assert np.array_equal(Yp, Yf)
    ok, st = orc.check_f16_tolerance(Yp, W, S, X, N, K, M)
    assert ok, st
