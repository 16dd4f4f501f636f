"""The two pair stream kernels (17 <= M <= 32, one prepacked projection):
the counted kernel (K = 1024, M = 32, N % 32 == 0: fixed memory operations
per step, its own waits) and the general pair kernel, which serves every
other shape and, with CUDALM_W4A16_STREAM_PAIR_COUNTED=0 (read once per
process), the counted kernel's shapes too. The general kernel runs in a
child process; both must equal the tile kernel bit for bit (the per-output
operation sequence every kernel shares), and the counted kernel's output
must be within the oracle's bound."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHAPES = [(4096, 32), (248320, 32), (1024, 32), (4096, 24)]  # (N, M), K = 1024

CHILD = r"""
import sys
import numpy as np
import torch
sys.path[:0] = [{repo!r}, {pkg!r}]
import cudalm_w4a16 as w4
import oracle
dev = torch.device("cuda:0")
for N, M in {shapes!r}:
    K = 1024
    W, S = oracle.synth_w4a16(0x5A1 + N + M, N, K)
    X = oracle.synth_act(0x5A2 + M, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    p = w4.repack(w, s, N, K)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv_prepacked(p, x, N, K, M, y=y)
    torch.cuda.synchronize()
    np.save({out!r} + f"/y_{{N}}_{{M}}.npy", y.view(torch.int16).cpu().numpy().view(np.uint16))
print("child ok", flush=True)
"""


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_counted_and_general_pair_kernels(w4, orc, dev, tmp_path):
    env = dict(os.environ, CUDALM_W4A16_STREAM_PAIR_COUNTED="0")
    code = CHILD.format(repo=REPO, pkg=os.path.join(REPO, "cudalm-agent_amd"), shapes=SHAPES,
                        out=str(tmp_path))
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=240)
    print(res.stdout + res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "child ok" in res.stdout
    for N, M in SHAPES:
        K = 1024
        W, S = orc.synth_w4a16(0x5A1 + N + M, N, K)
        X = orc.synth_act(0x5A2 + M, M, K)
        w = torch.from_numpy(W).to(dev)
        s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
        x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
        p = w4.repack(w, s, N, K)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.gemv_prepacked(p, x, N, K, M, y=y)
        yt = torch.empty_like(y)
        w4.gemv(w, s, x, N, K, M, y=yt, variant="tile32")
        torch.cuda.synchronize()
        Y = _bits(y)
        assert np.array_equal(Y, _bits(yt)), ("tile32", N, M)
        assert np.array_equal(Y, np.load(tmp_path / f"y_{N}_{M}.npy")), ("general pair kernel", N, M)
        if N <= 4096:
            ok, st = orc.check_tolerance(Y, W, S, X, N, K, M)
            assert ok, (N, M, st)
            print(f"  pair kernels N={N} M={M}: equal, max {st['max_ulp']:.3f} ulp", flush=True)
        del w, s, x, p, y, yt


def test_counted_pair_kernel_f16(w4, orc, dev):
    """The fp16-activation twin through the counted kernel (prepacked, K = 1024,
    M = 32, N % 32 == 0) equals the file-layout launch (the general pair
    kernel) bit for bit and is within the fp16 oracle bound."""
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
    Yf = y_file.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
    Yp = y_packed.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
    assert np.array_equal(Yp, Yf)
    ok, st = orc.check_f16_tolerance(Yp, W, S, X, N, K, M)
    assert ok, st
