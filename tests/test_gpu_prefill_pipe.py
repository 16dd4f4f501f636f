"""The opt-in pipelined prefill GEMM (w4a16_gemm.hip, selected by
CUDALM_W4A16_GEMM_CFG = 50 / 51, read once per process): run in a child
process with the setting, on K = 1024 shapes (the only K it serves) at
several M, both weight layouts. Its outputs must equal the tile kernel's
bit for bit (the per-output operation sequence every kernel shares) and be
within the oracle's bound."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
import numpy as np
import torch
sys.path[:0] = [{repo!r}, {pkg!r}]
import cudalm_w4a16 as w4
import oracle
dev = torch.device("cuda:0")
for N, M in ((3584, 512), (1000, 70), (16, 33), (2048, 129)):
    K = 1024
    W, S = oracle.synth_w4a16(0x919E + N + M, N, K)
    X = oracle.synth_act(0x919F + M, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv(w, s, x, N, K, M, y=y, variant="prefill")
    yt = torch.empty_like(y)
    w4.gemv(w, s, x, N, K, M, y=yt, variant="tile32")
    p = w4.repack(w, s, N, K)
    yp = torch.empty_like(y)
    w4.gemv_prepacked(p, x, N, K, M, y=yp, variant="prefill")
    torch.cuda.synchronize()
    Y = y.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(Y, yt.view(torch.int16).cpu().numpy().view(np.uint16)), ("tile32", N, M)
    assert np.array_equal(Y, yp.view(torch.int16).cpu().numpy().view(np.uint16)), ("prepacked", N, M)
    ok, st = oracle.check_tolerance(Y, W, S, X, N, K, M)
    assert ok, (N, M, st)
    print("pipe", N, K, M, st["max_ulp"], flush=True)
print("child ok", flush=True)
"""


@pytest.mark.parametrize("cfg", ["50", "51"])
def test_pipelined_prefill_gemm(cfg):
    env = dict(os.environ, CUDALM_W4A16_GEMM_CFG=cfg)
    code = CHILD.format(repo=REPO, pkg=os.path.join(REPO, "cudalm-agent_amd"))
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=180)
    print(res.stdout + res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "child ok" in res.stdout
