"""The measurement overrides (environment variables read once per process)
select other kernels, grids or fetch granularities for the same launches;
none may change a result bit. Each setting runs in a child process over
the same inputs (single projections at M = 1, 8, 17 and 32 through the
prepacked and file-layout entries, a fused multi-projection launch, and a
prefill chunk); every output must equal the default process's."""
import os
import subprocess
import sys

import numpy as np
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
out = {{}}
def run(tag, N, K, M, seed):
    W, S = oracle.synth_w4a16(seed, N, K)
    X = oracle.synth_act(seed + 1, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    p = w4.repack(w, s, N, K)
    yp = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv_prepacked(p, x, N, K, M, y=yp)
    yf = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv(w, s, x, N, K, M, y=yf)
    torch.cuda.synchronize()
    out[tag + "_p"] = yp.view(torch.int16).cpu().numpy()
    out[tag + "_f"] = yf.view(torch.int16).cpu().numpy()
for M in (1, 8, 17, 32):
    run(f"lm{{M}}", 40000, 1024, M, 0xE0 + M)
run("k2048", 1024, 2048, 8, 0xE9)
run("prefill", 2048, 1024, 96, 0xEA)
# fused launch of three projections sharing x (the q/k/v shape group)
projs = []
for j, N in enumerate((4096, 512, 512)):
    W, S = oracle.synth_w4a16(0xF0 + j, N, 1024)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    projs.append((w4.repack(w, s, N, 1024), N))
X = oracle.synth_act(0xF9, 8, 1024)
x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
ys = w4.gemv_multi([p for p, _ in projs], [None] * 3, x, [N for _, N in projs], 1024, 8,
                   prepacked=True)
torch.cuda.synchronize()
for j, y in enumerate(ys):
    out[f"multi{{j}}"] = y.view(torch.int16).cpu().numpy()
np.savez({path!r}, **out)
print("child ok", flush=True)
"""

SETTINGS = [
    {},
    {"CUDALM_W4A16_STREAM_PIECE": "0"},
    {"CUDALM_W4A16_STREAM_PIECE": "2"},
    {"CUDALM_W4A16_STREAM_WGS_PER_CU": "2"},
    {"CUDALM_W4A16_STREAM_TAIL": "150"},
    {"CUDALM_W4A16_STREAM_PAIR": "0"},
    {"CUDALM_W4A16_STREAM_PAIR": "4"},
    {"CUDALM_W4A16_PROJ_ONE": "0"},
    {"CUDALM_W4A16_GEMM_CFG": "23"},
    {"CUDALM_W4A16_GEMM_CFG": "9"},
]


def _child(env_extra, path):
    env = dict(os.environ, **env_extra)
    code = CHILD.format(repo=REPO, pkg=os.path.join(REPO, "cudalm-agent_amd"), path=path)
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0 and "child ok" in res.stdout, (env_extra, res.stdout + res.stderr[-2000:])


def test_overrides_never_change_results(tmp_path):
    ref = None
    for k, extra in enumerate(SETTINGS):
        path = str(tmp_path / f"o{k}.npz")
        print(f"  overrides {extra or 'default'}", flush=True)
        _child(extra, path)
        got = np.load(path)
        if ref is None:
            ref = {n: got[n] for n in got.files}
            continue
        for n in ref:
            assert np.array_equal(got[n], ref[n]), (extra, n)
