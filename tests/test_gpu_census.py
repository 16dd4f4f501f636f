"""Census traversal parity: one decode step's 186 W4A16 projections plus the
LM head of the 24-layer Qwen3.5-0.8B model (shapes of
benchmarks/profiling/v07b_w4a16_shape_census.txt, call order of
src/runtime/qwen35_deltanet.cpp:166-251 and qwen35_full_attention.cpp:211-340),
launched as the benchmark launches them: prepacked weights, captured into a
HIP graph and replayed, unfused (one launch per projection), fused
(cudalm_w4a16_gemv_bf16_multi for the projections that share x) and as one
stage chain (cudalm_w4a16_chain_run, every fused group a stage that waits
for the previous one), at M = 1, 8 and 32. Every projection has its own
weights (seed from layer and role).

Bars: every projection output of the replay within the oracle's bound
(|y - r| <= 2 ulp_bf16(r) + 2^-16 sum|q s x|, r the fp64 sum of the exact
fp32 terms); over the whole traversal, no more outputs beyond 2 ulp of r
than the reference's own fp32 CPU loop (ref_gemv_bf16) has on the same
inputs (those outputs are sums whose terms cancel); the fused and chained
traversals bit for bit equal to the unfused one. The north_star's bar as
written, the distance in bf16 ulps from the reference loop's fp32
accumulator, is printed (max, count beyond 2) and gated: beyond 2 ulp only
where both fp32 sums may differ by their accumulation error
(2^-16 sum|q s x| each).
"""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DELTANET = [("in_proj_qkv", 6144, 1024), ("in_proj_z", 2048, 1024), ("in_proj_b", 16, 1024),
            ("in_proj_a", 16, 1024), ("out_proj", 1024, 2048)]
FULL_ATTN = [("q_proj", 4096, 1024), ("k_proj", 512, 1024), ("v_proj", 512, 1024),
             ("o_proj", 1024, 2048)]
MLP = [("gate_proj", 3584, 1024), ("up_proj", 3584, 1024), ("down_proj", 1024, 3584)]
LM_HEAD = ("lm_head", 248320, 1024)
ROLES = [name for name, _, _ in DELTANET + FULL_ATTN + MLP] + ["lm_head"]
THREADS = max(1, min(16, os.cpu_count() or 1))  # the GPU box's host share


def _groups(fused):
    """Launch groups of one decode step in call order (lists of (layer, name, N, K))."""
    out = []
    for li in range(24):
        full = li % 4 == 3
        plan = ([FULL_ATTN[:3], FULL_ATTN[3:], MLP[:2], MLP[2:]] if full else
                [DELTANET[:4], DELTANET[4:], MLP[:2], MLP[2:]])
        for grp in plan:
            items = [(li, name, N, K) for name, N, K in grp]
            out.extend([items] if fused else [[it] for it in items])
    out.append([(-1,) + LM_HEAD])
    return out


@pytest.fixture(scope="module")
def census(orc, w4, dev):
    mats = {}
    for items in _groups(False):
        li, name, N, K = items[0]
        W, S = orc.synth_w4a16(0xCE000000 + 64 * (li + 1) + ROLES.index(name), N, K)
        w = torch.from_numpy(W).to(dev)
        s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
        mats[(li, name)] = (W, S, w4.repack(w, s, N, K))
        del w, s
    torch.cuda.synchronize()
    return mats


def _replay(w4, census, xs, M, mode, dev):
    """Capture the traversal (mode: unfused / fused / chain) into a graph,
    replay it once; {(layer, name): y bits}."""
    lib = w4.lib()
    ys = {(li, nm): torch.empty((M, N), dtype=torch.bfloat16, device=dev)
          for items in _groups(False) for li, nm, N, _ in items}
    plan = []
    for items in _groups(mode != "unfused"):
        K = items[0][3]
        arr = w4.proj_array([(census[(li, nm)][2].data_ptr(), None, ys[(li, nm)].data_ptr(), N)
                             for li, nm, N, _ in items])
        plan.append((arr, len(items), xs[K].data_ptr(), K))
    chain = None
    if mode == "chain":
        # every fused group but the LM head is a stage waiting for the previous one
        body = [(list(zip([a.weight for a in arr], [None] * cnt, [a.y for a in arr],
                          [a.N for a in arr])), xp, K, gi - 1)
                for gi, (arr, cnt, xp, K) in enumerate(plan[:-1])]
        chain = w4.Chain(body, M, prepacked=True)
        plan = plan[-1:]
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        sraw = stream.cuda_stream
        if chain is not None:
            chain.run(stream=stream)
        for arr, cnt, xp, K in plan:
            if cnt == 1:
                rc = lib.cudalm_w4a16_gemv_bf16_prepacked(arr[0].weight, xp, arr[0].y, arr[0].N, K,
                                                           M, sraw)
            else:
                rc = lib.cudalm_w4a16_gemv_bf16_multi(ctypes.cast(arr, ctypes.c_void_p), cnt, xp, K,
                                                      M, 1, sraw)
            assert rc == 0, rc
    for y in ys.values():
        y.fill_(-1.0)  # the replay must write every output
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    if chain is not None:
        chain.status()
    return {k: v.view(torch.int16).cpu().numpy().view(np.uint16) for k, v in ys.items()}


@pytest.mark.parametrize("M", [1, 8, 32])
def test_census_traversal(w4, orc, dev, census, M):
    xh = {K: orc.synth_act(0xCE5 + 31 * M + K, M, K) for K in (1024, 2048, 3584)}
    xs = {K: torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16) for K, X in xh.items()}
    unfused = _replay(w4, census, xs, M, "unfused", dev)
    fused = _replay(w4, census, xs, M, "fused", dev)
    chained = _replay(w4, census, xs, M, "chain", dev)
    worst, over, ref_over, n = 0.0, 0, 0, 0
    worst32, over32 = 0.0, 0
    for (li, nm), Y in unfused.items():
        assert np.array_equal(fused[(li, nm)], Y), ("fused != unfused", li, nm)
        assert np.array_equal(chained[(li, nm)], Y), ("chain != unfused", li, nm)
        W, S, _ = census[(li, nm)]
        N, K = W.shape[0], W.shape[1] * 2
        ok, st = orc.full_parity(Y, W, S, xh[K], N, K, M, THREADS)
        assert ok, (li, nm, st)  # both bounds, on every output
        worst = max(worst, st["max_ulp"])
        over += st["n_over_2ulp"]
        ref_over += st["ref_n_over_2ulp"]
        n += st["n"]
        # the bar as written: bf16 ulps from the reference loop's fp32 accumulator
        worst32 = max(worst32, st["max_ulp_vs_fp32_ref"])
        over32 += st["n_over_2ulp_vs_fp32_ref"]
    print(f"  census M={M}: {len(unfused)} projections, {n} outputs, worst {worst:.3f} ulp of the "
          f"fp64 sum, {over} beyond 2 ulp (reference CPU loop: {ref_over}); vs the reference "
          f"loop's fp32 accumulator: max {worst32:.3f} ulp, {over32} beyond 2 ulp", flush=True)
    # over the whole traversal, no more outputs beyond 2 ulp than the reference loop
    assert over <= ref_over, (over, ref_over)
