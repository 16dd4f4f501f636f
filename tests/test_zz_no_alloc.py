"""cudalm_w4a16_gemv_bf16_chain_noalloc: the stage chain with its plan, flags
and counters in the library's static device array (no caller workspace, no
allocation). Checked against cudalm_w4a16_gemv_bf16_chain (caller
workspace) on the same stages, bit for bit, on two calls in a row, the
second smaller (fewer stages, fewer rows), and for its stage limit. No
reference counterpart (the reference allocates nothing per call because it
runs one launch per projection, src/runtime/qwen35_model.cpp:469-491)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _chain_case(orc, w4, dev, M, n_stages, seed):
    """n_stages alternating 3584x1024 / 1024x3584 projections, each reading
    the previous stage's output (real dependencies), plus per-stage output
    buffers for two independent runs."""
    shapes = [(3584, 1024), (1024, 3584)]
    mats = []
    for s in range(n_stages):
        N, K = shapes[s % 2]
        W, S = orc.synth_w4a16(seed + 16 * s, N, K)
        w = torch.from_numpy(W).to(dev)
        sc = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
        mats.append((w4.repack(w, sc, N, K), N, K))
    x0 = torch.from_numpy(orc.synth_act(seed + 1, M, 1024).view(np.int16)).to(dev).view(torch.bfloat16)

    def outputs():
        return [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
                for _, N, _ in mats]

    def stages(ys):
        arrs, st = [], (w4.Stage * n_stages)()
        for s, ((p, N, K), y) in enumerate(zip(mats, ys)):
            arr = w4.proj_array([(p.data_ptr(), None, y.data_ptr(), N)])
            arrs.append(arr)
            x = x0 if s == 0 else ys[s - 1]
            st[s].projs, st[s].count, st[s].x, st[s].K, st[s].dep = (
                ctypes.cast(arr, ctypes.c_void_p), 1, x.data_ptr(), K, s - 1)
        return st, arrs

    return outputs, stages


def test_noalloc_chain_matches_workspace_chain(orc, w4, dev):
    lib = w4.lib()
    sraw = torch.cuda.current_stream().cuda_stream
    for call, (M, n_stages) in enumerate([(8, 12), (1, 5)]):  # second call: smaller
        print(f"  no-alloc chain call {call}: M={M} stages={n_stages}", flush=True)
        outputs, stages = _chain_case(orc, w4, dev, M, n_stages, 0xA110C000 + 64 * call)
        ys_ws, ys_na = outputs(), outputs()
        st_ws, keep_ws = stages(ys_ws)
        st_na, keep_na = stages(ys_na)
        nbytes = lib.cudalm_w4a16_chain_workspace_bytes(n_stages)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.cudalm_w4a16_gemv_bf16_chain(ctypes.cast(st_ws, ctypes.c_void_p), n_stages, M, 1,
                                              ws.data_ptr(), nbytes, sraw)
        assert rc == 0, rc
        rc = lib.cudalm_w4a16_gemv_bf16_chain_noalloc(ctypes.cast(st_na, ctypes.c_void_p),
                                                      n_stages, M, 1, sraw)
        assert rc == 0, rc
        for s in range(n_stages):
            a, b = _bits(ys_ws[s]), _bits(ys_na[s])
            assert not np.isnan(orc.bf16_to_f32(a)).any(), (call, s)
            assert np.array_equal(a, b), (call, s)
        del keep_ws, keep_na


def test_noalloc_chain_swiglu_stage(orc, w4, dev):
    """A SwiGLU stage (gate/up writing act) and the down stage reading act,
    through the allocation-free entry: equal to the workspace chain and to
    cudalm_w4a16_swiglu_bf16 + cudalm_w4a16_gemv_bf16, on two calls in a row,
    the second with fewer rows."""
    lib = w4.lib()
    sraw = torch.cuda.current_stream().cuda_stream
    I, H = 3584, 1024
    mats = []
    for r, (N, K) in enumerate([(I, H), (I, H), (H, I)]):
        W, S = orc.synth_w4a16(0xA110D000 + 16 * r, N, K)
        w = torch.from_numpy(W).to(dev)
        sc = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
        mats.append(w4.repack(w, sc, N, K))
    g, u, d = mats
    for call, M in enumerate([8, 3]):
        print(f"  no-alloc swiglu chain call {call}: M={M}", flush=True)
        x = torch.from_numpy(orc.synth_act(0xA110D100 + M, M, H).view(np.int16)).to(dev).view(
            torch.bfloat16)
        act_ref = w4.swiglu(g, None, u, None, x, I, H, M, prepacked=True)
        h_ref = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
        w4.gemv_prepacked(d, act_ref.view(M, I), H, I, M, y=h_ref)
        outs = []
        for noalloc in (False, True):
            act = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=dev)
            h = torch.full((M, H), float("nan"), dtype=torch.bfloat16, device=dev)
            gu = w4.proj_array([(g.data_ptr(), None, 0, I), (u.data_ptr(), None, 0, I)])
            dn = w4.proj_array([(d.data_ptr(), None, h.data_ptr(), H)])
            st = (w4.Stage * 2)()
            st[0].projs, st[0].count, st[0].x, st[0].K, st[0].dep = (
                ctypes.cast(gu, ctypes.c_void_p), 2, x.data_ptr(), H, -1)
            st[0].act = act.data_ptr()
            st[1].projs, st[1].count, st[1].x, st[1].K, st[1].dep = (
                ctypes.cast(dn, ctypes.c_void_p), 1, act.data_ptr(), I, 0)
            if noalloc:
                rc = lib.cudalm_w4a16_gemv_bf16_chain_noalloc(ctypes.cast(st, ctypes.c_void_p), 2, M,
                                                              1, sraw)
            else:
                nbytes = lib.cudalm_w4a16_chain_workspace_bytes(2)
                ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
                rc = lib.cudalm_w4a16_gemv_bf16_chain(ctypes.cast(st, ctypes.c_void_p), 2, M, 1,
                                                      ws.data_ptr(), nbytes, sraw)
            assert rc == 0, (call, noalloc, rc)
            outs.append((_bits(act), _bits(h)))
            del gu, dn
        for a, hh in outs:
            assert np.array_equal(a.ravel(), _bits(act_ref).ravel()), call
            assert np.array_equal(hh, _bits(h_ref)), call


def test_noalloc_chain_stage_limit(orc, w4, dev):
    lib = w4.lib()
    sraw = torch.cuda.current_stream().cuda_stream
    n = 129  # one more than the static array holds
    st = (w4.Stage * n)()
    assert lib.cudalm_w4a16_gemv_bf16_chain_noalloc(ctypes.cast(st, ctypes.c_void_p), n, 1, 1,
                                                    sraw) == w4.ERANGE
