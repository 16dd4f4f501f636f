"""Stage chains (cudalm_w4a16_chain_*): one persistent launch runs a list of
dependent projection stages. No reference counterpart: the reference
issues every projection as its own launch
(src/runtime/qwen35_model.cpp:469-491).

Bars:
  * every stage output bit-identical to the same stages run one launch at a
    time through cudalm_w4a16_gemv_bf16_multi (whose outputs the other GPU
    tests pin to the oracle, the restatement of the reference's
    ref_gemv_bf16, tests/cuda/test_int4_gemv_bf16.cpp:54-69);
  * real data dependencies: stage outputs are later stages' inputs, and
    buffers are reused (a stage overwrites the input of an earlier stage it
    depends on), so a stage that read x early or a lost store shows up as
    different bits;
  * each output also inside the oracle's bound on the inputs it actually read;
  * repeated runs and HIP-graph replays (with eager work between them) give
    the same bits every time, and no wait times out.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, __import__("os").cpu_count() or 1))


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


class Net:
    """Weights and buffers of a 9-stage chain with real dependencies."""

    # (name, N, K, seed-role)
    MATS = [("a0", 3584, 1024), ("b0", 1024, 3584), ("q", 2048, 1024), ("k", 512, 1024),
            ("t", 16, 1024), ("o", 1024, 2048), ("a1", 3584, 1024), ("b1", 1024, 3584),
            ("r16", 16, 1024), ("z", 1000, 1024), ("big", 6144, 1024)]

    def __init__(self, orc, w4, dev, M, prepacked, seed):
        self.M, self.prepacked = M, prepacked
        self.host = {}
        self.dev = {}
        for role, (name, N, K) in enumerate(self.MATS):
            W, S = orc.synth_w4a16(seed + 16 * role, N, K)
            w = torch.from_numpy(W).to(dev)
            s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
            self.host[name] = (W, S)
            self.dev[name] = (w4.repack(w, s, N, K), None) if prepacked else (w, s)
        self.x0 = orc.synth_act(seed + 1, M, 1024)
        self.xi = orc.synth_act(seed + 2, M, 1024)
        self.N = {name: N for name, N, _ in self.MATS}

    def buffers(self, dev):
        M = self.M
        mk = lambda n: torch.empty((M, n), dtype=torch.bfloat16, device=dev)  # noqa: E731
        return {"h": mk(1024), "u": mk(3584), "v": mk(1024), "r": mk(2048), "kk": mk(512),
                "tt": mk(16), "rr": mk(16), "xi": mk(1024), "zz": mk(1000), "bb": mk(6144)}

    def stages(self, B):
        """(items, x buffer, K, dep) with items (matrix name, output buffer)."""
        return [
            ([("a0", "u")], "h", 1024, -1),                          # 0
            ([("b0", "v")], "u", 3584, 0),                           # 1
            ([("q", "r"), ("k", "kk"), ("t", "tt")], "v", 1024, 1),  # 2 (fused)
            ([("o", "h")], "r", 2048, 2),                            # 3 overwrites stage 0's x
            ([("a1", "u")], "h", 1024, 3),                           # 4 overwrites stage 1's x
            ([("b1", "v")], "u", 3584, 4),                           # 5 overwrites stage 2's x
            ([("r16", "rr")], "v", 1024, 5),                         # 6
            ([("z", "zz")], "xi", 1024, -1),                         # 7 independent, ragged N
            ([("big", "bb")], "v", 1024, 5),                         # 8 non-adjacent dep
        ]

    def reset(self, B):
        for name, t in B.items():
            t.fill_(float("nan"))
        B["h"].copy_(torch.from_numpy(self.x0.view(np.int16)).view(torch.bfloat16))
        B["xi"].copy_(torch.from_numpy(self.xi.view(np.int16)).view(torch.bfloat16))

    def chain_stages(self, B):
        out = []
        for items, xb, K, dep in self.stages(B):
            its = [(self.dev[m][0].data_ptr(),
                    None if self.dev[m][1] is None else self.dev[m][1].data_ptr(),
                    B[yb].data_ptr(), self.N[m]) for m, yb in items]
            out.append((its, B[xb], K, dep))
        return out

    def run_sequential(self, w4, B):
        """The same stages, one launch each (stream-ordered); returns the
        inputs each stage read (host bits) for the oracle check."""
        seen = []
        for items, xb, K, dep in self.stages(B):
            torch.cuda.synchronize()
            seen.append(_bits(B[xb]).reshape(self.M, K))
            w4.gemv_multi([self.dev[m][0] for m, _ in items],
                          None if self.prepacked else [self.dev[m][1] for m, _ in items],
                          B[xb], [self.N[m] for m, _ in items], K, self.M,
                          ys=[B[yb] for _, yb in items], prepacked=self.prepacked)
        torch.cuda.synchronize()
        return seen


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("prepacked", [True, False])
def test_chain_real_dependencies(orc, w4, dev, M, prepacked):
    print(f"  chain real deps M={M} prepacked={prepacked}", flush=True)
    net = Net(orc, w4, dev, M, prepacked, 0xC4A10000 + 97 * M + int(prepacked))
    ref = net.buffers(dev)
    net.reset(ref)
    seen = net.run_sequential(w4, ref)
    want = {k: _bits(v) for k, v in ref.items()}

    # oracle bound on the inputs each stage really read (stages 2, 7, 8)
    for si in (2, 7, 8):
        items, xb, K, _ = net.stages(ref)[si]
        for m, yb in items:
            W, S = net.host[m]
            N = net.N[m]
            ok, st = orc.check_tolerance(want[yb].reshape(M, N), W, S, seen[si], N, K, M)
            assert ok, (si, m, st)

    B = net.buffers(dev)
    chain = w4.Chain(net.chain_stages(B), M, prepacked=prepacked)
    for rep in range(3):
        net.reset(B)
        torch.cuda.synchronize()
        chain.run()
        chain.status()
        for k, v in B.items():
            assert np.array_equal(_bits(v), want[k]), ("run", rep, k)

    # captured into a graph, replayed with eager work in between
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        chain.run(stream=stream)
    for rep in range(3):
        net.reset(B)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        chain.status()
        for k, v in B.items():
            assert np.array_equal(_bits(v), want[k]), ("replay", rep, k)


def test_chain_one_shot_and_errors(orc, w4, dev):
    """cudalm_w4a16_gemv_bf16_chain (plan + run) and the plan's rejections."""
    lib = w4.lib()
    N, K, M = 512, 1024, 4
    W, S = orc.synth_w4a16(0xC4A1F000, N, K)
    X = orc.synth_act(0xC4A1F001, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    y2 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    arr = w4.proj_array([(w.data_ptr(), s.data_ptr(), y.data_ptr(), N)])
    arr2 = w4.proj_array([(w.data_ptr(), s.data_ptr(), y2.data_ptr(), N)])
    st = (w4.Stage * 2)()
    st[0].projs, st[0].count, st[0].x, st[0].K, st[0].dep = ctypes.cast(arr, ctypes.c_void_p), 1, \
        x.data_ptr(), K, -1
    st[1].projs, st[1].count, st[1].x, st[1].K, st[1].dep = ctypes.cast(arr2, ctypes.c_void_p), 1, \
        x.data_ptr(), K, 0
    nbytes = lib.cudalm_w4a16_chain_workspace_bytes(2)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    sraw = torch.cuda.current_stream().cuda_stream
    rc = lib.cudalm_w4a16_gemv_bf16_chain(ctypes.cast(st, ctypes.c_void_p), 2, M, 0,
                                          ws.data_ptr(), nbytes, sraw)
    assert rc == 0, rc
    torch.cuda.synchronize()
    ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv(w, s, x, N, K, M, y=ref)
    assert np.array_equal(_bits(y), _bits(ref))
    assert np.array_equal(_bits(y2), _bits(ref))
    # rejections
    bad = lambda n, m, b: lib.cudalm_w4a16_gemv_bf16_chain(  # noqa: E731
        ctypes.cast(st, ctypes.c_void_p), n, m, 0, ws.data_ptr(), b, sraw)
    assert bad(2, 33, nbytes) == w4.EINVAL
    assert bad(2, 0, nbytes) == w4.EINVAL
    assert bad(2, M, nbytes - 1) == w4.EINVAL
    st[1].dep = 1
    assert bad(2, M, nbytes) == w4.EINVAL  # a stage cannot wait for itself
    st[1].dep = 0
    st[1].K = 4224
    assert bad(2, M, nbytes) == w4.EINVAL  # K > 4096
    st[1].K = K
    st[1].x = x.data_ptr() + 2
    assert bad(2, M, nbytes) == w4.EALIGN


def test_chain_infinite_activation(orc, w4, dev):
    """An infinity in x: each chain output equals cudalm_w4a16_gemv_bf16's,
    which gives the reference loop's +-Inf / NaN there."""
    N, K, M = 1024, 1024, 4
    W, S = orc.synth_w4a16(0xC4A1E000, N, K)
    X = orc.synth_act(0xC4A1E001, M, K)
    X[2, 17] = 0xFF80  # -Inf
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    p = w4.repack(w, s, N, K)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    chain = w4.Chain([([(p.data_ptr(), None, y.data_ptr(), N)], x, K, -1)], M, prepacked=True)
    chain.run()
    chain.status()
    ref = torch.empty_like(y)
    w4.gemv_prepacked(p, x, N, K, M, y=ref)
    assert np.array_equal(_bits(y), _bits(ref))
    r = orc.gemv_bf16(W, S, X, N, K, M)
    assert np.array_equal(np.isinf(orc.bf16_to_f32(_bits(y).reshape(M, N)[2])),
                          np.isinf(orc.bf16_to_f32(r[2])))


def test_chain_wait_bound_timeout(orc, w4, dev):
    """The timeout path, forced from the host: 48 one-tile stages, each
    waiting for the previous one, so the last stages' workgroups wait ~100 us
    from the launch; with a wait bound of 1 tick those waits give up (their
    stages proceed and every wave exits), status() reports the timeout once
    and clears it; with the default bound restored the same chain runs clean
    and gives the outputs of per-stage launches."""
    N, K, M, S = 16, 1024, 1, 48
    W, Sc = orc.synth_w4a16(0xC4A1B000, N, K)
    X = orc.synth_act(0xC4A1B001, M, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(Sc.view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    p = w4.repack(w, s, N, K)
    ys = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(S)]
    chain = w4.Chain([([(p.data_ptr(), None, ys[k].data_ptr(), N)], x, K, k - 1) for k in range(S)],
                     M, prepacked=True)
    chain.set_wait_bound(1)
    chain.run()
    with pytest.raises(w4.W4A16Error) as ei:
        chain.status()
    assert ei.value.code == w4.ETIMEOUT
    chain.status()  # the record was cleared
    chain.set_wait_bound(0)
    for y in ys:
        y.fill_(float("nan"))
    chain.run()
    chain.status()
    ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv_prepacked(p, x, N, K, M, y=ref)
    for y in ys:
        assert np.array_equal(_bits(y), _bits(ref))


def _dev_mat(orc, w4, dev, seed, N, K, prepacked):
    W, S = orc.synth_w4a16(seed, N, K)
    w = torch.from_numpy(W).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev).view(torch.float16)
    return (w4.repack(w, s, N, K), None) if prepacked else (w, s)


@pytest.mark.parametrize("M", [1, 8, 17, 32])
@pytest.mark.parametrize("prepacked", [True, False])
def test_chain_swiglu_mlp(orc, w4, dev, M, prepacked):
    """SwiGLU stages (stage.act): two MLP blocks in one launch, each a
    gate/up stage writing act = silu(gate) * up and a down stage reading act,
    the second block overwriting the first block's act and reading its
    output. Every output bit-identical to cudalm_w4a16_swiglu_bf16 followed
    by cudalm_w4a16_gemv_bf16, launch by launch. Shapes: the census MLP
    (3584 x 1024 gate/up), a ragged one at K = 2048 (two groups per wave,
    1000 rows: 63 tile pairs), a one-tile one and one that takes two rounds
    (5000 x 2048)."""
    print(f"  chain swiglu M={M} prepacked={prepacked}", flush=True)
    seed = 0xC4A15000 + 31 * M + int(prepacked)
    # (N of gate/up, K = hidden); 5000 x 2048 is 626 stage tiles at two per
    # workgroup: more than one round of the 256 workgroups a stage may use
    blocks = [(3584, 1024), (1000, 2048), (16, 1024), (5000, 2048)]
    mats = []
    for b, (N, K) in enumerate(blocks):
        g = _dev_mat(orc, w4, dev, seed + 8 * b, N, K, prepacked)
        u = _dev_mat(orc, w4, dev, seed + 8 * b + 1, N, K, prepacked)
        # down: [K, N], only where act's width is whole groups
        d = _dev_mat(orc, w4, dev, seed + 8 * b + 2, K, N, prepacked) if N % 128 == 0 else None
        mats.append((g, u, d))
    X = orc.synth_act(seed + 7, M, 2048)
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)

    for b, (N, K) in enumerate(blocks):
        (g, u, d) = mats[b]
        xk = x[:, :K].contiguous()
        down = N % 128 == 0
        # reference: one launch per step
        act_ref = w4.swiglu(g[0], g[1], u[0], u[1], xk, N, K, M, prepacked=prepacked)
        h_ref = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        act2_ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        h2_ref = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        if down:
            def lin(m, xin, yout, n, k):
                if prepacked:
                    w4.gemv_prepacked(m[0], xin, n, k, M, y=yout)
                else:
                    w4.gemv(m[0], m[1], xin, n, k, M, y=yout)
            lin(d, act_ref, h_ref, K, N)
            w4.swiglu(g[0], g[1], u[0], u[1], h_ref, N, K, M, y=act2_ref, prepacked=prepacked)
            lin(d, act2_ref, h2_ref, K, N)
        torch.cuda.synchronize()

        act = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        h = torch.full((M, K), float("nan"), dtype=torch.bfloat16, device=dev)
        h2 = torch.full((M, K), float("nan"), dtype=torch.bfloat16, device=dev)
        pw = lambda m: (m[0].data_ptr(), None if m[1] is None else m[1].data_ptr())  # noqa: E731
        gu = [(*pw(g), 0, N), (*pw(u), 0, N)]
        stages = [(gu, xk, K, -1, act)]
        if down:
            stages += [([(*pw(d), h.data_ptr(), K)], act, N, 0),
                       (gu, h, K, 1, act),
                       ([(*pw(d), h2.data_ptr(), K)], act, N, 2)]
        chain = w4.Chain(stages, M, prepacked=prepacked)
        for rep in range(2):
            chain.run()
            chain.status()
            if down:
                assert np.array_equal(_bits(h), _bits(h_ref)), (b, rep, "h")
                assert np.array_equal(_bits(h2), _bits(h2_ref)), (b, rep, "h2")
                assert np.array_equal(_bits(act), _bits(act2_ref)), (b, rep, "act")
            else:
                assert np.array_equal(_bits(act).ravel(), _bits(act_ref).ravel()), (b, rep, "act")
            act.fill_(float("nan"))
            h.fill_(float("nan"))
            h2.fill_(float("nan"))


def test_chain_swiglu_infinite_and_errors(orc, w4, dev):
    """An infinity in x reaches both projections of a SwiGLU stage (their
    NaN sums take the reference loop): act equals cudalm_w4a16_swiglu_bf16's
    bits. The plan rejects SwiGLU stages that are not gate/up pairs of one
    shape at K <= 2048."""
    N, K, M = 1024, 1024, 4
    g = _dev_mat(orc, w4, dev, 0xC4A1D000, N, K, True)
    u = _dev_mat(orc, w4, dev, 0xC4A1D001, N, K, True)
    X = orc.synth_act(0xC4A1D002, M, K)
    X[1, 5] = 0x7F80  # +Inf
    x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
    act = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    gu = [(g[0].data_ptr(), None, 0, N), (u[0].data_ptr(), None, 0, N)]
    chain = w4.Chain([(gu, x, K, -1, act)], M, prepacked=True)
    chain.run()
    chain.status()
    ref = w4.swiglu(g[0], None, u[0], None, x, N, K, M, prepacked=True)
    assert np.array_equal(_bits(act).ravel(), _bits(ref).ravel())
    assert not np.isfinite(orc.bf16_to_f32(_bits(act).reshape(M, N)[1])).all()

    with pytest.raises(ValueError):  # one projection
        w4.Chain([(gu[:1], x, K, -1, act)], M, prepacked=True)
    with pytest.raises(ValueError):  # gate and up of different N
        w4.Chain([([gu[0], (u[0].data_ptr(), None, 0, N - 16)], x, K, -1, act)], M, prepacked=True)
    big = torch.zeros((M, 4096), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):  # K > 2048
        w4.Chain([(gu, big, 4096, -1, act)], M, prepacked=True)
