"""GPU parity tests: the HIP kernels, called through the C ABI, against the
CPU oracle (a restatement of the reference's ref_gemv_bf16,
tests/cuda/test_int4_gemv_bf16.cpp:54-69) on the reference's own fixture
recipes, shapes, seeds and input classes
(tests/cuda/test_w4a16_qwen35_optimized.cpp:66-171,456).

Bars:
  * unpack and dequantized weights: bit-exact;
  * outputs: |y - r| <= 2 ulp_bf16(r) + 2^-16 * sum_k |q s x|, with r the
    fp64 sum of the exact fp32 terms (oracle.check_tolerance); the count of
    elements beyond 2 ulp is reported and must be 0 outside cancellation;
  * every kernel variant, both weight layouts and every batch row:
    bit-identical per output (the reference's row-parity and variant
    bit-identity gates, test_w4a16_qwen35_optimized.cpp:1-35).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# census (benchmarks/profiling/v07b_w4a16_shape_census.txt) + edge shapes
# (test_w4a16_qwen35_optimized.cpp:154-171)
CENSUS = [(16, 1024), (512, 1024), (1024, 2048), (1024, 3584), (2048, 1024), (3584, 1024),
          (4096, 1024), (6144, 1024)]
EDGE = [(1, 128), (3, 128), (5, 256), (9, 1024), (15, 1024), (1023, 1024)]
# LDS staging rows of the file-layout whole-line loads at M <= 16 (four
# waves of 16 rows: pieces of 4 groups in the stream kernel, units of 8 in
# the split kernel); these predicates are for file-layout weights
_STAGE_STREAM = 4 * 16 * (4 * 64 + 16)
_STAGE_SPLIT = 4 * 16 * (8 * 64 + 16)
VARIANTS_FOR_M = {
    # variant name -> predicate on (M, K) for applicability
    "stream": lambda M, K: M <= 32 and (M * (K // 8 + 2) * 16
                                        + (K // 128) * 64 * (2 if M > 16 else 1)
                                        + (_STAGE_STREAM if M <= 16 else 0)) <= 160 * 1024,
    "split": lambda M, K: M <= 32 and (M * (K // 8 + 2) * 16 + (K // 128) * 64 * (2 if M > 16 else 1)
                                       + max(1, 4 // -(-K // 1024)) * -(-K // 1024) * (2 if M > 16 else 1)
                                       * 1024 + (_STAGE_SPLIT if M <= 16 else 0)) <= 160 * 1024,
    "tile16": lambda M, K: True,
    "tile32": lambda M, K: True,
    "prefill": lambda M, K: True,
}


def up(dev, W, S, X):
    w = torch.from_numpy(np.ascontiguousarray(W)).to(dev)
    s = torch.from_numpy(np.ascontiguousarray(S).view(np.int16)).to(dev).view(torch.float16)
    x = torch.from_numpy(np.ascontiguousarray(X).view(np.int16)).to(dev).view(torch.bfloat16)
    return w, s, x


def down(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run(w4, w, s, x, N, K, M, variant="auto"):
    y = torch.empty((M, N), dtype=torch.bfloat16, device=w.device)
    w4.gemv(w, s, x, N, K, M, y=y, variant=variant)
    return down(y).reshape(M, N)


THREADS = max(1, min(16, __import__("os").cpu_count() or 1))  # the GPU box's host share


def assert_baseline(orc, Y, W, S, X, N, K, M, label=""):
    """BASELINE workloads: every output within the bound, and no more than 3
    more outputs beyond 2 ulp than the reference CPU loop has on the same
    inputs (a handful of cancelled sums either way; over whole census
    traversals tests/test_gpu_census.py gates the totals with no slack)."""
    _, st, _ = orc.check_against_reference_loop(Y, W, S, X, N, K, M, THREADS)
    print(f"  {label} N={N} K={K} M={M}: {st}", flush=True)
    assert st["n_bad"] == 0, (label, st)
    # outputs beyond 2 ulp are sums whose terms cancel: no more of them than
    # the reference loop has on the same inputs, up to a few for the other
    # accumulation order (either side can round one more of them badly)
    assert st["n_over_2ulp"] <= st["ref_n_over_2ulp"] + 3, (label, st)
    return st


def assert_tol(orc, Y, W, S, X, N, K, M, label=""):
    ok, st = orc.check_tolerance(Y, W, S, X, N, K, M)
    print(f"  {label} N={N} K={K} M={M}: {st}", flush=True)
    assert ok, (label, st)
    return st


# ---------------------------------------------------------------- dequant ---

@pytest.mark.parametrize("N,K,kind", [(16, 1024, "random"), (3, 128, "boundary"),
                                      (37, 256, "random"), (512, 1024, "boundary"),
                                      (1023, 1024, "small")])
def test_dequant_bitexact(w4, orc, dev, N, K, kind):
    W, S, _ = orc.fixture_kind(kind, 0x51ED, N, K, 1)
    w, s, _ = up(dev, W, S, np.zeros((1, K), np.uint16))
    q, wf = w4.dequant(w, s, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), orc.unpack(W, N, K))
    assert np.array_equal(wf.cpu().numpy().view(np.uint32), orc.dequant(W, S, N, K).view(np.uint32))


# ---------------------------------------------------------------- reference's GEMV tests ---

@pytest.mark.parametrize("N,K", [(4096, 1024), (512, 1024), (1024, 2048), (3584, 1024),
                                 (1024, 3584), (16, 1024), (3, 128)])
def test_reference_vectorized_shapes(w4, orc, dev, N, K):
    # test_int4_gemv_bf16.cpp:127-140, seed 0x51ed51 + N + K
    W, S, X = orc.fixture_gemv(0x51ED51 + N + K, N, K)
    Y = run(w4, *up(dev, W, S, X), N, K, 1)
    assert_tol(orc, Y, W, S, X, N, K, 1, "vectorized")
    if orc.ref is not None:
        ok, mx, idx = orc.ref.compare_bf16_stages(orc.gemv_bf16(W, S, X, N, K), Y)
        assert ok, (mx, idx)


def test_zero_group_exact_zero(w4, orc, dev):
    # test_int4_gemv_bf16.cpp:146-176
    N, K = 8, 256
    W = np.zeros((N, K // 2), np.uint8)
    S = np.zeros((N, K // 128), np.uint16)
    X = orc.f32_to_bf16((orc.xorshift32(123, K) * (2.0 / 4294967296.0) - 1.0).astype(np.float32))
    X = X.reshape(1, K)
    for M in (1, 3, 40):
        Xm = np.repeat(X, M, axis=0)
        Y = run(w4, *up(dev, W, S, Xm), N, K, M)
        assert not Y.any()
    # zero scales with nonzero nibbles also give exact zeros
    W2 = np.full((N, K // 2), 0x77, np.uint8)
    Y = run(w4, *up(dev, W2, S, X), N, K, 1)
    assert not Y.any()


def test_misaligned_bases_take_bytewise_path(w4, orc, dev):
    # test_int4_gemv_bf16.cpp:181-242: W and x offset by one byte
    N, K = 37, 256
    W, S, X = orc.fixture_gemv(777, N, K)
    wbuf = torch.zeros(W.size + 2, dtype=torch.uint8, device=dev)
    wbuf[1:1 + W.size] = torch.from_numpy(W.ravel()).to(dev)
    xbytes = X.view(np.uint8).ravel()
    xbuf = torch.zeros(xbytes.size + 2, dtype=torch.uint8, device=dev)
    xbuf[1:1 + xbytes.size] = torch.from_numpy(xbytes).to(dev)
    s = torch.from_numpy(S.view(np.int16)).to(dev)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    rc = w4.gemv_ptr(wbuf.data_ptr() + 1, s.data_ptr(), xbuf.data_ptr() + 1, y.data_ptr(), N, K, 1,
                     w4.VARIANT_AUTO, stream)
    assert rc == 0
    Yb = down(y).reshape(1, N)
    assert_tol(orc, Yb, W, S, X, N, K, 1, "bytewise")
    Yv = run(w4, *up(dev, W, S, X), N, K, 1)
    if orc.ref is not None:
        ok, mx, _ = orc.ref.compare_bf16_stages(Yv, Yb)
        assert ok, mx


# ---------------------------------------------------------------- variant / row parity gate ---

def _parity_case(w4, orc, dev, N, K, B, kind, seed):
    W, S, X = orc.fixture_kind(kind, seed, N, K, B)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, B)
    assert_tol(orc, Y, W, S, X, N, K, B, f"{kind}/{seed:#x}")
    # row parity: batch row b == single call on row b
    for b in range(B):
        yb = run(w4, w, s, x[b:b + 1], N, K, 1)
        assert np.array_equal(Y[b], yb[0]), ("row parity", b)
    # every applicable variant, file layout and prepacked
    p = w4.repack(w, s, N, K)
    for name, ok in VARIANTS_FOR_M.items():
        if not ok(B, K):
            continue
        assert np.array_equal(run(w4, w, s, x, N, K, B, name), Y), ("variant", name)
        yp = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
        w4.gemv_prepacked(p, x, N, K, B, y=yp, variant=name)
        assert np.array_equal(down(yp).reshape(B, N), Y), ("prepacked", name)


@pytest.mark.parametrize("N,K", EDGE + CENSUS[:2])
@pytest.mark.parametrize("kind", ["random", "zero", "small", "mixed_sign", "boundary"])
def test_parity_gate_small(w4, orc, dev, N, K, kind):
    for seed in orc.REFERENCE_SEEDS:
        _parity_case(w4, orc, dev, N, K, 3, kind, seed)


@pytest.mark.parametrize("N,K", CENSUS[2:])
@pytest.mark.parametrize("kind", ["random", "zero", "small", "mixed_sign", "boundary"])
def test_parity_gate_census(w4, orc, dev, N, K, kind):
    # test_w4a16_qwen35_optimized.cpp:154-171,456: every census shape x the
    # four reference seeds x the five input classes
    for seed in orc.REFERENCE_SEEDS:
        _parity_case(w4, orc, dev, N, K, 3, kind, seed)


# ---------------------------------------------------------------- BASELINE workloads ---

@pytest.mark.parametrize("N,K", CENSUS)
@pytest.mark.parametrize("M", [1, 8, 32])
def test_census_synthetic(w4, orc, dev, N, K, M):
    # N(0, 0.02) weights quantized per 128-group,
    # N(0, 1) bf16 activations, per-shape seeds
    W, S = orc.synth_w4a16(0xC0DA0000 + N + K, N, K)
    X = orc.synth_act(0xAC7 + M, M, K)
    Y = run(w4, *up(dev, W, S, X), N, K, M)
    assert_baseline(orc, Y, W, S, X, N, K, M, "census")


@pytest.mark.parametrize("N,K", CENSUS)
@pytest.mark.parametrize("M", [64, 100, 512])
def test_prefill_chunks(w4, orc, dev, N, K, M):
    # M-token prefill chunk GEMM
    W, S = orc.synth_w4a16(0xBEEF + N + K, N, K)
    X = orc.synth_act(0xF00D + M, M, K)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, M)
    assert_baseline(orc, Y, W, S, X, N, K, M, "prefill")
    for b in (0, 17, M - 1):
        assert np.array_equal(Y[b], run(w4, w, s, x[b:b + 1], N, K, 1)[0]), b


@pytest.mark.parametrize("N,K", [(37, 384), (1023, 1152), (129, 128), (300, 2176), (1, 128),
                                 (17, 4096)])
@pytest.mark.parametrize("M", [33, 70, 129])
def test_prefill_ragged(w4, orc, dev, N, K, M):
    # the prefill GEMM's partial paths: a last 8-group unit that is short
    # (K/128 % 8 != 0), scale rows not 16 B aligned in the file layout,
    # N not a multiple of the 16-row tile and M not a multiple of 32;
    # file layout, prepacked layout and the tile32 kernel agree bit for bit
    W, S = orc.synth_w4a16(0x9A61 + N * 3 + K, N, K)
    X = orc.synth_act(0x9A62 + M, M, K)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, M, "prefill")
    assert_tol(orc, Y, W, S, X, N, K, M, "prefill_ragged")
    assert np.array_equal(run(w4, w, s, x, N, K, M, "tile32"), Y)
    p = w4.repack(w, s, N, K)
    yp = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w4.gemv_prepacked(p, x, N, K, M, y=yp, variant="prefill")
    assert np.array_equal(down(yp).reshape(M, N), Y)
    for b in (0, M // 2, M - 1):
        assert np.array_equal(Y[b], run(w4, w, s, x[b:b + 1], N, K, 1)[0]), b


def test_lm_head_full_size(w4, orc, dev):
    # N = 248320, K = 1024, M = 1, whole output checked
    N, K = 248320, 1024
    W, S = orc.synth_w4a16(0x11AD, N, K)
    X = orc.synth_act(0x11AE, 1, K)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, 1)
    assert_baseline(orc, Y, W, S, X, N, K, 1, "lm_head")
    p = w4.repack(w, s, N, K)
    yp = w4.gemv_prepacked(p, x, N, K, 1)
    assert np.array_equal(down(yp).reshape(1, N), Y)
    # checksum of a second activation row: linearity in x (y(2x) == 2 y(x))
    x2 = (x.float() * 2).to(torch.bfloat16)
    Y2 = run(w4, w, s, x2, N, K, 1)
    assert np.array_equal(orc.bf16_to_f32(Y2), orc.bf16_to_f32(Y) * 2)


def _same_nonfinite(a, b):
    """bit-equal, NaN payloads aside (any NaN equals any NaN)"""
    fa, fb = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
    na = ((fa & 0x7F80) == 0x7F80) & ((fa & 0x7F) != 0)
    nb = ((fb & 0x7F80) == 0x7F80) & ((fb & 0x7F) != 0)
    return np.array_equal(na, nb) and np.array_equal(fa[~na], fb[~nb])


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan, "mixed"])
@pytest.mark.parametrize("M", [3, 40])
def test_nonfinite_activation(w4, orc, dev, bad, M):
    # Rows of x holding a non-finite value give the reference loop's outputs
    # (ref_gemv_bf16, tests/cuda/test_int4_gemv_bf16.cpp:54-69): +-Inf where
    # every infinite term has one sign, NaN where a term is NaN (a NaN x, a
    # zero weight or scale times an infinity, or +Inf and -Inf terms). The
    # kernels recompute an output whose fast sum is NaN with that loop, so
    # the rows equal the oracle's (NaN payloads aside); other rows are
    # untouched (row independence). Every kernel family, both layouts.
    N, K = 512, 1024
    W, S, X = orc.fixture_kind("random", 0x51, N, K, M)
    Xb = X.copy()
    if bad == "mixed":
        Xb[1, 77] = orc.f32_to_bf16(np.array([np.inf], np.float32))[0]
        Xb[1, 900] = orc.f32_to_bf16(np.array([-np.inf], np.float32))[0]
    else:
        Xb[1, 77] = orc.f32_to_bf16(np.array([bad], np.float32))[0]
    # a row whose only infinity meets no zero weight: every output +-Inf
    Xb[M - 1, 5] = orc.f32_to_bf16(np.array([np.inf], np.float32))[0]
    Wz = W.copy()
    Wz[:, 2] = np.where((Wz[:, 2] & 0xF0) == 0, Wz[:, 2] | 0x10, Wz[:, 2])  # q[n, 5] != 0
    ref = orc.gemv_bf16(Wz, S, Xb, N, K, M)
    assert np.isinf(orc.bf16_to_f32(ref[M - 1])).all()
    w, s, x = up(dev, Wz, S, Xb)
    x0 = up(dev, Wz, S, X)[2]
    p = w4.repack(w, s, N, K)
    variants = ("auto", "stream", "split", "tile16", "tile32", "prefill", "prefill32", "bytewise")
    for variant in variants:
        if variant in ("stream", "split") and M > 32:
            continue
        Y = run(w4, w, s, x, N, K, M, variant)
        for row in (1, M - 1):
            assert _same_nonfinite(Y[row], ref[row]), (variant, row)
        Y0 = run(w4, w, s, x0, N, K, M, variant)
        keep = [r for r in range(M) if r not in (1, M - 1)]
        assert np.array_equal(Y[keep], Y0[keep]), variant
        if variant != "bytewise":
            yp = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            w4.gemv_prepacked(p, x, N, K, M, y=yp, variant=variant)
            assert np.array_equal(down(yp).reshape(M, N), Y), ("prepacked", variant)


@pytest.mark.parametrize("N,M", [(248320, 8), (100003, 3), (100003, 1), (248320, 32)])
def test_large_n_small_m(w4, orc, dev, N, M):
    # launches large enough for the dispatcher-placed tail workgroups
    # (M <= 8; N = 100003 leaves a ragged last tile and a partial last tail
    # workgroup) and for the 8-wave two-column-tile grid (M = 32): tolerance
    # against the oracle, both layouts equal, and row b == the M = 1 call
    K = 1024
    W, S = orc.synth_w4a16(0x7A11 + N + M, N, K)
    X = orc.synth_act(0x7A12 + M, M, K)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, M)
    assert_baseline(orc, Y, W, S, X, N, K, M, "large_n")
    p = w4.repack(w, s, N, K)
    yp = w4.gemv_prepacked(p, x, N, K, M)
    assert np.array_equal(down(yp).reshape(M, N), Y)
    for b in sorted({0, M // 2, M - 1}):
        assert np.array_equal(Y[b], run(w4, w, s, x[b:b + 1], N, K, 1)[0]), b


def test_repack_device_equals_host(w4, orc, dev):
    for N, K in ((1, 128), (37, 384), (1023, 1024), (16, 3584)):
        W, S, _ = orc.fixture_gemv(N * 7 + K, N, K)
        w, s, _ = up(dev, W, S, np.zeros((1, K), np.uint16))
        p = w4.repack(w, s, N, K)
        torch.cuda.synchronize()
        assert np.array_equal(p.cpu().numpy(), w4.repack_host(W, S, N, K)), (N, K)


def test_nondefault_stream(w4, orc, dev):
    N, K, M = 3584, 1024, 8
    W, S, X = orc.fixture_gemv(99, N, K)
    X = np.repeat(X, M, axis=0)
    w, s, x = up(dev, W, S, X)
    ref = run(w4, w, s, x, N, K, M)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.gemv(w, s, x, N, K, M, y=y, stream=st)
    st.synchronize()
    assert np.array_equal(down(y).reshape(M, N), ref)


def test_cpp_reference_names(w4, orc, dev):
    # int4_gemv_bf16 / batch_int4_gemv_bf16 in the reference's argument order
    N, K, B = 512, 1024, 3
    W, S, X = orc.fixture_kind("random", 0x9E3779B9, N, K, B)
    w, s, x = up(dev, W, S, X)
    y1 = torch.empty(N, dtype=torch.bfloat16, device=dev)
    w4.int4_gemv_bf16(w, s, x[0], y1, N, K)
    yb = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
    w4.batch_int4_gemv_bf16(w, s, x, yb, N, K, B)
    assert np.array_equal(down(yb).reshape(B, N)[0], down(y1).reshape(N))
    assert w4.int4_gemv_bf16_rowtile4_regs() > 0


@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 32, 40])
@pytest.mark.parametrize("packed", [False, True])
def test_multi_projection_equals_single(w4, orc, dev, M, packed):
    # one launch for projections sharing x (in_proj_qkv/z/b/a group shapes
    # plus a ragged N) == one call per projection, bit for bit
    K = 1024
    Ns = [6144, 2048, 16, 16, 37]
    x = torch.from_numpy(orc.synth_act(0x3317 + M, M, K).view(np.int16)).to(dev).view(torch.bfloat16)
    ws, ss, refs = [], [], []
    for j, N in enumerate(Ns):
        W, S = orc.synth_w4a16(0x7000 + 31 * j, N, K)
        w, s, _ = up(dev, W, S, np.zeros((1, K), np.uint16))
        if packed:
            w = w4.repack(w, s, N, K)
        ws.append(w)
        ss.append(s)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if packed:
            w4.gemv_prepacked(w, x, N, K, M, y=y)
        else:
            w4.gemv(w, s, x, N, K, M, y=y)
        refs.append(down(y).reshape(M, N))
    ys = w4.gemv_multi(ws, ss, x, Ns, K, M, prepacked=packed)
    for j, N in enumerate(Ns):
        assert np.array_equal(down(ys[j]).reshape(M, N), refs[j]), (j, N)


@pytest.mark.parametrize("Ns", [[3584, 3584], [4096, 512, 512], [6144, 2048, 16, 16], [37, 1000]])
@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("packed", [False, True])
def test_multi_projection_small_groups(w4, orc, dev, Ns, M, packed):
    # the fused groups of the census (gate/up, q/k/v, qkv/z/b/a) travel in a
    # table of 4: bit for bit equal to one call per projection
    K = 1024
    x = torch.from_numpy(orc.synth_act(0x4417 + M, M, K).view(np.int16)).to(dev).view(torch.bfloat16)
    ws, ss, refs = [], [], []
    for j, N in enumerate(Ns):
        W, S = orc.synth_w4a16(0x7100 + 17 * j + N, N, K)
        w, s, _ = up(dev, W, S, np.zeros((1, K), np.uint16))
        if packed:
            w = w4.repack(w, s, N, K)
        ws.append(w)
        ss.append(s)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if packed:
            w4.gemv_prepacked(w, x, N, K, M, y=y, variant="stream")
        else:
            w4.gemv(w, s, x, N, K, M, y=y, variant="stream")
        refs.append(down(y).reshape(M, N))
    ys = w4.gemv_multi(ws, ss, x, Ns, K, M, prepacked=packed)
    for j, N in enumerate(Ns):
        assert np.array_equal(down(ys[j]).reshape(M, N), refs[j]), (j, N)


def test_multi_projection_rejects_bad_count(w4, dev):
    x = torch.zeros((1, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        w4.gemv_multi([], [], x, [], 128, 1)


@pytest.mark.parametrize("N,K", [(37, 384), (5000, 640), (1000, 1152), (300, 3584), (200, 4096),
                                 (9000, 1024), (16, 128), (1024, 3584)])
@pytest.mark.parametrize("M", [1, 3, 8, 17, 24, 32])
def test_piece_split_equals_stream(w4, orc, dev, N, K, M):
    # the piece split (a tile's groups spread over up to 8 waves, the unit's
    # fma chain finished in group order by the reducing wave) against the
    # tile-serial stream kernel, bit for bit: one group per wave, pieces of
    # 2 on 4, 8 and 16 waves, pieces of 4; short last units (K/128 = 3, 5,
    # 9) and ragged last tiles; both weight layouts
    # where x does not fit the LDS the stream kernel cannot run; the piece
    # split with x in registers still serves auto, against the tile kernel
    ref = "stream" if VARIANTS_FOR_M["stream"](M, K) else "tile16"
    W, S = orc.synth_w4a16(0x5917 + N + K, N, K)
    X = orc.synth_act(0x5A + M, M, K)
    w, s, x = up(dev, W, S, X)
    Y = run(w4, w, s, x, N, K, M, ref)
    if M in (1, 17):
        assert_tol(orc, Y, W, S, X, N, K, M, ref)
    assert np.array_equal(run(w4, w, s, x, N, K, M), Y), "auto"
    p = w4.repack(w, s, N, K)
    for name in ("auto", "split") if ref == "stream" else ("auto",):
        yp = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.gemv_prepacked(p, x, N, K, M, y=yp, variant=name)
        assert np.array_equal(down(yp).reshape(M, N), Y), ("prepacked", name)


@pytest.mark.parametrize("N,bad", [(100003, False), (100002, False), (40000, False), (100008, False),
                                   (100008, True)])
@pytest.mark.parametrize("M", [17, 24, 31, 32])
def test_two_tile_stream_edges(w4, orc, dev, N, bad, M):
    # the stream kernel with two activation tiles (one projection, M =
    # 17..32, many tiles) against the tile kernel bit for bit: odd and even
    # N, ragged last tiles, masked rows (M < 32), y at an odd element, an
    # infinite activation (the reference loop's +-Inf / NaN outputs), and
    # the element past y left untouched
    K = 1024
    W, S = orc.synth_w4a16(0x9A1 + N, N, K)
    X = orc.synth_act(0x9A2 + M, M, K)
    if bad:
        X[M - 2, 77] = 0x7F80  # +Inf
    w, s, x = up(dev, W, S, X)
    ref = run(w4, w, s, x, N, K, M, "tile16")
    p = w4.repack(w, s, N, K)
    for shift in (0, 1):
        buf = torch.full((M * N + 2,), float("nan"), dtype=torch.bfloat16, device=dev)
        y = buf[shift:shift + M * N].view(M, N)
        w4.gemv_prepacked(p, x, N, K, M, y=y, variant="stream")
        assert np.array_equal(down(y).reshape(M, N), ref), ("shift", shift)
        assert torch.isnan(buf[shift + M * N]).item(), ("guard", shift)


@pytest.mark.parametrize("N,K", [(1000, 640), (77, 3584), (4100, 2176), (33, 1024), (2050, 2048),
                                 (248, 4096)])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_file_layout_whole_line_loads(w4, orc, dev, N, K, M):
    # file-layout weights at M <= 16 are loaded in whole lines and re-laid
    # out through LDS (stream: pieces of 4 groups; split: units of 8; piece
    # split: pieces of 2 or 4): every variant that applies, bit for bit
    # against the tile kernel, over ragged last tiles (row clamps) and short
    # last pieces and units (group clamps: K/128 = 5, 17, 28)
    W, S = orc.synth_w4a16(0xF1E0 + N + K, N, K)
    X = orc.synth_act(0xF1E1 + M, M, K)
    w, s, x = up(dev, W, S, X)
    ref = run(w4, w, s, x, N, K, M, "tile16")
    assert_tol(orc, ref, W, S, X, N, K, M, "file-layout")
    for name in ("auto", "stream", "split"):
        if name != "auto" and not VARIANTS_FOR_M[name](M, K):
            continue
        assert np.array_equal(run(w4, w, s, x, N, K, M, name), ref), name


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_auto_equals_tile(w4, orc, dev, seed):
    # seeded random shapes across the dispatch plans (piece split of every
    # plan, unit split, stream, prefill GEMM, 16-row passes): the tile
    # kernel within tolerance of the oracle, and the auto path, file layout
    # and prepacked bit for bit equal to it
    rng = np.random.default_rng(0xD15 + seed)
    for _ in range(6):
        K = 128 * int(rng.integers(1, 33))
        N = int(rng.integers(1, max(2, min(20000, (12 << 20) // K))))
        M = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 24, 32, 33, 48]))
        W, S = orc.synth_w4a16(int(rng.integers(1 << 30)), N, K)
        X = orc.synth_act(int(rng.integers(1 << 30)), M, K)
        w, s, x = up(dev, W, S, X)
        ref = run(w4, w, s, x, N, K, M, "tile16")
        # the shared decode / offset / epilogue code itself, against the oracle
        assert_tol(orc, ref, W, S, X, N, K, M, "random")
        got = run(w4, w, s, x, N, K, M)
        assert np.array_equal(got, ref), ("auto", N, K, M)
        p = w4.repack(w, s, N, K)
        yp = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        w4.gemv_prepacked(p, x, N, K, M, y=yp)
        assert np.array_equal(down(yp).reshape(M, N), ref), ("prepacked", N, K, M)
