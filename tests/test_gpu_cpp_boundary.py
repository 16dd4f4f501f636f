"""The C++ drop-in surface on the GPU, called the way the reference's runtime
calls it: tests/cpp/boundary_check (built by build(), compiled against
include/cudalm/ and linked with libcudalm_w4a16.so) runs
cudalm::int4_gemv_bf16, kernels::batch_int4_gemv_bf16, repack_w4a16_host /
repack_w4a16 -> w4a16_forward_bf16, bf16_gemv, kernels::batch_bf16_gemv,
int4_gemv, kernels::qwen35_silu_mul_bf16 and w4a16_swiglu_forward_bf16, and
a two-stage chain over the C ABI (cudalm_w4a16_chain_* and the allocation-free
entry), on device buffers (reference headers: include/cudalm/kernels/int4_gemv_bf16.h:46-52,
batch_decode.h:61-79, bf16_gemv.h:19-38, int4_gemv.h:22-40,
qwen35_kernels.h:146-155; weight_loader.h:58-63). Inputs and outputs pass
through files; every output is checked here against the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "boundary_check")


def _ulp_diff(a, b):
    """bf16 bit patterns -> distance in ulps (sign-magnitude order)."""
    def key(v):
        v = v.astype(np.int64)
        return np.where(v & 0x8000, 0x8000 - (v & 0x7FFF), 0x8000 + v)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("N,K,M", [(3584, 1024, 4), (1000, 384, 3)])
def test_cpp_boundary(orc, tmp_path, N, K, M):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/boundary_check is not built (run __graft_entry__.build())")
    W, S = orc.synth_w4a16(0xB0 + N, N, K)
    Wg, Sg = orc.synth_w4a16(0xB1 + N, N, K)
    Wu, Su = orc.synth_w4a16(0xB2 + N, N, K)
    X = orc.synth_act(0xB3 + M, M, K)
    E = orc.f32_to_bf16(orc.synth_normal(0xB4, 0.02, N * K)).reshape(N, K)
    Xh = np.random.default_rng(K).normal(0, 1, (1, K)).astype(np.float16).view(np.uint16)
    d = str(tmp_path)
    (tmp_path / "shape.txt").write_text(f"{N} {K} {M}\n")
    for name, a in (("W", W), ("S", S), ("X", X), ("Wg", Wg), ("Sg", Sg), ("Wu", Wu), ("Su", Su),
                    ("E", E), ("Xh", Xh)):
        np.ascontiguousarray(a).tofile(os.path.join(d, name + ".bin"))
    res = subprocess.run([BIN, d], capture_output=True, text=True, timeout=120)
    print(res.stdout + res.stderr, flush=True)
    assert res.returncode == 0, res.stderr

    def out(name, rows):
        return np.fromfile(os.path.join(d, name + ".bin"), np.uint16).reshape(rows, N)

    # W4A16: single call, batched call, both repack forms of the packed forward
    y1, yB = out("int4_gemv_bf16", 1), out("batch", M)
    ok, st = orc.check_tolerance(y1, W, S, X[:1], N, K, 1)
    assert ok, ("int4_gemv_bf16", st)
    ok, st = orc.check_tolerance(yB, W, S, X, N, K, M)
    assert ok, ("batch_int4_gemv_bf16", st)
    assert np.array_equal(yB[0], y1[0]), "row parity"
    assert np.array_equal(out("forward_host", M), yB)
    assert np.array_equal(out("forward_dev", M), yB)
    # the tied bf16 LM head
    e1, eB = out("bf16_gemv", 1), out("batch_bf16", M)
    ok, st = orc.check_bf16_tolerance(e1, E, X[:1], N, K, 1)
    assert ok, ("bf16_gemv", st)
    ok, st = orc.check_bf16_tolerance(eB, E, X, N, K, M)
    assert ok, ("batch_bf16_gemv", st)
    assert np.array_equal(eB[0], e1[0])
    # the fp16-activation twin
    ok, st = orc.check_f16_tolerance(out("int4_gemv", 1), W, S, Xh, N, K, 1)
    assert ok, ("int4_gemv", st)
    # MLP front half: gate / up against the oracle, silu*mul against the
    # oracle's restatement (device expf vs glibc expf: at most 1 ulp, rarely),
    # and the fused launch bit for bit equal to the three-step sequence
    g, u = out("gate", M), out("up", M)
    assert orc.check_tolerance(g, Wg, Sg, X, N, K, M)[0]
    assert orc.check_tolerance(u, Wu, Su, X, N, K, M)[0]
    sm = out("silu_mul", M)
    dd = _ulp_diff(sm, orc.silu_mul_bf16(g, u))
    assert dd.max() <= 1 and (dd != 0).sum() * 1000 <= dd.size, (int(dd.max()), int((dd != 0).sum()))
    assert np.array_equal(out("swiglu", M), sm)
    # stage chains over the C ABI, and the allocation-free entry: the bits of
    # the per-projection calls
    assert np.array_equal(out("chain_gate", M), g)
    assert np.array_equal(out("chain_up", M), u)
    assert np.array_equal(out("chain_w", M), yB)
    assert np.array_equal(out("noalloc_w", M), yB)
