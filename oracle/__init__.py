"""CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, always as the checker (never as the product path). numpy bindings over
liborc_w4a16.so (w4a16_oracle.c), which restates the reference's CPU path;
every C function cites the reference file:line it follows.

`ref` exposes the reference's own stage_compare.h, compiled from the
reference tree into _ref/ (None where that build is absent, e.g. on a GPU
box without /root/reference; the shared library itself does travel).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc_w4a16.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_stage_compare.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} missing; run `python oracle/build_oracle.py`")

_lib = ctypes.CDLL(LIB_PATH)
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SIGS = {
    "orc_fp16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "orc_f32_to_fp16_rne": ([ctypes.c_float], ctypes.c_uint16),
    "orc_bf16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "orc_f32_to_bf16_rne": ([ctypes.c_float], ctypes.c_uint16),
    "orc_fp16_to_f32_array": ([_P, _P, ctypes.c_size_t], None),
    "orc_f32_to_fp16_array": ([_P, _P, ctypes.c_size_t], None),
    "orc_f32_to_bf16_array": ([_P, _P, ctypes.c_size_t], None),
    "orc_pack_byte": ([ctypes.c_int, ctypes.c_int], ctypes.c_uint8),
    "orc_unpack_byte": ([ctypes.c_uint8, _P, _P], None),
    "orc_unpack": ([_P, _I64, _I64, _P], None),
    "orc_dequant": ([_P, _P, _I64, _I64, _P], None),
    "orc_quantize": ([_P, _I64, _I64, _P, _P], ctypes.c_int),
    "orc_gemv_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64], None),
    "orc_gemv_bf16_mt": ([_P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
    "orc_gemv_f64": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], None),
    "orc_gemv_f32acc_mt": ([_P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
    "orc_gemv_f64_mt": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
    "orc_xorshift32_fill": ([ctypes.c_uint32, _P, ctypes.c_size_t], None),
    "orc_fixture_gemv": ([ctypes.c_uint32, _I64, _I64, _P, _P, _P], None),
    "orc_fixture_kind": ([ctypes.c_int, ctypes.c_uint32, _I64, _I64, _I64, _P, _P, _P], None),
    "orc_synth_normal_f32": ([ctypes.c_uint64, ctypes.c_float, _P, ctypes.c_size_t], None),
    "orc_synth_w4a16": ([ctypes.c_uint64, ctypes.c_float, _I64, _I64, _P, _P], ctypes.c_int),
    "orc_synth_act_bf16": ([ctypes.c_uint64, _I64, _I64, _P], None),
    "orc_time_gemv_bf16": ([_P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int],
                           ctypes.c_double),
    "orc_hardware_threads": ([], ctypes.c_int),
    "orc_silu_bf16": ([ctypes.c_uint16], ctypes.c_uint16),
    "orc_silu_mul_bf16": ([_P, _P, _P, ctypes.c_size_t], None),
    "orc_gemv_f16": ([_P, _P, _P, _P, _I64, _I64, _I64], None),
    "orc_gemv_f16_f64": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], None),
    "orc_fixture_gemv_f16": ([ctypes.c_uint32, _I64, _I64, _P, _P, _P], None),
    "orc_bf16_fixture": ([ctypes.c_uint32, _I64, _I64, _P, _P], None),
    "orc_bf16_gemv": ([_P, _P, _P, _I64, _I64, _I64], None),
    "orc_bf16_gemv_mt": ([_P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
    "orc_bf16_gemv_f64": ([_P, _P, _P, _P, _I64, _I64, _I64], None),
    "orc_time_bf16_gemv": ([_P, _P, _P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int],
                           ctypes.c_double),
}
for _n, (_a, _r) in _SIGS.items():
    _f = getattr(_lib, _n)
    _f.argtypes = _a
    _f.restype = _r

KIND_RANDOM, KIND_ZERO, KIND_SMALL, KIND_MIXED_SIGN, KIND_BOUNDARY = range(5)
KINDS = {"random": 0, "zero": 1, "small": 2, "mixed_sign": 3, "boundary": 4}
# tests/cuda/test_w4a16_qwen35_optimized.cpp:456
REFERENCE_SEEDS = (0x51ED, 0x1234ABCD, 0x9E3779B9, 0xCAFEBABE)


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def lib():
    return _lib


# ---- formats ---------------------------------------------------------------

def fp16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    _lib.orc_fp16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_fp16(x) -> np.ndarray:
    f = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    _lib.orc_f32_to_fp16_array(_p(f), _p(out), f.size)
    return out


def f32_to_bf16(x) -> np.ndarray:
    f = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    _lib.orc_f32_to_bf16_array(_p(f), _p(out), f.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


# ---- int4 ------------------------------------------------------------------

def unpack_byte(b: int) -> tuple[int, int]:
    lo, hi = ctypes.c_int(), ctypes.c_int()
    _lib.orc_unpack_byte(b, ctypes.byref(lo), ctypes.byref(hi))
    return lo.value, hi.value


def pack_byte(lo: int, hi: int) -> int:
    return _lib.orc_pack_byte(lo, hi)


def unpack(W: np.ndarray, N: int, K: int) -> np.ndarray:
    q = np.empty((N, K), np.int8)
    _lib.orc_unpack(_p(W), N, K, _p(q))
    return q


def dequant(W: np.ndarray, S: np.ndarray, N: int, K: int) -> np.ndarray:
    out = np.empty((N, K), np.float32)
    _lib.orc_dequant(_p(W), _p(S), N, K, _p(out))
    return out


def quantize(Wf: np.ndarray):
    Wf = np.ascontiguousarray(Wf, dtype=np.float32)
    N, K = Wf.shape
    Wp = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // 128), np.uint16)
    rc = _lib.orc_quantize(_p(Wf), N, K, _p(Wp), _p(S))
    if rc != 0:
        raise ValueError("orc_quantize rejected the input")
    return Wp, S


# ---- gemv ------------------------------------------------------------------

def gemv_bf16(W, S, X, N: int, K: int, M: int = 1, nthreads: int = 1) -> np.ndarray:
    """ref_gemv_bf16 (tests/cuda/test_int4_gemv_bf16.cpp:54-69): bf16 bits [M, N]."""
    Y = np.empty((M, N), np.uint16)
    if nthreads > 1:
        _lib.orc_gemv_bf16_mt(_p(W), _p(S), _p(X), _p(Y), N, K, M, nthreads)
    else:
        _lib.orc_gemv_bf16(_p(W), _p(S), _p(X), _p(Y), N, K, M)
    return Y


def gemv_f32acc(W, S, X, N: int, K: int, M: int = 1, nthreads: int = 1) -> np.ndarray:
    """The fp32 accumulator of ref_gemv_bf16 (tests/cuda/test_int4_gemv_bf16.cpp:
    54-69) before its bf16 rounding, float32 [M, N]: the fp32-accumulated
    reference the 2-ulp bar is stated against."""
    Y = np.empty((M, N), np.float32)
    _lib.orc_gemv_f32acc_mt(_p(W), _p(S), _p(X), _p(Y), N, K, M, max(1, nthreads))
    return Y


def ulp_vs_fp32_reference(y_bits, acc) -> dict:
    """Distance of bf16 outputs from the reference loop's fp32 accumulator,
    in bf16 ulps at the accumulator's magnitude: max and count beyond 2."""
    acc = np.asarray(acc, np.float64)
    y = bf16_to_f32(np.asarray(y_bits, np.uint16).reshape(acc.shape)).astype(np.float64)
    d = np.abs(y - acc) / bf16_ulp(acc)
    return {"max_ulp_vs_fp32_ref": float(d.max()) if d.size else 0.0,
            "n_over_2ulp_vs_fp32_ref": int((d > 2.0).sum()), "n": int(d.size)}


def gemv_f64(W, S, X, N: int, K: int, M: int = 1, nthreads: int = 1):
    """fp64 sum of the exact fp32 terms and the sum of their magnitudes
    (rows split over `nthreads` threads; the values do not depend on it)."""
    Y = np.empty((M, N), np.float64)
    A = np.empty((M, N), np.float64)
    if nthreads > 1:
        _lib.orc_gemv_f64_mt(_p(W), _p(S), _p(X), _p(Y), _p(A), N, K, M, nthreads)
    else:
        _lib.orc_gemv_f64(_p(W), _p(S), _p(X), _p(Y), _p(A), N, K, M)
    return Y, A


def time_gemv_bf16(W, S, X, N, K, M, nthreads, iters) -> float:
    Y = np.empty((M, N), np.uint16)
    return _lib.orc_time_gemv_bf16(_p(W), _p(S), _p(X), _p(Y), N, K, M, nthreads, iters)


def hardware_threads() -> int:
    return _lib.orc_hardware_threads()


# ---- fixtures --------------------------------------------------------------

def xorshift32(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    _lib.orc_xorshift32_fill(seed, _p(out), n)
    return out


def fixture_gemv(seed: int, N: int, K: int):
    """test_int4_gemv_bf16.cpp:77-88: (W u8 [N,K/2], S fp16 bits [N,K/128], x bf16 bits [1,K])."""
    W = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // 128), np.uint16)
    X = np.empty((1, K), np.uint16)
    _lib.orc_fixture_gemv(seed, N, K, _p(W), _p(S), _p(X))
    return W, S, X


def fixture_kind(kind, seed: int, N: int, K: int, B: int = 1):
    """test_w4a16_qwen35_optimized.cpp:66-135: (W, S, X [B, K])."""
    if isinstance(kind, str):
        kind = KINDS[kind]
    W = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // 128), np.uint16)
    X = np.empty((B, K), np.uint16)
    _lib.orc_fixture_kind(kind, seed, N, K, B, _p(W), _p(S), _p(X))
    return W, S, X


def synth_normal(seed: int, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    _lib.orc_synth_normal_f32(seed, sigma, _p(out), n)
    return out


def synth_w4a16(seed: int, N: int, K: int, sigma: float = 0.02):
    """BASELINE weights: N(0, sigma) fp32 -> reference quantizer."""
    W = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // 128), np.uint16)
    rc = _lib.orc_synth_w4a16(seed, sigma, N, K, _p(W), _p(S))
    if rc != 0:
        raise RuntimeError(f"orc_synth_w4a16 failed ({rc})")
    return W, S


def synth_act(seed: int, M: int, K: int) -> np.ndarray:
    X = np.empty((M, K), np.uint16)
    _lib.orc_synth_act_bf16(seed, M, K, _p(X))
    return X


# ---- tolerance -------------------------------------------------------------

def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (the unit in the last place)."""
    a = np.abs(np.asarray(v, np.float64))
    tiny = 2.0 ** -133  # smallest bf16 subnormal spacing
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.maximum(2.0 ** (e - 7), tiny)


# Floor for outputs whose terms cancel: a bound on fp32 accumulation error
# relative to sum_k |q s x| (2^-24 per add over a 256-deep effective chain).
CANCEL_FLOOR = 2.0 ** -16


def check_against_reference_loop(y_bits, W, S, X, N, K, M, nthreads: int = 1, slack: int = 0):
    """The W4A16 gate for the BASELINE workloads: (ok, stats, ref_stats).
    ok iff y is within the check_tolerance bound and has at most `slack`
    more outputs beyond 2 bf16 ulp of the fp64 value than the reference's
    own fp32 CPU loop (ref_gemv_bf16) has on the same inputs. Those are
    outputs whose terms cancel; the two accumulation orders round them
    differently, so on one shape either side can have one more."""
    r, a = gemv_f64(W, S, X, N, K, M, nthreads)
    ok, st = check_tolerance_f64(y_bits, r, a, M, N)
    _, sr = check_tolerance_f64(gemv_bf16(W, S, X, N, K, M, nthreads), r, a, M, N)
    st["ref_max_ulp"], st["ref_n_over_2ulp"] = sr["max_ulp"], sr["n_over_2ulp"]
    return ok and st["n_over_2ulp"] <= sr["n_over_2ulp"] + slack, st, sr


def full_parity(y_bits, W, S, X, N, K, M, nthreads: int = 1):
    """Every W4A16 parity figure of one output block, each sum computed once:
    (ok, stats). ok iff (a) every output is within check_tolerance's bound
    of the fp64 sum and (b) within 2 bf16 ulps of the reference loop's fp32
    accumulator plus both fp32 sums' accumulation error (2 * CANCEL_FLOOR *
    sum|terms|). stats: check_tolerance_f64's figures, the reference loop's
    ref_max_ulp / ref_n_over_2ulp against the fp64 sum, and
    ulp_vs_fp32_reference's max / count beyond 2."""
    r, a = gemv_f64(W, S, X, N, K, M, nthreads)
    ok, st = check_tolerance_f64(y_bits, r, a, M, N)
    acc = gemv_f32acc(W, S, X, N, K, M, nthreads)
    _, sr = check_tolerance_f64(f32_to_bf16(acc), r, a, M, N)
    st["ref_max_ulp"], st["ref_n_over_2ulp"] = sr["max_ulp"], sr["n_over_2ulp"]
    st.update(ulp_vs_fp32_reference(y_bits, acc))
    y = bf16_to_f32(np.asarray(y_bits, np.uint16).reshape(M, N)).astype(np.float64)
    lim = 2.0 * bf16_ulp(acc) + 2.0 * CANCEL_FLOOR * a
    st["n_bad_vs_fp32_ref"] = int((~(np.abs(y - acc.astype(np.float64)) <= lim)).sum())
    return ok and st["n_bad_vs_fp32_ref"] == 0, st


def check_tolerance(y_bits, W, S, X, N, K, M, ulps: float = 2.0, nthreads: int = 1):
    """Pass iff |y - r| <= ulps * ulp_bf16(r) + CANCEL_FLOOR * sum|terms|,
    r = fp64 sum of the exact fp32 terms. Returns (ok, stats dict)."""
    r, a = gemv_f64(W, S, X, N, K, M, nthreads)
    return check_tolerance_f64(y_bits, r, a, M, N, ulps)


# ---- fp16-activation twin (int4_gemv) ----------------------------------------

def fixture_gemv_f16(seed: int, N: int, K: int):
    """test_int4_gemv.cpp:70-83: (W u8, S fp16 bits, x fp16 bits [1, K])."""
    W = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // 128), np.uint16)
    X = np.empty((1, K), np.uint16)
    _lib.orc_fixture_gemv_f16(seed, N, K, _p(W), _p(S), _p(X))
    return W, S, X


def gemv_f16(W, S, X, N: int, K: int, M: int = 1) -> np.ndarray:
    """ref_gemv of test_int4_gemv.cpp:49-63, M rows: fp16 bits [M, N]."""
    Y = np.empty((M, N), np.uint16)
    _lib.orc_gemv_f16(_p(W), _p(S), _p(X), _p(Y), N, K, M)
    return Y


def gemv_f16_f64(W, S, X, N: int, K: int, M: int = 1):
    Y = np.empty((M, N), np.float64)
    A = np.empty((M, N), np.float64)
    _lib.orc_gemv_f16_f64(_p(W), _p(S), _p(X), _p(Y), _p(A), N, K, M)
    return Y, A


def fp16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of fp16 numbers at |v| (subnormal spacing 2^-24 below 2^-14)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def check_f16_tolerance(y_bits, W, S, X, N, K, M, ulps: float = 2.0):
    """|y - r| <= ulps * ulp_fp16(r) + CANCEL_FLOOR * sum|terms| for finite
    r within the fp16 range; outputs whose exact value overflows fp16 must
    be infinities of the right sign."""
    r, a = gemv_f16_f64(W, S, X, N, K, M)
    y = fp16_to_f32(np.asarray(y_bits, np.uint16).reshape(M, N)).astype(np.float64)
    big = np.abs(r) >= 65520.0  # rounds to +-inf in fp16
    err = np.abs(y - r)
    tol = ulps * fp16_ulp(r) + CANCEL_FLOOR * a
    bad = ~(err <= tol) & ~big
    bad |= big & ~(np.isinf(y) & (np.sign(y) == np.sign(r)))
    ulp_dist = np.where(big, 0.0, err / fp16_ulp(r))
    # the reference's own fp32 loop (ref_gemv) measured the same way, for scale
    yr = fp16_to_f32(gemv_f16(W, S, X, N, K, M)).astype(np.float64)
    ref_ulp = np.where(big, 0.0, np.abs(yr - r) / fp16_ulp(r))
    stats = {"max_ulp": float(ulp_dist.max()) if err.size else 0.0, "n_bad": int(bad.sum()),
             "n_over_2ulp": int((ulp_dist > 2.0).sum()), "n": int(err.size),
             "ref_max_ulp": float(ref_ulp.max()) if err.size else 0.0}
    return not bad.any(), stats


# ---- SwiGLU element-wise stage ---------------------------------------------

def silu_bf16(g_bits) -> np.ndarray:
    g = np.ascontiguousarray(g_bits, np.uint16)
    return np.array([_lib.orc_silu_bf16(int(v)) for v in g.ravel()], np.uint16).reshape(g.shape)


def silu_mul_bf16(gate, up) -> np.ndarray:
    """qwen35_silu_mul_kernel (qwen35_kernels.cu:458-476) on bf16 bit arrays."""
    g = np.ascontiguousarray(gate, np.uint16)
    u = np.ascontiguousarray(up, np.uint16)
    assert g.shape == u.shape
    y = np.empty(g.shape, np.uint16)
    _lib.orc_silu_mul_bf16(_p(g), _p(u), _p(y), g.size)
    return y


# ---- bf16 GEMV (tied LM head) ----------------------------------------------

def bf16_fixture(seed: int, N: int, K: int):
    """test_bf16_gemv.cpp:44-57: (W bf16 bits [N, K], x bf16 bits [1, K])."""
    W = np.empty((N, K), np.uint16)
    X = np.empty((1, K), np.uint16)
    _lib.orc_bf16_fixture(seed, N, K, _p(W), _p(X))
    return W, X


def bf16_gemv(W, X, N: int, K: int, M: int = 1, nthreads: int = 1) -> np.ndarray:
    """ref_gemv_bf16 of test_bf16_gemv.cpp:62-73, M rows: bf16 bits [M, N]."""
    Y = np.empty((M, N), np.uint16)
    if nthreads > 1:
        _lib.orc_bf16_gemv_mt(_p(W), _p(X), _p(Y), N, K, M, nthreads)
    else:
        _lib.orc_bf16_gemv(_p(W), _p(X), _p(Y), N, K, M)
    return Y


def bf16_gemv_f64(W, X, N: int, K: int, M: int = 1):
    Y = np.empty((M, N), np.float64)
    A = np.empty((M, N), np.float64)
    _lib.orc_bf16_gemv_f64(_p(W), _p(X), _p(Y), _p(A), N, K, M)
    return Y, A


def time_bf16_gemv(W, X, N, K, M, nthreads, iters) -> float:
    Y = np.empty((M, N), np.uint16)
    return _lib.orc_time_bf16_gemv(_p(W), _p(X), _p(Y), N, K, M, nthreads, iters)


def check_tolerance_f64(y_bits, r, a, M, N, ulps: float = 2.0):
    """Pass iff |y - r| <= ulps * ulp_bf16(r) + CANCEL_FLOOR * a for the exact
    sum r and the magnitude sum a. Returns (ok, stats dict)."""
    y = bf16_to_f32(np.asarray(y_bits, np.uint16).reshape(M, N)).astype(np.float64)
    err = np.abs(y - r)
    tol = ulps * bf16_ulp(r) + CANCEL_FLOOR * a
    bad = ~(err <= tol)
    ulp_dist = err / bf16_ulp(r)
    stats = {
        "max_abs_err": float(err.max()) if err.size else 0.0,
        "max_ulp": float(ulp_dist.max()) if err.size else 0.0,
        "n_bad": int(bad.sum()),
        "n_over_2ulp": int((ulp_dist > 2.0).sum()),
        "n": int(err.size),
    }
    return not bad.any(), stats


def check_bf16_tolerance(y_bits, W, X, N, K, M, ulps: float = 2.0):
    r, a = bf16_gemv_f64(W, X, N, K, M)
    return check_tolerance_f64(y_bits, r, a, M, N, ulps)


def check_bf16_against_reference_loop(y_bits, W, X, N, K, M, nthreads: int = 1, slack: int = 0):
    """check_against_reference_loop for the bf16 GEMV (ref_gemv_bf16 of
    tests/cuda/test_bf16_gemv.cpp:62-73 as the reference loop)."""
    r, a = bf16_gemv_f64(W, X, N, K, M)
    ok, st = check_tolerance_f64(y_bits, r, a, M, N)
    _, sr = check_tolerance_f64(bf16_gemv(W, X, N, K, M, nthreads), r, a, M, N)
    st["ref_max_ulp"], st["ref_n_over_2ulp"] = sr["max_ulp"], sr["n_over_2ulp"]
    return ok and st["n_over_2ulp"] <= sr["n_over_2ulp"] + slack, st, sr


# ---- the reference's own comparator (oracle/_ref) ---------------------------

class _Ref:
    def __init__(self, path: str):
        self.lib = ctypes.CDLL(path)
        self.lib.ref_fp16_bits_to_f32.argtypes = [ctypes.c_uint16]
        self.lib.ref_fp16_bits_to_f32.restype = ctypes.c_float
        self.lib.ref_fp16_bits_to_f32_bits.argtypes = [ctypes.c_uint16]
        self.lib.ref_fp16_bits_to_f32_bits.restype = ctypes.c_uint32
        self.lib.ref_bf16_bits_to_f32.argtypes = [ctypes.c_uint16]
        self.lib.ref_bf16_bits_to_f32.restype = ctypes.c_float
        self.lib.ref_compare_bf16_stages.argtypes = [_P, _P, ctypes.c_size_t, ctypes.c_double,
                                                     ctypes.c_double, _P, _P]
        self.lib.ref_compare_bf16_stages.restype = ctypes.c_int
        self.lib.ref_compare_fp16_stages.argtypes = self.lib.ref_compare_bf16_stages.argtypes
        self.lib.ref_compare_fp16_stages.restype = ctypes.c_int

    def fp16_to_f32(self, h: int) -> float:
        return self.lib.ref_fp16_bits_to_f32(h)

    def fp16_to_f32_bits(self, h: int) -> int:
        return self.lib.ref_fp16_bits_to_f32_bits(h)

    def compare_bf16_stages(self, ref_bits, act_bits, atol=1e-2, rtol=1e-2):
        r = np.ascontiguousarray(ref_bits, np.uint16).ravel()
        a = np.ascontiguousarray(act_bits, np.uint16).ravel()
        mx = ctypes.c_double()
        idx = ctypes.c_size_t()
        ok = self.lib.ref_compare_bf16_stages(_p(r), _p(a), r.size, atol, rtol, ctypes.byref(mx),
                                              ctypes.byref(idx))
        return bool(ok), mx.value, idx.value


    def compare_fp16_stages(self, ref_bits, act_bits, atol=1e-2, rtol=1e-2):
        r = np.ascontiguousarray(ref_bits, np.uint16).ravel()
        a = np.ascontiguousarray(act_bits, np.uint16).ravel()
        mx = ctypes.c_double()
        idx = ctypes.c_size_t()
        ok = self.lib.ref_compare_fp16_stages(_p(r), _p(a), r.size, atol, rtol, ctypes.byref(mx),
                                              ctypes.byref(idx))
        return bool(ok), mx.value, idx.value


ref = _Ref(REF_LIB_PATH) if os.path.exists(REF_LIB_PATH) else None
