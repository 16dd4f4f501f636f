"""Python host layer over the W4A16 engine's C ABI (include/cudalm_w4a16.h).

Mirrors the reference's W4A16 operator interface for tests, the smoke check
and benchmarks:

  int4_gemv_bf16(weight, scales, x, y, N, K)              int4_gemv_bf16.h:46-48
  batch_int4_gemv_bf16(weight, scale, x, y, N, K, B)      batch_decode.h:61-63
  int4_gemv_bf16_rowtile4_regs()                          int4_gemv_bf16.h:52
  bf16_gemv(weight, x, y, N, K)                           bf16_gemv.h:37-38
  batch_bf16_gemv(weight, x, y, N, K, B)                  batch_decode.h:77-79

plus the load-time repack and the prepacked path. Arguments are torch
tensors on the GPU (torch provides device memory and the stream; all
arithmetic runs in the HIP library). Precondition violations raise
ValueError (the reference aborts); launch failures raise RuntimeError.
There is no fallback: if libcudalm_w4a16.so is missing, importing this
module raises ImportError.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcudalm_w4a16.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `python cudalm-agent_amd/build.py` "
        "(or __graft_entry__.build()) first")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGS = {
    "cudalm_w4a16_version": ([], _I),
    "cudalm_w4a16_strerror": ([_I], ctypes.c_char_p),
    "cudalm_w4a16_gemv_bf16": ([_P, _P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_gemv_bf16_variant": ([_P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "cudalm_w4a16_packed_bytes": ([_I, _I], _SZ),
    "cudalm_w4a16_repack": ([_P, _P, _P, _I, _I, _P], _I),
    "cudalm_w4a16_repack_host": ([_P, _P, _P, _I, _I], _I),
    "cudalm_w4a16_gemv_bf16_prepacked": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_gemv_bf16_prepacked_variant": ([_P, _P, _P, _I, _I, _I, _I, _P], _I),
    "cudalm_w4a16_dequant_f32": ([_P, _P, _P, _P, _I, _I, _P], _I),
    "cudalm_w4a16_gemv_bf16_multi": ([_P, _I, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_kernel_regs": ([_I], _I),
    "cudalm_w4a16_gemv_f16": ([_P, _P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_gemv_f16_prepacked": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_swiglu_bf16": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "cudalm_silu_mul_bf16": ([_P, _P, _P, _SZ, _P], _I),
    "cudalm_bf16_gemv": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_v2_open": ([ctypes.c_char_p, _P, ctypes.c_char_p, _SZ], _I),
    "cudalm_v2_close": ([_P], None),
    "cudalm_v2_num_tensors": ([_P], _I),
    "cudalm_v2_tensor_at": ([_P, _I, _P], _I),
    "cudalm_v2_find": ([_P, ctypes.c_char_p, _P], _I),
    "cudalm_v2_meta": ([_P, ctypes.c_char_p], ctypes.c_char_p),
    "cudalm_v2_get_config": ([_P, _P], _I),
    "cudalm_v2_validate_layer": ([_P, _I, ctypes.c_char_p, _SZ], _I),
    "cudalm_v2_w4a16_shape": ([_P, ctypes.c_char_p, _P, _P], _I),
    "cudalm_v2_upload_w4a16_packed": ([_P, ctypes.c_char_p, _P, _SZ, _P], _I),
    "cudalm_v2_upload": ([_P, ctypes.c_char_p, _P, _SZ, _P], _I),
    "cudalm_bf16_gemv_variant": ([_P, _P, _P, _I, _I, _I, _I, _P], _I),
    "cudalm_bf16_gemv_kernel_regs": ([_I], _I),
    "cudalm_bf16_packed_bytes": ([_I, _I], _SZ),
    "cudalm_bf16_repack": ([_P, _P, _I, _I, _P], _I),
    "cudalm_bf16_gemv_prepacked": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "cudalm_w4a16_chain_workspace_bytes": ([_I], _SZ),
    "cudalm_w4a16_chain_plan": ([_P, _I, _I, _I, _P, _SZ, _P, _P], _I),
    "cudalm_w4a16_chain_run": ([_P, _P], _I),
    "cudalm_w4a16_chain_status": ([_P, _P], _I),
    "cudalm_w4a16_chain_set_wait_bound": ([_P, ctypes.c_uint32, _P], _I),
    "cudalm_w4a16_gemv_bf16_chain": ([_P, _I, _I, _I, _P, _SZ, _P], _I),
    "cudalm_w4a16_gemv_bf16_chain_noalloc": ([_P, _I, _I, _I, _P], _I),
}
for _name, (_args, _ret) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _ret

EXPORTED_SYMBOLS = tuple(_SIGS)

OK = 0
EINVAL = -1
ENULL = -2
EALIGN = -3
ELAUNCH = -4
ERANGE = -5
EVARIANT = -6
V2_EFORMAT = -7
V2_EIO = -8
V2_ENOTFOUND = -9
ETIMEOUT = -10

VARIANT_AUTO = 0
VARIANT_STREAM = 1
VARIANT_TILE16 = 2
VARIANT_TILE32 = 3
VARIANT_PREFILL = 4
VARIANT_BYTEWISE = 5
VARIANT_SPLIT = 6
VARIANT_SWIGLU = 7  # kernel_regs only
VARIANT_PREFILL32 = 8
VARIANTS = {
    "split": VARIANT_SPLIT,
    "auto": VARIANT_AUTO,
    "stream": VARIANT_STREAM,
    "tile16": VARIANT_TILE16,
    "tile32": VARIANT_TILE32,
    "prefill": VARIANT_PREFILL,
    "prefill32": VARIANT_PREFILL32,
    "bytewise": VARIANT_BYTEWISE,
}

BF16_VARIANT_AUTO = 0
BF16_VARIANT_STREAM = 1
BF16_VARIANT_SCALAR = 2
BF16_VARIANTS = {"auto": BF16_VARIANT_AUTO, "stream": BF16_VARIANT_STREAM,
                 "scalar": BF16_VARIANT_SCALAR}

GROUP = 128
MAX_PROJ = 8
MAX_STAGES = 256


class Proj(ctypes.Structure):
    """struct cudalm_w4a16_proj (include/cudalm_w4a16.h)."""
    _fields_ = [("weight", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("N", ctypes.c_int)]


class Stage(ctypes.Structure):
    """struct cudalm_w4a16_stage (include/cudalm_w4a16.h)."""
    _fields_ = [("projs", ctypes.c_void_p), ("count", ctypes.c_int), ("x", ctypes.c_void_p),
                ("K", ctypes.c_int), ("dep", ctypes.c_int), ("act", ctypes.c_void_p)]


class ChainHandle(ctypes.Structure):
    """struct cudalm_w4a16_chain (include/cudalm_w4a16.h), filled by the plan."""
    _fields_ = [("workspace", ctypes.c_void_p), ("n_stages", ctypes.c_int), ("M", ctypes.c_int),
                ("prepacked", ctypes.c_int), ("grid", ctypes.c_int), ("gt_max", ctypes.c_int)]


class W4A16Error(RuntimeError):
    def __init__(self, code: int, entry: str):
        self.code = code
        super().__init__(f"{entry}: {strerror(code)} (code {code})")


def lib() -> ctypes.CDLL:
    return _lib


def version() -> int:
    return _lib.cudalm_w4a16_version()


def strerror(code: int) -> str:
    return _lib.cudalm_w4a16_strerror(code).decode()


def _check(rc: int, entry: str) -> None:
    if rc == OK:
        return
    if rc in (EINVAL, ENULL, EALIGN, ERANGE, EVARIANT):
        raise ValueError(f"{entry}: {strerror(rc)} (code {rc})")
    raise W4A16Error(rc, entry)


def _ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def _stream(stream) -> int | None:
    import torch  # noqa: F401  (torch owns the streams)

    if isinstance(stream, int):
        return stream  # a raw hipStream_t (0 = the null stream)
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def packed_bytes(N: int, K: int) -> int:
    return _lib.cudalm_w4a16_packed_bytes(N, K)


def kernel_regs(variant: int = VARIANT_STREAM) -> int:
    return _lib.cudalm_w4a16_kernel_regs(variant)


# ---------------------------------------------------------------------------
# raw-pointer layer (addresses are plain ints; used by the C-ABI tests)
# ---------------------------------------------------------------------------

def gemv_ptr(w: int, s: int, x: int, y: int, N: int, K: int, M: int,
             variant: int = VARIANT_AUTO, stream: int | None = None) -> int:
    return _lib.cudalm_w4a16_gemv_bf16_variant(w, s, x, y, N, K, M, variant, stream)


def prepacked_ptr(p: int, x: int, y: int, N: int, K: int, M: int,
                  variant: int = VARIANT_AUTO, stream: int | None = None) -> int:
    return _lib.cudalm_w4a16_gemv_bf16_prepacked_variant(p, x, y, N, K, M, variant, stream)


# ---------------------------------------------------------------------------
# tensor layer
# ---------------------------------------------------------------------------

def _out(y, M: int, N: int, like):
    import torch

    if y is None:
        y = torch.empty((M, N) if M > 1 else (N,), dtype=torch.bfloat16, device=like.device)
    return y


def gemv(weight, scale, x, N: int, K: int, M: int = 1, y=None, variant: int | str = VARIANT_AUTO,
         stream=None):
    """y[M, N] = W4A16(weight[N, K/2] u8, scale[N, K/128] fp16) @ x[M, K] bf16."""
    if isinstance(variant, str):
        variant = VARIANTS[variant]
    y = _out(y, M, N, x)
    rc = _lib.cudalm_w4a16_gemv_bf16_variant(_ptr(weight), _ptr(scale), _ptr(x), _ptr(y), N, K, M,
                                             variant, _stream(stream))
    _check(rc, "cudalm_w4a16_gemv_bf16")
    return y


def int4_gemv_bf16(weight, scales, x, y, N: int, K: int, stream=None):
    """Reference name and argument order (int4_gemv_bf16.h:46-48)."""
    return gemv(weight, scales, x, N, K, 1, y=y, stream=stream)


def batch_int4_gemv_bf16(weight, scale, x, y, N: int, K: int, B: int, stream=None):
    """Reference name and argument order (batch_decode.h:61-63)."""
    return gemv(weight, scale, x, N, K, B, y=y, stream=stream)


def int4_gemv_bf16_rowtile4_regs() -> int:
    return kernel_regs(VARIANT_STREAM)


def repack(weight, scale, N: int, K: int, out=None, stream=None):
    """Device-side load-time repack; returns a uint8 tensor of packed_bytes(N, K)."""
    import torch

    if out is None:
        out = torch.empty(packed_bytes(N, K), dtype=torch.uint8, device=weight.device)
    rc = _lib.cudalm_w4a16_repack(_ptr(weight), _ptr(scale), _ptr(out), N, K, _stream(stream))
    _check(rc, "cudalm_w4a16_repack")
    return out


def repack_host(weight_np, scale_bits_np, N: int, K: int):
    """Host-side repack of numpy arrays (uint8 [N, K/2], uint16 [N, K/128])."""
    import numpy as np

    w = np.ascontiguousarray(weight_np, dtype=np.uint8)
    s = np.ascontiguousarray(scale_bits_np, dtype=np.uint16)
    out = np.empty(packed_bytes(N, K), dtype=np.uint8)
    rc = _lib.cudalm_w4a16_repack_host(w.ctypes.data, s.ctypes.data, out.ctypes.data, N, K)
    _check(rc, "cudalm_w4a16_repack_host")
    return out


def gemv_prepacked(packed, x, N: int, K: int, M: int = 1, y=None,
                   variant: int | str = VARIANT_AUTO, stream=None):
    if isinstance(variant, str):
        variant = VARIANTS[variant]
    y = _out(y, M, N, x)
    rc = _lib.cudalm_w4a16_gemv_bf16_prepacked_variant(_ptr(packed), _ptr(x), _ptr(y), N, K, M,
                                                       variant, _stream(stream))
    _check(rc, "cudalm_w4a16_gemv_bf16_prepacked")
    return y


def dequant(weight, scale, N: int, K: int, want_q: bool = True, want_w: bool = True, stream=None):
    """(q int8 [N, K], w fp32 [N, K]) through the kernels' nibble decoder."""
    import torch

    q = torch.empty((N, K), dtype=torch.int8, device=weight.device) if want_q else None
    w = torch.empty((N, K), dtype=torch.float32, device=weight.device) if want_w else None
    rc = _lib.cudalm_w4a16_dequant_f32(_ptr(weight), _ptr(scale), _ptr(q), _ptr(w), N, K,
                                       _stream(stream))
    _check(rc, "cudalm_w4a16_dequant_f32")
    return q, w


def proj_array(items):
    """items: (weight_ptr, scale_ptr_or_None, y_ptr, N) -> ctypes array of Proj."""
    arr = (Proj * len(items))()
    for k, (w, sc, y, n) in enumerate(items):
        arr[k].weight, arr[k].scale, arr[k].y, arr[k].N = w, sc, y, n
    return arr


def gemv_multi(weights, scales, x, Ns, K: int, M: int = 1, ys=None, prepacked: bool = False,
               stream=None):
    """Several projections sharing x in one launch; returns the list of y."""
    import torch

    if ys is None:
        ys = [torch.empty((M, n), dtype=torch.bfloat16, device=x.device) for n in Ns]
    items = [(_ptr(w), None if (prepacked or s is None) else _ptr(s), _ptr(y), n)
             for w, s, y, n in zip(weights, scales if scales is not None else [None] * len(Ns), ys, Ns)]
    arr = proj_array(items)
    rc = _lib.cudalm_w4a16_gemv_bf16_multi(ctypes.cast(arr, ctypes.c_void_p), len(items), _ptr(x),
                                           K, M, int(prepacked), _stream(stream))
    _check(rc, "cudalm_w4a16_gemv_bf16_multi")
    return ys


class Chain:
    """A planned stage chain (cudalm_w4a16_chain_plan) and its workspace.

    stages: list of (items, x, K, dep) or (items, x, K, dep, act) with items
    a list of (weight_ptr, scale_ptr_or_None, y_ptr, N) sharing x (a tensor
    or a raw address); dep is the index of an earlier stage or -1; act (a
    tensor or address, or None) makes the stage a SwiGLU stage: items are
    gate and up, and act = silu(gate(x)) * up(x) is its only output. run()
    is one kernel launch (capturable); status() synchronizes and raises
    W4A16Error on a timed-out wait."""

    def __init__(self, stages, M: int, prepacked: bool = True, device=None, stream=None):
        import torch

        stages = [tuple(sg) + (None,) * (5 - len(sg)) for sg in stages]
        self._arrays = [proj_array(sg[0]) for sg in stages]
        st = (Stage * len(stages))()
        for k, ((items, x, K, dep, act), arr) in enumerate(zip(stages, self._arrays)):
            st[k].projs = ctypes.cast(arr, ctypes.c_void_p)
            st[k].count = len(items)
            st[k].x = x if isinstance(x, int) else _ptr(x)
            st[k].K = K
            st[k].dep = dep
            st[k].act = act if (act is None or isinstance(act, int)) else _ptr(act)
        self._stages = st
        nbytes = _lib.cudalm_w4a16_chain_workspace_bytes(len(stages))
        if nbytes == 0:
            raise ValueError(f"chain of {len(stages)} stages: at most {MAX_STAGES}")
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=device or "cuda")
        self.handle = ChainHandle()
        rc = _lib.cudalm_w4a16_chain_plan(ctypes.cast(st, ctypes.c_void_p), len(stages), M,
                                          int(prepacked), self.workspace.data_ptr(), nbytes,
                                          ctypes.byref(self.handle), _stream(stream))
        _check(rc, "cudalm_w4a16_chain_plan")

    def run(self, stream=None) -> None:
        _check(_lib.cudalm_w4a16_chain_run(ctypes.byref(self.handle), _stream(stream)),
               "cudalm_w4a16_chain_run")

    def status(self, stream=None) -> None:
        _check(_lib.cudalm_w4a16_chain_status(ctypes.byref(self.handle), _stream(stream)),
               "cudalm_w4a16_chain_status")

    def set_wait_bound(self, ticks: int, stream=None) -> None:
        """Bound of every wait of later runs, in 100 MHz s_memrealtime ticks
        (0 = the default, ~0.5 s)."""
        _check(_lib.cudalm_w4a16_chain_set_wait_bound(ctypes.byref(self.handle), ticks,
                                                      _stream(stream)),
               "cudalm_w4a16_chain_set_wait_bound")


# ---------------------------------------------------------------------------
# fp16-activation twin (int4_gemv)
# ---------------------------------------------------------------------------

def gemv_f16(weight, scale, x, N: int, K: int, M: int = 1, y=None, stream=None):
    """y[M, N] fp16 = W4A16(weight, scale) @ x[M, K] fp16."""
    import torch

    if y is None:
        y = torch.empty((M, N) if M > 1 else (N,), dtype=torch.float16, device=x.device)
    rc = _lib.cudalm_w4a16_gemv_f16(_ptr(weight), _ptr(scale), _ptr(x), _ptr(y), N, K, M,
                                    _stream(stream))
    _check(rc, "cudalm_w4a16_gemv_f16")
    return y


def gemv_f16_prepacked(packed, x, N: int, K: int, M: int = 1, y=None, stream=None):
    import torch

    if y is None:
        y = torch.empty((M, N) if M > 1 else (N,), dtype=torch.float16, device=x.device)
    rc = _lib.cudalm_w4a16_gemv_f16_prepacked(_ptr(packed), _ptr(x), _ptr(y), N, K, M,
                                              _stream(stream))
    _check(rc, "cudalm_w4a16_gemv_f16_prepacked")
    return y


def int4_gemv(weight, scales, x, y, N: int, K: int, stream=None):
    """Reference name and argument order (int4_gemv.h:39-40)."""
    return gemv_f16(weight, scales, x, N, K, 1, y=y, stream=stream)


# ---------------------------------------------------------------------------
# SwiGLU: fused gate/up + silu*mul, and the element-wise stage
# ---------------------------------------------------------------------------

def swiglu(gate_w, gate_s, up_w, up_s, x, N: int, K: int, M: int = 1, y=None,
           prepacked: bool = False, stream=None):
    """y[M, N] = silu(gate(x)) * up(x), one launch (bf16 roundings of the
    reference's gate -> up -> qwen35_silu_mul_bf16 sequence)."""
    y = _out(y, M, N, x)
    rc = _lib.cudalm_w4a16_swiglu_bf16(_ptr(gate_w), _ptr(gate_s), _ptr(up_w), _ptr(up_s),
                                       _ptr(x), _ptr(y), N, K, M, int(prepacked), _stream(stream))
    _check(rc, "cudalm_w4a16_swiglu_bf16")
    return y


def qwen35_silu_mul_bf16(gate, up, y, n: int, stream=None):
    """Reference name and argument order (qwen35_kernels.h:146-155)."""
    rc = _lib.cudalm_silu_mul_bf16(_ptr(gate), _ptr(up), _ptr(y), n, _stream(stream))
    _check(rc, "cudalm_silu_mul_bf16")
    return y


# ---------------------------------------------------------------------------
# bf16 GEMV (tied LM head), include/cudalm_bf16_gemv.h
# ---------------------------------------------------------------------------

def bf16_gemv_ptr(w: int, x: int, y: int, N: int, K: int, M: int,
                  variant: int = BF16_VARIANT_AUTO, stream: int | None = None) -> int:
    return _lib.cudalm_bf16_gemv_variant(w, x, y, N, K, M, variant, stream)


def bf16_gemv_any(weight, x, N: int, K: int, M: int = 1, y=None,
                  variant: int | str = BF16_VARIANT_AUTO, stream=None):
    """y[M, N] = weight[N, K] bf16 @ x[M, K] bf16 (fp32 accumulation)."""
    if isinstance(variant, str):
        variant = BF16_VARIANTS[variant]
    y = _out(y, M, N, x)
    rc = _lib.cudalm_bf16_gemv_variant(_ptr(weight), _ptr(x), _ptr(y), N, K, M, variant,
                                       _stream(stream))
    _check(rc, "cudalm_bf16_gemv")
    return y


def bf16_repack(weight, N: int, K: int, out=None, stream=None):
    """Tile-major copy of a bf16 [N, K] weight for bf16_gemv_prepacked."""
    import torch

    if out is None:
        out = torch.empty(N * K, dtype=torch.bfloat16, device=weight.device)
    rc = _lib.cudalm_bf16_repack(_ptr(weight), _ptr(out), N, K, _stream(stream))
    _check(rc, "cudalm_bf16_repack")
    return out


def bf16_gemv_prepacked(packed, x, N: int, K: int, M: int = 1, y=None, stream=None):
    """bf16_gemv_any on a bf16_repack copy (same bits)."""
    y = _out(y, M, N, x)
    rc = _lib.cudalm_bf16_gemv_prepacked(_ptr(packed), _ptr(x), _ptr(y), N, K, M, _stream(stream))
    _check(rc, "cudalm_bf16_gemv_prepacked")
    return y


def bf16_gemv(weight, x, y, N: int, K: int, stream=None):
    """Reference name and argument order (bf16_gemv.h:37-38)."""
    return bf16_gemv_any(weight, x, N, K, 1, y=y, stream=stream)


def batch_bf16_gemv(weight, x, y, N: int, K: int, B: int, stream=None):
    """Reference name and argument order (batch_decode.h:77-79)."""
    return bf16_gemv_any(weight, x, N, K, B, y=y, stream=stream)


def bf16_gemv_kernel_regs(variant: int = BF16_VARIANT_STREAM) -> int:
    return _lib.cudalm_bf16_gemv_kernel_regs(variant)


# ---------------------------------------------------------------------------
# .cudalm v2 reader (include/cudalm_v2.h)
# ---------------------------------------------------------------------------

class V2Tensor(ctypes.Structure):
    """struct cudalm_v2_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("dims", ctypes.c_int64 * 8), ("offset", ctypes.c_uint64),
                ("byte_size", ctypes.c_uint64), ("align", ctypes.c_int), ("host", ctypes.c_void_p)]

    @property
    def shape(self):
        return tuple(self.dims[:self.ndim])

    def bytes(self) -> bytes:
        return ctypes.string_at(self.host, self.byte_size)


_CFG_FIELDS = ("hidden_size", "num_hidden_layers", "intermediate_size", "vocab_size", "n_heads",
               "n_kv_heads", "head_dim", "lin_num_k_heads", "lin_num_v_heads", "lin_key_head_dim",
               "lin_value_head_dim", "lin_conv_kernel_dim", "full_attention_interval",
               "group_size", "max_seq_len")


class V2Config(ctypes.Structure):
    """struct cudalm_v2_config."""
    _fields_ = ([(n, ctypes.c_int32) for n in _CFG_FIELDS] +
                [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
                 ("partial_rotary_factor", ctypes.c_float), ("mrope_section", ctypes.c_int32 * 3)])


class V2FormatError(ValueError):
    def __init__(self, code: int, reason: str):
        self.code = code
        self.reason = reason
        super().__init__(f"{reason} (code {code})")


class V2File:
    """A validated, memory-mapped .cudalm v2 file (WeightFileV2's role,
    weight_loader_v2.cpp:48-240)."""

    def __init__(self, path: str):
        self._h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        rc = _lib.cudalm_v2_open(os.fsencode(path), ctypes.byref(self._h), err, 512)
        if rc != OK:
            self._h = None
            raise V2FormatError(rc, err.value.decode())

    def close(self) -> None:
        if self._h:
            _lib.cudalm_v2_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def tensors(self):
        out = []
        for i in range(_lib.cudalm_v2_num_tensors(self._h)):
            t = V2Tensor()
            _check(_lib.cudalm_v2_tensor_at(self._h, i, ctypes.byref(t)), "cudalm_v2_tensor_at")
            out.append(t)
        return out

    def find(self, name: str):
        t = V2Tensor()
        rc = _lib.cudalm_v2_find(self._h, name.encode(), ctypes.byref(t))
        return t if rc == OK else None

    def meta(self, key: str):
        v = _lib.cudalm_v2_meta(self._h, key.encode())
        return None if v is None else v.decode()

    def config(self) -> V2Config:
        c = V2Config()
        _check(_lib.cudalm_v2_get_config(self._h, ctypes.byref(c)), "cudalm_v2_get_config")
        return c

    def validate_layer(self, idx: int):
        """None if the layer's tensor set is complete, else the reason."""
        err = ctypes.create_string_buffer(512)
        rc = _lib.cudalm_v2_validate_layer(self._h, idx, err, 512)
        return None if rc == OK else err.value.decode()

    def w4a16_shape(self, prefix: str):
        N, K = ctypes.c_int(), ctypes.c_int()
        rc = _lib.cudalm_v2_w4a16_shape(self._h, prefix.encode(), ctypes.byref(N), ctypes.byref(K))
        if rc != OK:
            raise KeyError(prefix)
        return N.value, K.value

    def load_w4a16_packed(self, prefix: str, device="cuda", stream=None):
        """Repack-at-load of one projection: (packed uint8 tensor, N, K)."""
        import torch

        N, K = self.w4a16_shape(prefix)
        out = torch.empty(packed_bytes(N, K), dtype=torch.uint8, device=device)
        rc = _lib.cudalm_v2_upload_w4a16_packed(self._h, prefix.encode(), _ptr(out), out.numel(),
                                                _stream(stream))
        _check(rc, "cudalm_v2_upload_w4a16_packed")
        return out, N, K

    def load_raw(self, name: str, device="cuda", stream=None):
        """A tensor's file bytes on the device, as a uint8 tensor."""
        import torch

        t = self.find(name)
        if t is None:
            raise KeyError(name)
        out = torch.empty(t.byte_size, dtype=torch.uint8, device=device)
        rc = _lib.cudalm_v2_upload(self._h, name.encode(), _ptr(out), out.numel(), _stream(stream))
        _check(rc, "cudalm_v2_upload")
        return out
