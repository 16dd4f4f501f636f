"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/cudalm_w4a16.h declares, rejects bad shapes before touching the
device, computes the packed size and host repack layout, and the C++
entry points with the reference's names abort on a violated precondition
(the reference's CUDALM_PRECONDITION model, cuda_check.h:53-63)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(REPO, "include", h)
           for h in ("cudalm_w4a16.h", "cudalm_bf16_gemv.h", "cudalm_v2.h")]


def declared_symbols():
    syms = set()
    for h in HEADERS:
        syms |= set(re.findall(r"\b(cudalm_[a-z0-9_]+)\s*\(", open(h).read()))
    return sorted(syms)


def test_library_exports_every_declared_symbol(w4):
    syms = declared_symbols()
    assert len(syms) >= 13
    for s in syms:
        assert hasattr(w4.lib(), s), s
    assert set(syms) == set(w4.EXPORTED_SYMBOLS)


def test_version_and_strerror(w4):
    assert w4.version() >= 100
    for code in range(-9, 1):
        assert w4.strerror(code)
    assert "unknown" in w4.strerror(-99)


def test_shape_preconditions_rejected_before_device(w4):
    # invalid shapes and null pointers return before any HIP call
    fake = 0x1000
    assert w4.gemv_ptr(fake, fake, fake, fake, 0, 128, 1) == w4.EINVAL
    assert w4.gemv_ptr(fake, fake, fake, fake, 4, 100, 1) == w4.EINVAL
    assert w4.gemv_ptr(fake, fake, fake, fake, 4, 0, 1) == w4.EINVAL
    assert w4.gemv_ptr(fake, fake, fake, fake, 4, 128, 0) == w4.EINVAL
    assert w4.gemv_ptr(None, fake, fake, fake, 4, 128, 1) == w4.ENULL
    assert w4.prepacked_ptr(fake, fake, fake, 4, 127, 1) == w4.EINVAL
    assert w4.prepacked_ptr(fake + 8, fake, fake, 4, 128, 1) == w4.EALIGN
    lib = w4.lib()
    assert lib.cudalm_w4a16_repack(fake, fake, fake, 0, 128, None) == w4.EINVAL
    assert lib.cudalm_w4a16_repack(fake, fake, fake + 4, 16, 128, None) == w4.EALIGN
    assert lib.cudalm_w4a16_dequant_f32(fake + 1, fake, None, None, 16, 128, None) == w4.EALIGN
    # misaligned bases are legal for the file-layout entry, but not with a
    # vectorized variant forced
    assert w4.gemv_ptr(fake + 1, fake, fake, fake, 4, 128, 1, w4.VARIANT_STREAM) == w4.EVARIANT


def test_chain_plan_preconditions_rejected_before_device(w4):
    # the stage checks of cudalm_w4a16_chain_plan return before any HIP
    # call, SwiGLU stages (stage.act) included
    import ctypes
    lib = w4.lib()
    fake = 0x100000
    ws_bytes = lib.cudalm_w4a16_chain_workspace_bytes(1)
    assert ws_bytes > 0 and lib.cudalm_w4a16_chain_workspace_bytes(0) == 0
    assert lib.cudalm_w4a16_chain_workspace_bytes(w4.MAX_STAGES + 1) == 0

    def plan(items, K, act, M=4, x=fake):
        arr = w4.proj_array(items)
        st = (w4.Stage * 1)()
        st[0].projs, st[0].count, st[0].x, st[0].K, st[0].dep = \
            ctypes.cast(arr, ctypes.c_void_p), len(items), x, K, -1
        st[0].act = act
        h = w4.ChainHandle()
        return lib.cudalm_w4a16_chain_plan(ctypes.cast(st, ctypes.c_void_p), 1, M, 1, fake, ws_bytes,
                                           ctypes.byref(h), None)

    gu = [(fake, None, 0, 3584), (fake, None, 0, 3584)]
    assert plan(gu[:1], 1024, fake) == w4.EINVAL                      # one projection
    assert plan(gu + [(fake, None, 0, 3584)], 1024, fake) == w4.EINVAL  # three
    assert plan([gu[0], (fake, None, 0, 3568)], 1024, fake) == w4.EINVAL  # N differs
    assert plan(gu, 2176, fake) == w4.EINVAL                          # K > 2048
    assert plan(gu, 1024, fake + 1) == w4.EALIGN                      # act not 2 B aligned
    assert plan(gu, 1024, fake, x=fake + 8) == w4.EALIGN              # x not 16 B aligned
    assert plan([(fake, None, 0, 3584)], 1024, None) == w4.ENULL      # no act: y is required
    assert plan(gu, 1024, fake, M=33) == w4.EINVAL


def test_bf16_gemv_preconditions_rejected_before_device(w4):
    # include/cudalm_bf16_gemv.h: N, K, M >= 1; 2-byte aligned bases; a
    # forced stream variant needs K % 8 == 0 and 16 B bases
    fake = 0x1000
    p = w4.bf16_gemv_ptr
    assert p(fake, fake, fake, 0, 8, 1) == w4.EINVAL
    assert p(fake, fake, fake, 4, 0, 1) == w4.EINVAL
    assert p(fake, fake, fake, 4, 8, 0) == w4.EINVAL
    assert p(None, fake, fake, 4, 8, 1) == w4.ENULL
    assert p(fake, fake, None, 4, 8, 1) == w4.ENULL
    assert p(fake + 1, fake, fake, 4, 8, 1) == w4.EALIGN
    assert p(fake, fake, fake + 1, 4, 8, 1) == w4.EALIGN
    assert p(fake, fake, fake, 4, 12, 1, w4.BF16_VARIANT_STREAM) == w4.EVARIANT
    assert p(fake + 2, fake, fake, 4, 16, 1, w4.BF16_VARIANT_STREAM) == w4.EVARIANT
    assert p(fake, fake, fake, 4, 16, 1, 7) == w4.EVARIANT
    assert p(fake, fake, fake, 1 << 30, 16, 1) == w4.ERANGE


def test_bf16_repack_preconditions_rejected_before_device(w4):
    # include/cudalm_bf16_gemv.h: the packed path needs N % 16 == 0,
    # K % 256 == 0 and 16-byte aligned bases
    fake = 0x1000
    lib = w4.lib()
    assert lib.cudalm_bf16_packed_bytes(32, 512) == 32 * 512 * 2
    assert lib.cudalm_bf16_packed_bytes(17, 512) == 0
    assert lib.cudalm_bf16_packed_bytes(32, 100) == 0
    assert lib.cudalm_bf16_packed_bytes(-16, 256) == 0
    assert lib.cudalm_bf16_repack(fake, fake, 17, 256, None) == w4.EINVAL
    assert lib.cudalm_bf16_repack(fake, fake, 16, 128, None) == w4.EINVAL
    assert lib.cudalm_bf16_repack(None, fake, 16, 256, None) == w4.ENULL
    assert lib.cudalm_bf16_repack(fake + 2, fake, 16, 256, None) == w4.EALIGN
    assert lib.cudalm_bf16_gemv_prepacked(fake, fake, fake, 16, 200, 1, None) == w4.EINVAL
    assert lib.cudalm_bf16_gemv_prepacked(fake, fake, None, 16, 256, 1, None) == w4.ENULL
    assert lib.cudalm_bf16_gemv_prepacked(fake, fake + 2, fake, 16, 256, 1, None) == w4.EALIGN
    assert lib.cudalm_bf16_gemv_prepacked(fake, fake, fake, 16, 256, 0, None) == w4.EINVAL


def test_packed_bytes(w4):
    assert w4.packed_bytes(16, 128) == 1024 + 256
    assert w4.packed_bytes(17, 128) == 2 * (1024 + 256)
    assert w4.packed_bytes(248320, 1024) == 15520 * 8 * 1056
    assert w4.packed_bytes(16, 3584) == 28 * 1024 + 16 * 64
    assert w4.packed_bytes(0, 128) == 0
    assert w4.packed_bytes(16, 100) == 0


def _numpy_repack(W, S, N, K):
    G = K // 128
    SP = 16 * ((G + 7) // 8)
    nt = (N + 15) // 16
    Wp = np.zeros((nt * 16, K // 2), np.uint8)
    Wp[:N] = W
    Sp = np.zeros((nt * 16, SP // 2), np.uint16)
    Sp[:N, :G] = S
    tiles = []
    for rt in range(nt):
        wpart = np.zeros((G, 64, 16), np.uint8)
        for lane in range(64):
            i, a = lane & 15, lane >> 4
            rows = Wp[rt * 16 + i].reshape(G, 64)
            wpart[:, lane, :] = rows[:, a * 16:a * 16 + 16]
        # each little-endian dword of 8 nibbles is stored rotated left by 3 bits
        d = wpart.reshape(-1).view("<u4")
        d = ((d << np.uint32(3)) | (d >> np.uint32(29))).astype("<u4")
        tiles.append(np.concatenate([d.view(np.uint8), Sp[rt * 16:rt * 16 + 16].view(np.uint8).ravel()]))
    return np.concatenate(tiles)


@pytest.mark.parametrize("N,K", [(1, 128), (16, 256), (37, 384), (64, 1024), (20, 3584), (5, 2304)])
def test_repack_host_layout(w4, orc, N, K):
    W, S, _ = orc.fixture_gemv(N + K, N, K)
    got = w4.repack_host(W, S, N, K)
    assert np.array_equal(got, _numpy_repack(W, S, N, K))


def test_cpp_headers_compile_and_link(tmp_path, w4):
    src = tmp_path / "use.cpp"
    src.write_text(r'''
#include "cudalm/kernels/int4_gemv_bf16.h"
#include "cudalm/kernels/batch_decode.h"
#include "cudalm/kernels/bf16_gemv.h"
#include "cudalm/kernels/int4_gemv.h"
#include "cudalm/kernels/swiglu.h"
#include "cudalm/w4a16_linear.h"
#include "cudalm_bf16_gemv.h"
#include "cudalm_v2.h"
#include "cudalm_w4a16.h"
#include <cstddef>
#include <cstdio>
int main() {
  std::printf("%zu %zu\n", cudalm::packed_w4a16_bytes(16, 128), cudalm_w4a16_packed_bytes(32, 256));
  // struct layouts the Python layer mirrors with ctypes
  std::printf("stage %zu %zu %zu %zu %zu %zu %zu\n", sizeof(cudalm_w4a16_stage),
              offsetof(cudalm_w4a16_stage, projs), offsetof(cudalm_w4a16_stage, count),
              offsetof(cudalm_w4a16_stage, x), offsetof(cudalm_w4a16_stage, K),
              offsetof(cudalm_w4a16_stage, dep), offsetof(cudalm_w4a16_stage, act));
  std::printf("proj %zu %zu %zu %zu %zu\n", sizeof(cudalm_w4a16_proj),
              offsetof(cudalm_w4a16_proj, weight), offsetof(cudalm_w4a16_proj, scale),
              offsetof(cudalm_w4a16_proj, y), offsetof(cudalm_w4a16_proj, N));
  std::printf("chain %zu %zu %zu %zu %zu %zu %zu\n", sizeof(cudalm_w4a16_chain),
              offsetof(cudalm_w4a16_chain, workspace), offsetof(cudalm_w4a16_chain, n_stages),
              offsetof(cudalm_w4a16_chain, M), offsetof(cudalm_w4a16_chain, prepacked),
              offsetof(cudalm_w4a16_chain, grid), offsetof(cudalm_w4a16_chain, gt_max));
  // the reference-named bf16 entry points resolve at link time
  void (*f1)(const __hip_bfloat16*, const __hip_bfloat16*, __hip_bfloat16*, int, int, hipStream_t) =
      cudalm::bf16_gemv;
  void (*f2)(const __hip_bfloat16*, const __hip_bfloat16*, __hip_bfloat16*, int, int, int,
             hipStream_t) = cudalm::kernels::batch_bf16_gemv;
  void (*f3)(const std::uint8_t*, const __half*, const __half*, __half*, int, int, hipStream_t) =
      cudalm::int4_gemv;
  void (*f4)(const __hip_bfloat16*, const __hip_bfloat16*, __hip_bfloat16*, std::size_t,
             hipStream_t) = cudalm::kernels::qwen35_silu_mul_bf16;
  return (f1 && f2 && f3 && f4) ? 0 : 1;
}
''')
    exe = tmp_path / "use"
    libdir = os.path.dirname(w4.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-I", os.path.join(REPO, "include"), str(src),
           "-L", libdir, "-lcudalm_w4a16", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    assert lines[0].split() == ["1280", str(2 * (2 * 1024 + 256))]
    for line in lines[1:]:
        name, *nums = line.split()
        cls = {"stage": w4.Stage, "proj": w4.Proj, "chain": w4.ChainHandle}[name]
        want = [ctypes.sizeof(cls)] + [getattr(cls, f).offset for f, _ in cls._fields_]
        assert [int(v) for v in nums] == want, (name, nums, want)


def test_cpp_entry_aborts_on_precondition(tmp_path, w4):
    src = tmp_path / "bad.cpp"
    src.write_text(r'''
#include "cudalm/kernels/int4_gemv_bf16.h"
int main() {
  // K % 128 != 0: the reference aborts (int4_gemv_bf16.cu:224-226)
  cudalm::int4_gemv_bf16(nullptr, nullptr, nullptr, nullptr, 8, 100, nullptr);
  return 0;
}
''')
    exe = tmp_path / "bad"
    libdir = os.path.dirname(w4.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-I", os.path.join(REPO, "include"), str(src),
           "-L", libdir, "-lcudalm_w4a16", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    assert subprocess.run(cmd, capture_output=True).returncode == 0
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode != 0
    assert "invalid shape" in res.stderr


def test_cpp_bf16_entry_aborts_on_precondition(tmp_path, w4):
    src = tmp_path / "bad_bf16.cpp"
    src.write_text(r'''
#include "cudalm/kernels/bf16_gemv.h"
int main() {
  // N < 1: the reference aborts (bf16_gemv.cu:113-114)
  cudalm::bf16_gemv(nullptr, nullptr, nullptr, 0, 1024, nullptr);
  return 0;
}
''')
    exe = tmp_path / "bad_bf16"
    libdir = os.path.dirname(w4.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-I", os.path.join(REPO, "include"), str(src),
           "-L", libdir, "-lcudalm_w4a16", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    assert subprocess.run(cmd, capture_output=True).returncode == 0
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode != 0
    assert "bf16_gemv" in res.stderr and "invalid shape" in res.stderr


def test_python_layer_raises_on_bad_shape(w4):
    import torch

    x = torch.zeros(128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        w4.gemv(x, x, x, 0, 128, 1, y=x, stream=0)
