"""The device fp32 -> bf16 conversion every kernel's output goes through
(f32_to_bf16_rne, cudalm-agent_amd/csrc/hip_common.h: one
v_cvt_pk_bf16_f32) equals the oracle's integer round-to-nearest-even form
(oracle/w4a16_oracle.c orc_f32_to_bf16_rne; NaN -> (x >> 16) | 0x40) on a
fixed set of edge patterns and 2^20 random ones. The device program
tests/cpp/bf16_round_check is built by build() with the library's flags."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "bf16_round_check")

EDGES = [
    0x00000000, 0x80000000,                          # +-0
    0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000,  # ties, even and odd kept bit
    0x3F807FFF, 0x3F808001, 0x3F817FFF, 0x3F818001,  # just below / above the ties
    0x00000001, 0x00008000, 0x00018000, 0x007FFFFF,  # denormals (ties among them)
    0x80000001, 0x80008000, 0x807FFFFF,
    0x00800000, 0x00808000,                          # smallest normal, a tie next to it
    0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0x7F7E8000,  # largest finite: kept, tie -> Inf, -> Inf
    0xFF7F8000, 0xFF7FFFFF,
    0x7F800000, 0xFF800000,                          # +-Inf
    0x7F800001, 0x7FA00000, 0x7FBFFFFF, 0xFF800001,  # signalling NaNs with payloads
    0x7FC00000, 0x7FC12345, 0xFFC00001, 0xFFFFFFFF,  # quiet NaNs with payloads
    0x7F80FFFF, 0x7F810000,                          # NaN payloads in both halves
]


def test_device_bf16_rounding(orc, tmp_path):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/bf16_round_check is not built (run __graft_entry__.build())")
    rng = np.random.default_rng(0xB16)
    pats = np.concatenate([np.array(EDGES, np.uint32),
                           rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    pats.tofile(src)
    res = subprocess.run([BIN, str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    got = np.fromfile(dst, np.uint16)
    want = orc.f32_to_bf16(pats.view(np.float32))
    bad = np.nonzero(got != want)[0]
    print(f"  {pats.size} patterns, {bad.size} differ", flush=True)
    assert bad.size == 0, [(hex(int(pats[k])), hex(int(got[k])), hex(int(want[k]))) for k in bad[:8]]
