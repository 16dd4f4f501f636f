"""The .cudalm v2 reader (include/cudalm_v2.h) on files written from the
container spec by tests/golden/v2_fixtures.py: the valid synthetic file
reads back field for field and byte for byte, and every corruption case of
the reference's format test (tests/cpu/test_cudalm_v2_format.cpp:47-160),
plus five more structural rules, is rejected."""
import os
import struct
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import v2_fixtures as fx  # noqa: E402


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("v2")
    valid, cases, sums = fx.make_all()
    (d / "valid.cudalm").write_bytes(valid)
    for name, raw in cases.items():
        (d / f"corrupt_{name}.cudalm").write_bytes(raw)
    return d, sums, sorted(cases)


def test_valid_file_reads_back(w4, files):
    d, sums, _ = files
    with w4.V2File(str(d / "valid.cudalm")) as f:
        assert f.meta("arch") == "synthetic-qwen3.5-format-test"
        assert f.meta("model_repo") == "cudalm/synthetic"
        assert f.meta("nope") is None
        c = f.config()
        want = fx.SYNTH_CONFIG
        for k in ("hidden_size", "num_hidden_layers", "intermediate_size", "vocab_size", "n_heads",
                  "n_kv_heads", "head_dim", "lin_num_k_heads", "lin_num_v_heads",
                  "lin_key_head_dim", "lin_value_head_dim", "lin_conv_kernel_dim",
                  "full_attention_interval", "group_size", "max_seq_len"):
            assert getattr(c, k) == want[k], k
        f32 = lambda v: struct.unpack("<f", struct.pack("<f", v))[0]  # noqa: E731
        assert c.eps == f32(1e-6) and c.rope_theta == f32(1e7) and c.partial_rotary_factor == 0.25
        assert list(c.mrope_section) == [3, 3, 2]
        ts = f.tensors()
        assert len(ts) == len(sums) == 41
        by = {t.name.decode(): t for t in ts}
        for name, size, total in sums:
            t = by[name]
            assert t.byte_size == size
            assert sum(t.bytes()) & (2 ** 64 - 1) == total
        # layers 0 (DeltaNet) and 3 (full attention) are complete; 1, 2 absent; 4 out of range
        assert f.validate_layer(0) is None and f.validate_layer(3) is None
        assert "missing" in f.validate_layer(1) and "missing" in f.validate_layer(2)
        assert "out of range" in f.validate_layer(4)
        norm = f.find("norm.weight")
        assert norm.dtype == fx.DT_BF16 and norm.shape == (256,) and norm.byte_size == 512
        assert f.w4a16_shape("layers.0.mlp.gate_proj") == (768, 256)
        assert f.w4a16_shape("layers.3.self_attn.o_proj") == (256, 128)
        with pytest.raises(KeyError):
            f.w4a16_shape("layers.0.mlp")
        with pytest.raises(KeyError):
            f.w4a16_shape("norm")


EXPECTED_REASON = {
    "bad_magic": "bad magic", "bad_version": "unsupported version", "bad_flags": "flags",
    "bad_config_size": "config_size", "section_overlap": "overlap",
    "payload_unaligned": "16B-aligned", "payload_oob": "out of payload bounds",
    "bad_dtype": "bad dtype", "entry_pad_nonzero": "reserved pad", "table_trailing": "",
    "dup_name": "duplicate", "bad_name_charset": "charset", "invalid_config": "validation",
    "config_reserved": "reserved word", "truncated": "out of bounds", "bad_align": "bad align",
    "bad_ndim": "bad ndim", "unused_dim_nonzero": "unused dim", "byte_size_mismatch": "byte_size",
}


def test_every_corruption_rejected(w4, files):
    d, _, cases = files
    assert set(cases) == set(EXPECTED_REASON)
    for case in cases:
        with pytest.raises(w4.V2FormatError) as ei:
            w4.V2File(str(d / f"corrupt_{case}.cudalm"))
        assert ei.value.code == w4.V2_EFORMAT, case
        assert EXPECTED_REASON[case] in ei.value.reason, (case, ei.value.reason)


def test_missing_and_tiny_files(w4, tmp_path):
    with pytest.raises(w4.V2FormatError) as ei:
        w4.V2File(str(tmp_path / "absent.cudalm"))
    assert ei.value.code == w4.V2_EIO
    p = tmp_path / "empty.cudalm"
    p.write_bytes(b"")
    with pytest.raises(w4.V2FormatError) as ei:
        w4.V2File(str(p))
    assert ei.value.code == w4.V2_EFORMAT and "too small" in ei.value.reason
