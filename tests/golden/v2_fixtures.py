"""Writes `.cudalm` v2 test files (CUDLMW02) from the container layout in
the reference's include/cudalm/weight_format_v2.h:31-100,129-151: one valid
synthetic file and one file per corruption case that its reader must
reject (the cases of tests/cpu/test_cudalm_v2_format.cpp:140-160).

The valid file carries the synthetic config and tensor set that test uses
(layer 3 full attention, layer 0 Gated DeltaNet, final norm: 41 tensors;
config hidden 256, 4 layers, intermediate 768, vocab 1000, ...), with
deterministic payload bytes; `sums` gives each tensor's byte size and
wrapped byte sum. Optionally it embeds real W4A16 projections (file-layout
weight and fp16 scale bytes supplied by the caller) and a bf16 embedding.

Standard library only; used by tests/ to build fixtures in a temp dir.
"""
from __future__ import annotations

import struct

DT_FP16, DT_INT4, DT_SCALE, DT_FP32, DT_BF16 = 1, 2, 3, 4, 5
ELEM = {DT_FP16: 2, DT_INT4: 1, DT_SCALE: 2, DT_FP32: 4, DT_BF16: 2}

SYNTH_CONFIG = dict(
    hidden_size=256, num_hidden_layers=4, intermediate_size=768, vocab_size=1000, n_heads=2,
    n_kv_heads=1, head_dim=64, lin_num_k_heads=2, lin_num_v_heads=2, lin_key_head_dim=32,
    lin_value_head_dim=64, lin_conv_kernel_dim=4, full_attention_interval=4, group_size=128,
    max_seq_len=512, eps=1e-6, rope_theta=1e7, partial_rotary_factor=0.25,
    mrope_section=(3, 3, 2))

_INT_FIELDS = ("hidden_size", "num_hidden_layers", "intermediate_size", "vocab_size", "n_heads",
               "n_kv_heads", "head_dim", "lin_num_k_heads", "lin_num_v_heads",
               "lin_key_head_dim", "lin_value_head_dim", "lin_conv_kernel_dim",
               "full_attention_interval", "group_size", "max_seq_len")


def config_blob(c: dict, reserved: int = 0) -> bytes:
    b = struct.pack("<15i", *[c[k] for k in _INT_FIELDS])
    b += struct.pack("<3f", c["eps"], c["rope_theta"], c["partial_rotary_factor"])
    b += struct.pack("<3i", *c["mrope_section"]) + struct.pack("<I", reserved)
    assert len(b) == 88
    return b


def det_bytes(n: int, seed: int) -> bytes:
    """Deterministic bytes (64-bit LCG, top byte)."""
    x = (seed * 0x9E3779B97F4A7C15 + 1) & (2 ** 64 - 1)
    out = bytearray(n)
    for i in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) & (2 ** 64 - 1)
        out[i] = x >> 56
    return bytes(out)


def write(config: dict, metadata: dict, tensors, align: int = 16) -> bytes:
    """tensors: list of (name, dtype, dims, payload bytes). Section order:
    header, config, metadata, table, payload (16 B aligned)."""
    meta = b""
    for k, v in metadata.items():
        kb, vb = k.encode(), v.encode()
        meta += struct.pack("<B", len(kb)) + kb + struct.pack("<H", len(vb)) + vb
    offsets, payload = [], b""
    for _, _, _, data in tensors:
        pad = (-len(payload)) % align
        payload += b"\0" * pad
        offsets.append(len(payload))
        payload += data
    table = b""
    for (name, dt, dims, data), off in zip(tensors, offsets):
        nb = name.encode()
        d8 = list(dims) + [0] * (8 - len(dims))
        table += struct.pack("<B", len(nb)) + nb + struct.pack("<BBH", dt, len(dims), 0)
        table += struct.pack("<8q", *d8) + struct.pack("<QQBB", off, len(data), align, 0)
    cfg_off = 88
    meta_off = cfg_off + 88
    tbl_off = meta_off + len(meta)
    pay_off = tbl_off + len(table)
    pay_off += (-pay_off) % 16
    head = b"CUDLMW02" + struct.pack("<IIIHH", 2, 0, len(tensors), len(metadata), 0)
    head += struct.pack("<8Q", cfg_off, 88, meta_off, len(meta), tbl_off, len(table), pay_off,
                        len(payload))
    assert len(head) == 88
    raw = head + config_blob(config) + meta + table
    raw += b"\0" * (pay_off - len(raw))
    return raw + payload


def synth_tensors(c: dict, extra=None):
    """The 41-tensor set of the reference format test; `extra` maps a name to
    replacement payload bytes (same dtype and shape)."""
    H, G, I = c["hidden_size"], c["group_size"], c["intermediate_size"]
    qo = c["n_heads"] * c["head_dim"] * 2
    kvo = c["n_kv_heads"] * c["head_dim"]
    oin = c["n_heads"] * c["head_dim"]
    cv = c["lin_num_v_heads"] * c["lin_value_head_dim"]
    cd = 2 * c["lin_num_k_heads"] * c["lin_key_head_dim"] + cv
    nv = c["lin_num_v_heads"]
    spec = []

    def proj(base, n, k):
        spec.append((base + ".weight", DT_INT4, (n, k // 2)))
        spec.append((base + ".scale", DT_SCALE, (n, k // G)))

    L = "layers.3."
    spec.append((L + "input_layernorm.weight", DT_BF16, (H,)))
    proj(L + "self_attn.q_proj", qo, H)
    proj(L + "self_attn.k_proj", kvo, H)
    proj(L + "self_attn.v_proj", kvo, H)
    proj(L + "self_attn.o_proj", H, oin)
    spec.append((L + "self_attn.q_norm.weight", DT_BF16, (c["head_dim"],)))
    spec.append((L + "self_attn.k_norm.weight", DT_BF16, (c["head_dim"],)))
    spec.append((L + "post_attention_layernorm.weight", DT_BF16, (H,)))
    proj(L + "mlp.gate_proj", I, H)
    proj(L + "mlp.up_proj", I, H)
    proj(L + "mlp.down_proj", H, I)
    L = "layers.0."
    spec.append((L + "input_layernorm.weight", DT_BF16, (H,)))
    proj(L + "linear_attn.in_proj_qkv", cd, H)
    proj(L + "linear_attn.in_proj_z", cv, H)
    proj(L + "linear_attn.in_proj_b", nv, H)
    proj(L + "linear_attn.in_proj_a", nv, H)
    proj(L + "linear_attn.out_proj", H, cv)
    spec.append((L + "linear_attn.conv1d.weight", DT_BF16, (cd, 1, c["lin_conv_kernel_dim"])))
    spec.append((L + "linear_attn.dt_bias", DT_BF16, (nv,)))
    spec.append((L + "linear_attn.A_log", DT_FP32, (nv,)))
    spec.append((L + "linear_attn.norm.weight", DT_FP32, (c["lin_value_head_dim"],)))
    spec.append((L + "post_attention_layernorm.weight", DT_BF16, (H,)))
    proj(L + "mlp.gate_proj", I, H)
    proj(L + "mlp.up_proj", I, H)
    proj(L + "mlp.down_proj", H, I)
    spec.append(("norm.weight", DT_BF16, (H,)))
    extra = extra or {}
    out = []
    for seed, (name, dt, dims) in enumerate(spec, start=1):
        n = ELEM[dt]
        for d in dims:
            n *= d
        data = extra.get(name, det_bytes(n, seed))
        assert len(data) == n, name
        out.append((name, dt, dims, data))
    return out


SYNTH_META = {"arch": "synthetic-qwen3.5-format-test", "model_repo": "cudalm/synthetic",
              "model_revision": "0000"}


def _entries(raw: bytes):
    """(name, position after the name) for each table entry."""
    tbl_off, tbl_size = struct.unpack_from("<QQ", raw, 56)
    pos, end = tbl_off, tbl_off + tbl_size
    while pos < end:
        n = raw[pos]
        yield raw[pos + 1:pos + 1 + n].decode(), pos + 1 + n
        pos += 1 + n + 86


def corruptions(valid: bytes, c: dict, tensors, meta):
    """name -> bytes for each case the reader must reject."""
    out = {}

    def patched(fmt, off, val):
        r = bytearray(valid)
        struct.pack_into(fmt, r, off, val)
        return bytes(r)

    out["bad_magic"] = b"X" + valid[1:]
    out["bad_version"] = patched("<I", 8, 3)
    out["bad_flags"] = patched("<I", 12, 1)
    out["bad_config_size"] = patched("<Q", 32, 87)
    out["section_overlap"] = patched("<Q", 40, 88)  # metadata offset onto the config blob
    pay_off, pay_size = struct.unpack_from("<QQ", valid, 72)
    out["payload_unaligned"] = patched("<Q", 72, pay_off - 4)
    _, f0 = next(_entries(valid))
    out["payload_oob"] = patched("<Q", f0 + 68, pay_size - 4)
    r = bytearray(valid)
    r[f0] = 9
    out["bad_dtype"] = bytes(r)
    out["entry_pad_nonzero"] = patched("<H", f0 + 2, 1)
    tbl_size = struct.unpack_from("<Q", valid, 64)[0]
    out["table_trailing"] = patched("<Q", 64, tbl_size + 4)
    out["dup_name"] = write(c, meta, [tensors[0], tensors[0]])
    out["bad_name_charset"] = write(c, meta, [tensors[0], ("bad name with spaces", DT_BF16, (4,),
                                                           b"\0" * 8)])
    bad = dict(c, n_kv_heads=3)  # 2 heads do not divide into 3 groups
    out["invalid_config"] = write(bad, meta, tensors)
    cfg_off = struct.unpack_from("<Q", valid, 24)[0]
    out["config_reserved"] = patched("<I", cfg_off + 84, 0xDEAD)
    # beyond the reference's list: bytes the other checks guard
    out["truncated"] = valid[:len(valid) - 1]
    out["bad_align"] = patched("<B", f0 + 84, 3)
    out["bad_ndim"] = patched("<B", f0 + 1, 0)
    out["unused_dim_nonzero"] = patched("<q", f0 + 4 + 8 * 7, 5)
    out["byte_size_mismatch"] = patched("<Q", f0 + 76, len(tensors[0][3]) - 2)
    return out


def make_all(c: dict = None, meta: dict = None, extra=None):
    """(valid bytes, {case: bytes}, [(name, byte_size, byte_sum)])."""
    c = c or SYNTH_CONFIG
    meta = meta or SYNTH_META
    tensors = synth_tensors(c, extra)
    valid = write(c, meta, tensors)
    sums = [(n, len(d), sum(d) & (2 ** 64 - 1)) for n, _, _, d in tensors]
    return valid, corruptions(valid, c, tensors, meta), sums
