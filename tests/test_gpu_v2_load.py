"""Repack-at-load from a .cudalm v2 file (include/cudalm_v2.h) on the GPU:
projections loaded through cudalm_v2_upload_w4a16_packed give exactly the
bits of the file-layout entry point on the same file bytes, and match the
CPU oracle; the tied bf16 embedding loaded raw serves the LM-head GEMV.
This is the reference's load path (src/runtime/weight_loader_v2.cpp:
416-500) followed by its projection calls (qwen35_deltanet.cpp:166-251)."""
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import v2_fixtures as fx  # noqa: E402

pytestmark = pytest.mark.gpu

PROJS = ["layers.0.mlp.gate_proj", "layers.0.mlp.up_proj", "layers.0.mlp.down_proj",
         "layers.0.linear_attn.in_proj_qkv", "layers.0.linear_attn.in_proj_b",
         "layers.3.self_attn.q_proj", "layers.3.self_attn.o_proj"]


@pytest.fixture(scope="module")
def model_file(tmp_path_factory, orc):
    c = fx.SYNTH_CONFIG
    shapes = {}
    for t in fx.synth_tensors(c):
        shapes[t[0]] = t[2]
    extra, arrays = {}, {}
    for j, p in enumerate(PROJS):
        n, half_k = shapes[p + ".weight"]
        W, S = orc.synth_w4a16(0x1000 + j, n, 2 * half_k)
        extra[p + ".weight"] = W.tobytes()
        extra[p + ".scale"] = S.tobytes()
        arrays[p] = (W, S, n, 2 * half_k)
    tensors = fx.synth_tensors(c, extra)
    E = orc.f32_to_bf16(orc.synth_normal(0xE4B, 0.02, c["vocab_size"] * c["hidden_size"]))
    E = E.reshape(c["vocab_size"], c["hidden_size"])
    tensors.append(("embed_tokens.weight", fx.DT_BF16, E.shape, E.tobytes()))
    path = tmp_path_factory.mktemp("v2gpu") / "model.cudalm"
    path.write_bytes(fx.write(c, dict(fx.SYNTH_META, tie_word_embeddings="true"), tensors))
    return str(path), arrays, E


@pytest.mark.parametrize("M", [1, 5, 64])
def test_packed_load_matches_file_layout(w4, orc, dev, model_file, M):
    path, arrays, _ = model_file
    with w4.V2File(path) as f:
        for j, p in enumerate(PROJS):
            W, S, N, K = arrays[p]
            packed, n2, k2 = f.load_w4a16_packed(p, device=dev)
            assert (n2, k2) == (N, K)
            assert torch.equal(packed.cpu(), torch.from_numpy(w4.repack_host(W, S, N, K)))
            X = orc.synth_act(0x77 + 13 * j + M, M, K)
            x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
            y_packed = w4.gemv_prepacked(packed, x, N, K, M)
            w = f.load_raw(p + ".weight", device=dev)
            s = f.load_raw(p + ".scale", device=dev).view(torch.float16)
            y_file = w4.gemv(w, s, x, N, K, M)
            torch.cuda.synchronize()
            a = y_packed.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
            b = y_file.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
            assert np.array_equal(a, b), p
            ok, st = orc.check_tolerance(a, W, S, X, N, K, M)
            assert ok, (p, st)


def test_tied_embedding_lm_head(w4, orc, dev, model_file):
    path, _, E = model_file
    with w4.V2File(path) as f:
        assert f.meta("tie_word_embeddings") == "true"
        e = f.load_raw("embed_tokens.weight", device=dev).view(torch.bfloat16)
        N, K = E.shape
        X = orc.synth_act(0x1E, 2, K)
        x = torch.from_numpy(X.view(np.int16)).to(dev).view(torch.bfloat16)
        y = w4.bf16_gemv_any(e, x, N, K, 2)
        torch.cuda.synchronize()
        Y = y.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, N)
        ok, st = orc.check_bf16_tolerance(Y, E, X, N, K, 2)
        assert ok, st


def test_upload_rejects_small_or_misaligned_destination(w4, dev, model_file):
    path, arrays, _ = model_file
    with w4.V2File(path) as f:
        p = PROJS[0]
        W, S, N, K = arrays[p]
        small = torch.empty(w4.packed_bytes(N, K) - 16, dtype=torch.uint8, device=dev)
        lib = w4.lib()
        st = torch.cuda.current_stream().cuda_stream
        assert lib.cudalm_v2_upload_w4a16_packed(f._h, p.encode(), small.data_ptr(), small.numel(),
                                                 st) == w4.ERANGE
        big = torch.empty(w4.packed_bytes(N, K) + 16, dtype=torch.uint8, device=dev)
        assert lib.cudalm_v2_upload_w4a16_packed(f._h, p.encode(), big.data_ptr() + 8,
                                                 big.numel() - 8, st) == w4.EALIGN
        assert lib.cudalm_v2_upload_w4a16_packed(f._h, b"layers.9.mlp.gate_proj", big.data_ptr(),
                                                 big.numel(), st) == w4.V2_ENOTFOUND
