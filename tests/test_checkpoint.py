"""The quantized-checkpoint file format (sapphire_amd/checkpoint.py), on the CPU: blocks
written as raw bytes come back bit for bit, plain tensors pass through, and the projection
names follow the reference's Gemma-3 tensor map (src/loader/gemma3_map.c)."""
import numpy as np
import pytest
import torch

from sapphire_amd import checkpoint, synth


def test_round_trip(tmp_path):
    q4 = synth.quant_matrix(synth.Q4_0, 48, 100, 1, 2)      # ragged K: 4 blocks per row
    q8 = synth.quant_matrix(synth.Q8_0, 16, 640, 1, 3)
    emb = torch.from_numpy(synth.bf16_normal((32, 64), 1, 4).view(np.int16)).view(torch.bfloat16)
    norm = synth.normal_f32(64, 1, 5)
    path = str(tmp_path / "m.safetensors")
    checkpoint.save(path, {"model.embed_tokens.weight": emb, "model.norm.weight": norm},
                    {"model.layers.0.self_attn.q_proj.weight": (synth.Q4_0, q4, 100),
                     "model.layers.0.mlp.down_proj.weight": (synth.Q8_0, q8, 640)}, {"origin": "test"})
    tensors, quantized = checkpoint.load(path)
    dt, b, k = quantized["model.layers.0.self_attn.q_proj.weight"]
    assert dt == synth.Q4_0 and k == 100 and b.tobytes() == q4.tobytes()
    dt, b, k = quantized["model.layers.0.mlp.down_proj.weight"]
    assert dt == synth.Q8_0 and k == 640 and b.tobytes() == q8.tobytes()
    assert torch.equal(tensors["model.embed_tokens.weight"].view(torch.int16), emb.view(torch.int16))
    assert np.array_equal(tensors["model.norm.weight"].numpy(), norm)
    # the stored form is the reference's block array, rows contiguous
    from safetensors import safe_open
    with safe_open(path, "pt") as f:
        raw = f.get_tensor("model.layers.0.self_attn.q_proj.weight").numpy()
        assert f.metadata()["sapphire.format"] == checkpoint.FORMAT and f.metadata()["origin"] == "test"
    assert raw.shape == (48, 4 * 20) and raw.tobytes() == q4.tobytes()


def test_bad_stored_shape():
    with pytest.raises(ValueError):
        checkpoint.bytes_to_blocks(np.zeros((4, 21), np.uint8), synth.Q4_0, 4, 32)


def test_projection_names():
    for l in (0, 17):
        for p in checkpoint.PROJECTIONS:
            assert checkpoint.is_projection(f"model.layers.{l}.{p}")
    for n in ("model.embed_tokens.weight", "model.layers.0.input_layernorm.weight",
              "model.layers.3.self_attn.q_norm.weight", "model.norm.weight"):
        assert not checkpoint.is_projection(n)
