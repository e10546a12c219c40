"""MLX safetensors ingestion of stacked switch_mlp tensors (CPU): naming, sharding, shape
checks, the per-expert files of the reference's split step, and the host-side refusal of
tensors that are not in device memory."""
import os

import numpy as np
import pytest
import torch

from kandiga_amd import synth, weights


def _same(layer, L):
    for k, v in layer.items():
        assert np.array_equal(L[k].cpu().numpy().view(v.dtype), v), k


@pytest.mark.parametrize("bits,scale_dtype,shards", [(3, "bf16", 1), (4, "bf16", 3), (3, "f16", 2)])
def test_stacked_roundtrip(tmp_path, bits, scale_dtype, shards):
    shape = synth.LayerShape(192, 128, 6, 2, bits)
    layer = synth.make_layer(shape, 31 + bits, scale_dtype)
    d = tmp_path / "ckpt"
    d.mkdir()
    weights.write_switch_mlp(str(d), layer, 7, scale_dtype, shards=shards)
    assert weights.moe_layers(str(d)) == [7]
    L, info = weights.read_switch_mlp(str(d), 7)
    assert info == weights.SwitchMlpInfo(192, 128, 6, bits, scale_dtype)
    _same(layer, L)
    # the exact MLX key names the reference reads (kandiga/_split_experts.py:62-117)
    import json
    wm = json.load(open(d / "model.safetensors.index.json"))["weight_map"]
    assert "language_model.model.layers.7.mlp.switch_mlp.down_proj.biases" in wm


def test_single_file_and_custom_prefix(tmp_path):
    shape = synth.LayerShape(128, 64, 3, 1, 4)
    layer = synth.make_layer(shape, 5, "bf16")
    f = str(tmp_path / "m.safetensors")
    weights.write_switch_mlp(f, layer, 0, "bf16", prefix="model.layers")
    assert weights.moe_layers(f, prefix="model.layers") == [0]
    L, info = weights.read_switch_mlp(f, 0, prefix="model.layers")
    assert info.bits == 4 and info.hidden == 128 and info.intermediate == 64
    _same(layer, L)
    with pytest.raises(KeyError):
        weights.read_switch_mlp(f, 1, prefix="model.layers")


def test_expert_files_stack_back(tmp_path):
    """layer_XX/expert_NNN.safetensors with keys {proj}.{part} (kandiga/_split_experts.py:106-115)."""
    from safetensors.torch import save_file

    shape = synth.LayerShape(128, 64, 4, 2, 3)
    layer = synth.make_layer(shape, 9, "bf16")
    d = tmp_path / "layer_00"
    d.mkdir()
    for e in range(4):
        t = {}
        for proj in ("gate", "up", "down"):
            t[f"{proj}_proj.weight"] = torch.from_numpy(layer[f"{proj}_w"][e].view(np.int32)).view(torch.uint32)
            t[f"{proj}_proj.scales"] = torch.from_numpy(layer[f"{proj}_s"][e].view(np.int16)).view(torch.bfloat16)
            t[f"{proj}_proj.biases"] = torch.from_numpy(layer[f"{proj}_b"][e].view(np.int16)).view(torch.bfloat16)
        save_file(t, str(d / f"expert_{e:03d}.safetensors"))
    L, info = weights.read_expert_files(str(d))
    assert info == weights.SwitchMlpInfo(128, 64, 4, 3, "bf16")
    _same(layer, L)
    os.remove(d / "expert_002.safetensors")
    with pytest.raises(ValueError):
        weights.read_expert_files(str(d))


def test_shape_mismatch_rejected(tmp_path):
    shape = synth.LayerShape(128, 128, 3, 1, 3)
    layer = synth.make_layer(shape, 11, "bf16")
    layer["down_s"] = layer["down_s"][:, :, :1].copy()   # one group per row instead of two
    layer["down_b"] = layer["down_b"][:, :, :1].copy()
    f = str(tmp_path / "bad.safetensors")
    weights.write_switch_mlp(f, layer, 0, "bf16")
    with pytest.raises(ValueError):
        weights.read_switch_mlp(f, 0)


def test_host_tensors_rejected_before_launch():
    """route / permute / combine refuse host tensors with a ValueError before any C call."""
    from kandiga_amd.moe import combine, permute, route

    with pytest.raises(ValueError):
        route(torch.zeros(2, 16), 2)
    with pytest.raises(ValueError):
        permute(torch.zeros(2, 2, dtype=torch.int32), 16)
    with pytest.raises(ValueError):
        combine(torch.zeros(2, 2, 64, dtype=torch.float16), torch.ones(2, 2))
    with pytest.raises(TypeError):
        route(np.zeros((2, 16), np.float32), 2)
