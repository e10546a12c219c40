"""Routed-expert weights from MLX safetensors checkpoints.

mlx_lm stores a quantized SwitchGLU as nine stacked tensors per MoE layer
(the keys kandiga/_split_experts.py:62-117 collects):

    {prefix}.{layer}.mlp.switch_mlp.{gate,up,down}_proj.{weight,scales,biases}

``weight`` is uint32 ``[E, rows, in*bits/32]``; ``scales`` / ``biases`` are bf16 (or fp16)
``[E, rows, in/64]``; gate/up rows are the expert intermediate size, down rows the hidden
size.  A checkpoint is one ``model.safetensors`` file or shards listed by
``model.safetensors.index.json`` (``weight_map``: tensor name -> shard file).  The reference's
split step also writes one file per expert, ``layer_XX/expert_NNN.safetensors`` with keys
``{gate,up,down}_proj.{weight,scales,biases}`` (kandiga/_split_experts.py:106-115), which
:func:`read_expert_files` stacks back.

The result is the stacked layer dict of :mod:`kandiga_amd.synth` (``gate_w`` uint32 bits,
``gate_s`` / ``gate_b`` 16-bit patterns, ...) as torch tensors, plus a :class:`SwitchMlpInfo`
with the dimensions, bit width and scale dtype read from the tensor shapes.
"""
from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass

import torch

from .layout import GROUP_SIZE

PROJS = ("gate_proj", "up_proj", "down_proj")
PARTS = ("weight", "scales", "biases")
DEFAULT_PREFIX = "language_model.model.layers"


@dataclass(frozen=True)
class SwitchMlpInfo:
    hidden: int
    intermediate: int
    num_experts: int
    bits: int
    scale_dtype: str   # "bf16" or "f16"


def _key(prefix: str, layer: int, proj: str, part: str) -> str:
    return f"{prefix}.{layer}.mlp.switch_mlp.{proj}.{part}"


def _weight_map(path: str) -> dict:
    """Tensor name -> file for a checkpoint directory or a single .safetensors file."""
    from safetensors import safe_open

    if os.path.isdir(path):
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                wm = json.load(f)["weight_map"]
            return {k: os.path.join(path, v) for k, v in wm.items()}
        single = os.path.join(path, "model.safetensors")
        if not os.path.exists(single):
            raise FileNotFoundError(f"{path}: neither model.safetensors.index.json nor model.safetensors")
        path = single
    with safe_open(path, framework="pt") as f:
        return {k: path for k in f.keys()}


def moe_layers(path: str, prefix: str = DEFAULT_PREFIX) -> list:
    """Indices of the layers whose switch_mlp tensors a checkpoint holds."""
    pat = re.compile(re.escape(prefix) + r"\.(\d+)\.mlp\.switch_mlp\.")
    found = set()
    for k in _weight_map(path):
        m = pat.match(k)
        if m:
            found.add(int(m.group(1)))
    return sorted(found)


def _info(t: dict) -> SwitchMlpInfo:
    gw, gs, dw, ds = t[("gate_proj", "weight")], t[("gate_proj", "scales")], t[("down_proj", "weight")], \
        t[("down_proj", "scales")]
    if gw.dim() != 3 or gs.dim() != 3:
        raise ValueError("switch_mlp tensors must be stacked [experts, rows, cols]")
    E, inter, gwords = gw.shape
    hidden = gs.shape[2] * GROUP_SIZE
    if gwords * 32 % hidden:
        raise ValueError(f"gate_proj.weight has {gwords} words per row for hidden {hidden}")
    bits = gwords * 32 // hidden
    if bits not in (3, 4):
        raise ValueError(f"{bits}-bit codes are not supported (3 or 4)")
    if gs.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"scales dtype {gs.dtype} is neither bfloat16 nor float16")
    want = {
        ("gate_proj", "weight"): (E, inter, hidden * bits // 32),
        ("up_proj", "weight"): (E, inter, hidden * bits // 32),
        ("down_proj", "weight"): (E, hidden, inter * bits // 32),
        ("gate_proj", "scales"): (E, inter, hidden // GROUP_SIZE),
        ("up_proj", "scales"): (E, inter, hidden // GROUP_SIZE),
        ("down_proj", "scales"): (E, hidden, inter // GROUP_SIZE),
    }
    for (proj, part), shape in want.items():
        for p in ((part,) if part == "weight" else ("scales", "biases")):
            got = tuple(t[(proj, p)].shape)
            if got != shape:
                raise ValueError(f"{proj}.{p}: shape {got}, expected {shape}")
            if p != "weight" and t[(proj, p)].dtype != gs.dtype:
                raise ValueError(f"{proj}.{p}: dtype {t[(proj, p)].dtype} differs from gate scales {gs.dtype}")
    if dw.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"weight dtype {dw.dtype} is not a 32-bit integer")
    del ds
    return SwitchMlpInfo(hidden, inter, E, bits, "bf16" if gs.dtype == torch.bfloat16 else "f16")


def _to_layer(t: dict, device) -> dict:
    layer = {}
    for proj in PROJS:
        name = proj.split("_")[0]
        w = t[(proj, "weight")]
        layer[f"{name}_w"] = (w.view(torch.int32) if w.dtype == torch.uint32 else w).to(device).contiguous()
        layer[f"{name}_s"] = t[(proj, "scales")].view(torch.int16).to(device).contiguous()
        layer[f"{name}_b"] = t[(proj, "biases")].view(torch.int16).to(device).contiguous()
    return layer


def read_switch_mlp(path: str, layer: int, prefix: str = DEFAULT_PREFIX, device="cpu"):
    """The nine stacked switch_mlp tensors of one MoE layer -> (layer dict, SwitchMlpInfo).

    ``path`` is a checkpoint directory (sharded or single-file) or one ``.safetensors`` file.
    Only the nine tensors are read (``safe_open`` per shard), optionally straight into
    ``device`` memory."""
    from safetensors import safe_open

    wm = _weight_map(path)
    keys = {(proj, part): _key(prefix, layer, proj, part) for proj in PROJS for part in PARTS}
    missing = [k for k in keys.values() if k not in wm]
    if missing:
        raise KeyError(f"layer {layer}: missing tensors {missing[:3]}{'...' if len(missing) > 3 else ''}")
    by_file: dict = {}
    for pk, k in keys.items():
        by_file.setdefault(wm[k], []).append((pk, k))
    t = {}
    for fname, entries in by_file.items():
        with safe_open(fname, framework="pt") as f:
            for pk, k in entries:
                t[pk] = f.get_tensor(k)
    info = _info(t)
    return _to_layer(t, device), info


def read_expert_files(layer_dir: str, device="cpu"):
    """Per-expert files ``expert_NNN.safetensors`` of one layer (the reference's split step)
    stacked back into (layer dict, SwitchMlpInfo)."""
    from safetensors import safe_open

    files = sorted(f for f in os.listdir(layer_dir) if re.fullmatch(r"expert_\d+\.safetensors", f))
    if not files:
        raise FileNotFoundError(f"{layer_dir}: no expert_NNN.safetensors files")
    ids = [int(f[7:-12]) for f in files]
    if ids != list(range(len(ids))):
        raise ValueError(f"{layer_dir}: expert files are not numbered 0..{len(ids) - 1}")
    parts: dict = {(p, c): [] for p in PROJS for c in PARTS}
    for f in files:
        with safe_open(os.path.join(layer_dir, f), framework="pt") as fh:
            for p in PROJS:
                for c in PARTS:
                    parts[(p, c)].append(fh.get_tensor(f"{p}.{c}"))
    t = {k: torch.stack(v) for k, v in parts.items()}
    info = _info(t)
    return _to_layer(t, device), info


def write_switch_mlp(path: str, layer_dict: dict, layer: int, scale_dtype: str, prefix: str = DEFAULT_PREFIX,
                     shards: int = 1) -> None:
    """Write a stacked layer dict as MLX-named safetensors (one file, or ``shards`` files plus
    ``model.safetensors.index.json`` when ``path`` is a directory).  The 16-bit arrays must be
    bit patterns of ``scale_dtype``."""
    import numpy as np
    from safetensors.torch import save_file

    sdt = {"bf16": torch.bfloat16, "f16": torch.float16}[scale_dtype]
    tensors = {}
    for proj in PROJS:
        name = proj.split("_")[0]
        for part, key in (("weight", "w"), ("scales", "s"), ("biases", "b")):
            a = layer_dict[f"{name}_{key}"]
            a = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a).view(
                np.int32 if key == "w" else np.int16))
            a = a.cpu().contiguous()
            tensors[_key(prefix, layer, proj, part)] = a.view(torch.uint32) if key == "w" else a.view(sdt)
    if not os.path.isdir(path):
        save_file(tensors, path)
        return
    names = sorted(tensors)
    wm = {}
    for i in range(shards):
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: tensors[k] for k in names[i::shards]}
        save_file(part, os.path.join(path, fname))
        wm.update({k: fname for k in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
