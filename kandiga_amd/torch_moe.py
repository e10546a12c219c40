"""The routed-expert layer inside a PyTorch model.

The reference swaps the ``switch_mlp`` attribute of every MoE block of an mlx_lm Qwen model for
its own expert-MLP wrapper and leaves the router and the combine to the block
(kandiga/engine.py:1085-1128: MoE layers are the ones whose ``mlp`` has a ``switch_mlp``; the
wrapper replaces ``layer.mlp.switch_mlp``).  This module gives the same two moves for a PyTorch
model:

* :class:`QwenMoeBlock` -- a Qwen-style sparse MoE block as a ``torch.nn.Module``: router
  ``gate`` (a linear layer) -> softmax top-K -> renormalise -> ``switch_mlp(x, inds)`` ->
  weighted combine, plus an optional ``shared_expert`` gated by ``sigmoid(shared_expert_gate(x))``.
  Routing and combine run through the library (``kmoe_route`` / ``kmoe_combine``); the expert
  MLP is whatever ``switch_mlp`` holds.
* :func:`install_switch_mlp` -- replaces ``mlp.switch_mlp`` of every MoE layer with a
  :class:`~kandiga_amd.moe.QuantizedSwitchGLU` over experts resident in HBM, as engine.py does.
* :func:`install_moe_block` -- replaces the whole ``layer.mlp`` by a
  :class:`~kandiga_amd.moe.MoEBlock` (one C call for the block).
"""
from __future__ import annotations

import torch

from .moe import MoEBlock, QuantizedExperts, QuantizedSwitchGLU, combine, route


class QwenMoeBlock(torch.nn.Module):
    """Qwen-style sparse MoE block: ``out = sum_k w_k switch_mlp(x)[k] (+ sigmoid(g . x) * shared(x))``.

    ``gate`` maps ``x [..., H]`` to router logits ``[..., E]`` (any module; its output is routed in
    fp32 with ties to the lower expert index), ``switch_mlp(x, inds) -> [..., K, H]``.
    """

    def __init__(self, gate: torch.nn.Module, switch_mlp, top_k: int, shared_expert=None,
                 shared_expert_gate: torch.nn.Module | None = None):
        super().__init__()
        self.gate = gate
        self.switch_mlp = switch_mlp
        self.top_k = top_k
        self.shared_expert = shared_expert
        self.shared_expert_gate = shared_expert_gate

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        logits = self.gate(x).float()
        inds, scores = route(logits, self.top_k)
        y = self.switch_mlp(x, inds)
        out = combine(y, scores)
        if self.shared_expert is not None:
            sh = self.shared_expert(x)
            if self.shared_expert_gate is not None:
                sh = torch.sigmoid(self.shared_expert_gate(x).float()) * sh.float()
            out = (out.float() + sh.float()).to(out.dtype)
        return out


def moe_layers(model: torch.nn.Module):
    """(name, block) of every module whose ``switch_mlp`` attribute holds the expert MLP."""
    return [(n, m) for n, m in model.named_modules() if hasattr(m, "switch_mlp")]


def install_switch_mlp(model: torch.nn.Module, experts: list) -> int:
    """Swap ``switch_mlp`` of the model's MoE blocks (in module order) for a QuantizedSwitchGLU over
    ``experts[i]`` (QuantizedExperts, one per MoE block); returns the number swapped."""
    blocks = moe_layers(model)
    if len(blocks) != len(experts):
        raise ValueError(f"model has {len(blocks)} MoE blocks, got experts for {len(experts)}")
    for (_name, blk), ex in zip(blocks, experts):
        if not isinstance(ex, QuantizedExperts):
            raise TypeError("experts must be QuantizedExperts")
        top_k = getattr(blk, "top_k", ex.shape.top_k)
        if top_k != ex.shape.top_k:
            raise ValueError(f"block routes top-{top_k}, experts were built for top-{ex.shape.top_k}")
        blk.switch_mlp = QuantizedSwitchGLU(ex)
    return len(blocks)


class _BlockModule(torch.nn.Module):
    """A MoEBlock in a module slot: ``forward(x) -> mlp(x)``."""

    def __init__(self, block: MoEBlock):
        super().__init__()
        self.block = block

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.block(x)


def install_moe_block(model: torch.nn.Module, blocks: list, attr: str = "mlp") -> int:
    """Replace ``<layer>.<attr>`` of every layer whose ``attr`` is a MoE block (has ``switch_mlp``)
    by the corresponding MoEBlock (router, experts, shared expert in one C call)."""
    owners = [m for _n, m in model.named_modules() if hasattr(getattr(m, attr, None), "switch_mlp")]
    if len(owners) != len(blocks):
        raise ValueError(f"model has {len(owners)} MoE blocks, got {len(blocks)}")
    for owner, blk in zip(owners, blocks):
        setattr(owner, attr, _BlockModule(blk))
    return len(owners)
