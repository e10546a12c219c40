"""Seeded synthetic MoE layers in the MLX stacked layout.

Weights: codes uniform in ``[0, 2**bits - 1]`` (uniformly random packed bits are
uniform codes for both 3- and 4-bit packing), scales ``|N(0, 0.02)|`` rounded to
bf16 and clamped to ``[2**-14, 4096]`` so every scale is exactly representable in
both fp16 and bf16, biases ``-2**(bits-1) * scale`` (exact in both formats).
Activations ``x`` are fp16 ``N(0, 1)``; router logits are fp32 ``N(0, 1)``,
optionally plus a Zipf(1.1) per-expert bias for skewed prefill routing.

Numpy generation (``make_layer``/``make_inputs``) feeds the CPU oracle; the torch
generators build the same distributions directly in device memory for
benchmark-sized stacks.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .layout import GROUP_SIZE, f16_bits, f16_to_bf16_bits, f32_to_bf16_bits, packed_row_words

SCALE_STD = 0.02
SCALE_MIN = 2.0 ** -14
SCALE_MAX = 4096.0
SHARED_STD = 0.02


@dataclass(frozen=True)
class LayerShape:
    hidden: int
    intermediate: int
    num_experts: int
    top_k: int
    bits: int
    shared_intermediate: int = 0

    @property
    def name(self) -> str:
        s = (f"h{self.hidden}-e{self.num_experts}-i{self.intermediate}"
             f"-k{self.top_k}-{self.bits}bit")
        if self.shared_intermediate:
            s += f"-shared{self.shared_intermediate}"
        return s

    @property
    def expert_bytes(self) -> int:
        H, I, b = self.hidden, self.intermediate, self.bits
        codes = 3 * H * I * b // 8
        sb = 2 * 2 * (2 * I * (H // GROUP_SIZE) + H * (I // GROUP_SIZE))
        return codes + sb

    @property
    def shared_bytes(self) -> int:
        return 3 * self.hidden * self.shared_intermediate * 2

    def with_top_k(self, k: int) -> "LayerShape":
        return LayerShape(self.hidden, self.intermediate, self.num_experts, k, self.bits,
                          self.shared_intermediate)


# The layer shapes of the workloads this library is measured on.
SHAPES = {
    s.name: s for s in (
        LayerShape(2048, 512, 256, 8, 4),
        LayerShape(2048, 512, 256, 8, 3),
        LayerShape(2560, 1024, 256, 8, 3, shared_intermediate=1024),
        LayerShape(4096, 1024, 512, 10, 3),
    )
}


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _scales_f16_bits(rng, shape) -> np.ndarray:
    s = np.abs(rng.standard_normal(shape, dtype=np.float32)) * np.float32(SCALE_STD)
    s = f32_to_bf16_bits(s)                               # round to bf16 ...
    s = (s.astype(np.uint32) << 16).view(np.float32)
    s = np.clip(s, SCALE_MIN, SCALE_MAX)                  # ... inside the fp16 normal range
    return f16_bits(s.astype(np.float16))


def make_layer(shape: LayerShape, seed: int, scale_dtype: str = "f16") -> dict:
    """Stacked layer dict: ``{gate,up,down}_{w,s,b}`` numpy arrays (+ shared expert).

    ``*_w`` are uint32 ``[E, rows, in*bits/32]``; ``*_s``/``*_b`` are uint16 bit
    patterns of ``scale_dtype`` (``'f16'`` or ``'bf16'``) with shape ``[E, rows, in/64]``.
    """
    rng = _rng(seed)
    E, H, I, b = shape.num_experts, shape.hidden, shape.intermediate, shape.bits
    layer = {}
    for proj, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
        words = packed_row_words(cols, b)
        layer[f"{proj}_w"] = rng.integers(0, 2 ** 32, size=(E, rows, words), dtype=np.uint32)
        s = _scales_f16_bits(rng, (E, rows, cols // GROUP_SIZE))
        bias = f16_bits(s.view(np.float16).astype(np.float32) * np.float32(-(2 ** (b - 1))))
        if scale_dtype == "bf16":
            s, bias = f16_to_bf16_bits(s), f16_to_bf16_bits(bias)
        elif scale_dtype != "f16":
            raise ValueError(scale_dtype)
        layer[f"{proj}_s"] = s
        layer[f"{proj}_b"] = bias
    if shape.shared_intermediate:
        Is = shape.shared_intermediate
        for name, dims in (("shared_gate", (Is, H)), ("shared_up", (Is, H)), ("shared_down", (H, Is))):
            layer[name] = f16_bits(rng.standard_normal(dims, dtype=np.float32) * np.float32(SHARED_STD))
    return layer


def zipf_expert_bias(num_experts: int, rng: np.random.Generator, alpha: float = 1.1) -> np.ndarray:
    """Per-expert logit bias ``-alpha*ln(r_e)`` (r a random permutation of 1..E), mean-centred.

    Softmax weights then follow a Zipf(alpha) law over experts, so expert loads are skewed.
    """
    r = rng.permutation(num_experts).astype(np.float64) + 1.0
    beta = -alpha * np.log(r)
    return (beta - beta.mean()).astype(np.float32)


def make_inputs(shape: LayerShape, tokens: int, seed: int, zipf: bool = False):
    """Activations ``x`` fp16 ``[T, H]`` and router logits fp32 ``[T, E]``."""
    rng = _rng(seed)
    x = rng.standard_normal((tokens, shape.hidden), dtype=np.float32).astype(np.float16)
    logits = rng.standard_normal((tokens, shape.num_experts), dtype=np.float32)
    if zipf:
        logits = logits + zipf_expert_bias(shape.num_experts, rng)[None, :]
    return x, logits.astype(np.float32)


# --------------------------------------------------------------------------------------
# Device-side generation (benchmark stacks)
# --------------------------------------------------------------------------------------
def make_layer_torch(shape: LayerShape, seed: int, device, scale_dtype: str = "f16") -> dict:
    """Same distributions as :func:`make_layer`, generated in device memory with torch."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    E, H, I, b = shape.num_experts, shape.hidden, shape.intermediate, shape.bits
    layer = {}
    for proj, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
        words = packed_row_words(cols, b)
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, rows, words), generator=g, device=device,
                          dtype=torch.int32)
        layer[f"{proj}_w"] = w
        s = torch.randn((E, rows, cols // GROUP_SIZE), generator=g, device=device,
                        dtype=torch.float32).abs_().mul_(SCALE_STD)
        s = s.to(torch.bfloat16).to(torch.float32).clamp_(SCALE_MIN, SCALE_MAX)
        bias = s * float(-(2 ** (b - 1)))
        tdt = torch.float16 if scale_dtype == "f16" else torch.bfloat16
        layer[f"{proj}_s"] = s.to(tdt).view(torch.int16)
        layer[f"{proj}_b"] = bias.to(tdt).view(torch.int16)
    if shape.shared_intermediate:
        Is = shape.shared_intermediate
        for name, dims in (("shared_gate", (Is, H)), ("shared_up", (Is, H)), ("shared_down", (H, Is))):
            layer[name] = (torch.randn(dims, generator=g, device=device) * SHARED_STD).to(
                torch.float16).view(torch.int16)
    return layer


def make_inputs_torch(shape: LayerShape, tokens: int, seed: int, device, zipf: bool = False):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.randn((tokens, shape.hidden), generator=g, device=device).to(torch.float16)
    logits = torch.randn((tokens, shape.num_experts), generator=g, device=device)
    if zipf:
        bias = zipf_expert_bias(shape.num_experts, _rng(seed))
        logits = logits + torch.from_numpy(bias).to(device)[None, :]
    return x, logits.contiguous()


# --------------------------------------------------------------------------------------
# The projections of the MoE block around the routed experts
# --------------------------------------------------------------------------------------
def make_block(shape: LayerShape, shared_intermediate: int, seed: int, bits: int = 4, scale_dtype: str = "bf16",
               shared: bool = True, gated: bool = True) -> dict:
    """Quantized router ``blk_router_{w,s,b}`` ``[E, H]``, shared expert ``blk_shared_{gate,up,down}_{w,s,b}``
    (gate/up ``[Is, H]``, down ``[H, Is]``) and shared gate ``blk_sgate_{w,s,b}`` ``[1, H]`` in the MLX
    layout with ``bits``-bit codes (the distributions of :func:`make_layer`, without the expert
    dimension)."""
    rng = _rng(seed)
    H, E, Is = shape.hidden, shape.num_experts, shared_intermediate
    out = {}
    projs = [("blk_router", E, H)]
    if shared:
        projs += [("blk_shared_gate", Is, H), ("blk_shared_up", Is, H), ("blk_shared_down", H, Is)]
        if gated:
            projs += [("blk_sgate", 1, H)]
    for name, rows, cols in projs:
        out[f"{name}_w"] = rng.integers(0, 2 ** 32, size=(rows, packed_row_words(cols, bits)), dtype=np.uint32)
        sc = _scales_f16_bits(rng, (rows, cols // GROUP_SIZE))
        bi = f16_bits(sc.view(np.float16).astype(np.float32) * np.float32(-(2 ** (bits - 1))))
        if scale_dtype == "bf16":
            sc, bi = f16_to_bf16_bits(sc), f16_to_bf16_bits(bi)
        out[f"{name}_s"] = sc
        out[f"{name}_b"] = bi
    return out
