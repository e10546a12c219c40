"""Shared helpers of the GPU parity tests (seeded layers, oracle subsets, error metrics)."""
from __future__ import annotations

import numpy as np
import torch

from kandiga_amd import synth
from oracle import moe_oracle as O

# Output tolerance of the routed layer against the fp32-accumulated oracle.
MAX_ABS = 2e-2
REL_L2 = 1e-3


def f16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of fp16 values at |v| (normal range; 2**-24 below it)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 10)


def assert_close(got, ref, max_abs=MAX_ABS, rel_l2=REL_L2, what="", fp16_out=None, slack=None):
    """max |got-ref| <= max_abs and rel-L2 <= rel_l2.

    For fp16 outputs (``got`` of dtype float16, or ``fp16_out=True``) an element may instead
    be within half an fp16 ulp of the fp32 reference plus 2e-3: above |out| = 32 the output
    rounding alone (half of a 1/32 spacing) exceeds 2e-2 even for a correctly rounded result,
    and the 2e-3 covers fp32 accumulation-order differences before that rounding.
    """
    is16 = (np.asarray(got).dtype == np.float16) if fp16_out is None else fp16_out
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    err = O.compare(g, r)
    diff = np.abs(g - r)
    allowed = np.maximum(max_abs, 0.5 * f16_ulp(r) + 2e-3) if is16 else np.full_like(r, max_abs)
    if slack is not None:   # a per-element allowance for an fp16 intermediate the reference rounds
        allowed = allowed + np.asarray(slack, dtype=np.float64)
    worst = float((diff - allowed).max()) if diff.size else 0.0
    print(f"  {what}: max_abs={err['max_abs']:.3e} rel_l2={err['rel_l2']:.3e} max|ref|="
          f"{float(np.abs(r).max()) if r.size else 0:.1f} fp16_out={is16}", flush=True)
    assert worst <= 0 and err["rel_l2"] <= rel_l2, f"{what}: {err} (worst excess {worst:.3e})"
    return err


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def torch_layer_subset(layer_t: dict, experts) -> dict:
    """Host copy of the listed experts of a device-generated layer (oracle input)."""
    ex = torch.as_tensor(np.asarray(experts, dtype=np.int64), device=layer_t["gate_w"].device)
    out = {}
    for k, v in layer_t.items():
        if k.startswith("shared_"):
            out[k] = to_np(v).view(np.uint16)
            continue
        sub = to_np(v.index_select(0, ex))
        out[k] = sub.view(np.uint32) if k.endswith("_w") else sub.view(np.uint16)
    return out


def oracle_rows(layer_np: dict, x: np.ndarray, idx: np.ndarray, bits: int, scale_dtype="f16", nthreads=8):
    """Oracle switch_mlp for the given tokens, on a layer that may be an expert subset:
    ``idx`` holds positions into the subset."""
    return O.switch_mlp(layer_np, x, idx, bits, scale_dtype, nthreads=nthreads)


def remap(idx: np.ndarray):
    """Distinct experts of idx and idx rewritten as positions into that list."""
    uniq, inv = np.unique(idx, return_inverse=True)
    return uniq, inv.reshape(idx.shape).astype(np.int32)


def host_layer(layer) -> dict:
    """Host numpy copy of a layer dict (numpy or device tensors), 32-bit words as uint32 and
    16-bit patterns as uint16."""
    out = {}
    for k, v in layer.items():
        a = to_np(v) if isinstance(v, torch.Tensor) else np.asarray(v)
        out[k] = a.view(np.uint32) if k.endswith("_w") else a.view(np.uint16)
    return out


def dense_reference(layer_h: dict, shape, x, idx, w, scale_dtype="f16", dtype=np.float64, exact_x=False):
    """Oracle output of every row of a full-size batch: routed combine through dense per-expert
    products (oracle.moe_out_dense) plus the shared expert when the layer has one."""
    out = O.moe_out_dense(lambda e: {k: v[e] for k, v in layer_h.items() if not k.startswith("shared_")},
                          x, idx, w, shape.bits, shape.hidden, shape.intermediate, scale_dtype, dtype=dtype,
                          exact_x=exact_x)
    if "shared_gate" in layer_h:
        out = out + O.shared_expert_f64(layer_h, x)
    return out
