"""GPU parity of the whole MoE block (kmoe_block_forward through MoEBlock): router logits,
routing, routed experts, the sigmoid-gated quantized shared expert and the residual blend,
against the oracle (moe_oracle.moe_block; moe_block.metal:194-584)."""
import numpy as np
import pytest
import torch

from kandiga_amd import synth
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


def _block(device, shape, Is, seed, shared=True, gated=True, bits=4, scale_dtype="bf16"):
    from kandiga_amd.moe import MoEBlock, QuantizedExperts

    layer = synth.make_layer(shape, seed)
    blk = synth.make_block(shape, Is, seed + 1, bits=bits, scale_dtype=scale_dtype, shared=shared, gated=gated)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    return layer, blk, MoEBlock.from_arrays(ex, blk, bits, scale_dtype)


def _check(device, layer, blk, mb, shape, T, seed, residual, bits, scale_dtype, what):
    x, _ = synth.make_inputs(shape, T, seed)
    res = (np.random.default_rng(seed + 7).standard_normal((T, shape.hidden)) * 2).astype(np.float16) \
        if residual else None
    xd = torch.from_numpy(x).to(device)
    rd = torch.from_numpy(res).to(device) if residual else None
    out, idx, w, lg = mb(xd, rd, return_routing=True, out_dtype=torch.float32)
    out16 = mb(xd, rd)
    lg_n = to_np(lg)
    # logits: fp32 accumulation of the quantized router against the float64 product
    ref_lg = O.qlinear_f64(blk["blk_router_w"], blk["blk_router_s"], blk["blk_router_b"], bits, x, scale_dtype)
    np.testing.assert_allclose(lg_n, ref_lg, rtol=1e-5, atol=1e-5 * float(np.abs(ref_lg).max()))
    # routing bit-exact on the device's own logits, and equal to the oracle's on its logits
    ref_idx, ref_w = O.route(lg_n, shape.top_k)
    assert np.array_equal(to_np(idx), ref_idx), f"{what}: routing"
    np.testing.assert_allclose(to_np(w), ref_w, rtol=2e-6, atol=2e-7)
    full = O.moe_block(layer, blk, x, shape.top_k, shape.bits, bits, "f16", scale_dtype, residual=res)
    assert np.array_equal(full["idx"], ref_idx), f"{what}: oracle logits route differently"
    ref = O.moe_block(layer, blk, x, shape.top_k, shape.bits, bits, "f16", scale_dtype, residual=res, logits=lg_n,
                      nthreads=8)
    # The reference stores the shared expert's output in fp16 before gating it
    # (moe_block.metal:324): a last-bit difference in its fp32 value may round to the
    # neighbouring fp16 value, one spacing of |shared| times the gate.
    assert_close(to_np(out), ref["out"], what=f"{what} fp32 out", slack=ref["shared_flip"])
    assert_close(to_np(out16), ref["out"], what=f"{what} fp16 out", slack=ref["shared_flip"])


@pytest.mark.parametrize("T", [1, 3, 8, 9, 100])
@pytest.mark.parametrize("residual", [False, True])
def test_block_small(device, T, residual):
    shape = synth.LayerShape(512, 256, 32, 8, 3)
    layer, blk, mb = _block(device, shape, 256, 500)
    _check(device, layer, blk, mb, shape, T, 510 + T, residual, 4, "bf16", f"block T={T} residual={residual}")
    assert mb.experts.device_status() == 0


@pytest.mark.parametrize("variant", ["ungated", "no-shared", "3bit-f16"])
def test_block_variants(device, variant):
    shape = synth.LayerShape(256, 128, 16, 4, 4)
    kw = dict(shared=variant != "no-shared", gated=variant == "3bit-f16")
    bits, sdt = (3, "f16") if variant == "3bit-f16" else (4, "bf16")
    layer, blk, mb = _block(device, shape, 192, 520, bits=bits, scale_dtype=sdt, **kw)
    for T in (2, 40):
        _check(device, layer, blk, mb, shape, T, 530 + T, True, bits, sdt, f"{variant} T={T}")


@pytest.mark.parametrize("T", [1, 8, 512])
def test_block_full_size(device, T):
    """Hidden 2048, 256 routed 3-bit experts (I=512, top-8), 4-bit bf16 router, shared expert
    (Is=512) and shared gate: the 35B-A3B-style block, decode and prefill."""
    shape = synth.SHAPES["h2048-e256-i512-k8-3bit"]
    layer, blk, mb = _block(device, shape, 512, 540)
    _check(device, layer, blk, mb, shape, T, 550 + T, True, 4, "bf16", f"full block T={T}")
