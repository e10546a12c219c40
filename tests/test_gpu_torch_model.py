"""A PyTorch model whose MoE blocks get the HIP expert MLP swapped in, as the reference swaps
layer.mlp.switch_mlp (kandiga/engine.py:1085-1128), checked end to end against the oracle."""
import numpy as np
import pytest
import torch

from kandiga_amd import synth
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


class DequantLinear(torch.nn.Module):
    """A quantized linear layer of the model under test (router / shared gate), dequantized once
    into an fp32 matrix; x @ W.T in fp32."""

    def __init__(self, w, s, b, bits, scale_dtype, device):
        super().__init__()
        H = s.shape[-1] * 64
        self.register_buffer("W", torch.from_numpy(O.dequantize(w, s, b, bits, H, scale_dtype)).float().to(device))

    def forward(self, x):
        return x.float() @ self.W.T


class PendingSwitch:
    """Stand-in for the model's original expert MLP; forward is never reached after the swap."""

    def __call__(self, x, inds):
        raise RuntimeError("switch_mlp was not replaced")


class Layer(torch.nn.Module):
    def __init__(self, mlp):
        super().__init__()
        self.mlp = mlp

    def forward(self, h):
        return h + self.mlp(h)


def _model(device, shape, nlayers, seed):
    from kandiga_amd.torch_moe import QwenMoeBlock

    layers, blks, lays = [], [], []
    for i in range(nlayers):
        lay = synth.make_layer(shape, seed + 10 * i)
        blk = synth.make_block(shape, 128, seed + 10 * i + 1, bits=4, scale_dtype="bf16", shared=False)
        router = DequantLinear(blk["blk_router_w"], blk["blk_router_s"], blk["blk_router_b"], 4, "bf16", device)
        layers.append(Layer(QwenMoeBlock(router, PendingSwitch(), shape.top_k)))
        blks.append(blk)
        lays.append(lay)
    return torch.nn.Sequential(*layers), lays, blks


@pytest.mark.parametrize("T", [1, 6, 50])
def test_switch_mlp_swap_end_to_end(device, T):
    """Two MoE layers with residuals: h1 = h0 + moe1(h0), h2 = h1 + moe2(h1).  Hooks capture each
    block's input, router logits and output; every block output is checked against the oracle on
    the same input and logits (routing bit-exact on those logits), and the model output is the
    fp16 chain of the block outputs."""
    from kandiga_amd.moe import QuantizedExperts
    from kandiga_amd.torch_moe import install_switch_mlp, moe_layers

    shape = synth.LayerShape(256, 128, 16, 4, 3)
    model, lays, blks = _model(device, shape, 2, 600)
    assert len(moe_layers(model)) == 2
    with pytest.raises(RuntimeError):
        model(torch.zeros((1, 256), dtype=torch.float16, device=device))
    n = install_switch_mlp(model, [QuantizedExperts.from_stacked(shape, L, device) for L in lays])
    assert n == 2
    seen = []
    hooks = []
    for _name, blk in moe_layers(model):
        rec = {}
        hooks.append(blk.gate.register_forward_hook(lambda m, i, o, rec=rec: rec.__setitem__("logits", to_np(o))))
        hooks.append(blk.register_forward_hook(
            lambda m, i, o, rec=rec: rec.update(x=to_np(i[0]), out=to_np(o))))
        seen.append(rec)
    x, _ = synth.make_inputs(shape, T, 610 + T)
    out = to_np(model(torch.from_numpy(x).to(device)))
    for h in hooks:
        h.remove()
    h = x
    for li, (lay, blk, rec) in enumerate(zip(lays, blks, seen)):
        assert np.array_equal(rec["x"], h)
        ref_lg = O.qlinear_f64(blk["blk_router_w"], blk["blk_router_s"], blk["blk_router_b"], 4, h, "bf16")
        np.testing.assert_allclose(rec["logits"], ref_lg, rtol=1e-5, atol=1e-5 * float(np.abs(ref_lg).max()))
        ref = O.moe_layer(lay, h, rec["logits"], shape.top_k, 3)
        assert_close(rec["out"], ref["out"], what=f"layer {li} T={T}")
        h = (h.astype(np.float32) + rec["out"].astype(np.float32)).astype(np.float16)
    assert np.array_equal(out, h)


def test_moe_block_install(device):
    """The whole mlp replaced by MoEBlock (router + experts + shared expert in one call)."""
    from kandiga_amd.moe import MoEBlock, QuantizedExperts
    from kandiga_amd.torch_moe import install_moe_block

    shape = synth.LayerShape(256, 128, 16, 4, 3)
    model, lays, blks = _model(device, shape, 1, 700)
    full = synth.make_block(shape, 128, 701, bits=4, scale_dtype="bf16")   # router + gated shared expert
    mb = MoEBlock.from_arrays(QuantizedExperts.from_stacked(shape, lays[0], device), full, 4, "bf16")
    assert install_moe_block(model, [mb]) == 1
    x, _ = synth.make_inputs(shape, 7, 711)
    out = to_np(model(torch.from_numpy(x).to(device)))
    r = O.moe_block(lays[0], full, x, shape.top_k, 3, 4, "f16", "bf16")
    want = x.astype(np.float32) + O.round_f16(r["out"]).astype(np.float32)
    assert_close(out, want, what="installed MoEBlock", slack=r["shared_flip"])
