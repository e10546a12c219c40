"""GPU parity of bf16 and fp32 activations (kmoe_forward_x / kmoe_expert_mlp_x, through
SparseMoeBlock and QuantizedSwitchGLU), decode (T <= 8) and grouped-GEMM (T > 8) paths.

The reference widens bf16 and fp32 activations to fp32 (kandiga_cpu_expert.m:471-552, 690-719);
the oracle takes them the same way (``exact_x``).  Each token's row is scaled by a power of two
into fp16's range, so:
* fp16-representable values given as fp32 (or as bf16, when bf16 holds them) give the fp16
  path's result bit for bit;
* rows far outside fp16's range (1e5, 1e-6) keep their precision: outputs in fp32 against the
  oracle with a relative bar (max |err| <= 1e-3 * max |ref|, rel-L2 <= 1e-4), since the SwiGLU
  output grows with the square of the row scale;
* general fp32 values (not fp16-representable) meet the layer bar against the fp32 oracle.
"""
import numpy as np
import pytest
import torch

from kandiga_amd import synth
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, dense_reference, f16_ulp, host_layer, to_np

pytestmark = pytest.mark.gpu

SHAPES = {
    "3bit": synth.LayerShape(256, 128, 16, 4, 3),
    "4bit": synth.LayerShape(256, 128, 16, 4, 4),
}


def _layer(device, shape, seed, prefill_copy=False):
    from kandiga_amd.moe import QuantizedExperts

    layer = synth.make_layer(shape, seed)
    return layer, QuantizedExperts.from_stacked(shape, layer, device, prefill_copy=prefill_copy)


def _bf16_values(a: np.ndarray) -> np.ndarray:
    """float32 values rounded to bf16 (round to nearest even), as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def _rel_close(got, ref, what):
    g, r = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.abs(g - r).max()
    scale = np.abs(r).max()
    rel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-300)
    print(f"  {what}: max|err| {err:.3e} of max|ref| {scale:.3e}, rel-L2 {rel:.2e}", flush=True)
    assert err <= 1e-3 * scale and rel <= 1e-4, what


@pytest.mark.parametrize("name", sorted(SHAPES))
@pytest.mark.parametrize("T", [1, 3, 8, 9, 300])
def test_fp16_values_as_fp32_and_bf16_are_bit_identical(device, name, T):
    from kandiga_amd.moe import QuantizedSwitchGLU, SparseMoeBlock

    shape = SHAPES[name]
    _layer_np, ex = _layer(device, shape, 9100 + T)
    x, lg = synth.make_inputs(shape, T, 9200 + T)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)
    blk, sw = SparseMoeBlock(ex), QuantizedSwitchGLU(ex)
    ref, idx, _w = blk(xd, ld, return_routing=True, out_dtype=torch.float32)
    got32 = blk(xd.float(), ld, out_dtype=torch.float32)
    assert torch.equal(got32, ref), f"fp32 copy of fp16 x, T={T}"
    y16 = sw(xd, idx)
    assert torch.equal(sw(xd.float(), idx), y16)
    # bf16 holds these values only where their mantissa fits 8 bits: round x to bf16 first
    xb = torch.from_numpy(_bf16_values(x.astype(np.float32))).to(device)
    assert torch.equal(xb.half().float(), xb)  # inside fp16's normal range, so fp16 holds them too
    assert torch.equal(blk(xb.bfloat16(), ld, out_dtype=torch.float32), blk(xb.half(), ld, out_dtype=torch.float32))
    assert torch.equal(sw(xb.bfloat16(), idx), sw(xb.half(), idx))
    assert ex.device_status() == 0


@pytest.mark.parametrize("name", sorted(SHAPES))
@pytest.mark.parametrize("T", [1, 5, 8, 40])
def test_fp32_activations_against_oracle(device, name, T):
    from kandiga_amd.moe import QuantizedSwitchGLU, SparseMoeBlock

    shape = SHAPES[name]
    layer, ex = _layer(device, shape, 9300 + T)
    rng = np.random.default_rng(9400 + T)
    x = rng.standard_normal((T, shape.hidden)).astype(np.float32)
    _, lg = synth.make_inputs(shape, T, 9500 + T)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)
    out, idx, w = SparseMoeBlock(ex)(xd, ld, return_routing=True, out_dtype=torch.float32)
    ref_idx, ref_w = O.route(lg, shape.top_k)
    assert np.array_equal(to_np(idx), ref_idx)
    y_ref = O.switch_mlp(layer, x, ref_idx, shape.bits, exact_x=True)
    assert_close(to_np(out), O.combine(y_ref, ref_w), what=f"{name} fp32 x T={T} layer")
    y = QuantizedSwitchGLU(ex)(xd, idx)
    assert_close(to_np(y), y_ref, what=f"{name} fp32 x T={T} switch_mlp")
    # fp16-rounded x would be a different answer: the layer output (fp32) sits far closer to the
    # fp32-x oracle than the fp16-x oracle does
    ref = O.combine(y_ref, ref_w).astype(np.float64)
    ref16 = O.combine(O.switch_mlp(layer, x, ref_idx, shape.bits), ref_w).astype(np.float64)
    assert np.abs(to_np(out) - ref).max() < 0.1 * np.abs(ref16 - ref).max()


@pytest.mark.parametrize("T", [1, 6, 300])
@pytest.mark.parametrize("xdt", ["bf16", "fp32"])
def test_rows_outside_fp16_range(device, T, xdt):
    """Rows scaled by 1e5 (past fp16's largest value) and by 1e-6 (below its normal range), and
    a row mixing magnitudes 1e3..1e-3: fp32 outputs against the oracle on the same values."""
    from kandiga_amd.moe import QuantizedSwitchGLU, SparseMoeBlock

    shape = SHAPES["3bit"]
    layer, ex = _layer(device, shape, 9600 + T)
    rng = np.random.default_rng(9700 + T)
    x = rng.standard_normal((T, shape.hidden))
    scales = np.array([1e5, 1e-6, 1.0])[np.arange(T) % 3][:, None]
    x = x * scales
    if T >= 3:
        x[2] = x[2] * np.logspace(3, -3, shape.hidden)
    x = x.astype(np.float32)
    if xdt == "bf16":
        x = _bf16_values(x)
    _, lg = synth.make_inputs(shape, T, 9800 + T)
    xt = torch.from_numpy(x).to(device)
    xt = xt.bfloat16() if xdt == "bf16" else xt
    ld = torch.from_numpy(lg).to(device)
    out, idx, w = SparseMoeBlock(ex)(xt, ld, return_routing=True, out_dtype=torch.float32)
    ref_idx, ref_w = O.route(lg, shape.top_k)
    assert np.array_equal(to_np(idx), ref_idx)
    ref = dense_reference(host_layer(layer), shape, x, ref_idx, ref_w, exact_x=True)
    got = to_np(out)
    for t in range(T):   # each row on its own scale
        _rel_close(got[t], ref[t], f"{xdt} T={T} row {t} (scale {scales[t % 3, 0]:g})")
    # switch_mlp: fp16 y, as the reference's fp16 output; the 1e5 rows overflow it to inf there
    y = to_np(QuantizedSwitchGLU(ex)(xt, idx)).astype(np.float64)
    y_ref = O.switch_mlp(layer, x, ref_idx, shape.bits, exact_x=True).astype(np.float64)
    with np.errstate(over="ignore"):
        y_ref16 = y_ref.astype(np.float16).astype(np.float64)
    assert np.array_equal(np.isinf(y), np.isinf(y_ref16)) and np.array_equal(np.sign(y), np.sign(y_ref16))
    # each finite element within one fp16 ulp of the fp32 oracle, plus fp32 accumulation noise
    # of its (token, k) row's scale (elements far below the row's largest cancel)
    fin = np.isfinite(y_ref16)
    row_max = np.abs(y_ref).max(axis=-1, keepdims=True)   # the row's scale, overflowed elements included
    allowed = f16_ulp(y_ref) + 2e-5 * row_max
    err = np.where(fin, np.abs(y - y_ref), 0.0)
    print(f"  {xdt} switch_mlp T={T}: {int((~fin).sum())} overflowed, worst err/allowed "
          f"{float((err / allowed).max()):.2f}", flush=True)
    assert (err <= allowed).all()


def test_fp32_prefill_copy_matches_mlx_layout(device):
    """fp32 activations take 128-row tiles with both planes; the prefill copy gives the same
    bits as the MLX layout."""
    from kandiga_amd.moe import SparseMoeBlock

    shape = synth.LayerShape(512, 256, 32, 8, 3)
    layer, ex = _layer(device, shape, 9900)
    packed = ex.with_prefill_copy()
    rng = np.random.default_rng(9901)
    x = rng.standard_normal((300, shape.hidden)).astype(np.float32)
    _, lg = synth.make_inputs(shape, 300, 9902, zipf=True)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)
    a = SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32)
    b = SparseMoeBlock(packed)(xd, ld, out_dtype=torch.float32)
    assert torch.equal(a, b)
    idx, w = O.route(lg, shape.top_k)
    assert_close(to_np(a), dense_reference(host_layer(layer), shape, x, idx, w, exact_x=True),
                 what="fp32 x prefill copy")


def test_shared_expert_layer_refuses_bf16(device):
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(256, 128, 16, 4, 3, shared_intermediate=128)
    layer = synth.make_layer(shape, 9950)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    x, lg = synth.make_inputs(shape, 2, 9951)
    with pytest.raises(TypeError):
        SparseMoeBlock(ex)(torch.from_numpy(x).to(device).bfloat16(), torch.from_numpy(lg).to(device))
