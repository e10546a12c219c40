"""GPU parity of the HIP path (through the C ABI) against the oracle.

Bit-exact: dequantized codes, top-K indices, permutation order, histogram.
Tolerance (layer and switch_mlp outputs vs the fp32-accumulated oracle):
max |err| <= 2e-2 and relative L2 <= 1e-3.
"""
import numpy as np
import pytest
import torch

from kandiga_amd import synth
from kandiga_amd.layout import unpack_codes
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, dense_reference, host_layer, to_np, remap, torch_layer_subset

pytestmark = pytest.mark.gpu

SMALL = {
    "3bit": synth.LayerShape(256, 128, 16, 4, 3),
    "4bit": synth.LayerShape(256, 128, 16, 4, 4),
    "3bit-h320-i192": synth.LayerShape(320, 192, 12, 3, 3),
}


def _experts(shape, seed, device, scale_dtype="f16", activation="swiglu"):
    from kandiga_amd.moe import QuantizedExperts

    layer = synth.make_layer(shape, seed, scale_dtype)
    return layer, QuantizedExperts.from_stacked(shape, layer, device, scale_dtype, activation)


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("scale_dtype", ["f16", "bf16"])
def test_dequantize_bitexact(device, name, scale_dtype):
    shape = SMALL[name]
    layer, ex = _experts(shape, 11, device, scale_dtype)
    for proj, rows, in_dim in (("gate", shape.intermediate, shape.hidden), ("up", shape.intermediate, shape.hidden),
                               ("down", shape.hidden, shape.intermediate)):
        for e in (0, shape.num_experts - 1):
            codes, w16 = ex.dequantize(proj, e, 0, rows)
            ref_codes = O.unpack_codes(layer[f"{proj}_w"][e], shape.bits, in_dim)
            assert np.array_equal(to_np(codes), ref_codes), f"{proj} expert {e} codes differ"
            ref_w = O.dequantize(layer[f"{proj}_w"][e], layer[f"{proj}_s"][e], layer[f"{proj}_b"][e], shape.bits,
                                 in_dim, scale_dtype).astype(np.float16)
            assert np.array_equal(to_np(w16).view(np.uint16), ref_w.view(np.uint16)), f"{proj} expert {e} weights"


def _general_scale_bias(rng, shape, scale_dtype):
    """Independent random scales and biases of both signs, 2**-13 .. 2**3 in magnitude."""
    from kandiga_amd import layout

    mag = np.exp2(rng.uniform(-13, 3, size=shape)) * rng.choice([-1.0, 1.0], size=shape)
    if scale_dtype == "f16":
        return layout.f16_bits(mag.astype(np.float16))
    return layout.f32_to_bf16_bits(mag.astype(np.float32))


@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("scale_dtype", ["f16", "bf16"])
def test_dequantize_bitexact_general_scales(device, bits, scale_dtype):
    """round(q*s + b) to fp16, bit for bit, on scale/bias pairs that are not tied together
    (b != -2**(bits-1)*s): the rounding of the dequantized weight itself is checked, including
    results in the fp16 subnormal range."""
    from kandiga_amd.moe import QuantizedExperts

    shape = synth.LayerShape(256, 192, 3, 2, bits)
    layer = synth.make_layer(shape, 13 + bits, scale_dtype)
    rng = np.random.default_rng(17 + bits)
    for proj in ("gate", "up", "down"):
        layer[f"{proj}_s"] = _general_scale_bias(rng, layer[f"{proj}_s"].shape, scale_dtype)
        layer[f"{proj}_b"] = _general_scale_bias(rng, layer[f"{proj}_b"].shape, scale_dtype)
    # groups whose bias cancels q*s: b = -s gives exact zeros at q = 1; s = 2**-13 with
    # b = -(2**-10 - 2**-17) gives q = 8 -> 2**-17 and nearby codes in the fp16 subnormal range
    tiny = _general_scale_bias(rng, (2,), scale_dtype)
    tiny[0] = np.float16(2.0 ** -13).view(np.uint16) if scale_dtype == "f16" else 0x3900
    tiny[1] = np.float16(-(2.0 ** -10 - 2.0 ** -17)).view(np.uint16) if scale_dtype == "f16" else 0xBA7E
    for proj in ("gate", "up", "down"):
        layer[f"{proj}_b"][0, 0, :2] = layer[f"{proj}_s"][0, 0, :2] ^ 0x8000
        layer[f"{proj}_s"][0, 1, 0], layer[f"{proj}_b"][0, 1, 0] = tiny
    ex = QuantizedExperts.from_stacked(shape, layer, device, scale_dtype)
    n_sub = 0
    for proj, rows, in_dim in (("gate", shape.intermediate, shape.hidden), ("up", shape.intermediate, shape.hidden),
                               ("down", shape.hidden, shape.intermediate)):
        for e in range(shape.num_experts):
            _codes, w16 = ex.dequantize(proj, e, 0, rows)
            ref = O.dequantize(layer[f"{proj}_w"][e], layer[f"{proj}_s"][e], layer[f"{proj}_b"][e], bits, in_dim,
                               scale_dtype).astype(np.float16)
            got = to_np(w16)
            bad = np.nonzero(got.view(np.uint16) != ref.view(np.uint16))
            assert bad[0].size == 0, f"{proj} expert {e}: {bad[0].size} weights differ, first at {bad[0][0]},{bad[1][0]}"
            n_sub += int(((np.abs(ref) < 2 ** -14) & (ref != 0)).sum())
    print(f"  subnormal fp16 weights checked: {n_sub}")


@pytest.mark.parametrize("E,K,T", [(16, 4, 5), (256, 8, 1), (256, 8, 333), (256, 4, 8), (512, 10, 67),
                                   (64, 1, 3), (1000, 16, 9)])
def test_route_bitexact(device, E, K, T):
    from kandiga_amd.moe import route

    rng = np.random.default_rng(E * 31 + K * 7 + T)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    # ties: duplicated values, a row of equal logits, signed zeros, -inf
    if T > 2:
        logits[1, ::3] = logits[1, 0]
        logits[2, :] = 0.25
    logits[0, : min(E, 4)] = -np.inf
    logits[0, min(E, 4):min(E, 8)] = [-0.0, 0.0, -0.0, 0.0][: max(0, min(E, 8) - min(E, 4))]
    # NaN ranks below every number: some NaNs among normal logits, and a row of NaNs and -inf
    if T > 3:
        logits[3, ::5] = np.nan
    if T > 4:
        logits[4, :] = np.nan
        logits[4, E // 2] = -np.inf
    idx, w = route(torch.from_numpy(logits).to(device), K)
    ref_idx, ref_w = O.route(logits, K)
    assert np.array_equal(to_np(idx), ref_idx)
    np.testing.assert_allclose(to_np(w), ref_w, rtol=2e-6, atol=2e-7)


@pytest.mark.parametrize("T,K,E,zipf", [(1, 8, 256, False), (8, 8, 256, False), (512, 8, 256, True),
                                        (4096, 8, 256, True), (333, 10, 512, False), (2000, 4, 7, False),
                                        (1500, 16, 1024, True)])
def test_permute_bitexact(device, T, K, E, zipf):
    from kandiga_amd.moe import permute, route

    shape = synth.LayerShape(64, 64, E, K, 3)
    _x, logits = synth.make_inputs(shape, T, 5, zipf=zipf)
    ref_idx, _ = O.route(logits, K)
    got = permute(torch.from_numpy(ref_idx).to(device), E)
    ref = O.permute(ref_idx, E)
    assert np.array_equal(to_np(got["perm"]), ref["perm"])
    assert np.array_equal(to_np(got["counts"]), ref["counts"])
    assert np.array_equal(to_np(got["offsets"]), ref["offsets"])
    assert np.array_equal(to_np(got["unique"]), ref["unique"])


def test_permute_rejects_bad_index(device):
    from kandiga_amd import _capi
    from kandiga_amd.moe import permute

    idx = torch.tensor([[0, 3], [9, 1]], dtype=torch.int32, device=device)
    with pytest.raises(_capi.KmoeError):
        permute(idx, 4)


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("T", [1, 3, 8, 40, 300])
def test_switch_mlp_small(device, name, T):
    from kandiga_amd.moe import QuantizedSwitchGLU

    shape = SMALL[name]
    layer, ex = _experts(shape, 21, device)
    x, logits = synth.make_inputs(shape, T, 22)
    idx, _w = O.route(logits, shape.top_k)
    y = QuantizedSwitchGLU(ex)(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    assert ex.device_status() == 0
    ref = O.switch_mlp(layer, x, idx, shape.bits)
    assert_close(to_np(y), ref, what=f"{name} T={T} switch_mlp")


@pytest.mark.parametrize("K,T,pattern", [(4, 1, "same"), (4, 3, "same"), (4, 8, "same"), (4, 8, "random"),
                                          (4, 12, "same"), (16, 5, "random"), (16, 8, "same"), (16, 8, "random")])
def test_switch_mlp_repeated_experts(device, K, T, pattern):
    """Given indices may repeat an expert within a token (the reference computes every (t, k)
    independently, kandiga_cpu_expert.m:471-552): one expert's run then exceeds the token count.
    K=16 puts up to 128 assignments through the block-wide grouping of the decode path."""
    from kandiga_amd.moe import QuantizedSwitchGLU

    shape = synth.LayerShape(256, 128, 32, K, 3)
    layer, ex = _experts(shape, 23, device)
    x, _ = synth.make_inputs(shape, T, 24)
    rng = np.random.default_rng(25 + T)
    if pattern == "same":
        idx = np.full((T, K), 5, dtype=np.int32)
        idx[:, -1] = 7
    else:
        idx = rng.integers(0, 6, size=(T, K)).astype(np.int32)  # few experts, many repeats
    y = QuantizedSwitchGLU(ex)(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    assert ex.device_status() == 0
    ref = O.switch_mlp(layer, x, idx, shape.bits)
    assert_close(to_np(y), ref, what=f"K={K} T={T} {pattern} switch_mlp")


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("T", [1, 2, 5, 8, 9, 64, 700])
def test_forward_small(device, name, T):
    from kandiga_amd.moe import SparseMoeBlock

    shape = SMALL[name]
    layer, ex = _experts(shape, 31, device)
    x, logits = synth.make_inputs(shape, T, 32, zipf=T > 50)
    out, idx, w = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                                     return_routing=True)
    ref = O.moe_layer(layer, x, logits, shape.top_k, shape.bits)
    assert np.array_equal(to_np(idx), ref["idx"])
    np.testing.assert_allclose(to_np(w), ref["w"], rtol=2e-6, atol=2e-7)
    assert_close(to_np(out), ref["out"], what=f"{name} T={T} layer")
    out32 = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                               out_dtype=torch.float32)
    assert_close(to_np(out32), ref["out"], what=f"{name} T={T} layer fp32 out")


@pytest.mark.parametrize("layout", ["expert", "stacked"])
@pytest.mark.parametrize("T", [1, 8, 300])
def test_forward_both_weight_layouts(device, layout, T):
    """Expert-contiguous blocks (BKEX body) and one-tensor-per-part stacks give the same layer."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = SMALL["3bit-h320-i192"]
    layer = synth.make_layer(shape, 51)
    ex = QuantizedExperts.from_stacked(shape, layer, device, layout=layout)
    x, logits = synth.make_inputs(shape, T, 52 + T)
    out = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                             out_dtype=torch.float32)
    ref = O.moe_layer(layer, x, logits, shape.top_k, shape.bits)
    assert_close(to_np(out), ref["out"], what=f"{layout} T={T}")
    sub = ex.host_subset([3, 0, 11])
    for k, v in sub.items():
        assert np.array_equal(v, layer[k][[3, 0, 11]]), k


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("scale_dtype", ["f16", "bf16"])
def test_prefill_copy_matches_mlx_layout(device, name, scale_dtype):
    """The grouped GEMMs give bit-identical layers from the prefill copy and from the MLX
    tensors (even and odd group counts, both weight layouts); decode sizes are unaffected."""
    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU, SparseMoeBlock

    shape = SMALL[name]
    layer = synth.make_layer(shape, 61, scale_dtype)
    plain = QuantizedExperts.from_stacked(shape, layer, device, scale_dtype)
    for layout in ("expert", "stacked"):
        packed = QuantizedExperts.from_stacked(shape, layer, device, scale_dtype, layout=layout, prefill_copy=True)
        for T in (3, 9, 300):
            x, logits = synth.make_inputs(shape, T, 62 + T, zipf=T > 50)
            xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
            a = SparseMoeBlock(plain)(xd, ld, out_dtype=torch.float32)
            b = SparseMoeBlock(packed)(xd, ld, out_dtype=torch.float32)
            assert torch.equal(a, b), f"{name} {scale_dtype} {layout} T={T}"
            ref = O.moe_layer(layer, x, logits, shape.top_k, shape.bits, scale_dtype=scale_dtype)
            assert_close(to_np(b), ref["out"], what=f"{name} {scale_dtype} {layout} T={T} prefill copy")
            # the switch_mlp contract (per-assignment fp16 outputs) reads the copy too
            ix = torch.from_numpy(O.route(logits, shape.top_k)[0]).to(device)
            assert torch.equal(QuantizedSwitchGLU(plain)(xd, ix), QuantizedSwitchGLU(packed)(xd, ix))
        assert packed.device_status() == 0


TINY = {
    "h64-i64-e1-k1-3bit": synth.LayerShape(64, 64, 1, 1, 3),
    "h64-i128-e2-k2-4bit": synth.LayerShape(64, 128, 2, 2, 4),
    "h128-i64-e3-k2-3bit": synth.LayerShape(128, 64, 3, 2, 3),
}


@pytest.mark.parametrize("name", sorted(TINY))
def test_tiny_shapes(device, name):
    """Smallest legal layers: one quantization group per row (odd group counts, padded scale
    pairs), a single expert with top-1, decode and prefill sizes, with and without the copy."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = TINY[name]
    layer = synth.make_layer(shape, 71)
    plain = QuantizedExperts.from_stacked(shape, layer, device)
    packed = QuantizedExperts.from_stacked(shape, layer, device, prefill_copy=True)
    for T in (1, 5, 8, 9, 77, 300):
        x, logits = synth.make_inputs(shape, T, 72 + T)
        xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
        out, idx, _w = SparseMoeBlock(plain)(xd, ld, out_dtype=torch.float32, return_routing=True)
        ref = O.moe_layer(layer, x, logits, shape.top_k, shape.bits)
        assert np.array_equal(to_np(idx), ref["idx"]), f"{name} T={T} routing"
        assert_close(to_np(out), ref["out"], what=f"{name} T={T}")
        assert torch.equal(SparseMoeBlock(packed)(xd, ld, out_dtype=torch.float32), out), f"{name} T={T} copy"
    assert plain.device_status() == 0 and packed.device_status() == 0


@pytest.mark.parametrize("inter", [512, 1024])
def test_decode_stage2_unit_counts(device, inter):
    """Every decode batch (1..8 tokens) at top-K 1, 3, 10, 12 and 16: at intermediate 1024 the
    down stage gives its waves one to four units each (three included), so every exit of its
    two-stage unit loop runs.  Fused layer and switch_mlp outputs against the oracle."""
    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU, SparseMoeBlock

    base = synth.LayerShape(512, inter, 32, 16, 3)
    layer = synth.make_layer(base, 81)
    for K in (1, 3, 10, 12, 16):
        shape = base.with_top_k(K)
        ex = QuantizedExperts.from_stacked(shape, layer, device)
        for T in range(1, 9):
            x, logits = synth.make_inputs(shape, T, 82 + 10 * T + K)
            xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
            out, idx, _w = SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32, return_routing=True)
            ref = O.moe_layer(layer, x, logits, K, 3)
            assert np.array_equal(to_np(idx), ref["idx"]), f"I={inter} K={K} T={T} routing"
            assert_close(to_np(out), ref["out"], what=f"I={inter} K={K} T={T} layer")
            y = QuantizedSwitchGLU(ex)(xd, torch.from_numpy(ref["idx"]).to(device))
            assert_close(to_np(y), ref["y"], what=f"I={inter} K={K} T={T} switch_mlp")
        assert ex.device_status() == 0


def test_kernel_timing_covers_decode_and_prefill(device):
    from kandiga_amd.moe import SparseMoeBlock, profile_kernels

    shape = SMALL["3bit"]
    _layer, ex = _experts(shape, 61, device)
    blk = SparseMoeBlock(ex)
    ins = [tuple(torch.from_numpy(a).to(device) for a in synth.make_inputs(shape, T, 62 + T)) for T in (1, 300)]
    ref = [blk(*a) for a in ins]
    with profile_kernels(64) as prof:
        got = [blk(*a) for a in ins]
    for r, g in zip(ref, got):
        assert torch.equal(r, g)
    names = ("dec_stage1_kernel", "dec_stage2_kernel", "route_xpair_kernel", "permute_rank_kernel",
             "permute_scatter_kernel", "gemm_gateup_kernel", "gemm_down_kernel", "combine_kernel")
    for n in names:
        assert prof.result[n]["launches"] == 1, n
        assert 0 < prof.result[n]["mean_ms"] < 100, n


def test_forward_bf16_scales_gelu(device):
    from kandiga_amd.moe import SparseMoeBlock

    shape = synth.LayerShape(256, 128, 16, 4, 3)
    layer = synth.make_layer(shape, 41, "bf16")
    from kandiga_amd.moe import QuantizedExperts

    ex = QuantizedExperts.from_stacked(shape, layer, device, "bf16", "gelu_tanh")
    for T in (2, 100):
        x, logits = synth.make_inputs(shape, T, 42 + T)
        out = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device))
        idx, w = O.route(logits, shape.top_k)
        y = O.switch_mlp(layer, x, idx, 3, "bf16", act="gelu")
        assert_close(to_np(out), O.combine(y, w), what=f"bf16 gelu T={T}")


def test_combine_matches_closed_form(device):
    from kandiga_amd.moe import combine

    rng = np.random.default_rng(3)
    y = (rng.standard_normal((37, 6, 192)) * 3).astype(np.float16)
    w = rng.random((37, 6)).astype(np.float32)
    out = combine(torch.from_numpy(y).to(device), torch.from_numpy(w).to(device))
    ref = O.combine(y.astype(np.float32), w)
    assert_close(to_np(out), ref, what="combine")


# ---- benchmark-sized layers -------------------------------------------------------------
@pytest.mark.parametrize("name", ["h256_e16_i128_k4_3bit", "h256_e16_i128_k4_4bit", "h320_e12_i192_k3_3bit"])
def test_stored_golden_fixture(device, name):
    """The stored fixture (tests/golden/moe_small.npz): its inputs through the HIP path give its
    stored routing bit for bit, its stored per-(token, k) expert outputs and its combined output
    (layers regenerated from the seed, checked against the stored SHA-256)."""
    import os

    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU, SparseMoeBlock
    from tests.golden.make_golden import CASES, layer_sha256

    data = np.load(os.path.join(os.path.dirname(__file__), "golden", "moe_small.npz"))
    shape, seed, _tokens = CASES[name]
    layer = synth.make_layer(shape, seed)
    assert layer_sha256(layer) == str(data[f"{name}.layer_sha256"])
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    x = torch.from_numpy(data[f"{name}.x"]).to(device)
    lg = torch.from_numpy(data[f"{name}.logits"]).to(device)
    out, idx, w = SparseMoeBlock(ex)(x, lg, return_routing=True)
    assert np.array_equal(to_np(idx), data[f"{name}.idx"])
    np.testing.assert_allclose(to_np(w), data[f"{name}.w"], rtol=2e-6, atol=2e-7)
    y = QuantizedSwitchGLU(ex)(x, idx)
    assert_close(to_np(y), data[f"{name}.y"], what=f"{name} stored y")
    assert_close(to_np(out), data[f"{name}.out"], what=f"{name} stored out")


@pytest.fixture(scope="module")
def full3(device):
    shape = synth.SHAPES["h2048-e256-i512-k8-3bit"]
    layer, ex = _experts(shape, 1001, device)
    return shape, layer, ex


@pytest.mark.parametrize("T", [1, 4, 8])
def test_decode_full_3bit(device, full3, T):
    from kandiga_amd.moe import SparseMoeBlock

    shape, layer, ex = full3
    x, logits = synth.make_inputs(shape, T, 2000 + T)
    out, idx, w = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                                     return_routing=True)
    ref = O.moe_layer(layer, x, logits, shape.top_k, 3, nthreads=8)
    assert np.array_equal(to_np(idx), ref["idx"])
    assert_close(to_np(out), ref["out"], what=f"h2048 3bit decode T={T}")


def test_decode_full_3bit_fast_mode(device, full3):
    """K=4 'fast mode' (engine.py:1132-1147): the same experts, top-4 renormalised."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape, layer, _ex = full3
    s4 = shape.with_top_k(4)
    ex4 = QuantizedExperts.from_stacked(s4, layer, device)
    for T in (1, 8):
        x, logits = synth.make_inputs(s4, T, 2100 + T)
        out = SparseMoeBlock(ex4)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device))
        ref = O.moe_layer(layer, x, logits, 4, 3, nthreads=8)
        assert_close(to_np(out), ref["out"], what=f"h2048 3bit K=4 T={T}")


@pytest.mark.parametrize("T", [512, 2048, 4096])
def test_prefill_full_3bit_zipf(device, full3, T):
    """Every row of the 512/2048/4096-token Zipf-routed prefill against the oracle's dense
    per-expert products (float64), plus sampled rows through the C restatement."""
    from kandiga_amd.moe import SparseMoeBlock

    shape, layer, ex = full3
    x, logits = synth.make_inputs(shape, T, 3000 + T, zipf=True)
    out, idx, w = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                                     return_routing=True, out_dtype=torch.float32)
    ref_idx, ref_w = O.route(logits, shape.top_k)
    assert np.array_equal(to_np(idx), ref_idx)
    assert_close(to_np(out), dense_reference(layer, shape, x, ref_idx, ref_w), what=f"h2048 3bit prefill T={T} all rows")
    rows = np.random.default_rng(T).choice(T, 16, replace=False)
    y = O.switch_mlp(layer, x[rows], ref_idx[rows], 3, nthreads=8)
    assert_close(to_np(out)[rows], O.combine(y, ref_w[rows]), what=f"h2048 3bit prefill T={T} C-oracle rows")


@pytest.mark.parametrize("bits", [3, 4])
def test_prefill_copy_full_size(device, full3, bits):
    """4096-token prefill from the prefill copy equals the MLX-layout result bit for bit."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    if bits == 3:
        shape, layer, plain = full3
    else:
        shape = synth.SHAPES["h2048-e256-i512-k8-4bit"]
        layer = synth.make_layer(shape, 1002)
        plain = QuantizedExperts.from_stacked(shape, layer, device)
    packed = QuantizedExperts.from_stacked(shape, layer, device, prefill_copy=True)
    x, logits = synth.make_inputs(shape, 4096, 3100 + bits, zipf=True)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
    assert torch.equal(SparseMoeBlock(plain)(xd, ld), SparseMoeBlock(packed)(xd, ld))
    assert packed.device_status() == 0


def test_decode_full_4bit(device):
    from kandiga_amd.moe import SparseMoeBlock

    shape = synth.SHAPES["h2048-e256-i512-k8-4bit"]
    layer, ex = _experts(shape, 1002, device)
    for T in (1, 8, 64):
        x, logits = synth.make_inputs(shape, T, 2200 + T)
        xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
        out = SparseMoeBlock(ex)(xd, ld)
        out32 = SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32)
        ref = O.moe_layer(layer, x, logits, 8, 4, nthreads=8)
        assert_close(to_np(out), ref["out"], what=f"h2048 4bit T={T}")
        assert_close(to_np(out32), ref["out"], what=f"h2048 4bit T={T} fp32 out")


@pytest.mark.parametrize("T", [512, 2048])
def test_prefill_full_4bit_zipf(device, T):
    """Every row of a Zipf-routed 4-bit prefill (activations reach ~240 and outputs ~125 in
    magnitude) against the oracle's dense per-expert products, fp32 and fp16 outputs."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.SHAPES["h2048-e256-i512-k8-4bit"]
    layer = synth.make_layer(shape, 1002)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    x, logits = synth.make_inputs(shape, T, 3000 + T, zipf=True)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
    idx, w = O.route(logits, 8)
    ref = dense_reference(layer, shape, x, idx, w)
    assert_close(to_np(SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32)), ref, what=f"h2048 4bit prefill T={T}")
    assert_close(to_np(SparseMoeBlock(ex)(xd, ld)), ref, what=f"h2048 4bit prefill T={T} fp16 out")


def test_wide_layer_h4096_e512_k10(device):
    """H=4096, E=512, I=1024, K=10 generated on the device; every row against the oracle (dense
    per-expert products, float32 for the 1 TFLOP of the 4096-token batch: relative error near
    1e-6), up to the 4096-token prefill (also from the prefill copy, bit for bit)."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.SHAPES["h4096-e512-i1024-k10-3bit"]
    layer_t = synth.make_layer_torch(shape, 5001, device)
    ex = QuantizedExperts.from_stacked(shape, layer_t, device)
    packed = ex.with_prefill_copy()
    layer_h = host_layer(layer_t)
    for T, zipf in ((1, False), (8, False), (300, True), (4096, True)):
        x, logits = synth.make_inputs(shape, T, 5100 + T, zipf=zipf)
        xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
        out = SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32)
        if T > 8:
            assert torch.equal(SparseMoeBlock(packed)(xd, ld, out_dtype=torch.float32), out), f"prefill copy T={T}"
        idx, w = O.route(logits, shape.top_k)
        ref = dense_reference(layer_h, shape, x, idx, w, dtype=np.float32 if T > 1000 else np.float64)
        assert_close(to_np(out), ref, what=f"h4096 e512 T={T} all rows")
        if T <= 8:
            uniq, pos = remap(idx)
            y = O.switch_mlp(torch_layer_subset(layer_t, uniq), x, pos, 3, nthreads=8)
            assert_close(to_np(out), O.combine(y, w), what=f"h4096 e512 T={T} C oracle")


@pytest.mark.parametrize("T", [1, 3, 8, 9, 200])
def test_forward_with_shared_expert_small(device, T):
    """Dense fp16 shared expert added after the routed combine (decode GEMVs and prefill GEMMs)."""
    from kandiga_amd.moe import SparseMoeBlock

    shape = synth.LayerShape(256, 128, 16, 4, 3, shared_intermediate=192)
    layer, ex = _experts(shape, 71, device)
    x, logits = synth.make_inputs(shape, T, 72 + T, zipf=T > 50)
    ref = O.moe_layer(layer, x, logits, shape.top_k, shape.bits)
    blk = SparseMoeBlock(ex)
    xt, lt = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
    out32 = to_np(blk(xt, lt, out_dtype=torch.float32))
    assert_close(out32, ref["out"], what=f"shared T={T} fp32 out")
    assert_close(to_np(blk(xt, lt)), ref["out"], what=f"shared T={T}")
    # the shared term itself: layer output minus the oracle's routed part
    routed = O.combine(O.switch_mlp(layer, x, ref["idx"], 3), ref["w"]).astype(np.float64)
    shared = O.shared_expert_f64(layer, x)
    assert np.abs(shared).max() > 1e-2
    np.testing.assert_allclose(out32 - routed, shared, rtol=0, atol=1e-3)


def test_hidden2560_layer_with_shared_expert(device):
    """H=2560, E=256, I=1024, K=8, 3-bit + fp16 shared expert I=1024: every row against the
    oracle (dense per-expert products + the shared expert, float64)."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.SHAPES["h2560-e256-i1024-k8-3bit-shared1024"]
    layer_t = synth.make_layer_torch(shape, 6001, device)
    ex = QuantizedExperts.from_stacked(shape, layer_t, device)
    layer_h = host_layer(layer_t)
    for T, zipf in ((1, False), (8, False), (2048, True)):
        x, logits = synth.make_inputs(shape, T, 6100 + T, zipf=zipf)
        out = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                                 out_dtype=torch.float32)
        idx, w = O.route(logits, shape.top_k)
        assert_close(to_np(out), dense_reference(layer_h, shape, x, idx, w), what=f"h2560 shared T={T} all rows")


def test_decode_graph_replays_match_eager(device):
    """Several replays of a captured stack of decode layers, with eager work between them
    (including a larger call that grows the workspaces), each bit-identical to the eager
    result."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(512, 256, 32, 8, 3)
    blocks, ins = [], []
    for i in range(3):
        layer = synth.make_layer(shape, 600 + i)
        ex = QuantizedExperts.from_stacked(shape, layer, device)
        ex.reserve(4)
        blocks.append(SparseMoeBlock(ex))
        x, lg = synth.make_inputs(shape, 1 + i, 700 + i)
        ins.append((torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)))
    eager = [b(*a).clone() for b, a in zip(blocks, ins)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for b, a in zip(blocks, ins):
            b(*a)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    outs = [None] * 3
    with torch.cuda.graph(g):
        for i, (b, a) in enumerate(zip(blocks, ins)):
            outs[i] = b(*a)
    big = [tuple(torch.from_numpy(a).to(device) for a in synth.make_inputs(shape, 64, 750 + i)) for i in range(3)]
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for i in range(3):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} layer {i}"
        _ = [b(*a) for b, a in zip(blocks, ins)]   # eager work between replays
        if rep == 1:
            # a larger eager call grows the workspace; the captured graph keeps its own
            _ = [b(*a) for b, a in zip(blocks, big)]
        torch.cuda.synchronize()
    for b in blocks:
        assert b.experts.device_status() == 0


def test_decode_repeated_calls_deterministic(device, full3):
    from kandiga_amd.moe import SparseMoeBlock

    shape, layer, ex = full3
    x, logits = synth.make_inputs(shape, 3, 4242)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
    blk = SparseMoeBlock(ex)
    first = blk(xd, ld).clone()
    for _ in range(20):
        assert torch.equal(blk(xd, ld), first)
    assert ex.device_status() == 0


def test_prefill_graph_replays_match_eager(device):
    """A captured sequence of prefill calls (route, permute, grouped GEMMs, combine) and a decode
    call on one layer, replayed several times with eager work between replays: every replay is
    bit-identical to the eager result (the kernels rewrite all the workspace they read)."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(512, 256, 32, 8, 3)
    layer = synth.make_layer(shape, 810)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    ex.reserve(300)
    blk = SparseMoeBlock(ex)
    ins = []
    for T in (300, 8, 97):
        x, lg = synth.make_inputs(shape, T, 820 + T, zipf=T > 8)
        ins.append((torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)))
    eager = [blk(*a).clone() for a in ins]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for a in ins:
            blk(*a)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    outs = [None] * len(ins)
    with torch.cuda.graph(g):
        for i, a in enumerate(ins):
            outs[i] = blk(*a)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for i in range(len(ins)):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} call {i}"
        _ = [blk(*a) for a in reversed(ins)]  # eager work between replays
        torch.cuda.synchronize()
    assert ex.device_status() == 0


def test_prefill_repeated_calls_deterministic(device, full3):
    """The grouped-GEMM path has no atomics and a fixed combine order: repeated calls are
    bit-identical."""
    from kandiga_amd.moe import SparseMoeBlock

    shape, layer, ex = full3
    x, logits = synth.make_inputs(shape, 600, 4343, zipf=True)
    xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
    blk = SparseMoeBlock(ex)
    first = blk(xd, ld).clone()
    for _ in range(5):
        assert torch.equal(blk(xd, ld), first)
    assert ex.device_status() == 0

