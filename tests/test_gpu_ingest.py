"""GPU checks of the weight ingestion paths and of the boundary's error behaviour.

BKEX files (kandiga/_pack_experts.py:95-182, scripts/repack_experts_3bit.py:145-166 write them
with bf16 scales) and MLX safetensors checkpoints (stacked switch_mlp tensors,
kandiga/_split_experts.py:62-117) loaded into HBM and run against the oracle; bad expert
indices on the grouped-GEMM path; host tensors refused before any launch.
"""
import numpy as np
import pytest
import torch

from kandiga_amd import layout, synth
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [3, 4])
def test_bkex_file_to_hbm(device, tmp_path, bits):
    """write_bkex (bf16 scales, the dtype the reference's packer stores) -> from_bkex -> layer
    outputs against the oracle at decode and prefill sizes."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(512, 256, 24, 4, bits)
    layer = synth.make_layer(shape, 90 + bits, "bf16")
    path = str(tmp_path / "layer_00.bin")
    layout.write_bkex(path, layer, layout.ExpertGeometry(512, 256, bits), "bf16")
    ex = QuantizedExperts.from_bkex(path, top_k=4, device=device)
    assert ex.scale_dtype == "bf16" and ex.shape.bits == bits and ex.shape.num_experts == 24
    blk = SparseMoeBlock(ex)
    for T in (1, 8, 100):
        x, logits = synth.make_inputs(shape, T, 95 + T, zipf=T > 8)
        out, idx, _w = blk(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                           out_dtype=torch.float32, return_routing=True)
        ref = O.moe_layer(layer, x, logits, 4, bits, scale_dtype="bf16")
        assert np.array_equal(to_np(idx), ref["idx"])
        assert_close(to_np(out), ref["out"], what=f"bkex {bits}-bit T={T}")
    assert ex.device_status() == 0


@pytest.mark.parametrize("bits,shards", [(3, 1), (4, 2)])
def test_safetensors_checkpoint_to_hbm(device, tmp_path, bits, shards):
    """Stacked switch_mlp tensors of an MLX checkpoint (sharded, bf16 scales) -> from_safetensors
    -> switch_mlp and layer outputs against the oracle."""
    from kandiga_amd import weights
    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU, SparseMoeBlock

    shape = synth.LayerShape(256, 192, 16, 4, bits)
    layer = synth.make_layer(shape, 110 + bits, "bf16")
    d = tmp_path / "ckpt"
    d.mkdir()
    weights.write_switch_mlp(str(d), layer, 3, "bf16", shards=shards)
    ex = QuantizedExperts.from_safetensors(str(d), 3, top_k=4, device=device)
    for T in (2, 50):
        x, logits = synth.make_inputs(shape, T, 120 + T)
        xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device)
        ref = O.moe_layer(layer, x, logits, 4, bits, scale_dtype="bf16")
        assert_close(to_np(SparseMoeBlock(ex)(xd, ld, out_dtype=torch.float32)), ref["out"], what=f"st T={T}")
        y = QuantizedSwitchGLU(ex)(xd, torch.from_numpy(ref["idx"]).to(device))
        assert_close(to_np(y), ref["y"], what=f"st switch_mlp T={T}")


@pytest.mark.parametrize("T", [5, 40])
def test_switch_mlp_bad_index_rows_are_zero(device, T):
    """An expert index outside [0, E) gives a zero row and the device flag on both paths (the
    decode GEMVs at T <= 8 and the grouped GEMMs above); the other rows are unaffected."""
    from kandiga_amd import _capi
    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU

    shape = synth.LayerShape(256, 128, 16, 4, 3)
    layer = synth.make_layer(shape, 130)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    x, logits = synth.make_inputs(shape, T, 131)
    idx, _ = O.route(logits, 4)
    bad = idx.copy()
    bad[1, 2] = 16
    bad[T - 1, 0] = -3
    y = to_np(QuantizedSwitchGLU(ex)(torch.from_numpy(x).to(device), torch.from_numpy(bad).to(device)))
    assert ex.device_status() & _capi.DEVERR_BAD_EXPERT
    assert not y[1, 2].any() and not y[T - 1, 0].any()
    ref = O.switch_mlp(layer, x, idx, 3)
    keep = np.ones(idx.shape, bool)
    keep[1, 2] = keep[T - 1, 0] = False
    assert_close(y[keep], ref[keep], what=f"bad-index T={T} other rows")
    assert ex.device_status() == 0   # read-and-clear


@pytest.mark.parametrize("T", [3, 300])
def test_forward_1024_experts_top16(device, T):
    """The largest expert count (1024) and top-K (16): routing, permutation and the layer."""
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(256, 128, 1024, 16, 3)
    layer = synth.make_layer(shape, 140)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    x, logits = synth.make_inputs(shape, T, 141 + T, zipf=T > 8)
    out, idx, w = SparseMoeBlock(ex)(torch.from_numpy(x).to(device), torch.from_numpy(logits).to(device),
                                     out_dtype=torch.float32, return_routing=True)
    ref = O.moe_layer(layer, x, logits, 16, 3, nthreads=8)
    assert np.array_equal(to_np(idx), ref["idx"])
    np.testing.assert_allclose(to_np(w), ref["w"], rtol=2e-6, atol=2e-7)
    assert_close(to_np(out), ref["out"], what=f"E=1024 K=16 T={T}")
    assert ex.device_status() == 0


def test_host_tensors_rejected(device):
    """CPU tensors handed to a layer on the GPU raise ValueError before anything is launched."""
    from kandiga_amd.moe import QuantizedExperts, QuantizedSwitchGLU, SparseMoeBlock

    shape = synth.LayerShape(128, 64, 8, 2, 3)
    ex = QuantizedExperts.from_stacked(shape, synth.make_layer(shape, 150), device)
    x, logits = synth.make_inputs(shape, 2, 151)
    xc, lc = torch.from_numpy(x), torch.from_numpy(logits)
    with pytest.raises(ValueError):
        SparseMoeBlock(ex)(xc, lc.to(device))
    with pytest.raises(ValueError):
        SparseMoeBlock(ex)(xc.to(device), lc)
    with pytest.raises(ValueError):
        QuantizedSwitchGLU(ex)(xc.to(device), torch.zeros(2, 2, dtype=torch.int32))
    torch.cuda.synchronize()
    assert ex.device_status() == 0
