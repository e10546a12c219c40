"""kmoe_forward_noalloc (the routed layer on the library's static scratch) against kmoe_forward
(the same layer on a caller workspace), through the C ABI: bit-identical outputs and routing on
consecutive calls, each later call smaller than the one before, on both the decode and the
grouped-GEMM paths; a call too large for the scratch is refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from kandiga_amd import _capi, synth
from oracle import moe_oracle as O
from tests.gpu_helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


def _noalloc(ex, x, lg, out_dtype=torch.float16):
    T = x.shape[0]
    out = torch.empty((T, ex.shape.hidden), dtype=out_dtype, device=x.device)
    idx = torch.empty((T, ex.shape.top_k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, ex.shape.top_k), dtype=torch.float32, device=x.device)
    odt = _capi.OUT_F32 if out_dtype == torch.float32 else _capi.OUT_F16
    rc = _capi.lib().kmoe_forward_noalloc(ex._handle, x.data_ptr(), lg.data_ptr(), T, out.data_ptr(), odt,
                                          idx.data_ptr(), w.data_ptr(), torch.cuda.current_stream().cuda_stream)
    _capi.check(rc, "kmoe_forward_noalloc")
    return out, idx, w


def test_noalloc_matches_workspace_entry(device):
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    shape = synth.LayerShape(512, 256, 32, 8, 3)
    layer = synth.make_layer(shape, 910)
    ex = QuantizedExperts.from_stacked(shape, layer, device)
    blk = SparseMoeBlock(ex)
    for T in (200, 37, 8, 3, 1):   # each call smaller than the one before; grouped GEMM, then decode
        x, lg = synth.make_inputs(shape, T, 920 + T, zipf=T > 8)
        xd, ld = torch.from_numpy(x).to(device), torch.from_numpy(lg).to(device)
        ref_out, ref_idx, ref_w = blk(xd, ld, return_routing=True)
        for odt in (torch.float16, torch.float32):
            out, idx, w = _noalloc(ex, xd, ld, odt)
            torch.cuda.synchronize()
            assert torch.equal(idx, ref_idx) and torch.equal(w, ref_w), f"T={T} routing"
            if odt == torch.float16:
                assert torch.equal(out, ref_out), f"T={T} fp16 output"
            assert_close(to_np(out), O.moe_layer(layer, x, lg, 8, 3)["out"], what=f"noalloc T={T}")


def test_noalloc_rejects_calls_beyond_the_scratch(device):
    from kandiga_amd.moe import QuantizedExperts

    shape = synth.LayerShape(2048, 512, 16, 8, 3)
    ex = QuantizedExperts.from_stacked(shape, synth.make_layer(shape, 930), device)
    need = ex.workspace_bytes(4096)
    assert need > _capi.NOALLOC_SCRATCH_BYTES
    T = 4096
    x = torch.zeros((T, 2048), dtype=torch.float16, device=device)
    lg = torch.zeros((T, 16), dtype=torch.float32, device=device)
    out = torch.empty((T, 2048), dtype=torch.float16, device=device)
    rc = _capi.lib().kmoe_forward_noalloc(ex._handle, x.data_ptr(), lg.data_ptr(), T, out.data_ptr(),
                                          _capi.OUT_F16, None, None, torch.cuda.current_stream().cuda_stream)
    assert rc == _capi.ERR_WORKSPACE
    assert b"static scratch" in _capi.lib().kmoe_last_error()
