"""GPU parity of the TQ3 codebook kernels (kmoe_tq3_gemv, kmoe_tq3_expert_mlp) against the
float64 oracle (oracle/tq3_oracle.py: dequantize the blocks, then a dense product).

The GEMV output is fp32: the bar is 2e-6 of sum|W||x| per element (fp32 accumulation of at most
4096 products and the transform of the input, in a different order than the oracle's).  The
expert MLP output is fp16 (gate/up and the activation stay fp32 in between): half an fp16 ulp
plus 2e-3, as for the routed layer."""
import os

import numpy as np
import pytest
import torch

from kandiga_amd import tq3
from oracle import tq3_oracle as Q
from tests.gpu_helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


def _gemv_case(device, rows, cols, T, seed, x_f32):
    rng = np.random.default_rng(seed)
    blocks = tq3.random_blocks(rows * cols // 32, rng)
    x = rng.standard_normal((T, cols)).astype(np.float32 if x_f32 else np.float16)
    got = to_np(tq3.gemv(torch.from_numpy(blocks).to(device), rows, cols, torch.from_numpy(x).to(device)))
    W = Q.dequantize_matrix(blocks, rows, cols)
    ref = x.astype(np.float64) @ W.T
    bound = 2e-6 * (np.abs(x.astype(np.float64)) @ np.abs(W).T) + 1e-30
    excess = np.abs(got - ref) - bound
    print(f"  gemv rows={rows} cols={cols} T={T} f32={x_f32}: max|err|={np.abs(got - ref).max():.3e}", flush=True)
    assert excess.max() <= 0, f"worst excess {excess.max():.3e}"


@pytest.mark.parametrize("rows,cols,T", [(64, 32, 1), (96, 256, 3), (512, 2048, 1), (1024, 512, 4),
                                         (33, 4096, 2), (2048, 3072, 1)])
def test_tq3_gemv_fp16_input(device, rows, cols, T):
    _gemv_case(device, rows, cols, T, rows + cols + T, False)


@pytest.mark.parametrize("rows,cols,T", [(128, 1024, 1), (100, 96, 5)])
def test_tq3_gemv_fp32_input(device, rows, cols, T):
    _gemv_case(device, rows, cols, T, 7 + rows, True)


def test_tq3_gemv_quantized_weights_match_dense(device):
    """Blocks from the library's quantizer of a dense matrix: the GEMV is the product with the
    dequantized matrix, and close to the dense one (quantization error only)."""
    rng = np.random.default_rng(5)
    Wd = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    blocks = tq3.quantize(Wd)
    x = rng.standard_normal((2, 512)).astype(np.float16)
    got = to_np(tq3.gemv(torch.from_numpy(blocks).to(device), 256, 512, torch.from_numpy(x).to(device)))
    ref = Q.gemv_f64(blocks, 256, 512, x)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5 * float(np.abs(ref).max()))
    dense = x.astype(np.float64) @ Wd.T.astype(np.float64)
    assert np.linalg.norm(got - dense) / np.linalg.norm(dense) < 0.25


def _experts(E, H, I, seed):
    rng = np.random.default_rng(seed)
    return np.stack([tq3.random_blocks(3 * H * I // 32, rng, scale=0.05).reshape(-1) for _ in range(E)])


@pytest.mark.parametrize("E,H,I,T,K", [(8, 256, 128, 1, 2), (16, 512, 256, 3, 4), (32, 2048, 512, 1, 8),
                                       (4, 1024, 1536, 2, 2)])
def test_tq3_expert_mlp(device, E, H, I, T, K):
    body = _experts(E, H, I, E + H + I)
    rng = np.random.default_rng(T * 31 + K)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ex = tq3.TQ3Experts(body, H, I, device)
    y = to_np(ex(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)))
    ref = np.stack([np.stack([Q.expert_mlp_f64(body[idx[t, k]], H, I, x[t])[0] for k in range(K)])
                    for t in range(T)])
    assert_close(y, ref, what=f"tq3 mlp E={E} H={H} I={I} T={T} K={K}")


def test_tq3_expert_mlp_invalid_expert_rows_are_zero(device):
    E, H, I = 4, 256, 128
    body = _experts(E, H, I, 3)
    x = np.random.default_rng(4).standard_normal((2, H)).astype(np.float16)
    idx = np.array([[1, -1], [E, 2]], dtype=np.int32)
    y = to_np(tq3.TQ3Experts(body, H, I, device)(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)))
    assert not y[0, 1].any() and not y[1, 0].any()
    assert_close(y[0, 0], Q.expert_mlp_f64(body[1], H, I, x[0])[0], what="valid row 0")
    assert_close(y[1, 1], Q.expert_mlp_f64(body[2], H, I, x[1])[0], what="valid row 1")


def test_tq3_experts_from_file(device, tmp_path):
    """A TQ3X file of experts converted from dense weights by the library's quantizer."""
    E, H, I = 3, 256, 128
    rng = np.random.default_rng(9)
    dense = [tuple((rng.standard_normal(s) * 0.03).astype(np.float32) for s in ((I, H), (I, H), (H, I)))
             for _ in range(E)]
    body = tq3.convert_layer(dense, H, I)
    path = os.path.join(tmp_path, "layer_000.tq3x")
    tq3.write_tq3x(path, body, H, I)
    ex = tq3.TQ3Experts.from_file(path, device)
    x = (rng.standard_normal((2, H)) * 0.5).astype(np.float16)
    idx = np.array([[0, 2], [1, 0]], dtype=np.int32)
    y = to_np(ex(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)))
    for t in range(2):
        for k in range(2):
            assert_close(y[t, k], Q.expert_mlp_f64(body[idx[t, k]], H, I, x[t])[0], what=f"file t={t} k={k}")


def test_tq3_empty_and_bad_shapes(device):
    from kandiga_amd import _capi

    blocks = torch.zeros((64 * 32 // 32, 20), dtype=torch.uint8, device=device)
    out = tq3.gemv(blocks, 64, 32, torch.zeros((0, 32), dtype=torch.float16, device=device))
    assert out.shape == (0, 64)
    with pytest.raises(_capi.KmoeError):
        tq3.gemv(blocks, 64, 48, torch.zeros((1, 48), dtype=torch.float16, device=device))
