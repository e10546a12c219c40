"""TQ3 format checks on the CPU: the oracle's transform and dequantization against closed forms
and the reference quantizer's own vectors (tests/golden/tq3_quantize.npz, written by
tests/golden/make_tq3_golden.py), and the library's quantizer, packing and TQ3X file."""
import os

import numpy as np
import pytest

from kandiga_amd import tq3
from oracle import tq3_oracle as Q

GOLD = os.path.join(os.path.dirname(__file__), "golden", "tq3_quantize.npz")


def test_sign_table_is_the_golden_ratio_hash():
    """sign[i] = -1 where bit 31 of (i * 0x9E3779B9 mod 2^32) is set (quantize.py:39)."""
    want = np.array([-1.0 if ((i * 0x9E3779B9) & 0xFFFFFFFF) >> 31 else 1.0 for i in range(32)])
    assert np.array_equal(Q.SIGNS, want) and np.array_equal(tq3.SIGNS, want)


def test_tables_agree_and_boundaries_are_midpoints():
    assert np.array_equal(Q.CENTROIDS, tq3.CENTROIDS) and np.array_equal(Q.BOUNDARIES, tq3.BOUNDARIES)
    assert (np.diff(Q.CENTROIDS) > 0).all()
    np.testing.assert_allclose(Q.BOUNDARIES, (Q.CENTROIDS[1:] + Q.CENTROIDS[:-1]) / 2, atol=2e-6)


def test_hadamard_closed_forms():
    """H H = 32 I; H e0 = all ones; inverse(forward(x)) = x; the dot identity w.x = r.WHT(x)."""
    eye = np.eye(32)
    Hm = Q.hadamard_butterfly(eye)
    np.testing.assert_allclose(Hm @ Hm, 32 * eye, atol=1e-12)
    assert np.array_equal(Hm[0], np.ones(32)) and set(np.unique(Hm)) == {-1.0, 1.0}
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 32))
    np.testing.assert_allclose(Q.wht_inverse(Q.wht_forward(x)), x, atol=1e-12)
    r = rng.standard_normal((5, 32))
    np.testing.assert_allclose((Q.wht_inverse(r) * x).sum(1), (r * Q.wht_forward(x)).sum(1), atol=1e-12)


def test_dequantize_constant_block_closed_form():
    """All indices c with d = 1, m = 0 in both halves: the rotated block is C[c] everywhere, and
    its inverse transform is sqrt(32) * C[c] at element 0 and zero elsewhere."""
    for c in range(8):
        blk = np.zeros((1, 20), np.uint8)
        blk[0, :8] = np.array([1.0, 1.0, 0.0, 0.0], np.float16).view(np.uint8)
        blk[0, 8:] = tq3.pack_indices(np.full((1, 32), c))
        w = Q.dequantize_blocks(blk)[0]
        want = np.zeros(32)
        want[0] = np.sqrt(32.0) * float(Q.CENTROIDS[c])
        np.testing.assert_allclose(w, want, atol=1e-6)
    # a mean alone behaves the same way, half by half
    blk = np.zeros((1, 20), np.uint8)
    blk[0, :8] = np.array([0.0, 0.0, 0.5, 0.0], np.float16).view(np.uint8)
    w = Q.dequantize_blocks(blk)[0]
    np.testing.assert_allclose(w, Q.wht_inverse(np.r_[np.full(16, 0.5), np.zeros(16)]), atol=1e-12)


def test_index_packing_matches_the_unpacker():
    rng = np.random.default_rng(2)
    idx = rng.integers(0, 8, size=(7, 32))
    assert np.array_equal(Q.unpack_indices(tq3.pack_indices(idx)), idx)
    # known bytes: indices 0..7 in a group -> 0xFAC688 little-endian (the MLX 3-bit order)
    assert tq3.pack_indices(np.tile(np.arange(8), 4)[None])[0, :3].tobytes() == bytes([0x88, 0xC6, 0xFA])


def test_quantizer_matches_reference_vectors():
    """The library's quantizer writes the reference's bytes; the oracle reads its weights back."""
    g = np.load(GOLD)
    for name in ("a", "b", "c", "d"):
        w = g[f"{name}.input"]
        blocks = tq3.quantize(w)
        assert np.array_equal(blocks, g[f"{name}.blocks"]), name
        deq = Q.dequantize_blocks(g[f"{name}.blocks"]).reshape(-1)[: w.size]
        np.testing.assert_allclose(deq, g[f"{name}.dequant"].reshape(-1), rtol=1e-5, atol=1e-6)


def test_quantizer_error_is_small():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    deq = Q.dequantize_blocks(tq3.quantize(w)).reshape(64, 256)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < 0.2, rel


def test_tq3x_file_roundtrip(tmp_path):
    rng = np.random.default_rng(4)
    H, I, E = 128, 64, 3
    body = np.stack([tq3.random_blocks(3 * H * I // 32, rng).reshape(-1) for _ in range(E)])
    p = str(tmp_path / "layer_00.bin")
    tq3.write_tq3x(p, body, H, I)
    got, gh, gi = tq3.read_tq3x(p)
    assert (gh, gi) == (H, I) and np.array_equal(got, body)
    with open(p, "r+b") as f:
        f.write(b"BKEX")
    with pytest.raises(ValueError):
        tq3.read_tq3x(p)


def test_gemv_oracle_against_dense_product():
    rng = np.random.default_rng(5)
    rows, cols = 6, 96
    raw = tq3.random_blocks(rows * cols // 32, rng)
    x = rng.standard_normal((3, cols)).astype(np.float16)
    W = Q.dequantize_matrix(raw, rows, cols)
    np.testing.assert_allclose(Q.gemv_f64(raw, rows, cols, x), x.astype(np.float64) @ W.T, rtol=1e-12)
