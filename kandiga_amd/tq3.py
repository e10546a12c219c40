"""TQ3: the reference's 3-bit codebook weight format, as an alternative expert format.

A TQ3 block holds 32 weights in 20 bytes (kandiga/tq3/quantize.py:120-143, 390-463): fp16
``d0, d1`` (scales of elements 0-15 and 16-31), fp16 ``m0, m1`` (their means), and 12 bytes of
3-bit indices into an 8-entry Lloyd-Max codebook, 8 per 3-byte group, index ``r`` of group ``g``
at bits ``3r..3r+2`` of ``b0 | b1<<8 | b2<<16`` (quantize.py:98-117).  The weights are those
codebook values, scaled and shifted per half, taken back through the randomized Walsh-Hadamard
transform of the block: ``w = S (H (C[q]*d + m)) / sqrt(32)`` (H the 32-point Hadamard butterfly,
S a fixed sign pattern).  Since ``H`` and ``S`` are symmetric, ``w . x = (C[q]*d + m) . WHT(x)``
with ``WHT(x) = H (S x) / sqrt(32)``: the GEMV rotates the activation once per 32-block and dots
it with the codebook values directly (kandiga/tq3/fused_kernel.py:170-251,
kandiga/tq3/tq3_metal.metal:55-141).

This module holds the format (tables, index packing), the quantizer that turns float weights
into blocks (quantize.py:190-236, 390-463: per half, mean removal, a 9-point scale search and 6
least-squares refinements), the ``TQ3X`` per-layer expert file (kandiga/tq3/convert_experts.py:
171-200: a 4096-byte header "TQ3X", version 1, experts, expert_size, hidden, intermediate,
group; then each expert's gate, up and down blocks in turn) and :class:`TQ3Experts`, the
experts resident in HBM with the switch_mlp contract run by the TQ3 kernels.
"""
from __future__ import annotations

import ctypes
import os
import struct

import numpy as np

BLOCK = 32
BLOCK_BYTES = 20
TQ3X_MAGIC = b"TQ3X"
TQ3X_HEADER = 4096

# The format's codebook, decision boundaries and sign pattern (quantize.py:29-46).
CENTROIDS = np.array([-1.996684, -1.291398, -0.740341, -0.247508,
                      0.230106, 0.725222, 1.277503, 1.988943], dtype=np.float32)
BOUNDARIES = np.array([-1.644041, -1.015870, -0.493924, -0.008701,
                       0.477664, 1.001362, 1.633223], dtype=np.float32)
SIGNS = np.array([+1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1,
                  -1, -1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1], dtype=np.float32)
_SCALE_MULTS = np.array([0.60, 0.70, 0.80, 0.90, 1.00, 1.10, 1.20, 1.35, 1.50])


def pack_indices(idx: np.ndarray) -> np.ndarray:
    """Indices ``[..., 32]`` (values < 8) -> ``[..., 12]`` bytes."""
    q = np.asarray(idx, dtype=np.uint32).reshape(*np.shape(idx)[:-1], 4, 8)
    t = np.bitwise_or.reduce(q << (3 * np.arange(8, dtype=np.uint32)), axis=-1)
    out = np.stack([t & 0xFF, (t >> 8) & 0xFF, (t >> 16) & 0xFF], axis=-1).astype(np.uint8)
    return out.reshape(*np.shape(idx)[:-1], 12)


def _wht_forward(blocks: np.ndarray) -> np.ndarray:
    """Rows of 32 through sign flips, the Hadamard butterfly and 1/sqrt(32) (quantize.py:330-342)."""
    out = blocks * SIGNS[None, :]
    step = 1
    while step < BLOCK:
        o = out.reshape(out.shape[0], BLOCK // (2 * step), 2, step)
        a, b = o[:, :, 0, :].copy(), o[:, :, 1, :].copy()
        o[:, :, 0, :], o[:, :, 1, :] = a + b, a - b
        step *= 2
    return out / np.sqrt(32.0)


def _choose(v: np.ndarray) -> np.ndarray:
    idx = np.zeros(v.shape, dtype=np.uint8)
    for b in range(7):
        idx[v > BOUNDARIES[b]] = b + 1
    return idx


def _half_scales(halves: np.ndarray, rms: np.ndarray, means: np.ndarray) -> np.ndarray:
    """Scale search and least-squares refinement of mean-centred half blocks (quantize.py:190-236)."""
    n = halves.shape[0]
    centred = halves - means[:, None]
    best_s, best_e = rms.copy(), np.full(n, np.inf)
    for mult in _SCALE_MULTS:
        sc = np.maximum(rms * mult, 1e-10)
        q = _choose(centred * (1.0 / sc)[:, None])
        err = np.sum((halves - (CENTROIDS[q] * sc[:, None] + means[:, None])) ** 2, axis=1)
        better = err < best_e
        best_e[better], best_s[better] = err[better], sc[better]
    sc = best_s.copy()
    for _ in range(6):
        q = _choose(centred * (1.0 / np.maximum(sc, 1e-10))[:, None])
        cv = CENTROIDS[q]
        num, den = np.sum(centred * cv, axis=1), np.sum(cv ** 2, axis=1)
        new = np.maximum(np.where(den > 1e-12, num / den, sc), 1e-10)
        err = np.sum((halves - (CENTROIDS[q] * new[:, None] + means[:, None])) ** 2, axis=1)
        better = err < best_e
        best_e[better], best_s[better] = err[better], new[better]
        sc = new
    return best_s


def quantize(weights: np.ndarray) -> np.ndarray:
    """Float weights (any shape, flattened row-major, zero-padded to whole blocks) -> blocks
    ``[N, 20]`` uint8 (quantize.py:390-463)."""
    flat = np.asarray(weights, dtype=np.float32).reshape(-1)
    pad = (-flat.size) % BLOCK
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, np.float32)])
    rot = _wht_forward(flat.reshape(-1, BLOCK))
    h0, h1 = rot[:, :16], rot[:, 16:]
    m0, m1 = h0.mean(axis=1), h1.mean(axis=1)
    r0 = np.sqrt(np.mean((h0 - m0[:, None]) ** 2, axis=1))
    r1 = np.sqrt(np.mean((h1 - m1[:, None]) ** 2, axis=1))
    r0[r0 < 1e-10] = 1.0
    r1[r1 < 1e-10] = 1.0
    d0, d1 = _half_scales(h0, r0, m0), _half_scales(h1, r1, m1)
    idx = np.concatenate([_choose((h0 - m0[:, None]) / np.maximum(d0, 1e-10)[:, None]),
                          _choose((h1 - m1[:, None]) / np.maximum(d1, 1e-10)[:, None])], axis=1)
    lim = 65504.0
    head = np.stack([np.clip(d0, -lim, lim), np.clip(d1, -lim, lim), np.clip(m0, -lim, lim),
                     np.clip(m1, -lim, lim)], axis=1).astype(np.float16)
    out = np.empty((idx.shape[0], BLOCK_BYTES), np.uint8)
    out[:, :8] = head.view(np.uint8)
    out[:, 8:] = pack_indices(idx)
    return out


def random_blocks(n: int, rng: np.random.Generator, scale: float = 0.02) -> np.ndarray:
    """``n`` synthetic blocks: uniform indices, scales ``|N(0, scale)|``, means ``N(0, scale/8)``."""
    out = np.empty((n, BLOCK_BYTES), np.uint8)
    d = np.abs(rng.standard_normal((n, 2))) * scale
    m = rng.standard_normal((n, 2)) * (scale / 8)
    out[:, :8] = np.concatenate([d, m], axis=1).astype(np.float16).view(np.uint8)
    out[:, 8:] = pack_indices(rng.integers(0, 8, size=(n, BLOCK)))
    return out


# ---- TQ3X expert files ------------------------------------------------------------------
def expert_bytes(hidden: int, inter: int) -> int:
    return 3 * hidden * inter // BLOCK * BLOCK_BYTES


def tq3x_header(num_experts: int, hidden: int, inter: int) -> bytes:
    h = bytearray(TQ3X_HEADER)
    h[0:4] = TQ3X_MAGIC
    struct.pack_into("<IIQIII", h, 4, 1, num_experts, expert_bytes(hidden, inter), hidden, inter, 64)
    return bytes(h)


def write_tq3x(path: str, experts: np.ndarray, hidden: int, inter: int) -> None:
    """``experts`` uint8 ``[E, expert_bytes]`` (gate, up, down blocks of each expert)."""
    experts = np.ascontiguousarray(experts, dtype=np.uint8)
    if experts.shape[1] != expert_bytes(hidden, inter):
        raise ValueError("expert body size does not match hidden/intermediate")
    with open(path, "wb") as f:
        f.write(tq3x_header(experts.shape[0], hidden, inter))
        f.write(experts.tobytes())


def read_tq3x(path: str):
    """-> (experts uint8 [E, expert_bytes], hidden, intermediate)."""
    with open(path, "rb") as f:
        hdr = f.read(TQ3X_HEADER)
    if len(hdr) < TQ3X_HEADER or hdr[:4] != TQ3X_MAGIC:
        raise ValueError(f"{path}: not a TQ3X file")
    version, E, size, H, I, _g = struct.unpack_from("<IIQIII", hdr, 4)
    if version != 1 or size != expert_bytes(H, I):
        raise ValueError(f"{path}: unsupported TQ3X header (version {version}, expert_size {size})")
    body = np.fromfile(path, dtype=np.uint8, offset=TQ3X_HEADER)
    if body.size != E * size:
        raise ValueError(f"{path}: truncated TQ3X body")
    return body.reshape(E, size), H, I


def convert_layer(dense_experts, hidden: int, inter: int) -> np.ndarray:
    """TQ3X bodies of float experts: ``dense_experts(e)`` -> (gate [I,H], up [I,H], down [H,I])
    for e in range(E) (kandiga/tq3/convert_experts.py:140-160 does this from 4-bit experts)."""
    out = []
    for g, u, d in dense_experts:
        out.append(np.concatenate([quantize(g).reshape(-1), quantize(u).reshape(-1), quantize(d).reshape(-1)]))
    body = np.stack(out)
    if body.shape[1] != expert_bytes(hidden, inter):
        raise ValueError("converted expert has the wrong size")
    return body


# ---- experts in HBM ----------------------------------------------------------------------
class TQ3Experts:
    """TQ3X expert bodies resident in device memory, with the switch_mlp contract
    (``__call__(x [..., H] fp16, indices [..., K]) -> y [..., K, H]`` fp16) run by the TQ3 kernels
    (kmoe_tq3_expert_mlp)."""

    def __init__(self, body, hidden: int, inter: int, device="cuda"):
        import torch

        t = body if isinstance(body, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(body, dtype=np.uint8))
        self.body = t.to(device).contiguous()
        self.num_experts = self.body.shape[0]
        self.hidden, self.intermediate = hidden, inter
        self.device = self.body.device
        if self.body.shape[1] != expert_bytes(hidden, inter):
            raise ValueError("expert body size does not match hidden/intermediate")
        self._ws = None
        self._ws_retired = []  # earlier workspaces, kept alive for graphs captured with them

    def reserve(self, tokens: int, top_k: int) -> None:
        """Allocate the workspace for calls of up to ``tokens`` x ``top_k`` assignments (do this
        before capturing calls into a graph; growing under a capture is refused)."""
        import torch

        from . import _capi

        n = ctypes.c_size_t()
        _capi.check(_capi.lib().kmoe_tq3_workspace_size(int(tokens), int(top_k), self.intermediate, ctypes.byref(n)),
                    "kmoe_tq3_workspace_size")
        if self._ws is None or self._ws.numel() < n.value:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"TQ3 workspace for {tokens}x{top_k} assignments was not reserved before graph "
                                   "capture; call reserve() first")
            if self._ws is not None:
                self._ws_retired.append(self._ws)
            self._ws = torch.empty(max(n.value, 256), dtype=torch.uint8, device=self.device)

    @classmethod
    def from_file(cls, path: str, device="cuda") -> "TQ3Experts":
        body, H, I = read_tq3x(path)
        return cls(body, H, I, device)

    def __call__(self, x, indices):
        import torch

        from . import _capi
        from .moe import _check_x, _on_device, _stream

        _on_device(x, self.device, "x")
        _on_device(indices, self.device, "indices")
        K = indices.shape[-1]
        xf = _check_x(x, self.hidden)
        idx = indices.reshape(-1, K).to(torch.int32).contiguous()
        T = xf.shape[0]
        if idx.shape[0] != T:
            raise ValueError("x and indices disagree on the number of tokens")
        L = _capi.lib()
        self.reserve(T, K)
        y = torch.empty((T, K, self.hidden), dtype=torch.float16, device=self.device)
        _capi.check(L.kmoe_tq3_expert_mlp(self.body.data_ptr(), self.body.shape[1], self.num_experts, self.hidden,
                                          self.intermediate, xf.data_ptr(), idx.data_ptr(), T, K, y.data_ptr(),
                                          self._ws.data_ptr(), self._ws.numel(), _stream(self.device)),
                    "kmoe_tq3_expert_mlp")
        return y.reshape(*indices.shape, self.hidden)


def gemv(blocks, rows: int, cols: int, x):
    """``x @ W.T`` (fp32 ``[T, rows]``) for a TQ3 matrix in device memory (kmoe_tq3_gemv); x fp16 or
    fp32 ``[T, cols]``."""
    import torch

    from . import _capi
    from .moe import _on_device, _stream

    _on_device(blocks, None, "blocks")
    _on_device(x, blocks.device, "x")
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError("x must be float16 or float32")
    xx = x.reshape(-1, cols).contiguous()
    T = xx.shape[0]
    out = torch.empty((T, rows), dtype=torch.float32, device=blocks.device)
    _capi.check(_capi.lib().kmoe_tq3_gemv(blocks.data_ptr(), rows, cols, xx.data_ptr(),
                                          1 if x.dtype == torch.float32 else 0, T, out.data_ptr(), _stream()),
                "kmoe_tq3_gemv")
    return out.reshape(*x.shape[:-1], rows)
