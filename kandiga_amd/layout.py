"""MLX-layout group-quantized expert weights and the BKEX packed-expert file.

MLX affine quantization with group size 64 stores a projection ``W[out, in]`` as

* ``weight``  uint32 ``[out, in*bits/32]`` -- each row's codes as one little-endian
  bit stream;
* ``scales``  fp16 or bf16 ``[out, in/64]``;
* ``biases``  fp16 or bf16 ``[out, in/64]``;

and dequantizes code ``q`` of column ``c`` as ``w = q * scales[c//64] + biases[c//64]``.

Bit order (kandiga/metal/kandiga_cpu_expert.m:194-201 for 3 bits, :285-293 for 4 bits):

* 4 bits: column ``c`` is nibble ``c % 8`` of word ``c // 8``: ``(word >> 4*(c%8)) & 0xF``.
* 3 bits: every 3-byte triplet holds 8 codes.  With ``t = b0 | b1<<8 | b2<<16`` the
  code of column ``8*j + i`` is ``(t >> 3*i) & 7`` (the same order as
  kandiga/tq3/quantize.py:98-107).  A row of ``in`` columns is ``in*3/8`` bytes.

Expert stacks follow mlx_lm's SwitchGLU tensors ``switch_mlp.{gate,up,down}_proj.*``:
the expert index is the leading dimension, gate/up are ``[E, I, H]`` and down is
``[E, H, I]`` (before packing).

BKEX (kandiga/_pack_experts.py:6-20, 95-132) is the reference's per-layer file: a
4096-byte header followed by ``E`` expert blocks of ``expert_size`` bytes, each block
``[gate.w][gate.s][gate.b][up.w][up.s][up.b][down.w][down.s][down.b]``.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

GROUP_SIZE = 64
BKEX_HEADER_SIZE = 4096
BKEX_MAGIC = b"BKEX"
BKEX_VERSION = 1

# Tensor order inside a BKEX expert block (kandiga/_pack_experts.py:35-45).
TENSOR_NAMES = (
    "gate_proj.weight", "gate_proj.scales", "gate_proj.biases",
    "up_proj.weight", "up_proj.scales", "up_proj.biases",
    "down_proj.weight", "down_proj.scales", "down_proj.biases",
)

# BKEX dtype byte.  0 and 1 are the reference's codes (uint32, bfloat16);
# 2 marks fp16 scale/bias tensors, which the reference never writes.
DTYPE_U32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2


def _check_bits(bits: int) -> None:
    if bits not in (3, 4):
        raise ValueError(f"bits must be 3 or 4, got {bits}")


def packed_row_words(in_dim: int, bits: int) -> int:
    """uint32 words per packed row of ``in_dim`` codes."""
    _check_bits(bits)
    if in_dim % 32:
        raise ValueError(f"in_dim {in_dim} must be a multiple of 32")
    return in_dim * bits // 32


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes ``[..., in]`` (values < 2**bits) into MLX uint32 words."""
    _check_bits(bits)
    codes = np.asarray(codes)
    in_dim = codes.shape[-1]
    if in_dim % 32:
        raise ValueError(f"in_dim {in_dim} must be a multiple of 32")
    if codes.size and int(codes.max()) >= (1 << bits):
        raise ValueError(f"code out of range for {bits}-bit packing")
    lead = codes.shape[:-1]
    c = codes.astype(np.uint32).reshape(*lead, in_dim // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * bits)
    t = np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)   # [..., in/8]
    if bits == 4:
        return np.ascontiguousarray(t)
    tri = np.stack([t & 0xFF, (t >> 8) & 0xFF, (t >> 16) & 0xFF], axis=-1).astype(np.uint8)
    return np.ascontiguousarray(tri.reshape(*lead, in_dim * 3 // 8)).view(np.uint32)


def unpack_codes(words: np.ndarray, bits: int, in_dim: int) -> np.ndarray:
    """Inverse of :func:`pack_codes`: uint32 words ``[..., in*bits/32]`` -> uint8 codes."""
    _check_bits(bits)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    lead = words.shape[:-1]
    if words.shape[-1] != packed_row_words(in_dim, bits):
        raise ValueError("packed row length does not match in_dim")
    if bits == 4:
        t = words.reshape(*lead, in_dim // 8)
    else:
        b = words.view(np.uint8).reshape(*lead, in_dim // 8, 3).astype(np.uint32)
        t = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    shifts = np.arange(8, dtype=np.uint32) * bits
    c = (t[..., None] >> shifts) & ((1 << bits) - 1)
    return c.reshape(*lead, in_dim).astype(np.uint8)


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16)).view(np.uint16)


def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)
    rounded = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return rounded.astype(np.uint16)


def scale_bits_to_f32(bits16: np.ndarray, scale_dtype: str) -> np.ndarray:
    if scale_dtype == "f16":
        return np.asarray(bits16, dtype=np.uint16).view(np.float16).astype(np.float32)
    if scale_dtype == "bf16":
        return bf16_bits_to_f32(bits16)
    raise ValueError(f"scale_dtype must be 'f16' or 'bf16', got {scale_dtype!r}")


def f16_to_bf16_bits(bits16: np.ndarray) -> np.ndarray:
    """Re-encode fp16 bit patterns as bf16 (RNE).  Exact for values with <= 8 mantissa bits."""
    return f32_to_bf16_bits(np.asarray(bits16, dtype=np.uint16).view(np.float16).astype(np.float32))


def bf16_to_f16_bits(bits16: np.ndarray) -> np.ndarray:
    """Re-encode bf16 bit patterns as fp16 (RNE, as ``astype(float16)`` in engine.py:475-482)."""
    return f16_bits(bf16_bits_to_f32(bits16).astype(np.float16))


# --------------------------------------------------------------------------------------
# Expert block geometry
# --------------------------------------------------------------------------------------
@dataclass(frozen=True)
class ExpertGeometry:
    """Byte layout of one expert block (gate/up ``[I, H]``, down ``[H, I]``)."""

    hidden: int
    intermediate: int
    bits: int
    group_size: int = GROUP_SIZE

    def __post_init__(self):
        _check_bits(self.bits)
        if self.group_size != GROUP_SIZE:
            raise ValueError("only group size 64 is supported")
        for d in (self.hidden, self.intermediate):
            if d % GROUP_SIZE:
                raise ValueError(f"dimension {d} is not a multiple of {GROUP_SIZE}")

    def tensor_shapes(self):
        """(name, shape, kind) in BKEX order; kind is 'w' (uint32) or 's' (16-bit)."""
        H, I, b = self.hidden, self.intermediate, self.bits
        gh, gi = H // GROUP_SIZE, I // GROUP_SIZE
        out = []
        for proj, rows, cols in (("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
            out.append((f"{proj}.weight", (rows, cols * b // 32), "w"))
            g = gh if cols == H else gi
            out.append((f"{proj}.scales", (rows, g), "s"))
            out.append((f"{proj}.biases", (rows, g), "s"))
        return out

    def tensor_nbytes(self):
        res = []
        for name, shape, kind in self.tensor_shapes():
            res.append((name, shape, kind, shape[0] * shape[1] * (4 if kind == "w" else 2)))
        return res

    def offsets(self) -> dict:
        """Byte offset of each tensor inside the expert block."""
        off, res = 0, {}
        for name, _shape, _kind, nb in self.tensor_nbytes():
            res[name] = off
            off += nb
        return res

    @property
    def expert_size(self) -> int:
        return sum(nb for *_x, nb in self.tensor_nbytes())


# --------------------------------------------------------------------------------------
# BKEX files
# --------------------------------------------------------------------------------------
def build_bkex_header(num_experts: int, geom: ExpertGeometry, scale_dtype: str = "bf16") -> bytes:
    """4096-byte BKEX header (field layout of kandiga/_pack_experts.py:95-132)."""
    sdt = {"bf16": DTYPE_BF16, "f16": DTYPE_F16}[scale_dtype]
    buf = bytearray(BKEX_HEADER_SIZE)
    buf[0:4] = BKEX_MAGIC
    struct.pack_into("<I", buf, 4, BKEX_VERSION)
    struct.pack_into("<I", buf, 8, num_experts)
    struct.pack_into("<Q", buf, 12, geom.expert_size)
    tensors = geom.tensor_nbytes()
    struct.pack_into("<I", buf, 20, len(tensors))
    pos, off = 24, 0
    for name, shape, kind, nb in tensors:
        nm = name.encode("ascii")
        buf[pos] = len(nm)
        buf[pos + 1:pos + 1 + len(nm)] = nm
        pos += 25
        struct.pack_into("<IIII", buf, pos, off, nb, shape[0], shape[1])
        pos += 16
        buf[pos] = DTYPE_U32 if kind == "w" else sdt
        pos += 1
        off += nb
    return bytes(buf)


@dataclass
class BkexHeader:
    version: int
    num_experts: int
    expert_size: int
    tensors: list          # dicts: name, offset, nbytes, shape, dtype
    hidden: int
    intermediate: int
    bits: int
    scale_dtype: str


def parse_bkex_header(hdr: bytes) -> BkexHeader:
    """Parse and validate a BKEX header (kandiga/metal/kandiga_cpu_expert_lg.m:67-117)."""
    if len(hdr) < BKEX_HEADER_SIZE or hdr[:4] != BKEX_MAGIC:
        raise ValueError("not a BKEX file (bad magic)")
    version, num_experts = struct.unpack_from("<II", hdr, 4)
    (expert_size,) = struct.unpack_from("<Q", hdr, 12)
    (ntensors,) = struct.unpack_from("<I", hdr, 20)
    if ntensors != 9:
        raise ValueError(f"BKEX file has {ntensors} tensors, expected 9")
    tensors, pos = [], 24
    for _ in range(ntensors):
        nlen = hdr[pos]
        name = hdr[pos + 1:pos + 1 + min(nlen, 24)].decode("ascii")
        pos += 25
        off, nb, d0, d1 = struct.unpack_from("<IIII", hdr, pos)
        pos += 16
        dt = hdr[pos]
        pos += 1
        tensors.append(dict(name=name, offset=off, nbytes=nb, shape=(d0, d1), dtype=dt))
    by = {t["name"]: t for t in tensors}
    if tuple(t["name"] for t in tensors) != TENSOR_NAMES:
        raise ValueError("BKEX tensor order differs from gate/up/down weight/scales/biases")
    inter = by["gate_proj.weight"]["shape"][0]
    hidden = by["gate_proj.scales"]["shape"][1] * GROUP_SIZE
    wbytes = by["gate_proj.weight"]["nbytes"]
    if wbytes * 8 == inter * hidden * 4:
        bits = 4
    elif wbytes * 8 == inter * hidden * 3:
        bits = 3
    else:
        raise ValueError("gate_proj.weight size matches neither 3- nor 4-bit codes")
    sdt = by["gate_proj.scales"]["dtype"]
    scale_dtype = {DTYPE_BF16: "bf16", DTYPE_F16: "f16"}.get(sdt)
    if scale_dtype is None:
        raise ValueError(f"unknown scale dtype code {sdt}")
    geom = ExpertGeometry(hidden, inter, bits)
    expect = geom.offsets()
    for t in tensors:
        if t["offset"] != expect[t["name"]]:
            raise ValueError(f"tensor {t['name']} at offset {t['offset']}, expected {expect[t['name']]}")
    if geom.expert_size != expert_size:
        raise ValueError(f"expert_size {expert_size} != sum of tensors {geom.expert_size}")
    return BkexHeader(version, num_experts, expert_size, tensors, hidden, inter, bits, scale_dtype)


def read_bkex_header(path: str) -> BkexHeader:
    with open(path, "rb") as f:
        return parse_bkex_header(f.read(BKEX_HEADER_SIZE))


def expert_block_bytes(layer: dict, e: int, geom: ExpertGeometry) -> bytes:
    """Concatenate expert ``e`` of a stacked layer dict into one BKEX block."""
    parts = []
    for name, shape, kind, nb in geom.tensor_nbytes():
        proj, field = name.split(".")
        key = {"weight": "w", "scales": "s", "biases": "b"}[field]
        arr = layer[f"{proj.split('_')[0]}_{key}"][e]
        raw = np.ascontiguousarray(arr).tobytes()
        if len(raw) != nb:
            raise ValueError(f"{name}: {len(raw)} bytes, expected {nb}")
        parts.append(raw)
    return b"".join(parts)


def write_bkex(path: str, layer: dict, geom: ExpertGeometry, scale_dtype: str) -> None:
    """Write a stacked layer (dict from :mod:`kandiga_amd.synth`) as one BKEX file.

    ``scale_dtype`` is the dtype the file stores; the layer dict's 16-bit scale/bias
    arrays must already be bit patterns of that dtype.
    """
    num_experts = layer["gate_w"].shape[0]
    with open(path, "wb") as f:
        f.write(build_bkex_header(num_experts, geom, scale_dtype))
        for e in range(num_experts):
            f.write(expert_block_bytes(layer, e, geom))
    if os.path.getsize(path) != BKEX_HEADER_SIZE + num_experts * geom.expert_size:
        raise IOError(f"short write to {path}")


def read_bkex_layer(path: str) -> tuple:
    """Read a BKEX file back into the stacked layer dict layout.  Returns (layer, header)."""
    hdr = read_bkex_header(path)
    geom = ExpertGeometry(hdr.hidden, hdr.intermediate, hdr.bits)
    raw = np.fromfile(path, dtype=np.uint8, offset=BKEX_HEADER_SIZE)
    if raw.size != hdr.num_experts * hdr.expert_size:
        raise ValueError("BKEX file is truncated")
    blocks = raw.reshape(hdr.num_experts, hdr.expert_size)
    layer = {}
    for name, shape, kind, nb in geom.tensor_nbytes():
        off = geom.offsets()[name]
        proj, field = name.split(".")
        key = {"weight": "w", "scales": "s", "biases": "b"}[field]
        dt = np.uint32 if kind == "w" else np.uint16
        layer[f"{proj.split('_')[0]}_{key}"] = np.ascontiguousarray(blocks[:, off:off + nb]).view(dt).reshape(
            hdr.num_experts, *shape)
    return layer, hdr
