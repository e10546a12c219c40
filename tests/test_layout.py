"""MLX bit layout, BKEX format and synthetic-generator checks (CPU).

Known answers come from the reference: the BKEX header constants its pack test asserts
(tests/test_pack.py:13-30: magic, version 1, 256 experts, expert_size 1 769 472,
9 tensors, 4096-byte header) and the per-tensor byte offsets its CPU library hard-codes
(kandiga/metal/kandiga_cpu_expert.m:42-65).
"""
import numpy as np
import pytest

from kandiga_amd import layout, synth
from oracle import moe_oracle as O


def test_pack_3bit_known_bytes():
    # codes 0..7 in one triplet: t = sum(i << 3i) = 0xFAC688 -> bytes 88 C6 FA
    codes = np.tile(np.arange(8, dtype=np.uint8), 4)[None, :]
    w = layout.pack_codes(codes, 3)
    assert w.view(np.uint8)[0, :3].tobytes() == bytes([0x88, 0xC6, 0xFA])
    # code 7 at position 2 straddles bytes 0/1 (kandiga_cpu_expert.m:196: bits 6,7 of b0 and bit 0 of b1)
    c = np.zeros((1, 32), dtype=np.uint8)
    c[0, 2] = 7
    assert layout.pack_codes(c, 3).view(np.uint8)[0, :3].tobytes() == bytes([0xC0, 0x01, 0x00])
    c = np.zeros((1, 32), dtype=np.uint8)
    c[0, 5] = 7  # bit 7 of b1 and bits 0,1 of b2 (:199)
    assert layout.pack_codes(c, 3).view(np.uint8)[0, :3].tobytes() == bytes([0x00, 0x80, 0x03])


def test_pack_4bit_known_word():
    codes = (np.arange(32) % 16).astype(np.uint8)[None, :]
    w = layout.pack_codes(codes, 4)
    assert w[0, 0] == 0x76543210 and w[0, 1] == 0xFEDCBA98


@pytest.mark.parametrize("bits", [3, 4])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 2 ** bits, size=(7, 5, 192), dtype=np.uint8)
    w = layout.pack_codes(codes, bits)
    assert w.dtype == np.uint32 and w.shape == (7, 5, 192 * bits // 32)
    assert np.array_equal(layout.unpack_codes(w, bits, 192), codes)
    # the oracle's byte-by-byte restatement agrees with the vectorised unpack
    assert np.array_equal(O.unpack_codes(w, bits, 192), codes)


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        layout.pack_codes(np.full((1, 32), 8, dtype=np.uint8), 3)
    with pytest.raises(ValueError):
        layout.pack_codes(np.zeros((1, 40), dtype=np.uint8), 3)


def test_bkex_header_known_answers_4bit():
    """The 35B layer geometry of the reference's pack test (tests/test_pack.py:13-30)."""
    geom = layout.ExpertGeometry(2048, 512, 4)
    hdr = layout.build_bkex_header(256, geom, "bf16")
    assert len(hdr) == layout.BKEX_HEADER_SIZE == 4096
    assert hdr[:4] == b"BKEX"
    import struct

    assert struct.unpack_from("<I", hdr, 4)[0] == 1
    assert struct.unpack_from("<I", hdr, 8)[0] == 256
    assert struct.unpack_from("<Q", hdr, 12)[0] == 1_769_472
    assert struct.unpack_from("<I", hdr, 20)[0] == 9
    parsed = layout.parse_bkex_header(hdr)
    assert (parsed.hidden, parsed.intermediate, parsed.bits, parsed.scale_dtype) == (2048, 512, 4, "bf16")


def test_expert_offsets_match_reference_constants():
    """Byte offsets of kandiga/metal/kandiga_cpu_expert.m:42-65."""
    o4 = layout.ExpertGeometry(2048, 512, 4).offsets()
    assert [o4[n] for n in layout.TENSOR_NAMES] == [0, 524288, 557056, 589824, 1114112, 1146880, 1179648,
                                                     1703936, 1736704]
    assert layout.ExpertGeometry(2048, 512, 4).expert_size == 1769472
    o3 = layout.ExpertGeometry(2048, 512, 3).offsets()
    assert [o3[n] for n in layout.TENSOR_NAMES] == [0, 393216, 425984, 458752, 851968, 884736, 917504,
                                                     1310720, 1343488]
    assert layout.ExpertGeometry(2048, 512, 3).expert_size == 1376256
    # header-derived sizes of the larger layers
    assert layout.ExpertGeometry(2560, 1024, 3).expert_size == 3440640
    assert layout.ExpertGeometry(4096, 1024, 3).expert_size == 5505024


def test_bkex_roundtrip(tmp_path):
    shape = synth.LayerShape(128, 64, 5, 2, 3)
    layer = synth.make_layer(shape, 3, "bf16")
    geom = layout.ExpertGeometry(128, 64, 3)
    p = tmp_path / "layer_00.bin"
    layout.write_bkex(str(p), layer, geom, "bf16")
    back, hdr = layout.read_bkex_layer(str(p))
    assert hdr.num_experts == 5 and hdr.bits == 3 and hdr.scale_dtype == "bf16"
    for k in ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b"):
        assert np.array_equal(back[k], layer[k]), k


def test_bkex_rejects_bad_files(tmp_path):
    with pytest.raises(ValueError):
        layout.parse_bkex_header(b"XXXX" + bytes(4092))
    geom = layout.ExpertGeometry(128, 64, 4)
    hdr = bytearray(layout.build_bkex_header(3, geom, "f16"))
    hdr[12] ^= 0xFF  # corrupt expert_size
    with pytest.raises(ValueError):
        layout.parse_bkex_header(bytes(hdr))


def test_synthetic_scales_dual_representable():
    shape = synth.LayerShape(256, 128, 4, 2, 3)
    layer = synth.make_layer(shape, 9)
    s = layer["gate_s"].view(np.float16).astype(np.float32)
    assert (s >= 2 ** -14).all()
    # every scale is a bf16 value (low 16 bits of its fp32 pattern are zero)
    assert (s.view(np.uint32) & 0xFFFF == 0).all()
    b = layer["gate_b"].view(np.float16).astype(np.float32)
    assert np.array_equal(b, -4 * s)
    bf = synth.make_layer(shape, 9, "bf16")
    assert np.array_equal(layout.bf16_bits_to_f32(bf["gate_s"]), s)


def test_synthetic_codes_uniform():
    shape = synth.LayerShape(512, 256, 8, 2, 3)
    layer = synth.make_layer(shape, 10)
    c = layout.unpack_codes(layer["gate_w"], 3, 512)
    hist = np.bincount(c.reshape(-1), minlength=8) / c.size
    assert np.abs(hist - 1 / 8).max() < 0.005


def test_zipf_bias_skews_loads():
    shape = synth.LayerShape(64, 64, 256, 8, 3)
    _x, logits = synth.make_inputs(shape, 2048, 4, zipf=True)
    idx, _ = O.route(logits, 8)
    counts = np.sort(np.bincount(idx.reshape(-1), minlength=256))[::-1]
    assert counts[0] > 8 * counts[128]  # heavy head, light tail
    _x, logits = synth.make_inputs(shape, 2048, 4, zipf=False)
    idx, _ = O.route(logits, 8)
    counts = np.bincount(idx.reshape(-1), minlength=256)
    assert counts.max() < 3 * counts.mean()
