"""C ABI checks that need no GPU: the library loads, exports every symbol that
include/kandiga_amd.h declares, and rejects bad arguments on the host before launching."""
import ctypes
import os
import re

import pytest

from kandiga_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    text = open(os.path.join(ROOT, "include", "kandiga_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:kmoe|bakan)_\w+)\s*\(", text)))


def test_header_declarations_match_binding_table():
    assert sorted(_capi.EXPORTS) == _declared_functions()


def test_library_exports_every_declared_symbol():
    L = _capi.lib()
    for name in _declared_functions():
        assert hasattr(L, name), f"{name} not exported"
    assert L.kmoe_version() >= 100


def test_strerror_strings():
    L = _capi.lib()
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9):
        assert L.kmoe_strerror(code)
    assert L.kmoe_strerror(-99) == b"unknown status"


def _desc(**kw):
    d = _capi.LayerDesc()
    d.hidden, d.intermediate, d.num_experts, d.top_k, d.bits, d.group_size = 2048, 512, 256, 8, 3, 64
    fake = 1 << 20  # aligned, never dereferenced by layer_create
    for p in ("gate", "up", "down"):
        q = getattr(d, p)
        q.weight, q.scales, q.biases = fake, fake, fake
        rows = 512 if p != "down" else 2048
        cols = 2048 if p != "down" else 512
        q.weight_expert_stride = rows * cols * 3 // 8
        q.scale_expert_stride = rows * cols // 64 * 2
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def _create(d):
    L = _capi.lib()
    h = ctypes.c_void_p()
    rc = L.kmoe_layer_create(ctypes.byref(d), ctypes.byref(h))
    return rc, h


def test_layer_create_valid_and_workspace_size():
    L = _capi.lib()
    rc, h = _create(_desc())
    assert rc == 0 and h.value
    n1, n2 = ctypes.c_size_t(), ctypes.c_size_t()
    assert L.kmoe_workspace_size(h, 1, ctypes.byref(n1)) == 0
    assert L.kmoe_workspace_size(h, 4096, ctypes.byref(n2)) == 0
    assert 256 <= n1.value < n2.value
    # prefill workspace holds act (2 planes) and per-assignment outputs
    assert n2.value >= 4096 * 8 * 512 * 4 + 4096 * 8 * 2048 * 2
    assert L.kmoe_layer_destroy(h) == 0


@pytest.mark.parametrize("field,value,code", [
    ("bits", 5, _capi.ERR_UNSUPPORTED), ("group_size", 32, _capi.ERR_UNSUPPORTED),
    ("hidden", 2000, _capi.ERR_UNSUPPORTED), ("intermediate", 0, _capi.ERR_UNSUPPORTED),
    ("num_experts", 2000, _capi.ERR_UNSUPPORTED), ("top_k", 0, _capi.ERR_INVALID_ARG),
    ("top_k", 17, _capi.ERR_INVALID_ARG), ("scale_dtype", 7, _capi.ERR_INVALID_ARG),
    ("activation", 9, _capi.ERR_INVALID_ARG),
])
def test_layer_create_rejects(field, value, code):
    rc, h = _create(_desc(**{field: value}))
    assert rc == code and not h.value
    assert _capi.lib().kmoe_last_error()


def test_layer_create_rejects_misaligned_and_short_strides():
    d = _desc()
    d.gate.weight = (1 << 20) + 2
    assert _create(d)[0] == _capi.ERR_ALIGNMENT
    d = _desc(bits=4)
    for p, rows, cols in (("gate", 512, 2048), ("up", 512, 2048), ("down", 2048, 512)):
        getattr(d, p).weight_expert_stride = rows * cols // 2
    d.up.weight = (1 << 20) + 4            # 4-bit codes need 16-byte alignment
    assert _create(d)[0] == _capi.ERR_ALIGNMENT
    d = _desc()
    d.down.weight_expert_stride = 100
    assert _create(d)[0] in (_capi.ERR_ALIGNMENT, _capi.ERR_INVALID_ARG)
    d = _desc()
    d.gate.scales = None
    assert _create(d)[0] == _capi.ERR_INVALID_ARG


def test_calls_validate_before_launch():
    L = _capi.lib()
    null = None
    assert L.kmoe_route(null, 4, 256, 0, null, null, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_route(null, 4, 256, 8, null, null, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_route(null, 0, 256, 8, null, null, null) == 0          # empty batch is a no-op
    assert L.kmoe_route(null, -1, 256, 8, null, null, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_expert_mlp(null, null, null, 1, null, null, 0, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_forward(null, null, null, 1, null, 0, null, null, null, 0, null) == _capi.ERR_INVALID_ARG
    rc, h = _create(_desc())
    assert L.kmoe_forward(h, null, null, 0, null, 0, null, null, null, 0, null) == 0
    assert L.kmoe_forward(h, 256, 256, 1, 256, 5, null, null, 256, 1 << 30, null) == _capi.ERR_INVALID_ARG
    # misaligned x
    assert L.kmoe_forward(h, 258, 256, 1, 256, 0, null, null, 256, 1 << 30, null) == _capi.ERR_ALIGNMENT
    # workspace too small
    assert L.kmoe_forward(h, 256, 256, 4, 256, 0, null, null, 256, 512, null) == _capi.ERR_WORKSPACE
    assert L.kmoe_dequantize(h, 3, 0, 0, 1, 256, 256, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_dequantize(h, 0, 256, 0, 1, 256, 256, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_dequantize(h, 2, 0, 2040, 9, 256, 256, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_combine(null, null, 3, 0, 64, null, null) == _capi.ERR_INVALID_ARG
    n = ctypes.c_size_t()
    assert L.kmoe_permute_workspace_size(4096, 8, 256, ctypes.byref(n)) == 0 and n.value > 4096 * 8 * 8
    assert L.kmoe_permute(null, 4, 8, 2000, null, null, null, null, null, null, 0, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_device_status(null, 0, None, null) == _capi.ERR_INVALID_ARG
    L.kmoe_layer_destroy(h)


def test_activation_dtypes_validate_before_launch():
    """kmoe_forward_x / kmoe_expert_mlp_x: unknown dtypes are refused, and a layer with the dense
    fp16 shared expert refuses bf16/fp32 activations, all before anything is launched."""
    L = _capi.lib()
    null = None
    rc, h = _create(_desc())
    assert L.kmoe_forward_x(h, 256, 3, 256, 1, 256, 0, null, null, 256, 1 << 30, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_forward_x(h, 256, -1, 256, 1, 256, 0, null, null, 256, 1 << 30, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_expert_mlp_x(h, 256, 5, 256, 1, 256, 256, 1 << 30, null) == _capi.ERR_INVALID_ARG
    assert L.kmoe_forward_x(h, 256, _capi.X_BF16, 256, 0, 256, 0, null, null, 256, 1 << 30, null) == 0
    assert L.kmoe_forward_x(h, 258, _capi.X_F32, 256, 1, 256, 0, null, null, 256, 1 << 30, null) == _capi.ERR_ALIGNMENT
    L.kmoe_layer_destroy(h)
    fake = 1 << 20
    rc, hs = _create(_desc(shared_gate=fake, shared_up=fake, shared_down=fake, shared_intermediate=1024))
    assert rc == 0
    assert L.kmoe_forward_x(hs, 256, _capi.X_BF16, 256, 1, 256, 0, null, null, 256, 1 << 30, null) == \
        _capi.ERR_UNSUPPORTED
    L.kmoe_layer_destroy(hs)


def test_prefill_copy_size_and_validation():
    L = _capi.lib()
    n = ctypes.c_size_t()
    assert L.kmoe_prefill_pack_size(ctypes.byref(_desc()), ctypes.byref(n)) == 0
    # H=2048, I=512, E=256, 3-bit: 3 x 256 x 512x2048x3/8 code bytes, then per projection
    # 256 experts x rows x group pairs x 8 bytes (16 pairs x 512 rows; 4 pairs x 2048 rows)
    assert n.value == 3 * 256 * 393216 + 3 * 256 * 65536
    # odd group counts are padded to whole pairs: H=320 (5 groups), I=192 (3 groups), E=12
    d = _desc(hidden=320, intermediate=192, num_experts=12, top_k=3)
    for p, rows, cols in (("gate", 192, 320), ("up", 192, 320), ("down", 320, 192)):
        getattr(d, p).weight_expert_stride = rows * cols * 3 // 8
        getattr(d, p).scale_expert_stride = rows * cols // 64 * 2
    assert L.kmoe_prefill_pack_size(ctypes.byref(d), ctypes.byref(n)) == 0
    up = lambda v: (v + 255) // 256 * 256
    codes = 2 * up(12 * 192 * 320 * 3 // 8) + up(12 * 320 * 192 * 3 // 8)
    assert n.value == codes + 2 * up(12 * 192 * 3 * 8) + up(12 * 320 * 2 * 8)
    assert L.kmoe_prefill_pack_size(ctypes.byref(_desc(bits=5)), ctypes.byref(n)) == _capi.ERR_UNSUPPORTED
    # the copy must be aligned and whole before a layer uses it
    full = 3 * 256 * 393216 + 3 * 256 * 65536
    assert _create(_desc(prefill_pack=(1 << 20) + 128, prefill_pack_bytes=full))[0] == _capi.ERR_ALIGNMENT
    assert _create(_desc(prefill_pack=1 << 20, prefill_pack_bytes=full - 1))[0] == _capi.ERR_INVALID_ARG
    rc, h = _create(_desc(prefill_pack=1 << 20, prefill_pack_bytes=full))
    assert rc == 0 and h.value
    L.kmoe_layer_destroy(h)
    # kmoe_prefill_pack checks its buffer before launching
    assert L.kmoe_prefill_pack(ctypes.byref(_desc()), 1 << 20, full - 1, None) == _capi.ERR_INVALID_ARG
    assert L.kmoe_prefill_pack(ctypes.byref(_desc()), (1 << 20) + 64, full, None) == _capi.ERR_ALIGNMENT
    assert L.kmoe_prefill_pack(ctypes.byref(_desc()), None, full, None) == _capi.ERR_INVALID_ARG


def test_kernel_timing_validates_arguments():
    L = _capi.lib()
    assert L.kmoe_profile_begin(0) == _capi.ERR_INVALID_ARG
    assert L.kmoe_profile_begin(16385) == _capi.ERR_INVALID_ARG
    n = ctypes.c_int32()
    assert L.kmoe_profile_end(None, 0, ctypes.byref(n)) == _capi.ERR_INVALID_ARG  # timing is not on
    assert ctypes.sizeof(_capi.KernelTime) == 80


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setattr(_capi, "LIB_PATH", str(tmp_path / "libkandiga_amd.so"))
    with pytest.raises(ImportError):
        _capi.lib()
