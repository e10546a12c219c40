"""ctypes binding of ``libkandiga_amd.so`` (the C ABI declared in ``include/kandiga_amd.h``).

The library is built in-tree (``kandiga_amd/libkandiga_amd.so``).  Loading fails loudly
when it is missing: there is no fallback implementation.  ``torch`` is imported before
the library so both share the HIP runtime torch ships (the library's ``libamdhip64.so.7``
dependency then resolves to the already-loaded copy).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkandiga_amd.so")

# Every symbol include/kandiga_amd.h declares, in declaration order.
EXPORTS = (
    "kmoe_version", "kmoe_strerror", "kmoe_last_error",
    "kmoe_layer_create", "kmoe_layer_destroy", "kmoe_workspace_size",
    "kmoe_route", "kmoe_permute_workspace_size", "kmoe_permute",
    "kmoe_expert_mlp", "kmoe_expert_mlp_x", "kmoe_combine", "kmoe_forward", "kmoe_forward_x",
    "kmoe_block_create", "kmoe_block_destroy", "kmoe_block_workspace_size", "kmoe_block_forward",
    "kmoe_tq3_gemv", "kmoe_tq3_workspace_size", "kmoe_tq3_expert_mlp",
    "kmoe_forward_noalloc",
    "kmoe_prefill_pack_size", "kmoe_prefill_pack",
    "kmoe_dequantize", "kmoe_device_status",
    "kmoe_profile_begin", "kmoe_profile_end",
)

OK = 0
ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_ALIGNMENT, ERR_WORKSPACE = -1, -2, -3, -4
ERR_HIP, ERR_IO, ERR_FORMAT, ERR_DEVICE, ERR_NO_MEMORY = -5, -6, -7, -8, -9
SCALE_F16, SCALE_BF16 = 0, 1
ACT_SWIGLU, ACT_GELU_TANH = 0, 1
OUT_F16, OUT_F32 = 0, 1
X_F16, X_BF16, X_F32 = 0, 1, 2
DEVERR_BAD_EXPERT = 1
NOALLOC_SCRATCH_BYTES = 16 << 20


class KmoeError(RuntimeError):
    """A C ABI call returned a negative status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class QProjDesc(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("weight_expert_stride", ctypes.c_int64), ("scale_expert_stride", ctypes.c_int64)]


class LayerDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32), ("num_experts", ctypes.c_int32),
                ("top_k", ctypes.c_int32), ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32),
                ("scale_dtype", ctypes.c_int32), ("activation", ctypes.c_int32),
                ("gate", QProjDesc), ("up", QProjDesc), ("down", QProjDesc),
                ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p), ("shared_down", ctypes.c_void_p),
                ("shared_intermediate", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("prefill_pack", ctypes.c_void_p), ("prefill_pack_bytes", ctypes.c_int64)]


class BlockDesc(ctypes.Structure):
    _fields_ = [("routed", ctypes.c_void_p), ("router", QProjDesc), ("shared_gate_proj", QProjDesc),
                ("shared_up_proj", QProjDesc), ("shared_down_proj", QProjDesc), ("shared_expert_gate", QProjDesc),
                ("bits", ctypes.c_int32), ("scale_dtype", ctypes.c_int32), ("shared_intermediate", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("total_ms", ctypes.c_double), ("min_ms", ctypes.c_double), ("max_ms", ctypes.c_double)]


_lib = None
_vp, _i32, _sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t


def _declare(L):
    P = ctypes.POINTER
    sig = {
        "kmoe_version": ([], ctypes.c_int),
        "kmoe_strerror": ([ctypes.c_int], ctypes.c_char_p),
        "kmoe_last_error": ([], ctypes.c_char_p),
        "kmoe_layer_create": ([P(LayerDesc), P(_vp)], ctypes.c_int),
        "kmoe_layer_destroy": ([_vp], ctypes.c_int),
        "kmoe_workspace_size": ([_vp, _i32, P(_sz)], ctypes.c_int),
        "kmoe_route": ([_vp, _i32, _i32, _i32, _vp, _vp, _vp], ctypes.c_int),
        "kmoe_permute_workspace_size": ([_i32, _i32, _i32, P(_sz)], ctypes.c_int),
        "kmoe_permute": ([_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_expert_mlp": ([_vp, _vp, _vp, _i32, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_expert_mlp_x": ([_vp, _vp, _i32, _vp, _i32, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_combine": ([_vp, _vp, _i32, _i32, _i32, _vp, _vp], ctypes.c_int),
        "kmoe_forward": ([_vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_forward_x": ([_vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_block_create": ([P(BlockDesc), P(_vp)], ctypes.c_int),
        "kmoe_block_destroy": ([_vp], ctypes.c_int),
        "kmoe_block_workspace_size": ([_vp, _i32, P(_sz)], ctypes.c_int),
        "kmoe_block_forward": ([_vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
        "kmoe_tq3_gemv": ([_vp, _i32, _i32, _vp, _i32, _i32, _vp, _vp], ctypes.c_int),
        "kmoe_tq3_workspace_size": ([_i32, _i32, _i32, P(_sz)], ctypes.c_int),
        "kmoe_tq3_expert_mlp": ([_vp, ctypes.c_int64, _i32, _i32, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _sz, _vp],
                                ctypes.c_int),
        "kmoe_forward_noalloc": ([_vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp], ctypes.c_int),
        "kmoe_prefill_pack_size": ([P(LayerDesc), P(_sz)], ctypes.c_int),
        "kmoe_prefill_pack": ([P(LayerDesc), _vp, _sz, _vp], ctypes.c_int),
        "kmoe_dequantize": ([_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp], ctypes.c_int),
        "kmoe_device_status": ([_vp, _sz, P(_i32), _vp], ctypes.c_int),
        "kmoe_profile_begin": ([_i32], ctypes.c_int),
        "kmoe_profile_end": ([P(KernelTime), _i32, P(_i32)], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def lib():
    """The loaded library; raises ``ImportError`` if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `make -C kandiga_amd/csrc` "
                              "(or __graft_entry__.build()); there is no fallback implementation")
        import torch  # noqa: F401  -- share torch's HIP runtime

        L = ctypes.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != OK:
        L = lib()
        msg = L.kmoe_last_error().decode() or L.kmoe_strerror(rc).decode()
        raise KmoeError(rc, f"{what}: {L.kmoe_strerror(rc).decode()} ({msg})" if what else msg)
