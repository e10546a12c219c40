"""ORACLE -- test infrastructure only (see ``oracle/__init__.py``).

Numpy restatements of the routed-expert MoE layer of the reference, plus a ctypes
binding of the C restatement of its expert MLP (``oracle/expert_mlp.c``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
GROUP = 64


# --------------------------------------------------------------------------------------
# Codes and dequantization
# --------------------------------------------------------------------------------------
def unpack_codes(words: np.ndarray, bits: int, in_dim: int) -> np.ndarray:
    """Codes of packed rows, byte by byte.

    3 bits follows the scalar unpack of kandiga/metal/kandiga_cpu_expert.m:194-201
    literally (each 3-byte pack gives 8 values); 4 bits follows :285-293
    (nibble n of each uint32 word).
    """
    words = np.ascontiguousarray(words, dtype=np.uint32)
    lead = words.shape[:-1]
    rows = int(np.prod(lead)) if lead else 1
    out = np.empty((rows, in_dim), dtype=np.uint8)
    if bits == 4:
        w = words.reshape(rows, in_dim // 8)
        for n in range(8):
            out[:, n::8] = (w >> (4 * n)) & 0xF
    elif bits == 3:
        b = words.view(np.uint8).reshape(rows, in_dim // 8, 3).astype(np.uint16)
        b0, b1, b2 = b[..., 0], b[..., 1], b[..., 2]
        vals = [
            b0 & 0x07,
            (b0 >> 3) & 0x07,
            ((b0 >> 6) & 0x03) | ((b1 & 0x01) << 2),
            (b1 >> 1) & 0x07,
            (b1 >> 4) & 0x07,
            ((b1 >> 7) & 0x01) | ((b2 & 0x03) << 1),
            (b2 >> 2) & 0x07,
            (b2 >> 5) & 0x07,
        ]
        for i, v in enumerate(vals):
            out[:, i::8] = v
    else:
        raise ValueError(bits)
    return out.reshape(*lead, in_dim)


def scale_to_f64(bits16: np.ndarray, scale_dtype: str) -> np.ndarray:
    u = np.asarray(bits16, dtype=np.uint16)
    if scale_dtype == "f16":
        return u.view(np.float16).astype(np.float64)
    if scale_dtype == "bf16":
        return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    raise ValueError(scale_dtype)


def dequantize(words, scales, biases, bits: int, in_dim: int, scale_dtype: str = "f16") -> np.ndarray:
    """``w = q * s + b`` per group of 64 columns, in float64 (exact for 16-bit s, b)."""
    q = unpack_codes(words, bits, in_dim).astype(np.float64)
    s = np.repeat(scale_to_f64(scales, scale_dtype), GROUP, axis=-1)
    b = np.repeat(scale_to_f64(biases, scale_dtype), GROUP, axis=-1)
    return q * s + b


# --------------------------------------------------------------------------------------
# Router: softmax -> top-K -> renormalise
# --------------------------------------------------------------------------------------
def route(logits: np.ndarray, top_k: int):
    """Top-K experts per token with weights renormalised over the selected K.

    Selection key: logit descending, expert index ascending on equal logits; NaN logits
    rank below every number (-inf included).  The
    reference's router (kandiga/metal/moe_block.metal:419-505; mlx_lm's
    softmax -> argpartition -> renorm on the live path) selects on the softmax
    probabilities with lowest-index ties; softmax is monotone in the logit, so the two
    agree except where distinct logits round to the same fp32 probability, which
    :func:`route_prob_ties` reports.

    Weights: ``w_k = p_k / sum_{j in topK} p_j`` with ``p = softmax(logits)``
    (:499-503), evaluated as ``exp(l_k - l_max) / sum_j exp(l_j - l_max)`` in float64
    (the full-softmax denominator cancels).  Returns ``idx`` int32 ``[T,K]`` and ``w``
    float32 ``[T,K]``.
    """
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    if not 0 < top_k <= E:
        raise ValueError("top_k out of range")
    order = np.argsort(-logits, axis=1, kind="stable")       # ties: lower index first
    idx = order[:, :top_k].astype(np.int32)
    sel = np.take_along_axis(logits, idx, axis=1).astype(np.float64)
    with np.errstate(invalid="ignore"):   # NaN or infinite logits give NaN weights
        e = np.exp(sel - sel[:, :1])
        w = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


def route_by_probs(logits: np.ndarray, top_k: int):
    """The reference kernel's literal fp32 steps (moe_block.metal:419-505).

    max, ``exp(l - max)``, sum, multiply by ``1/sum``; then K argmax passes with a strict
    ``>`` (lowest index wins ties); scores times ``1/sum(scores)``.
    """
    l = np.asarray(logits, dtype=np.float32)
    m = l.max(axis=1, keepdims=True)
    p = np.exp(l - m).astype(np.float32)
    p = (p * (np.float32(1.0) / p.sum(axis=1, keepdims=True, dtype=np.float32))).astype(np.float32)
    idx = np.argsort(-p, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    sc = np.take_along_axis(p, idx, axis=1)
    w = (sc * (np.float32(1.0) / sc.sum(axis=1, keepdims=True, dtype=np.float32))).astype(np.float32)
    return idx, w


def route_prob_ties(logits: np.ndarray, top_k: int) -> np.ndarray:
    """Tokens whose probability-keyed selection differs from the logit-keyed one."""
    a, _ = route(logits, top_k)
    b, _ = route_by_probs(logits, top_k)
    return np.nonzero((a != b).any(axis=1))[0]


# --------------------------------------------------------------------------------------
# Token -> expert permutation
# --------------------------------------------------------------------------------------
def permute(idx: np.ndarray, num_experts: int) -> dict:
    """Stable grouping of the T*K assignments by expert (kandiga/engine.py:407-418).

    ``flat_tok = repeat(arange(T), K)``, ``flat_k = tile(arange(K), T)``, mergesort of
    ``idx.ravel()``; group boundaries at expert changes; unique experts ascending;
    plus the dense per-expert histogram and its exclusive scan.
    """
    idx = np.asarray(idx, dtype=np.int32)
    T, K = idx.shape
    flat_exp = idx.reshape(-1)
    order = np.argsort(flat_exp, kind="mergesort").astype(np.int32)
    s_exp = flat_exp[order]
    counts = np.bincount(flat_exp, minlength=num_experts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    if s_exp.size:
        changes = np.concatenate([[0], np.nonzero(np.diff(s_exp))[0] + 1, [s_exp.size]]).astype(np.int32)
        unique = s_exp[changes[:-1]].astype(np.int32)
    else:
        changes = np.zeros(1, dtype=np.int32)
        unique = np.zeros(0, dtype=np.int32)
    return dict(perm=order, s_tok=(order // K).astype(np.int32), s_k=(order % K).astype(np.int32),
                s_exp=s_exp.astype(np.int32), counts=counts, offsets=offsets, unique=unique,
                group_starts=changes)


# --------------------------------------------------------------------------------------
# Combine and the dense shared expert
# --------------------------------------------------------------------------------------
def combine(y: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``out[t] = sum_k w[t,k] * y[t,k]`` accumulated in fp32 in k order (moe_block.metal:530-538)."""
    y = np.asarray(y, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    out = np.zeros((y.shape[0], y.shape[2]), dtype=np.float32)
    for k in range(y.shape[1]):
        out += y[:, k, :] * w[:, k:k + 1]
    return out


def silu64(g):
    with np.errstate(over="ignore"):   # exp(-g) = inf for very negative g gives silu = -0, as it should
        return g / (1.0 + np.exp(-g))


def shared_expert_f64(layer: dict, x: np.ndarray) -> np.ndarray:
    """Ungated dense fp16 SwiGLU expert added after the routed combine, in float64."""
    xs = np.asarray(x, dtype=np.float16).astype(np.float64)
    g = xs @ layer["shared_gate"].view(np.float16).astype(np.float64).T
    u = xs @ layer["shared_up"].view(np.float16).astype(np.float64).T
    return (silu64(g) * u) @ layer["shared_down"].view(np.float16).astype(np.float64).T


# --------------------------------------------------------------------------------------
# Expert MLP: float64 closed form and the C restatement
# --------------------------------------------------------------------------------------
def dequantize_dense(words, scales, biases, bits: int, in_dim: int, scale_dtype: str = "f16",
                     dtype=np.float64) -> np.ndarray:
    """:func:`dequantize` with broadcast unpacking (whole 3-byte triplets / 4-byte words at
    once), for the full-size checks.  Equal to :func:`dequantize` in float64; in float32 the
    result is exact whenever ``q*s + b`` is (always for the synthetic scales)."""
    words = np.ascontiguousarray(words)
    lead = words.shape[:-1]
    rows = int(np.prod(lead)) if lead else 1
    if bits == 4:
        q = (words.reshape(rows, in_dim // 8, 1) >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF
    elif bits == 3:
        b = words.view(np.uint8).reshape(rows, in_dim // 8, 3).astype(np.uint32)
        t = (b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16))[..., None]
        q = (t >> (np.arange(8, dtype=np.uint32) * 3)) & 7
    else:
        raise ValueError(bits)
    q = q.reshape(rows, in_dim // GROUP, GROUP).astype(dtype)
    sc = scale_to_f64(scales, scale_dtype).reshape(rows, in_dim // GROUP, 1).astype(dtype)
    bi = scale_to_f64(biases, scale_dtype).reshape(rows, in_dim // GROUP, 1).astype(dtype)
    return (q * sc + bi).reshape(*lead, in_dim)


def moe_out_dense(expert_arrays, x: np.ndarray, idx: np.ndarray, w: np.ndarray, bits: int, hidden: int,
                  inter: int, scale_dtype: str = "f16", act: str = "silu", dtype=np.float64,
                  threads: int = 8, exact_x: bool = False) -> np.ndarray:
    """Routed combine ``out[t] = sum_k w[t,k] * expert_{idx[t,k]}(x[t])`` for every token of a
    full-size batch, through dense matrix products one expert at a time: all the rows routed
    to an expert go through its dequantized gate/up/down matrices together.

    ``expert_arrays(e)`` returns expert e's nine arrays (``gate_w``, ``gate_s``, ...,
    ``down_b``, without the expert dimension).  Experts are spread over ``threads`` workers,
    each with a single-threaded BLAS.  float64 by default; float32 keeps the relative error
    near 1e-6, three orders below the layer tolerance, at half the time.  ``x`` is rounded to
    fp16 unless ``exact_x`` (bf16 / fp32 activations, taken as given)."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits

    idx = np.asarray(idx)
    T, K = idx.shape
    xs = np.asarray(x, dtype=dtype if exact_x else np.float16).astype(dtype)
    wts = np.asarray(w, dtype=np.float64)
    experts = np.unique(idx)

    def one(e):
        a = expert_arrays(int(e))
        tok, kk = np.nonzero(idx == e)
        g = dequantize_dense(a["gate_w"], a["gate_s"], a["gate_b"], bits, hidden, scale_dtype, dtype)
        u = dequantize_dense(a["up_w"], a["up_s"], a["up_b"], bits, hidden, scale_dtype, dtype)
        d = dequantize_dense(a["down_w"], a["down_s"], a["down_b"], bits, inter, scale_dtype, dtype)
        xr = xs[tok]
        gv, uv = xr @ g.T, xr @ u.T
        if act == "silu":
            av = silu64(gv) * uv
        else:
            av = 0.5 * gv * (1 + np.tanh(0.7978845608 * (gv + 0.044715 * gv ** 3))) * uv
        return tok, (av @ d.T).astype(np.float64) * wts[tok, kk][:, None]

    out = np.zeros((T, hidden), dtype=np.float64)
    with threadpool_limits(limits=1, user_api="blas"), ThreadPoolExecutor(max(1, threads)) as pool:
        for tok, contrib in pool.map(one, experts):
            np.add.at(out, tok, contrib)
    return out


def expert_weights_f64(layer: dict, e: int, bits: int, hidden: int, inter: int, scale_dtype: str = "f16"):
    g = dequantize(layer["gate_w"][e], layer["gate_s"][e], layer["gate_b"][e], bits, hidden, scale_dtype)
    u = dequantize(layer["up_w"][e], layer["up_s"][e], layer["up_b"][e], bits, hidden, scale_dtype)
    d = dequantize(layer["down_w"][e], layer["down_s"][e], layer["down_b"][e], bits, inter, scale_dtype)
    return g, u, d


def expert_mlp_f64(layer: dict, e: int, x: np.ndarray, bits: int, scale_dtype: str = "f16",
                   act: str = "silu", exact_x: bool = False) -> np.ndarray:
    """One expert on rows of ``x`` via float64 matrix products of the dequantized weights (``x``
    rounded to fp16, or with ``exact_x`` taken as given)."""
    H = layer["gate_s"].shape[-1] * GROUP
    I = layer["down_s"].shape[-1] * GROUP
    g_w, u_w, d_w = expert_weights_f64(layer, e, bits, H, I, scale_dtype)
    xs = np.atleast_2d(np.asarray(x, dtype=np.float64 if exact_x else np.float16).astype(np.float64))
    g = xs @ g_w.T
    u = xs @ u_w.T
    if act == "silu":
        a = silu64(g) * u
    else:
        a = 0.5 * g * (1.0 + np.tanh(0.7978845608 * (g + 0.044715 * g ** 3))) * u
    return a @ d_w.T


class _Proj(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("b", ctypes.c_void_p),
                ("w_stride", ctypes.c_int64), ("s_stride", ctypes.c_int64)]


class _Layer(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("bits", ctypes.c_int),
                ("scale_bf16", ctypes.c_int), ("act", ctypes.c_int),
                ("gate", _Proj), ("up", _Proj), ("down", _Proj)]


_lib = None


def build_lib(force: bool = False) -> str:
    """Compile ``oracle/expert_mlp.c`` with ``oracle/Makefile``."""
    if force or not os.path.exists(_LIB_PATH) or not os.path.exists(os.path.join(_HERE, "_build", "librefscalar.so")):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build_lib()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_switch_mlp.argtypes = [ctypes.POINTER(_Layer), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.oracle_switch_mlp.restype = ctypes.c_int
        L.oracle_switch_mlp_f32.argtypes = [ctypes.POINTER(_Layer), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.oracle_switch_mlp_f32.restype = ctypes.c_int
        L.oracle_round_f16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _proj(layer, name):
    w, s, b = layer[f"{name}_w"], layer[f"{name}_s"], layer[f"{name}_b"]
    for a in (w, s, b):
        if not a.flags.c_contiguous:
            raise ValueError(f"{name} arrays must be C-contiguous")
    return _Proj(w.ctypes.data, s.ctypes.data, b.ctypes.data,
                 w[0].nbytes if w.shape[0] > 0 else 0, s[0].size if s.shape[0] > 0 else 0)


def switch_mlp(layer: dict, x: np.ndarray, idx: np.ndarray, bits: int, scale_dtype: str = "f16",
               act: str = "silu", nthreads: int = 1, exact_x: bool = False) -> np.ndarray:
    """``y[t, k] = expert idx[t, k] (x[t])`` in fp32 via the C restatement -> ``[T, K, H]``.

    ``x`` is rounded to fp16 (``bakan_cpu_expert_mlp_f16``), or with ``exact_x`` taken as fp32
    values as they are (``bakan_cpu_expert_mlp``; bf16 activations are widened to fp32 exactly
    and passed this way, as ``bakan_cpu_expert_mlp_bf16`` does)."""
    H = layer["gate_s"].shape[-1] * GROUP
    I = layer["down_s"].shape[-1] * GROUP
    if exact_x:
        xa = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    else:
        xa = np.ascontiguousarray(np.asarray(x, dtype=np.float16)).view(np.uint16)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    if idx.size and (idx.min() < 0 or idx.max() >= layer["gate_w"].shape[0]):
        raise ValueError("expert index out of range")
    y = np.empty((T, K, H), dtype=np.float32)
    desc = _Layer(H, I, bits, 1 if scale_dtype == "bf16" else 0, 0 if act == "silu" else 1,
                  _proj(layer, "gate"), _proj(layer, "up"), _proj(layer, "down"))
    fn = lib().oracle_switch_mlp_f32 if exact_x else lib().oracle_switch_mlp
    rc = fn(ctypes.byref(desc), xa.ctypes.data, idx.ctypes.data, T, K, y.ctypes.data, int(nthreads))
    if rc != 0:
        raise RuntimeError("oracle_switch_mlp failed")
    return y


_rs_lib = None


def ref_scalar_switch_mlp(layer: dict, x: np.ndarray, idx: np.ndarray, bits: int, scale_dtype: str = "f16",
                          nthreads: int = 1) -> np.ndarray:
    """The CPU baseline (``oracle/ref_scalar.c``): the reference's portable scalar expert MLP at
    its own optimisation level, K experts of a token on an OpenMP team -> ``[T, K, H]`` fp32."""
    global _rs_lib
    if _rs_lib is None:
        path = os.path.join(_HERE, "_build", "librefscalar.so")
        if not os.path.exists(path):
            build_lib()
        L = ctypes.CDLL(path)
        L.refscalar_switch_mlp.argtypes = [ctypes.POINTER(_Layer), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.refscalar_switch_mlp.restype = ctypes.c_int
        _rs_lib = L
    H = layer["gate_s"].shape[-1] * GROUP
    I = layer["down_s"].shape[-1] * GROUP
    x16 = np.ascontiguousarray(np.asarray(x, dtype=np.float16)).view(np.uint16)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    if idx.size and (idx.min() < 0 or idx.max() >= layer["gate_w"].shape[0]):
        raise ValueError("expert index out of range")
    y = np.empty((T, K, H), dtype=np.float32)
    desc = _Layer(H, I, bits, 1 if scale_dtype == "bf16" else 0, 0,
                  _proj(layer, "gate"), _proj(layer, "up"), _proj(layer, "down"))
    if _rs_lib.refscalar_switch_mlp(ctypes.byref(desc), x16.ctypes.data, idx.ctypes.data, T, K, y.ctypes.data,
                                    int(nthreads)) != 0:
        raise RuntimeError("refscalar_switch_mlp failed")
    return y


def round_f16(a: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 with the C restatement's RNE conversion."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_round_f16(a.ctypes.data, out.ctypes.data, a.size)
    return out.view(np.float16)


def moe_layer(layer: dict, x: np.ndarray, logits: np.ndarray, top_k: int, bits: int,
              scale_dtype: str = "f16", nthreads: int = 1) -> dict:
    """Whole routed layer: route -> switch_mlp (fp32) -> combine (+ shared expert)."""
    idx, w = route(logits, top_k)
    y = switch_mlp(layer, x, idx, bits, scale_dtype, nthreads=nthreads)
    out = combine(y, w)
    if "shared_gate" in layer:
        out = (out.astype(np.float64) + shared_expert_f64(layer, x)).astype(np.float32)
    return dict(idx=idx, w=w, y=y, out=out)


def qlinear_f64(words, scales, biases, bits: int, x: np.ndarray, scale_dtype: str = "f16") -> np.ndarray:
    """``x @ W.T`` for a group-quantized projection ``W [rows, in]`` (MLX layout), float64 (the
    router and shared-gate projections, moe_block.metal:194-227, 300-336)."""
    xs = np.atleast_2d(np.asarray(x, dtype=np.float16).astype(np.float64))
    w = dequantize(words, scales, biases, bits, xs.shape[1], scale_dtype)
    return xs @ w.T


def block_shared_layer(block: dict) -> dict:
    """The block's quantized shared expert as a one-expert stacked layer dict."""
    return {f"{p}_{k}": np.ascontiguousarray(block[f"blk_shared_{p}_{k}"][None]) for p in ("gate", "up", "down")
            for k in ("w", "s", "b")}


def moe_block(layer: dict, block: dict, x: np.ndarray, top_k: int, bits: int, block_bits: int,
              scale_dtype: str = "f16", block_scale_dtype: str = "bf16", residual=None, logits=None,
              nthreads: int = 1) -> dict:
    """The whole MoE block (moe_block.metal:194-584; bakan_forward.h:111-140):

    logits = router . x (fp32); softmax -> top-K -> renorm; the routed experts' weighted sum
    (C restatement, fp32, k order); the shared expert (C restatement) rounded to fp16 as the
    reference's shared_expert_down_kernel stores it (:324); its gate sigmoid(shared_gate . x);
    out = (residual + routed) + shared16 * gate (:577-583; without a residual :536-538).
    ``logits`` given: route on those instead (to check the rest of the block on a device's
    own logits)."""
    lg = qlinear_f64(block["blk_router_w"], block["blk_router_s"], block["blk_router_b"], block_bits, x,
                     block_scale_dtype).astype(np.float32)
    use = lg if logits is None else np.asarray(logits, dtype=np.float32)
    idx, w = route(use, top_k)
    out = combine(switch_mlp(layer, x, idx, bits, scale_dtype, nthreads=nthreads), w).astype(np.float64)
    if residual is not None:
        out = np.asarray(residual, dtype=np.float16).astype(np.float64) + out
    if "blk_shared_gate_w" in block:
        T = np.atleast_2d(x).shape[0]
        sh = switch_mlp(block_shared_layer(block), x, np.zeros((T, 1), np.int32), block_bits, block_scale_dtype)[:, 0]
        sh16 = round_f16(sh).astype(np.float64)
        g = np.ones((T, 1))
        if "blk_sgate_w" in block:
            gl = qlinear_f64(block["blk_sgate_w"], block["blk_sgate_s"], block["blk_sgate_b"], block_bits, x,
                             block_scale_dtype)
            g = 1.0 / (1.0 + np.exp(-gl))
        out = out + sh16 * g
        # one fp16 spacing of the shared output, gated: how far a device whose fp32 shared value
        # differs in the last bits can land after the fp16 rounding
        a = np.maximum(np.abs(sh).astype(np.float64), 2.0 ** -14)
        flip = np.exp2(np.floor(np.log2(a)) - 10) * g
    else:
        flip = np.zeros_like(out)
    return dict(logits=lg, idx=idx, w=w, out=out.astype(np.float32), shared_flip=flip)


def compare(got: np.ndarray, ref: np.ndarray) -> dict:
    """max-abs and relative-L2 error of ``got`` against ``ref`` (both taken as float64)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    diff = g - r
    denom = np.linalg.norm(r)
    return dict(max_abs=float(np.abs(diff).max()) if diff.size else 0.0,
                rel_l2=float(np.linalg.norm(diff) / denom) if denom > 0 else float(np.linalg.norm(diff)))
