"""Host side of the routed-expert MoE layer: torch tensors in HBM, HIP kernels via the C ABI.

Mirrors the reference's operator interface for this path:

* :class:`QuantizedSwitchGLU` -- drop-in for ``_CPUSwitchGLU`` / mlx_lm ``SwitchGLU``
  (kandiga/engine.py:327-739): ``__call__(x [..., H], indices [..., K]) -> y [..., K, H]``,
  the per-(token, k) expert outputs, not combined, fp16.
* :class:`SparseMoeBlock` -- the routed block around it (router softmax -> top-K ->
  renorm, switch_mlp, weighted combine; mlx_lm's SparseMoeBlock as driven by
  engine.py:1090-1139, restated in kandiga/metal/moe_block.metal:419-584) with the router
  logits as input: ``__call__(x [..., H], logits [..., E]) -> out [..., H]``.
* :func:`route`, :func:`permute`, :func:`combine` -- the individual stages.

Errors raise :class:`~kandiga_amd._capi.KmoeError` (the reference raises RuntimeError on a
nonzero status, engine.py:185-186); a missing library raises ImportError.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _capi
from .layout import GROUP_SIZE, ExpertGeometry, read_bkex_header, BKEX_HEADER_SIZE
from .synth import LayerShape

_PROJS = ("gate", "up", "down")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device | None = None) -> int:
    """The hipStream_t of the current stream of ``dev`` (default: the current device).  The raw
    query costs ~0.1 us against ~2.5 us for ``torch.cuda.current_stream().cuda_stream``, which
    matters on the per-token path of eager callers."""
    idx = dev.index if dev is not None and dev.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def _as_u16(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype in (torch.float16, torch.bfloat16, torch.int16, torch.uint16) else t


@dataclass
class _Proj:
    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    weight_stride: int   # bytes between experts
    scale_stride: int    # bytes between experts


def _block_projs(buf: "torch.Tensor", geom: ExpertGeometry, expert_size: int | None = None) -> dict:
    """Projection descriptors over expert-contiguous blocks (BKEX body layout): expert e's
    tensor starts at buf + e*expert_size + its offset within the block."""
    offs = geom.offsets()
    stride = expert_size or geom.expert_size
    flat = buf.reshape(-1)
    projs = {}
    for name in _PROJS:
        off_w = offs[f"{name}_proj.weight"]
        if (flat.data_ptr() + off_w) % (16 if geom.bits == 4 else 4):
            raise ValueError("expert weight tensor is misaligned")
        projs[name] = _Proj(flat[off_w:], flat[offs[f"{name}_proj.scales"]:], flat[offs[f"{name}_proj.biases"]:],
                            stride, stride)
    return projs


class QuantizedExperts:
    """All experts of one layer resident in device memory (MLX affine layout, group 64).

    Holds the ``kmoe_layer`` handle and a workspace that grows with the largest token
    count seen (allocate it up front with :meth:`reserve` to keep allocation out of
    timed regions).  ``prefill_copy=True`` also keeps the experts in the layout the
    grouped prefill GEMMs read with whole cache lines (``kmoe_prefill_pack``; about one
    more copy of the weights); results are the same either way.
    """

    def __init__(self, shape: LayerShape, projs: dict, scale_dtype: str = "f16", activation: str = "swiglu",
                 shared: dict | None = None, keepalive=None, prefill_copy: bool = False):
        if scale_dtype not in ("f16", "bf16"):
            raise ValueError("scale_dtype must be 'f16' or 'bf16'")
        if activation not in ("swiglu", "gelu_tanh"):
            raise ValueError("activation must be 'swiglu' or 'gelu_tanh'")
        self.shape = shape
        self.scale_dtype = scale_dtype
        self.activation = activation
        self.projs = projs
        self.shared = shared
        self._keepalive = keepalive
        dev = projs["gate"].weight.device
        if dev.type != "cuda":
            raise ValueError("expert weights must be on a cuda (HIP) device")
        self.device = dev
        d = _capi.LayerDesc()
        d.hidden, d.intermediate = shape.hidden, shape.intermediate
        d.num_experts, d.top_k, d.bits, d.group_size = shape.num_experts, shape.top_k, shape.bits, GROUP_SIZE
        d.scale_dtype = _capi.SCALE_BF16 if scale_dtype == "bf16" else _capi.SCALE_F16
        d.activation = _capi.ACT_GELU_TANH if activation == "gelu_tanh" else _capi.ACT_SWIGLU
        for name in _PROJS:
            p = projs[name]
            q = getattr(d, name)
            q.weight, q.scales, q.biases = p.weight.data_ptr(), p.scales.data_ptr(), p.biases.data_ptr()
            q.weight_expert_stride, q.scale_expert_stride = p.weight_stride, p.scale_stride
        if shared:
            d.shared_gate = shared["gate"].data_ptr()
            d.shared_up = shared["up"].data_ptr()
            d.shared_down = shared["down"].data_ptr()
            d.shared_intermediate = shape.shared_intermediate
        L = _capi.lib()
        self._pack = None
        if prefill_copy:
            n = ctypes.c_size_t()
            _capi.check(L.kmoe_prefill_pack_size(ctypes.byref(d), ctypes.byref(n)), "kmoe_prefill_pack_size")
            pack = torch.empty(n.value, dtype=torch.uint8, device=dev)
            if pack.data_ptr() % 256:
                raise RuntimeError("prefill copy allocation is not 256-byte aligned")
            _capi.check(L.kmoe_prefill_pack(ctypes.byref(d), pack.data_ptr(), n.value, _stream()),
                        "kmoe_prefill_pack")
            d.prefill_pack, d.prefill_pack_bytes = pack.data_ptr(), n.value
            self._pack = pack
        self._desc = d
        h = ctypes.c_void_p()
        _capi.check(L.kmoe_layer_create(ctypes.byref(d), ctypes.byref(h)), "kmoe_layer_create")
        self._handle = h
        self._ws = None
        self._ws_tokens = -1
        self._ws_captured = False   # the current workspace was used by a captured call
        self._ws_retired = []       # earlier workspaces still referenced by captured graphs

    # ---- construction helpers ---------------------------------------------------------
    @classmethod
    def from_stacked(cls, shape: LayerShape, layer: dict, device="cuda", scale_dtype: str = "f16",
                     activation: str = "swiglu", layout: str = "expert",
                     prefill_copy: bool = False) -> "QuantizedExperts":
        """From a stacked layer dict (numpy from :func:`synth.make_layer` or torch tensors).

        ``layout="expert"`` (default) packs each expert's nine tensors into one contiguous
        block at the BKEX offsets, as a ``layer_XX.bin`` body holds them
        (kandiga/metal/kandiga_cpu_expert.m:42-65): one expert then spans at most two 2 MiB
        pages, which keeps address translation cheap when a decode step touches a few
        experts out of hundreds.  ``layout="stacked"`` keeps one tensor per projection part
        (expert stride = one expert's slice)."""
        if layout not in ("expert", "stacked"):
            raise ValueError(f"unknown layout {layout!r}")
        tensors = {}
        for name in _PROJS:
            for key in ("w", "s", "b"):
                a = layer[f"{name}_{key}"]
                t = a if isinstance(a, torch.Tensor) else torch.from_numpy(a.view(a.dtype.str.replace("u", "i")))
                tensors[(name, key)] = t.to(device).contiguous()
        shared = None
        if shape.shared_intermediate and "shared_gate" in layer:
            shared = {}
            for name in _PROJS:
                a = layer[f"shared_{name}"]
                t = a if isinstance(a, torch.Tensor) else torch.from_numpy(a.view("i2"))
                shared[name] = t.to(device).contiguous()
        if layout == "stacked":
            projs = {}
            for name in _PROJS:
                w, s, b = (tensors[(name, k)] for k in ("w", "s", "b"))
                projs[name] = _Proj(w, _as_u16(s), _as_u16(b), w[0].numel() * w.element_size(),
                                    s[0].numel() * s.element_size())
            return cls(shape, projs, scale_dtype, activation, shared, list(tensors.values()), prefill_copy)
        geom = ExpertGeometry(shape.hidden, shape.intermediate, shape.bits)
        offs, E = geom.offsets(), shape.num_experts
        body = torch.empty((E, geom.expert_size), dtype=torch.uint8, device=device)
        for name in _PROJS:
            for key, part in (("w", "weight"), ("s", "scales"), ("b", "biases")):
                t = tensors[(name, key)].reshape(E, -1).view(torch.uint8)
                off = offs[f"{name}_proj.{part}"]
                body[:, off:off + t.shape[1]] = t
        del tensors
        return cls(shape, _block_projs(body, geom), scale_dtype, activation, shared, [body], prefill_copy)

    @classmethod
    def from_bkex(cls, path: str, top_k: int, device="cuda", activation: str | None = None,
                  prefill_copy: bool = False) -> "QuantizedExperts":
        """Load a BKEX ``layer_XX.bin`` file: the expert blocks are uploaded as one buffer and
        described with the block size as expert stride (no repacking).  The activation
        defaults to GELU-tanh for intermediate size 704 and SwiGLU otherwise, as the
        header-driven reference does (kandiga/metal/kandiga_cpu_expert_lg.m:109-111)."""
        hdr = read_bkex_header(path)
        geom = ExpertGeometry(hdr.hidden, hdr.intermediate, hdr.bits)
        import numpy as np
        body = np.fromfile(path, dtype=np.uint8, offset=BKEX_HEADER_SIZE)
        if body.size != hdr.num_experts * hdr.expert_size:
            raise ValueError(f"{path}: truncated BKEX body")
        buf = torch.from_numpy(body).to(device)
        shape = LayerShape(hdr.hidden, hdr.intermediate, hdr.num_experts, top_k, hdr.bits)
        act = activation or ("gelu_tanh" if hdr.intermediate == 704 else "swiglu")
        return cls(shape, _block_projs(buf, geom, hdr.expert_size), hdr.scale_dtype, act, None, [buf], prefill_copy)

    @classmethod
    def from_safetensors(cls, path: str, layer: int, top_k: int, device="cuda", prefix: str | None = None,
                         activation: str = "swiglu", layout: str = "expert",
                         prefill_copy: bool = False) -> "QuantizedExperts":
        """Load one MoE layer's stacked ``switch_mlp`` tensors from an MLX safetensors checkpoint
        (a directory with ``model.safetensors.index.json`` or ``model.safetensors``, or one
        file); dimensions, bit width and scale dtype come from the tensor shapes
        (kandiga/_split_experts.py:62-117 reads the same nine tensors)."""
        from . import weights

        L, info = weights.read_switch_mlp(path, layer, prefix or weights.DEFAULT_PREFIX)
        shape = LayerShape(info.hidden, info.intermediate, info.num_experts, top_k, info.bits)
        return cls.from_stacked(shape, L, device, info.scale_dtype, activation, layout, prefill_copy)

    @classmethod
    def from_expert_files(cls, layer_dir: str, top_k: int, device="cuda", activation: str = "swiglu",
                          layout: str = "expert", prefill_copy: bool = False) -> "QuantizedExperts":
        """Load a ``layer_XX/expert_NNN.safetensors`` directory, the per-expert files of the
        reference's split step (kandiga/_split_experts.py:106-115)."""
        from . import weights

        L, info = weights.read_expert_files(layer_dir)
        shape = LayerShape(info.hidden, info.intermediate, info.num_experts, top_k, info.bits)
        return cls.from_stacked(shape, L, device, info.scale_dtype, activation, layout, prefill_copy)

    def with_prefill_copy(self) -> "QuantizedExperts":
        """The same experts (sharing these tensors) with a prefill copy made for them."""
        return QuantizedExperts(self.shape, self.projs, self.scale_dtype, self.activation, self.shared,
                                self._keepalive, prefill_copy=True)

    # ---- workspace --------------------------------------------------------------------
    def workspace_bytes(self, tokens: int) -> int:
        n = ctypes.c_size_t()
        _capi.check(_capi.lib().kmoe_workspace_size(self._handle, int(tokens), ctypes.byref(n)),
                    "kmoe_workspace_size")
        return n.value

    def reserve(self, tokens: int) -> None:
        """Allocate (zeroed) workspace for calls of up to ``tokens`` tokens.

        A larger request replaces the workspace.  A workspace that was handed to a call under
        CUDA-graph capture is never released: the captured graph keeps its address, so it is
        retained for the life of this object (a later, larger eager call then gets a new one).
        Growing is refused while a capture is in progress (allocate with ``reserve`` before
        capturing)."""
        if tokens > self._ws_tokens:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"workspace for {tokens} tokens was not reserved before graph capture "
                                   f"(reserved: {self._ws_tokens}); call reserve({tokens}) first")
            if self._ws is not None and self._ws_captured:
                self._ws_retired.append(self._ws)
            self._ws = torch.zeros(max(self.workspace_bytes(tokens), 256), dtype=torch.uint8, device=self.device)
            self._ws_tokens = tokens
            self._ws_captured = False

    def workspace(self, tokens: int) -> torch.Tensor:
        self.reserve(tokens)
        if torch.cuda.is_current_stream_capturing():
            self._ws_captured = True
        return self._ws

    def host_subset(self, experts) -> dict:
        """Host copies of the given experts' tensors, stacked in the listed order, as the dict of
        numpy arrays (``gate_w`` uint32, ``gate_s`` / ``gate_b`` uint16, ...) that
        :func:`synth.make_layer` produces.  Works for either weight layout."""
        import numpy as np

        geom = ExpertGeometry(self.shape.hidden, self.shape.intermediate, self.shape.bits)
        ids = [int(e) for e in experts]
        out = {}
        for name, shape, kind, nbytes in geom.tensor_nbytes():
            proj, part = name.split("_proj.")
            p = self.projs[proj]
            base = p.weight if part == "weight" else p.scales if part == "scales" else p.biases
            stride = p.weight_stride if part == "weight" else p.scale_stride
            flat = base.reshape(-1).view(torch.uint8)
            rows = [flat[e * stride:e * stride + nbytes] for e in ids]
            a = torch.stack(rows).cpu().numpy()
            key = f"{proj}_{part[0]}"
            out[key] = a.view(np.uint32 if kind == "w" else np.uint16).reshape((len(ids),) + tuple(shape))
        return out

    def device_status(self) -> int:
        """Read and clear the device error flags (synchronises the current stream)."""
        if self._ws is None:
            return 0
        f = ctypes.c_int32()
        _capi.check(_capi.lib().kmoe_device_status(self._ws.data_ptr(), self._ws.numel(), ctypes.byref(f),
                                                   _stream()), "kmoe_device_status")
        return f.value

    def dequantize(self, proj: str, expert: int, row0: int = 0, nrows: int = 1):
        """(codes uint8 [nrows, in], fp16 weights [nrows, in]) as the kernels unpack them."""
        pi = _PROJS.index(proj)
        in_dim = self.shape.intermediate if proj == "down" else self.shape.hidden
        codes = torch.empty((nrows, in_dim), dtype=torch.uint8, device=self.device)
        w16 = torch.empty((nrows, in_dim), dtype=torch.float16, device=self.device)
        _capi.check(_capi.lib().kmoe_dequantize(self._handle, pi, expert, row0, nrows, codes.data_ptr(),
                                                w16.data_ptr(), _stream()), "kmoe_dequantize")
        return codes, w16

    def __del__(self):
        h = getattr(self, "_handle", None)
        lib = getattr(_capi, "_lib", None) if _capi is not None else None  # None at interpreter exit
        if h is not None and lib is not None:
            lib.kmoe_layer_destroy(h)
            self._handle = None


def _on_device(t: torch.Tensor, dev: torch.device, name: str) -> None:
    """Raise before any launch unless ``t`` lives in device memory of ``dev``: a host tensor's
    pointer handed to a kernel would be a GPU memory fault."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} is on {t.device}; move it to {dev} first")
    if dev is not None and t.device.index != dev.index:
        raise ValueError(f"{name} is on {t.device}, the experts are on {dev}")


_X_DTYPES = {torch.float16: _capi.X_F16, torch.bfloat16: _capi.X_BF16, torch.float32: _capi.X_F32}


def _x_arg(x: torch.Tensor, H: int):
    """(rows [T, H] contiguous, KMOE_X_* code) for the entry points that take fp16, bf16 or fp32
    activations natively (kmoe_expert_mlp_x / kmoe_forward_x)."""
    if x.shape[-1] != H:
        raise ValueError(f"last dimension of x is {x.shape[-1]}, expected {H}")
    code = _X_DTYPES.get(x.dtype)
    if code is None:
        raise TypeError(f"x must be float16, bfloat16 or float32, got {x.dtype}")
    if x.dim() == 2 and x.is_contiguous():
        return x, code
    return x.reshape(-1, H).contiguous(), code


def _logits_arg(logits: torch.Tensor, E: int) -> torch.Tensor:
    """Router logits as contiguous float32 rows [T, E] (a view when they already are)."""
    if logits.dtype == torch.float32 and logits.dim() == 2 and logits.shape[1] == E and logits.is_contiguous():
        return logits
    return logits.reshape(-1, E).to(torch.float32).contiguous()


def _check_x(x: torch.Tensor, H: int) -> torch.Tensor:
    if x.shape[-1] != H:
        raise ValueError(f"last dimension of x is {x.shape[-1]}, expected {H}")
    if x.dtype == torch.bfloat16:
        x = x.to(torch.float16)
    if x.dtype != torch.float16:
        raise TypeError(f"x must be float16 or bfloat16, got {x.dtype}")
    return x.reshape(-1, H).contiguous()


class QuantizedSwitchGLU:
    """``switch_mlp(x, indices)``: per-(token, k) SwiGLU expert outputs ``[..., K, H]`` (fp16).

    Same contract as the reference's ``_CPUSwitchGLU.__call__`` (kandiga/engine.py:670-739).
    """

    def __init__(self, experts: QuantizedExperts):
        self.experts = experts

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        E = self.experts
        _on_device(x, E.device, "x")
        _on_device(indices, E.device, "indices")
        K = indices.shape[-1]
        if K != E.shape.top_k:
            raise ValueError(f"indices have {K} experts per token, layer was built for top_k={E.shape.top_k}")
        xf, xdt = _x_arg(x, E.shape.hidden)
        if indices.dtype == torch.int32 and indices.dim() == 2 and indices.is_contiguous():
            idx = indices
        else:
            idx = indices.reshape(-1, K).to(torch.int32).contiguous()
        T = xf.shape[0]
        if idx.shape[0] != T:
            raise ValueError("x and indices disagree on the number of tokens")
        y = torch.empty((T, K, E.shape.hidden), dtype=torch.float16, device=E.device)
        ws = E.workspace(T)
        _capi.check(_capi.lib().kmoe_expert_mlp_x(E._handle, xf.data_ptr(), xdt, idx.data_ptr(), T, y.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), _stream(E.device)), "kmoe_expert_mlp_x")
        return y.reshape(*indices.shape, E.shape.hidden)


class SparseMoeBlock:
    """Routed MoE block: route(logits) -> switch_mlp -> weighted combine (+ shared expert)."""

    def __init__(self, experts: QuantizedExperts):
        self.experts = experts
        self.switch_mlp = QuantizedSwitchGLU(experts)

    @property
    def top_k(self) -> int:
        return self.experts.shape.top_k

    def __call__(self, x: torch.Tensor, logits: torch.Tensor, return_routing: bool = False,
                 out_dtype: torch.dtype = torch.float16):
        """``x`` float16, bfloat16 or float32 (taken natively; a layer with the dense fp16 shared
        expert takes float16 only); ``out_dtype`` float16 (default) or float32 (the combine result
        before fp16 rounding)."""
        E = self.experts
        if out_dtype not in (torch.float16, torch.float32):
            raise TypeError("out_dtype must be torch.float16 or torch.float32")
        _on_device(x, E.device, "x")
        _on_device(logits, E.device, "logits")
        lead = x.shape[:-1]
        xf, xdt = _x_arg(x, E.shape.hidden)
        if xdt != _capi.X_F16 and E.shared:
            raise TypeError("a layer with the dense fp16 shared expert takes float16 x only")
        lg = _logits_arg(logits, E.shape.num_experts)
        T = xf.shape[0]
        if lg.shape[0] != T:
            raise ValueError("x and logits disagree on the number of tokens")
        out = torch.empty((T, E.shape.hidden), dtype=out_dtype, device=E.device)
        idx = w = None
        if return_routing:
            idx = torch.empty((T, E.shape.top_k), dtype=torch.int32, device=E.device)
            w = torch.empty((T, E.shape.top_k), dtype=torch.float32, device=E.device)
        ws = E.workspace(T)
        odt = _capi.OUT_F32 if out_dtype == torch.float32 else _capi.OUT_F16
        _capi.check(_capi.lib().kmoe_forward_x(E._handle, xf.data_ptr(), xdt, lg.data_ptr(), T, out.data_ptr(), odt,
                                               _ptr(idx), _ptr(w), ws.data_ptr(), ws.numel(), _stream(E.device)),
                    "kmoe_forward_x")
        out = out.reshape(*lead, E.shape.hidden)
        if return_routing:
            return out, idx.reshape(*lead, -1), w.reshape(*lead, -1)
        return out


class MoEBlock:
    """The whole MoE block ``mlp(x)`` of a Qwen-style decoder layer, one C call (kmoe_block_forward):

    router projection over the quantized ``mlp.gate`` -> softmax top-K -> renorm -> the routed
    experts -> weighted combine, plus the quantized shared expert ``mlp.shared_expert`` gated by
    ``sigmoid(mlp.shared_expert_gate . x)`` and an optional residual:
    ``out = (residual + sum_k w_k y_k) + fp16(shared(x)) * sigmoid(gate . x)``
    (kandiga/metal/moe_block.metal:194-584; the bakan_forward_moe_block step,
    kandiga/metal/bakan_forward.h:111-140).

    ``router``, ``shared`` and ``shared_gate`` hold device tensors: router ``{"w","s","b"}``
    ``[E, H]``, shared ``{"gate","up","down"}`` each a ``{"w","s","b"}`` dict, shared_gate
    ``{"w","s","b"}`` ``[1, H]`` (MLX layout, ``bits``-bit codes, ``scale_dtype`` scales).
    """

    def __init__(self, experts: QuantizedExperts, router: dict, shared: dict | None = None,
                 shared_gate: dict | None = None, bits: int = 4, scale_dtype: str = "bf16"):
        if experts.shared:
            raise ValueError("the routed experts of a block must not carry a dense shared expert")
        self.experts = experts
        self.bits = bits
        self.scale_dtype = scale_dtype
        dev = experts.device
        keep = []

        def qp(d: dict, rows: int) -> _capi.QProjDesc:
            q = _capi.QProjDesc()
            t = {k: d[k].to(dev).contiguous() for k in ("w", "s", "b")}
            for k, v in t.items():
                _on_device(v, dev, f"block projection {k}")
            if t["w"].shape[0] != rows:
                raise ValueError(f"projection has {t['w'].shape[0]} rows, expected {rows}")
            keep.extend(t.values())
            q.weight, q.scales, q.biases = t["w"].data_ptr(), t["s"].data_ptr(), t["b"].data_ptr()
            return q

        H, E = experts.shape.hidden, experts.shape.num_experts
        d = _capi.BlockDesc()
        d.routed = experts._handle.value
        d.router = qp(router, E)
        self.shared_intermediate = 0
        if shared:
            Is = shared["gate"]["w"].shape[0]
            self.shared_intermediate = Is
            d.shared_gate_proj = qp(shared["gate"], Is)
            d.shared_up_proj = qp(shared["up"], Is)
            d.shared_down_proj = qp(shared["down"], H)
            d.shared_intermediate = Is
        if shared_gate:
            d.shared_expert_gate = qp(shared_gate, 1)
        d.bits = bits
        d.scale_dtype = _capi.SCALE_BF16 if scale_dtype == "bf16" else _capi.SCALE_F16
        h = ctypes.c_void_p()
        _capi.check(_capi.lib().kmoe_block_create(ctypes.byref(d), ctypes.byref(h)), "kmoe_block_create")
        self._handle = h
        self._keep = keep
        self._ws = None
        self._ws_tokens = -1
        self._ws_captured = False
        self._ws_retired = []

    @classmethod
    def from_arrays(cls, experts: QuantizedExperts, block: dict, bits: int = 4, scale_dtype: str = "bf16") -> "MoEBlock":
        """From the ``blk_*`` arrays of :func:`synth.make_block` (numpy or torch)."""
        dev = experts.device

        def t(a):
            if isinstance(a, torch.Tensor):
                return a.to(dev)
            return torch.from_numpy(a.view(a.dtype.str.replace("u", "i"))).to(dev)

        def proj(name):
            return {k: t(block[f"{name}_{k}"]) for k in ("w", "s", "b")}

        shared = None
        if "blk_shared_gate_w" in block:
            shared = {p: proj(f"blk_shared_{p}") for p in ("gate", "up", "down")}
        gate = proj("blk_sgate") if "blk_sgate_w" in block else None
        return cls(experts, proj("blk_router"), shared, gate, bits, scale_dtype)

    def workspace(self, tokens: int) -> torch.Tensor:
        if tokens > self._ws_tokens:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"block workspace for {tokens} tokens was not reserved before graph capture")
            n = ctypes.c_size_t()
            _capi.check(_capi.lib().kmoe_block_workspace_size(self._handle, int(tokens), ctypes.byref(n)),
                        "kmoe_block_workspace_size")
            if self._ws is not None and self._ws_captured:
                self._ws_retired.append(self._ws)
            self._ws = torch.zeros(max(n.value, 256), dtype=torch.uint8, device=self.experts.device)
            self._ws_tokens = tokens
            self._ws_captured = False
        if torch.cuda.is_current_stream_capturing():
            self._ws_captured = True
        return self._ws

    def __call__(self, x: torch.Tensor, residual: torch.Tensor | None = None, return_routing: bool = False,
                 out_dtype: torch.dtype = torch.float16):
        E = self.experts
        if out_dtype not in (torch.float16, torch.float32):
            raise TypeError("out_dtype must be torch.float16 or torch.float32")
        _on_device(x, E.device, "x")
        lead = x.shape[:-1]
        xf = _check_x(x, E.shape.hidden)
        T = xf.shape[0]
        res = None
        if residual is not None:
            _on_device(residual, E.device, "residual")
            res = _check_x(residual, E.shape.hidden)
            if res.shape[0] != T:
                raise ValueError("x and residual disagree on the number of tokens")
        out = torch.empty((T, E.shape.hidden), dtype=out_dtype, device=E.device)
        idx = w = lg = None
        if return_routing:
            idx = torch.empty((T, E.shape.top_k), dtype=torch.int32, device=E.device)
            w = torch.empty((T, E.shape.top_k), dtype=torch.float32, device=E.device)
            lg = torch.empty((T, E.shape.num_experts), dtype=torch.float32, device=E.device)
        ws = self.workspace(T)
        odt = _capi.OUT_F32 if out_dtype == torch.float32 else _capi.OUT_F16
        _capi.check(_capi.lib().kmoe_block_forward(self._handle, xf.data_ptr(), _ptr(res), T, out.data_ptr(), odt,
                                                   _ptr(idx), _ptr(w), _ptr(lg), ws.data_ptr(), ws.numel(),
                                                   _stream(E.device)), "kmoe_block_forward")
        out = out.reshape(*lead, E.shape.hidden)
        if return_routing:
            return out, idx.reshape(*lead, -1), w.reshape(*lead, -1), lg.reshape(*lead, -1)
        return out

    def __del__(self):
        h = getattr(self, "_handle", None)
        lib = getattr(_capi, "_lib", None) if _capi is not None else None  # None at interpreter exit
        if h is not None and lib is not None:
            lib.kmoe_block_destroy(h)
            self._handle = None


def route(logits: torch.Tensor, top_k: int):
    """Top-K experts per token (ties -> lower index) and renormalised softmax weights."""
    _on_device(logits, None, "logits")
    lg = logits.to(torch.float32).contiguous()
    T, E = lg.reshape(-1, lg.shape[-1]).shape
    idx = torch.empty((T, top_k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=lg.device)
    _capi.check(_capi.lib().kmoe_route(lg.data_ptr(), T, E, top_k, idx.data_ptr(), w.data_ptr(), _stream()),
                "kmoe_route")
    lead = logits.shape[:-1]
    return idx.reshape(*lead, top_k), w.reshape(*lead, top_k)


def permute(idx: torch.Tensor, num_experts: int) -> dict:
    """Stable token->expert grouping: perm, counts, offsets, unique experts (engine.py:407-418)."""
    _on_device(idx, None, "idx")
    K = idx.shape[-1]
    ii = idx.reshape(-1, K).to(torch.int32).contiguous()
    T = ii.shape[0]
    dev = ii.device
    L = _capi.lib()
    n = ctypes.c_size_t()
    _capi.check(L.kmoe_permute_workspace_size(T, K, num_experts, ctypes.byref(n)), "kmoe_permute_workspace_size")
    ws = torch.zeros(max(n.value, 256), dtype=torch.uint8, device=dev)
    perm = torch.empty(T * K, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    unique = torch.empty(num_experts, dtype=torch.int32, device=dev)
    nu = torch.empty(1, dtype=torch.int32, device=dev)
    _capi.check(L.kmoe_permute(ii.data_ptr(), T, K, num_experts, perm.data_ptr(), counts.data_ptr(),
                               offsets.data_ptr(), unique.data_ptr(), nu.data_ptr(), ws.data_ptr(), ws.numel(),
                               _stream()), "kmoe_permute")
    f = ctypes.c_int32()
    _capi.check(L.kmoe_device_status(ws.data_ptr(), ws.numel(), ctypes.byref(f), _stream()), "kmoe_device_status")
    if f.value & _capi.DEVERR_BAD_EXPERT:
        raise _capi.KmoeError(_capi.ERR_DEVICE, "kmoe_permute: expert index out of range")
    u = int(nu.item())
    return dict(perm=perm, s_tok=perm // K, s_k=perm % K, counts=counts, offsets=offsets,
                unique=unique[:u], num_unique=u)


def combine(y: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """``out[t] = sum_k w[t,k] * y[t,k]`` (fp32 accumulate, fp16 out) for y ``[..., K, H]`` fp16."""
    _on_device(y, None, "y")
    _on_device(weights, y.device, "weights")
    K, H = y.shape[-2], y.shape[-1]
    yy = y.reshape(-1, K, H).to(torch.float16).contiguous()
    ww = weights.reshape(-1, K).to(torch.float32).contiguous()
    T = yy.shape[0]
    out = torch.empty((T, H), dtype=torch.float16, device=y.device)
    _capi.check(_capi.lib().kmoe_combine(yy.data_ptr(), ww.data_ptr(), T, K, H, out.data_ptr(), _stream()),
                "kmoe_combine")
    return out.reshape(*y.shape[:-2], H)


class profile_kernels:
    """Time every kernel the library launches from this thread inside the ``with`` block.

    Each launch is bracketed by a HIP event pair on its stream (kmoe_profile_begin/end), so
    use it around eager calls, not graph capture.  ``result`` maps kernel name to a dict of
    launches, total_ms, mean_ms, min_ms, max_ms.
    """

    def __init__(self, max_launches: int = 4096):
        self.max_launches = int(max_launches)
        self.result: dict = {}

    def __enter__(self) -> "profile_kernels":
        _capi.check(_capi.lib().kmoe_profile_begin(self.max_launches), "kmoe_profile_begin")
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        buf = (_capi.KernelTime * 64)()
        n = ctypes.c_int32()
        rc = _capi.lib().kmoe_profile_end(buf, 64, ctypes.byref(n))
        if exc_type is None:
            _capi.check(rc, "kmoe_profile_end")
        for i in range(min(n.value, 64)):
            t = buf[i]
            self.result[t.name.decode()] = dict(launches=t.launches, total_ms=t.total_ms,
                                                mean_ms=t.total_ms / max(t.launches, 1), min_ms=t.min_ms,
                                                max_ms=t.max_ms)

