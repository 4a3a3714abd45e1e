"""MoE layer over PyTorch device buffers, driven through the C ABI.

Mirrors the Swift block API of FFAI (Sources/FFAI/Models/MoELayer.swift:
MoEGatingMode :71, MoERouter :97-124, MoELayer.init :440-498, decode :530,
decodeMany :677) on top of libmoehip.so. PyTorch only provides device memory
and the stream; every computation is a libmoehip.so kernel.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import LayerDesc, LayerTrace, QProj, check

_DT = {torch.float32: _lib.MOE_F32, torch.float16: _lib.MOE_F16, torch.bfloat16: _lib.MOE_BF16}


def moe_dtype(t: torch.dtype) -> int:
    return _DT[t]


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class MoEGatingMode:
    """MoELayer.swift:71-78, plus the NemotronH sigmoid router
    (NemotronHText.swift:838-868)."""
    softmaxThenTopK = _lib.MOE_SOFTMAX_THEN_TOPK
    topKThenSoftmax = _lib.MOE_TOPK_THEN_SOFTMAX
    sigmoidTopK = _lib.MOE_SIGMOID_TOPK


@dataclass
class MoERouter:
    """MoERouter (MoELayer.swift:97-124): the gating configuration, with the
    routing scales of the NemotronH (routed_scaling_factor,
    NemotronHText.swift:867) and Gemma 4 (hidden^-0.5 logit scale and
    per_expert_scale, Gemma4Text.swift:938-950) routers."""
    nExperts: int
    topK: int
    gatingMode: int = MoEGatingMode.softmaxThenTopK
    normTopKProb: bool = True
    expertBias: Optional[torch.Tensor] = None  # [nExperts] float32 on device
    logitScale: float = 1.0
    routedScale: float = 1.0
    expertScale: Optional[torch.Tensor] = None  # [nExperts] float32 on device

    def __post_init__(self):
        if self.nExperts <= 0:
            raise ValueError("MoERouter: nExperts must be positive")
        if not (0 < self.topK <= self.nExperts):
            raise ValueError(f"MoERouter: topK ({self.topK}) must be in 1...nExperts ({self.nExperts})")
        if self.expertBias is not None and self.expertBias.numel() != self.nExperts:
            raise ValueError("MoERouter: expertBias must have nExperts entries")
        if self.expertScale is not None and self.expertScale.numel() != self.nExperts:
            raise ValueError("MoERouter: expertScale must have nExperts entries")


@dataclass
class StackedExperts:
    """One stacked mlx-affine projection: weight [E, N, K*bits/32] (int32
    storage of u32 words), scales/biases [E, N, K/gs], optional per-expert
    output bias [E, N] in the activation dtype."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    bits: int
    group_size: int
    out_bias: Optional[torch.Tensor] = None

    @property
    def n_experts(self) -> int:
        return self.weight.shape[0]

    @property
    def n(self) -> int:
        return self.weight.shape[1]

    @property
    def k(self) -> int:
        return self.scales.shape[-1] * self.group_size

    def struct(self) -> QProj:
        return QProj(self.weight.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr(),
                     None if self.out_bias is None else self.out_bias.data_ptr(),
                     self.bits, self.group_size, moe_dtype(self.scales.dtype),
                     self.n, self.k, self.n_experts)


class MoELayer:
    """MoE feed-forward layer (router -> dispatch -> grouped expert products
    -> combine [+ shared expert]) on one GPU. With MOE_ACT_RELU2 the experts
    have no gate projection: pass gate=None (and None as the shared gate).
    The router weight and the shared expert's sigmoid gate are either dense
    tensors ([E, hidden], [1, hidden]) or, as loadLinear returns them for a
    quantised checkpoint (Layers.swift:371-400), one-expert StackedExperts
    ([1, E, hidden], [1, 1, hidden])."""

    def __init__(self, *, router_weight, router: MoERouter,
                 gate: Optional[StackedExperts], up: StackedExperts, down: StackedExperts,
                 hidden: int, act_dtype: torch.dtype,
                 router_bias: Optional[torch.Tensor] = None,
                 activation: int = _lib.MOE_ACT_SWIGLU, alpha: float = 1.702, limit: float = 7.0,
                 shared: Optional[tuple] = None, shared_gate_weight: Optional[torch.Tensor] = None):
        self.router_weight, self.router, self.router_bias = router_weight, router, router_bias
        self.gate, self.up, self.down = gate, up, down
        self.hidden, self.act_dtype = hidden, act_dtype
        self.activation, self.alpha, self.limit = activation, alpha, limit
        self.shared, self.shared_gate_weight = shared, shared_gate_weight
        self._desc = self._build_desc()
        check(_lib.load().moe_validate_layer(C.byref(self._desc)))
        self._ws = None

    def _build_desc(self) -> LayerDesc:
        d = LayerDesc()
        d.hidden, d.n_experts, d.top_k = self.hidden, self.router.nExperts, self.router.topK
        d.intermediate = self.up.n
        d.act_dtype = moe_dtype(self.act_dtype)
        if isinstance(self.router_weight, StackedExperts):
            d.router_q = self.router_weight.struct()
            d.router_dtype = d.act_dtype
        else:
            d.router_weight = self.router_weight.data_ptr()
            d.router_dtype = moe_dtype(self.router_weight.dtype)
        d.router_bias = None if self.router_bias is None else self.router_bias.data_ptr()
        d.gating, d.norm_topk_prob = self.router.gatingMode, int(bool(self.router.normTopKProb))
        d.expert_bias = None if self.router.expertBias is None else self.router.expertBias.data_ptr()
        d.gate = QProj() if self.gate is None else self.gate.struct()
        d.up, d.down = self.up.struct(), self.down.struct()
        d.activation, d.act_alpha, d.act_limit = self.activation, self.alpha, self.limit
        if self.shared is not None:
            d.has_shared = 1
            d.shared_gate, d.shared_up, d.shared_down = (
                QProj() if p is None else p.struct() for p in self.shared)
            sgw = self.shared_gate_weight
            if isinstance(sgw, StackedExperts):
                d.shared_gate_q = sgw.struct()
            else:
                d.shared_gate_weight = None if sgw is None else sgw.data_ptr()
        r = self.router
        d.logit_scale, d.routed_scale = r.logitScale, r.routedScale
        d.expert_scale = None if r.expertScale is None else r.expertScale.data_ptr()
        return d

    @property
    def desc(self) -> LayerDesc:
        return self._desc

    @property
    def device(self) -> torch.device:
        return self.up.weight.device

    def parameters(self):
        """(name, tensor) pairs in the order and with the names of
        MoELayer.parameters() (MoELayer.swift:500-522): the router, then each
        expert's projections as views of the stacked tensors, then the
        shared expert; plus the sigmoid gate of the shared expert under its
        checkpoint name (Qwen3xText.swift:660-661)."""
        out = []

        def linear(prefix, w):  # a dense weight or a one-expert quantised stack
            if isinstance(w, StackedExperts):
                return [(f"{prefix}.weight", w.weight[0]), (f"{prefix}.scales", w.scales[0]),
                        (f"{prefix}.biases", w.biases[0])]
            return [(f"{prefix}.weight", w)]

        out += linear("gate", self.router_weight)
        if self.router_bias is not None:
            out.append(("gate.bias", self.router_bias))

        def proj(prefix, p):
            if p is None:
                return []
            items = [(f"{prefix}.weight", p.weight), (f"{prefix}.scales", p.scales),
                     (f"{prefix}.biases", p.biases)]
            if p.out_bias is not None:
                items.append((f"{prefix}.bias", p.out_bias))
            return items

        for name, p in (("gate_proj", self.gate), ("up_proj", self.up), ("down_proj", self.down)):
            if p is None:
                continue
            for e in range(p.n_experts):
                for n, t in proj(f"experts.{e}.{name}", p):
                    out.append((n, t[e]))
        if self.shared is not None:
            for name, p in zip(("gate_proj", "up_proj", "down_proj"), self.shared):
                if p is not None:
                    out += [(n, t[0]) for n, t in proj(f"shared_expert.{name}", p)]
            if self.shared_gate_weight is not None:
                out += linear("shared_expert_gate", self.shared_gate_weight)
        return out

    def paths(self, T: int) -> dict:
        """The kernels a call of T rows runs per stage (moe_layer_path):
        'decode1', 'gemv', 'gemv_mma', 'gemm' or 'none'."""
        p = _lib.LayerPaths()
        check(_lib.load().moe_layer_path(C.byref(self._desc), T, C.byref(p)))
        return p.names()

    def _check_rows(self, name: str, t: Optional[torch.Tensor], T: Optional[int] = None):
        """Rows handed to the C ABI: [T, hidden], the layer's activation dtype,
        contiguous, on the layer's device (the kernels read and write them
        through raw pointers)."""
        if t is None:
            return
        dev = self.device
        if t.dim() != 2 or t.shape[1] != self.hidden or (T is not None and t.shape[0] != T):
            want = f"[{'T' if T is None else T}, {self.hidden}]"
            raise ValueError(f"MoELayer: {name} must be {want}, got {list(t.shape)}")
        if t.dtype != self.act_dtype:
            raise ValueError(f"MoELayer: {name} dtype {t.dtype} is not the layer's {self.act_dtype}")
        if not t.is_contiguous():
            raise ValueError(f"MoELayer: {name} must be contiguous")
        if t.device != dev:
            raise ValueError(f"MoELayer: {name} is on {t.device}, the layer on {dev}")

    def workspace_bytes(self, T: int) -> int:
        return _lib.load().moe_layer_workspace_bytes(C.byref(self._desc), T)

    def workspace(self, T: int) -> torch.Tensor:
        need = self.workspace_bytes(T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, trace: bool = False,
                stream=None, router_x: Optional[torch.Tensor] = None):
        """decodeMany: x [T, hidden] -> [T, hidden]. router_x (default x) is
        the router's input, for Gemma 4 whose router and experts read
        differently normalised rows. With trace=True also returns the
        routing (logits, topk_idx, topk_weight, perm, offsets)."""
        self._check_rows("x", x)
        T = x.shape[0]
        if T <= 0:
            raise ValueError("MoELayer.decodeMany: T must be positive")
        self._check_rows("router_x", router_x, T)
        if out is None:
            out = torch.empty_like(x)
        self._check_rows("out", out, T)
        ws = self.workspace(T)
        tr = None
        tensors = None
        if trace:
            dev = x.device
            E, k = self.router.nExperts, self.router.topK
            tensors = dict(
                logits=torch.empty(T, E, dtype=self.act_dtype, device=dev),
                topk_idx=torch.empty(T, k, dtype=torch.int32, device=dev),
                topk_weight=torch.empty(T, k, dtype=torch.float32, device=dev),
                perm=torch.empty(T * k, dtype=torch.int32, device=dev),
                offsets=torch.empty(E + 1, dtype=torch.int32, device=dev))
            tr = LayerTrace(*(tensors[n].data_ptr() for n in
                              ("logits", "topk_idx", "topk_weight", "perm", "offsets")))
        check(_lib.load().moe_layer_forward_routed(C.byref(self._desc), _ptr(x), _ptr(router_x),
                                                   T, _ptr(out), _ptr(ws), ws.numel(),
                                                   C.byref(tr) if tr is not None else None,
                                                   _stream(stream)))
        return (out, tensors) if trace else out

    def forward_residual(self, h: torch.Tensor, mixer_out: torch.Tensor, norm_weight: torch.Tensor,
                         eps: float, out: Optional[torch.Tensor] = None,
                         residual_out: Optional[torch.Tensor] = None, stream=None):
        """The block between the decoder steps (Qwen3xText.swift:2640-2670,
        1015-1035): r = h + mixer_out, y = r + MoE(rmsnorm(r) * norm_weight).
        Returns y; residual_out (optional) receives r."""
        self._check_rows("h", h)
        T = h.shape[0]
        if T <= 0:
            raise ValueError("MoELayer.decodeMany: T must be positive")
        self._check_rows("mixer_out", mixer_out, T)
        if (norm_weight.dim() != 1 or norm_weight.numel() != self.hidden
                or norm_weight.dtype != self.act_dtype or not norm_weight.is_contiguous()
                or norm_weight.device != h.device):
            raise ValueError("MoELayer.forward_residual: norm_weight must be a contiguous "
                             f"[{self.hidden}] vector of the layer's dtype on its device")
        if out is None:
            out = torch.empty_like(h)
        self._check_rows("out", out, T)
        self._check_rows("residual_out", residual_out, T)
        ws = self.workspace(T)
        check(_lib.load().moe_layer_forward_residual(
            C.byref(self._desc), _ptr(h), _ptr(mixer_out), _ptr(norm_weight), float(eps), T,
            _ptr(out), _ptr(residual_out), _ptr(ws), ws.numel(), None, _stream(stream)))
        return out

    # Swift-API names
    def decode(self, h: torch.Tensor, stream=None) -> torch.Tensor:
        return self.forward(h.reshape(1, -1), stream=stream).reshape(-1)

    def decodeMany(self, hFlat: torch.Tensor, t: int, stream=None) -> torch.Tensor:
        return self.forward(hFlat.reshape(t, self.hidden), stream=stream).reshape(-1)
