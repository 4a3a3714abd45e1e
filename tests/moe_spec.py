"""Synthetic MoE layers for the parity tests and the
glue that hands the same numpy arrays to the CPU oracle and to libmoehip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

import oracle as orc

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16


def store(a, dt):
    """float32 values -> storage array of dt (RNE)."""
    return orc.from_f32(np.asarray(a, dtype=np.float32), dt)


def load(a, dt):
    return orc.to_f32(a, dt)


def gen_qproj(rng, E, N, K, bits, gs, sb_dt, s_range=(0.005, 0.02), b_range=(-0.1, 0.1),
              out_bias_dt=None):
    """Uniform codes (random u32 words are uniform codes at every width),
    scales ~U(s_range), biases ~U(b_range) stored in sb_dt."""
    words = K * bits // 32
    w = rng.integers(0, 2**32, size=(E, N, words), dtype=np.uint64).astype(np.uint32)
    s = store(rng.uniform(*s_range, size=(E, N, K // gs)), sb_dt)
    b = store(rng.uniform(*b_range, size=(E, N, K // gs)), sb_dt)
    ob = None
    if out_bias_dt is not None:
        ob = store(rng.normal(0, 0.1, size=(E, N)), out_bias_dt)
    return orc.QProj(w, s, b, bits, gs, sb_dt, out_bias=ob)


def affine_quantize(W, bits, gs, sb_dt):
    """mlx's affine quantiser on a dense [N, K] float matrix, per group of gs
    values: scale = (max - min) / (2^bits - 1), bias = min, code = round((w -
    bias) / scale) clamped to the code range; scale and bias stored in sb_dt.
    Returns a one-expert QProj [1, N, K] (the layout loadLinear gives a
    quantised router or shared-expert gate)."""
    W = np.asarray(W, dtype=np.float64)
    N, K = W.shape
    g = W.reshape(N, K // gs, gs)
    lo, hi = g.min(axis=2), g.max(axis=2)
    scale = (hi - lo) / (2 ** bits - 1)
    scale = np.where(scale == 0, 1.0, scale)
    s_st, b_st = store(scale, sb_dt), store(lo, sb_dt)
    s_f, b_f = load(s_st, sb_dt).astype(np.float64), load(b_st, sb_dt).astype(np.float64)
    q = np.clip(np.rint((g - b_f[..., None]) / s_f[..., None]), 0, 2 ** bits - 1).astype(np.uint8)
    w = orc.pack_codes(q.reshape(N, K), bits).reshape(1, N, K * bits // 32)
    return orc.QProj(w, s_st.reshape(1, N, K // gs), b_st.reshape(1, N, K // gs), bits, gs, sb_dt)


def with_quantised_router(spec, bits=None, shared_gate_bits=None, gs=64, sb_dt=None):
    """spec with its dense router (and/or shared-expert gate) replaced by the
    mlx affine quantisation of the same weights."""
    import copy
    out = copy.copy(spec)
    sb = spec.act_dt if sb_dt is None else sb_dt
    if bits is not None:
        out.router_weight = affine_quantize(load(spec.router_weight, spec.router_dt), bits, gs, sb)
        out.name = f"{spec.name}+router{bits}b"
    if shared_gate_bits is not None:
        out.shared_gate_weight = affine_quantize(load(spec.shared_gate_weight, spec.router_dt),
                                                 shared_gate_bits, gs, sb)
        out.name = f"{out.name}+sgate{shared_gate_bits}b"
    return out


@dataclass
class LayerSpec:
    hidden: int
    n_experts: int
    top_k: int
    intermediate: int
    act_dt: int
    router_weight: np.ndarray
    router_dt: int
    gate: Optional[orc.QProj]  # None for squared-ReLU experts
    up: orc.QProj
    down: orc.QProj
    gating: int = orc.SOFTMAX_THEN_TOPK
    norm_topk: bool = True
    router_bias: Optional[np.ndarray] = None
    expert_bias: Optional[np.ndarray] = None
    activation: int = orc.ACT_SWIGLU
    alpha: float = 1.702
    limit: float = 7.0
    shared: Optional[tuple] = None
    shared_gate_weight: Optional[np.ndarray] = None
    logit_scale: float = 1.0
    routed_scale: float = 1.0
    expert_scale: Optional[np.ndarray] = None  # [E] float32
    split_router_input: bool = False  # the router reads its own rows (Gemma 4)
    name: str = ""
    meta: dict = field(default_factory=dict)

    # ---- CPU oracle view -------------------------------------------------
    def oracle_struct(self) -> orc.OrLayer:
        L = orc.OrLayer()
        L.hidden, L.n_experts, L.top_k = self.hidden, self.n_experts, self.top_k
        L.intermediate, L.act_dt = self.intermediate, self.act_dt
        if isinstance(self.router_weight, orc.QProj):
            L.router_q = self.router_weight.c()
        else:
            L.router_weight = self.router_weight.ctypes.data
        L.router_dt = self.router_dt
        L.router_bias = None if self.router_bias is None else self.router_bias.ctypes.data
        L.gating, L.norm_topk = self.gating, int(self.norm_topk)
        L.expert_bias = None if self.expert_bias is None else self.expert_bias.ctypes.data
        L.gate = orc.OrQProj() if self.gate is None else self.gate.c()
        L.up, L.down = self.up.c(), self.down.c()
        L.activation, L.alpha, L.limit = self.activation, self.alpha, self.limit
        if self.shared is not None:
            L.has_shared = 1
            L.shared_gate, L.shared_up, L.shared_down = (
                orc.OrQProj() if p is None else p.c() for p in self.shared)
            sgw = self.shared_gate_weight
            if isinstance(sgw, orc.QProj):
                L.shared_gate_q = sgw.c()
            else:
                L.shared_gate_weight = None if sgw is None else sgw.ctypes.data
        L.logit_scale, L.routed_scale = self.logit_scale, self.routed_scale
        L.expert_scale = None if self.expert_scale is None else self.expert_scale.ctypes.data
        self._keep = L
        return L

    # ---- device view (GPU tests) ----------------------------------------
    def device(self):
        import torch
        from ffai_amd import layer as fl

        def T(a):
            if a is None:
                return None
            if a.dtype == np.uint16:
                return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
            if a.dtype == np.uint32:
                return torch.from_numpy(a.view(np.int32)).cuda()
            return torch.from_numpy(np.ascontiguousarray(a)).cuda()

        def P(q):
            if q is None:
                return None
            return fl.StackedExperts(T(q.weight), T(q.scales), T(q.biases), q.bits, q.gs,
                                     out_bias=T(q.out_bias))

        def W(a):  # dense router / gate weight or a one-expert quantised stack
            return P(a) if isinstance(a, orc.QProj) else T(a)

        act = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[self.act_dt]
        router = fl.MoERouter(self.n_experts, self.top_k, self.gating, self.norm_topk,
                              T(self.expert_bias), self.logit_scale, self.routed_scale,
                              T(self.expert_scale))
        shared = None if self.shared is None else tuple(P(q) for q in self.shared)
        return fl.MoELayer(router_weight=W(self.router_weight), router=router, gate=P(self.gate),
                           up=P(self.up), down=P(self.down), hidden=self.hidden, act_dtype=act,
                           router_bias=T(self.router_bias), activation=self.activation,
                           alpha=self.alpha, limit=self.limit, shared=shared,
                           shared_gate_weight=W(self.shared_gate_weight))

    def oracle_logits(self, rx):
        """The router logits the oracle computes for router input rows rx."""
        if isinstance(self.router_weight, orc.QProj):
            return orc.router_logits_q(rx, self.act_dt, self.router_weight, self.router_bias)
        return orc.router_logits(rx, self.act_dt, self.router_weight, self.router_dt,
                                 self.router_bias)

    def logits_tolerance(self, ref):
        """Allowed |GPU - oracle| per logit: two storage ulps (a bias add rounds
        twice); a quantised router also differs in fp32 summation order over
        terms much larger than a small logit, so it gets 1e-4 of its row's
        largest logit on top."""
        ulp = np.abs(ref) * (2.0 ** -7 if self.act_dt == BF16 else 2.0 ** -10 if self.act_dt == F16
                             else 2.0 ** -20) + 1e-6
        tol = 2.02 * ulp
        if isinstance(self.router_weight, orc.QProj):
            tol = tol + 1e-4 * (1.0 + np.abs(ref).max(axis=1, keepdims=True))
        return tol

    def x(self, T, seed=0):
        rng = np.random.default_rng(seed + 1000)
        return store(rng.normal(0, 1, size=(T, self.hidden)), self.act_dt)

    def router_x(self, T, seed=0):
        """The router's own input rows when split_router_input, else None."""
        if not self.split_router_input:
            return None
        rng = np.random.default_rng(seed + 5000)
        return store(rng.normal(0, 1, size=(T, self.hidden)), self.act_dt)


def to_torch(a):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_numpy_f32(t):
    import torch
    return t.detach().float().cpu().numpy() if t.dtype != torch.float32 else t.detach().cpu().numpy()


# ---------------------------------------------------------------- configs --

def cfg_tiny(seed=0, act_dt=F16):
    """hidden=256, 8 experts, top-2, I=512, 4-bit gs64, f16."""
    rng = np.random.default_rng(seed)
    H, E, k, I = 256, 8, 2, 512
    return LayerSpec(H, E, k, I, act_dt,
                     router_weight=store(rng.normal(0, 0.02, size=(E, H)), F16), router_dt=F16,
                     gate=gen_qproj(rng, E, I, H, 4, 64, F16), up=gen_qproj(rng, E, I, H, 4, 64, F16),
                     down=gen_qproj(rng, E, H, I, 4, 64, F16), name="tiny")


def cfg_gptoss(seed=0, n_experts=32, hidden=2880, inter=2880, expert_bias=False):
    """GPT-OSS-20B-shaped decode layer (4-bit gs64, bf16)."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, 4, inter
    ob = BF16 if expert_bias else None
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), BF16),
                     router_dt=BF16, router_bias=store(rng.normal(0, 0.1, size=E), BF16),
                     gating=orc.TOPK_THEN_SOFTMAX,
                     gate=gen_qproj(rng, E, I, H, 4, 64, BF16, out_bias_dt=ob),
                     up=gen_qproj(rng, E, I, H, 4, 64, BF16, out_bias_dt=ob),
                     down=gen_qproj(rng, E, H, I, 4, 64, BF16, out_bias_dt=ob),
                     activation=orc.ACT_GPTOSS, alpha=1.702, limit=7.0, name="gptoss")


def cfg_qwen3(seed=0, n_experts=128, hidden=2048, inter=768, router_bias=None):
    """configs[2]/[3]: Qwen3-MoE shape, 4-bit gs64, fp16 scales, bf16 acts."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, 8, inter
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), BF16),
                     router_dt=BF16,
                     router_bias=None if router_bias is None else store(router_bias, BF16),
                     gate=gen_qproj(rng, E, I, H, 4, 64, F16), up=gen_qproj(rng, E, I, H, 4, 64, F16),
                     down=gen_qproj(rng, E, H, I, 4, 64, F16), name="qwen3")


# Router-bias strength for configs[3]: beta * log p with p Zipf(1.1) gives a
# hottest-expert load of about 10x the median at 0.33 (4096 tokens, 128
# experts, top-8: max / median 9.9-10.0 over two seeds; beta = 1.0 gives
# about 230x, nearly every token on the hottest expert).
ZIPF_BETA = 0.33


def zipf_router_bias(E, s=1.1, beta=ZIPF_BETA, seed=0):
    """beta * log p_e with p Zipf(s) over a random permutation of ranks."""
    rng = np.random.default_rng(seed + 7)
    ranks = rng.permutation(E) + 1
    p = ranks.astype(np.float64) ** (-s)
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def cfg_mixed(seed=0, n_experts=256, hidden=2048, inter=512, shared_inter=512):
    """3-bit gate/up, 6-bit down, bf16 scales, shared expert with
    a sigmoid gate."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, 8, inter
    shared = (gen_qproj(rng, 1, shared_inter, H, 3, 64, BF16),
              gen_qproj(rng, 1, shared_inter, H, 3, 64, BF16),
              gen_qproj(rng, 1, H, shared_inter, 6, 64, BF16))
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), BF16),
                     router_dt=BF16,
                     gate=gen_qproj(rng, E, I, H, 3, 64, BF16), up=gen_qproj(rng, E, I, H, 3, 64, BF16),
                     down=gen_qproj(rng, E, H, I, 6, 64, BF16), shared=shared,
                     shared_gate_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(1, H)), BF16),
                     name="mixed")


def cfg_bits(gu_bits, down_bits, gs, sb_dt, act_dt, seed=0, hidden=512, inter=384, n_experts=16,
             top_k=3):
    """Small layers over every packed width, group size and dtype pairing.
    Scales shrink with the code range (x 15 / (2^bits - 1)) so every width
    spans the weight range of the 4-bit configs and fp16 outputs stay finite."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, top_k, inter

    def proj(n, kk, bits):
        f = 15.0 / (2 ** bits - 1)
        return gen_qproj(rng, E, n, kk, bits, gs, sb_dt, s_range=(0.005 * f, 0.02 * f))

    return LayerSpec(H, E, k, I, act_dt,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), act_dt),
                     router_dt=act_dt,
                     gate=proj(I, H, gu_bits), up=proj(I, H, gu_bits), down=proj(H, I, down_bits),
                     name=f"bits{gu_bits}/{down_bits} gs{gs}")


def cfg_nemotron(seed=0, n_experts=64, hidden=1024, inter=512, shared_inter=1024, top_k=6):
    """NemotronH MoE (NemotronHText.swift:694-868): sigmoid router with a
    correction bias for the selection, renormalised top-6 weights times
    routed_scaling_factor 2.5, squared-ReLU experts with no gate projection
    and an always-on squared-ReLU shared expert. Nemotron-3-Nano-shaped
    ratios at a smaller width; 4-bit gs64, bf16."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, top_k, inter
    shared = (None, gen_qproj(rng, 1, shared_inter, H, 4, 64, BF16),
              gen_qproj(rng, 1, H, shared_inter, 4, 64, BF16))
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), BF16),
                     router_dt=BF16, gating=orc.SIGMOID_TOPK, norm_topk=True,
                     expert_bias=rng.uniform(-0.05, 0.05, size=E).astype(np.float32),
                     gate=None, up=gen_qproj(rng, E, I, H, 4, 64, BF16),
                     down=gen_qproj(rng, E, H, I, 4, 64, BF16), activation=orc.ACT_RELU2,
                     shared=shared, routed_scale=2.5, name="nemotron")


def cfg_gemma4(seed=0, n_experts=64, hidden=1024, inter=384, top_k=8):
    """Gemma 4 MoE (Gemma4Text.swift:928-978): top-8 of the logits scaled by
    hidden^-0.5, softmax over the 8, times per_expert_scale[e]; GELU-gated
    experts; the router reads its own normalised rows. 4-bit gs64, bf16."""
    rng = np.random.default_rng(seed)
    H, E, k, I = hidden, n_experts, top_k, inter
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1, size=(E, H)), BF16), router_dt=BF16,
                     gating=orc.TOPK_THEN_SOFTMAX, logit_scale=float(np.float32(H ** -0.5)),
                     expert_scale=rng.uniform(0.5, 1.5, size=E).astype(np.float32),
                     gate=gen_qproj(rng, E, I, H, 4, 64, BF16), up=gen_qproj(rng, E, I, H, 4, 64, BF16),
                     down=gen_qproj(rng, E, H, I, 4, 64, BF16), activation=orc.ACT_GEGLU,
                     split_router_input=True, name="gemma4")


# ------------------------------------------------------------- tolerance --

def check_close(got, ref, dt, label="", mean_tol=1e-3):
    """The layer's float bar against the fp32-accumulated oracle.

    fp16/bf16: max |d| <= 2e-2 on each element's own scale, max(1, |ref|,
    rms(ref)), and mean |d| / mean |ref| <= 1e-3. The synthetic layers (codes
    uniform over the full range, positive scales) produce outputs far above 1,
    where one storage ulp of a large element is already well above 2e-2 in
    absolute terms: a rounding flip of the largest elements is 2^-8..2^-7 of
    their value, while a wrong expert, a dropped term or a wrong scale moves
    the error to order 1 on the RMS scale. Elements below the RMS are judged on
    the RMS scale, since the combine adds rounded per-expert outputs whose
    rounding is set by the summands, not by a cancelled result.
    f32: |d| <= 1e-3 * max(1, |ref|) elementwise (MoELayerTests.swift:224).
    mean_tol overrides the mean bar for single products whose operands the
    kernel rounds on purpose (the matrix-core path); layer tests keep 1e-3."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    d = np.abs(got - ref)
    mean_rel = float(d.mean() / max(np.abs(ref).mean(), 1e-30)) if d.size else 0.0
    if dt == F32:
        max_scaled = float((d / np.maximum(1.0, np.abs(ref))).max()) if d.size else 0.0
        assert max_scaled <= 1e-3, f"{label}: max |d|/max(1,|ref|) = {max_scaled:.3e} > 1e-3"
        return max_scaled, mean_rel
    rms = float(np.sqrt(np.mean(ref * ref))) if d.size else 1.0
    scale = np.maximum(np.maximum(1.0, rms), np.abs(ref))
    max_scaled = float((d / scale).max()) if d.size else 0.0
    assert max_scaled <= 2e-2, f"{label}: max |d| / max(1, |ref|, rms) = {max_scaled:.3e} > 2e-2"
    assert mean_rel <= mean_tol, f"{label}: mean relative error {mean_rel:.3e} > {mean_tol:.1e}"
    return max_scaled, mean_rel
