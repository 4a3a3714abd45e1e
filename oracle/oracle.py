"""ctypes binding of the CPU oracle (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py as the checker / timed CPU baseline.
The product package ``ffai_amd`` never imports it.

Arrays cross the boundary as numpy buffers: float32 for f32, float16 for f16
and uint16 bit patterns for bf16.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

F32, F16, BF16 = 0, 1, 2
SOFTMAX_THEN_TOPK, TOPK_THEN_SOFTMAX, SIGMOID_TOPK = 0, 1, 2
ACT_SWIGLU, ACT_GPTOSS, ACT_GEGLU, ACT_RELU2 = 0, 1, 2, 3

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


class OrQProj(C.Structure):
    _fields_ = [
        ("weight", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
        ("out_bias", C.c_void_p),
        ("bits", C.c_int), ("group_size", C.c_int), ("sb_dt", C.c_int),
        ("n", C.c_int), ("k", C.c_int),
    ]


class OrLayer(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
        ("intermediate", C.c_int), ("act_dt", C.c_int),
        ("router_weight", C.c_void_p), ("router_dt", C.c_int), ("router_bias", C.c_void_p),
        ("gating", C.c_int), ("norm_topk", C.c_int), ("expert_bias", C.c_void_p),
        ("gate", OrQProj), ("up", OrQProj), ("down", OrQProj),
        ("activation", C.c_int), ("alpha", C.c_float), ("limit", C.c_float),
        ("has_shared", C.c_int),
        ("shared_gate", OrQProj), ("shared_up", OrQProj), ("shared_down", OrQProj),
        ("shared_gate_weight", C.c_void_p),
        ("logit_scale", C.c_float), ("routed_scale", C.c_float), ("expert_scale", C.c_void_p),
        ("router_q", OrQProj), ("shared_gate_q", OrQProj),
    ]


def _declare(L):
    vp, i, f, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
    L.or_bf16_to_f32.argtypes = [C.c_uint16]; L.or_bf16_to_f32.restype = f
    L.or_f32_to_bf16.argtypes = [f]; L.or_f32_to_bf16.restype = C.c_uint16
    L.or_f16_to_f32.argtypes = [C.c_uint16]; L.or_f16_to_f32.restype = f
    L.or_f32_to_f16.argtypes = [f]; L.or_f32_to_f16.restype = C.c_uint16
    L.or_round_dt.argtypes = [f, i]; L.or_round_dt.restype = f
    L.or_load.argtypes = [vp, i, sz, vp]; L.or_load.restype = None
    L.or_store.argtypes = [vp, i, sz, vp]; L.or_store.restype = None
    L.or_expf.argtypes = [f]; L.or_expf.restype = f
    L.or_unpack_codes.argtypes = [vp, i, sz, vp]; L.or_unpack_codes.restype = i
    L.or_pack_codes.argtypes = [vp, i, sz, vp]; L.or_pack_codes.restype = i
    L.or_packed_u32_count.argtypes = [C.c_long, i]; L.or_packed_u32_count.restype = C.c_long
    L.or_derive_bits.argtypes = [C.c_long, C.c_long, C.c_long]; L.or_derive_bits.restype = i
    L.or_dequantize_affine.argtypes = [vp, vp, vp, i, i, i, sz, vp]
    L.or_dequantize_affine.restype = i
    L.or_router_logits.argtypes = [vp, i, i, i, vp, i, vp, i, vp]
    L.or_router_logits.restype = None
    L.or_router_logits_q.argtypes = [vp, i, i, i, C.POINTER(OrQProj), vp, i, vp]
    L.or_router_logits_q.restype = i
    L.or_topk_indices.argtypes = [vp, i, i, vp]; L.or_topk_indices.restype = i
    L.or_softmax.argtypes = [vp, i, vp]; L.or_softmax.restype = None
    L.or_route.argtypes = [vp, i, i, i, i, i, vp, vp, vp]; L.or_route.restype = i
    L.or_route_scaled.argtypes = [vp, i, i, i, i, i, vp, f, f, vp, vp, vp]
    L.or_route_scaled.restype = i
    L.or_gelu.argtypes = [f]; L.or_gelu.restype = f
    L.or_act_dt.argtypes = [f, f, i, f, f, i]; L.or_act_dt.restype = f
    L.or_dispatch_plan.argtypes = [vp, i, i, i, vp, vp, vp, vp]
    L.or_dispatch_plan.restype = i
    L.or_qgemm_rows.argtypes = [C.POINTER(OrQProj), vp, i, vp, vp]
    L.or_qgemm_rows.restype = i
    L.or_act.argtypes = [f, f, i, f, f]; L.or_act.restype = f
    L.or_unpermute.argtypes = [vp, vp, vp, i, i, i, i, vp]; L.or_unpermute.restype = None
    L.or_moe_layer.argtypes = [C.POINTER(OrLayer), vp, i, vp, vp, vp, vp, vp]
    L.or_moe_layer.restype = i
    L.or_moe_layer_routed.argtypes = [C.POINTER(OrLayer), vp, vp, i, vp, vp, vp, vp, vp]
    L.or_moe_layer_routed.restype = i
    L.or_add_rmsnorm.argtypes = [vp, vp, vp, f, i, i, i, vp, vp]
    L.or_add_rmsnorm.restype = None
    L.or_residual_combine.argtypes = [vp, vp, vp, f, i, i, vp]
    L.or_residual_combine.restype = None
    L.or_moe_layer_residual.argtypes = [C.POINTER(OrLayer), vp, vp, vp, f, i, vp, vp, vp, vp, vp,
                                        vp, vp]
    L.or_moe_layer_residual.restype = i
    L.or_mxfp4_value.argtypes = [i]; L.or_mxfp4_value.restype = f
    L.or_mxfp4_to_affine.argtypes = [vp, vp, C.c_long, vp, vp, vp, i]
    L.or_mxfp4_to_affine.restype = None


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- dtypes ---

def np_dtype(dt: int):
    return {F32: np.float32, F16: np.float16, BF16: np.uint16}[dt]


def to_f32(a: np.ndarray, dt: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if dt == F32:
        return a.astype(np.float32)
    if dt == F16:
        return a.astype(np.float32)
    return (a.astype(np.uint32) << 16).view(np.float32)


def from_f32(a: np.ndarray, dt: int) -> np.ndarray:
    """Round float32 values to dt storage (RNE) with the oracle's converters."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np_dtype(dt))
    lib().or_store(_p(a), dt, a.size, _p(out))
    return out


def round_dt(a: np.ndarray, dt: int) -> np.ndarray:
    return to_f32(from_f32(a, dt), dt)


# ------------------------------------------------------------ bit stream ---

def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n = codes.size
    if (n * bits) % 32:
        raise ValueError("numel*bits must be a multiple of 32")
    w = np.zeros(n * bits // 32, dtype=np.uint32)
    if lib().or_pack_codes(_p(codes), bits, n, _p(w)) != 0:
        raise ValueError("bad bits")
    return w.reshape(codes.shape[:-1] + (codes.shape[-1] * bits // 32,))


def unpack_codes(w: np.ndarray, bits: int, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    out = np.zeros(n, dtype=np.uint8)
    if lib().or_unpack_codes(_p(w), bits, n, _p(out)) != 0:
        raise ValueError("bad bits / size")
    return out


def dequantize_affine(w, scales, biases, sb_dt, bits, gs, numel):
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    out = np.zeros(numel, dtype=np.float32)
    rc = lib().or_dequantize_affine(_p(w), _p(scales), _p(biases), sb_dt, bits, gs, numel, _p(out))
    if rc != 0:
        raise ValueError("invalid affine dequantize arguments")
    return out


def derive_bits(packed_cols, scale_cols, gs) -> int:
    return lib().or_derive_bits(packed_cols, scale_cols, gs)


def packed_u32_count(numel, bits) -> int:
    return lib().or_packed_u32_count(numel, bits)


def expf(x: float) -> float:
    return lib().or_expf(float(x))


# ---------------------------------------------------------------- router ---

def router_logits(x, x_dt, W, w_dt, bias=None):
    x = np.ascontiguousarray(x)
    W = np.ascontiguousarray(W)
    T, H = x.shape
    E = W.shape[0]
    out = np.zeros((T, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias)
    lib().or_router_logits(_p(x), x_dt, T, H, _p(W), w_dt, _p(b), E, _p(out))
    return out


def router_logits_q(x, x_dt, q, bias=None):
    """Router logits with an affine-quantised weight: q is a QProj holding one
    expert [1, E, H]."""
    x = np.ascontiguousarray(x)
    T, H = x.shape
    E = q.n
    out = np.zeros((T, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias)
    qc = q.c()
    if lib().or_router_logits_q(_p(x), x_dt, T, H, C.byref(qc), _p(b), E, _p(out)) != 0:
        raise ValueError("invalid quantised router")
    return out


def topk_indices(v, k):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(k, dtype=np.int32)
    if lib().or_topk_indices(_p(v), v.size, k, _p(out)) != 0:
        raise ValueError("k out of range")
    return out


def softmax(v):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros_like(v)
    lib().or_softmax(_p(v), v.size, _p(out))
    return out


def route(logits, k, gating=SOFTMAX_THEN_TOPK, norm_topk=True, expert_bias=None,
          logit_scale=1.0, routed_scale=1.0, expert_scale=None):
    logits = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    T, E = logits.shape
    idx = np.zeros((T, k), dtype=np.uint32)
    w = np.zeros((T, k), dtype=np.float32)
    eb = None if expert_bias is None else np.ascontiguousarray(expert_bias, dtype=np.float32)
    es = None if expert_scale is None else np.ascontiguousarray(expert_scale, dtype=np.float32)
    rc = lib().or_route_scaled(_p(logits), T, E, k, gating, int(bool(norm_topk)), _p(eb),
                               float(logit_scale), float(routed_scale), _p(es), _p(idx), _p(w))
    if rc != 0:
        raise ValueError("invalid router arguments")
    return idx, w


def dispatch_plan(idx, E):
    idx = np.ascontiguousarray(np.atleast_2d(idx), dtype=np.uint32)
    T, k = idx.shape
    M = T * k
    counts = np.zeros(E, dtype=np.uint32)
    offsets = np.zeros(E + 1, dtype=np.uint32)
    perm = np.zeros(M, dtype=np.uint32)
    inv = np.zeros(M, dtype=np.uint32)
    rc = lib().or_dispatch_plan(_p(idx), T, k, E, _p(counts), _p(offsets), _p(perm), _p(inv))
    if rc != 0:
        raise ValueError("expert id out of range")
    return counts, offsets, perm, inv


# ----------------------------------------------------------- projections ---

class QProj:
    """Stacked affine projection: weight [E, N, K*bits/32] u32, scales/biases
    [E, N, K/gs] in sb_dt, optional out_bias [E, N] in the activation dtype."""

    def __init__(self, weight, scales, biases, bits, gs, sb_dt, out_bias=None):
        self.weight = np.ascontiguousarray(weight, dtype=np.uint32)
        self.scales = np.ascontiguousarray(scales)
        self.biases = np.ascontiguousarray(biases)
        self.out_bias = None if out_bias is None else np.ascontiguousarray(out_bias)
        self.bits, self.gs, self.sb_dt = bits, gs, sb_dt
        self.E, self.n = self.weight.shape[0], self.weight.shape[1]
        self.k = self.scales.shape[2] * gs

    def c(self) -> OrQProj:
        return OrQProj(_p(self.weight), _p(self.scales), _p(self.biases), _p(self.out_bias),
                       self.bits, self.gs, self.sb_dt, self.n, self.k)

    def dense(self, e: int) -> np.ndarray:
        """Dequantised [N, K] float32 matrix of expert e."""
        N, K = self.n, self.k
        out = dequantize_affine(self.weight[e].ravel(), self.scales[e].ravel(),
                                self.biases[e].ravel(), self.sb_dt, self.bits, self.gs, N * K)
        return out.reshape(N, K)


def qgemm_rows(p: QProj, a: np.ndarray, row_expert: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    row_expert = np.ascontiguousarray(row_expert, dtype=np.uint32)
    M = a.shape[0]
    out = np.zeros((M, p.n), dtype=np.float32)
    c = p.c()
    if lib().or_qgemm_rows(C.byref(c), _p(a), M, _p(row_expert), _p(out)) != 0:
        raise ValueError("invalid projection")
    return out


def act(g, u, kind=ACT_SWIGLU, alpha=1.702, limit=7.0, dt=F32) -> float:
    return lib().or_act_dt(float(g), float(u), kind, float(alpha), float(limit), dt)


def gelu(g) -> float:
    return lib().or_gelu(float(g))


def unpermute(Y, inv_perm, w, T, H, k, dt):
    Y = np.ascontiguousarray(Y, dtype=np.float32)
    inv_perm = np.ascontiguousarray(inv_perm, dtype=np.uint32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros((T, H), dtype=np.float32)
    lib().or_unpermute(_p(Y), _p(inv_perm), _p(w), T, H, k, dt, _p(out))
    return out


# ---------------------------------------------------------------- layer ----

def moe_layer(spec, x, given_logits=None, router_x=None):
    """Run the whole layer on the CPU. ``spec`` is a tests' LayerSpec-like
    object (see tests/moe_spec.py). ``router_x`` (default x) is what the
    router reads. Returns (y, logits, idx, weights)."""
    x = np.ascontiguousarray(x)
    rx = x if router_x is None else np.ascontiguousarray(router_x)
    assert rx.shape == x.shape and rx.dtype == x.dtype
    T = x.shape[0]
    L = spec.oracle_struct()
    y = np.zeros((T, spec.hidden), dtype=np_dtype(spec.act_dt))
    logits = np.zeros((T, spec.n_experts), dtype=np.float32)
    idx = np.zeros((T, spec.top_k), dtype=np.uint32)
    w = np.zeros((T, spec.top_k), dtype=np.float32)
    gl = None if given_logits is None else np.ascontiguousarray(given_logits, dtype=np.float32)
    rc = lib().or_moe_layer_routed(C.byref(L), _p(x), _p(rx), T, _p(y), _p(gl), _p(logits),
                                   _p(idx), _p(w))
    if rc != 0:
        raise ValueError("invalid layer description")
    return y, logits, idx, w


# ------------------------------------------------------- decoder steps ----

def add_rmsnorm(a, b, w, eps, dt=F32):
    """(residual, normed) float32 arrays [T, H] (values rounded to dt)."""
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.float32)
    b = np.ascontiguousarray(np.atleast_2d(b), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    T, H = a.shape
    res = np.zeros_like(a)
    xn = np.zeros_like(a)
    lib().or_add_rmsnorm(_p(a), _p(b), _p(w), float(eps), T, H, dt, _p(res), _p(xn))
    return res, xn


def residual_combine(res, base, value=None, gate=1.0, dt=F32):
    base = np.ascontiguousarray(base, dtype=np.float32).ravel()
    r = None if res is None else np.ascontiguousarray(res, dtype=np.float32).ravel()
    v = None if value is None else np.ascontiguousarray(value, dtype=np.float32).ravel()
    out = np.zeros_like(base)
    lib().or_residual_combine(_p(r), _p(base), _p(v), float(gate), base.size, dt, _p(out))
    return out


def moe_layer_residual(spec, h, m, norm_w, eps, given_logits=None):
    """The block between the decoder steps. h, m: storage arrays [T, H] of
    spec.act_dt; norm_w: float32 [H] (values of the act dtype). Returns
    (y, xn, residual, logits, idx, weights)."""
    h = np.ascontiguousarray(h)
    m = np.ascontiguousarray(m)
    T, H = h.shape
    L = spec.oracle_struct()
    nw = np.ascontiguousarray(norm_w, dtype=np.float32)
    y = np.zeros((T, H), dtype=np_dtype(spec.act_dt))
    xn = np.zeros((T, H), dtype=np.float32)
    res = np.zeros((T, H), dtype=np.float32)
    logits = np.zeros((T, spec.n_experts), dtype=np.float32)
    idx = np.zeros((T, spec.top_k), dtype=np.uint32)
    w = np.zeros((T, spec.top_k), dtype=np.float32)
    gl = None if given_logits is None else np.ascontiguousarray(given_logits, dtype=np.float32)
    rc = lib().or_moe_layer_residual(C.byref(L), _p(h), _p(m), _p(nw), float(eps), T, _p(y),
                                     _p(gl), _p(xn), _p(res), _p(logits), _p(idx), _p(w))
    if rc != 0:
        raise ValueError("invalid layer description")
    return y, xn, res, logits, idx, w


# ----------------------------------------------------- MXFP4 transcode ----

def mxfp4_value(code: int) -> float:
    return lib().or_mxfp4_value(int(code))


def mxfp4_to_affine(packed, e8m0, sb_dt=BF16):
    """packed: u32 [..., K/8], e8m0: u8 [..., K/32] -> (codes u32 like packed,
    scales, biases [..., K/32] as sb_dt storage arrays)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    e8m0 = np.ascontiguousarray(e8m0, dtype=np.uint8)
    groups = e8m0.size
    assert packed.size == 4 * groups
    out_w = np.zeros_like(packed)
    sdt = np_dtype(sb_dt)
    out_s = np.zeros(e8m0.shape, dtype=sdt)
    out_b = np.zeros(e8m0.shape, dtype=sdt)
    lib().or_mxfp4_to_affine(_p(packed), _p(e8m0), groups, _p(out_w), _p(out_s), _p(out_b), sb_dt)
    return out_w, out_s, out_b

