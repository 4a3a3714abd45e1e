"""GPT-OSS's MXFP4 -> affine 4-bit transcode (GPTOSSText.swift:941-1236).

The reference has no test for it, so the oracle (oracle/moe_oracle.c
or_mxfp4_to_affine) is pinned by the format's table (GPTOSSText.swift:
947-957) and by what the per-group fit must satisfy: levels in 0..15, the
group minimum on level 0 exactly, every value reconstructed within half a
step, each code the nearest level, flat groups on a zero scale, and an
exponent step that doubles scale and bias and keeps the codes. On the GPU
the kernel must match the oracle bit for bit (codes, scales, biases), alone
and through the checkpoint reader, and a GPT-OSS-shaped layer on the
transcoded experts meets the layer bar."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import oracle as orc
from ffai_amd import _lib
from moe_spec import BF16, F16, F32, LayerSpec, check_close, load, store

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def random_groups(G, seed=0, e_range=(100, 140)):
    """Packed codes and e8m0 bytes for G groups, with flat groups, all-zero
    groups mixing +0/-0 codes, narrow groups and full-range groups."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(G, 32))
    codes[0::7] = rng.integers(0, 16)                         # flat
    codes[1::7] = rng.choice([0, 8], size=(len(codes[1::7]), 32))  # +-0 only
    codes[2::7] = rng.integers(1, 4, size=(len(codes[2::7]), 32))  # narrow, positive
    codes[3::7] = rng.integers(9, 12, size=(len(codes[3::7]), 32))  # narrow, negative
    e8 = rng.integers(e_range[0], e_range[1], size=G).astype(np.uint8)
    packed = orc.pack_codes(codes.reshape(-1).astype(np.uint8), 4).reshape(G, 4)
    return packed, e8, codes


def affine_values(out_w, s, b, sb_dt, G):
    q = orc.unpack_codes(out_w.reshape(-1), 4, G * 32).reshape(G, 32).astype(np.float64)
    return load(s, sb_dt).astype(np.float64)[:, None] * q + load(b, sb_dt).astype(np.float64)[:, None], q


def test_table_kat():
    g = GOLD["mxfp4_lut"]
    got = [orc.mxfp4_value(c) for c in range(16)]
    assert got == g["lut"]
    assert [np.signbit(np.float32(v)) for v in got] == [np.signbit(np.float32(v)) for v in g["lut"]]


@pytest.mark.parametrize("sb_dt", [F32, BF16, F16])
def test_per_group_fit_properties(sb_dt):
    G = 4000
    # f16 scales of small exponents are subnormal: keep f16 in its normal range
    packed, e8, codes = random_groups(G, seed=sb_dt, e_range=(125, 140) if sb_dt == F16 else (100, 140))
    out_w, s, b = orc.mxfp4_to_affine(packed, e8, sb_dt)
    lut = np.array(GOLD["mxfp4_lut"]["lut"])
    mx = 2.0 ** (e8.astype(np.float64) - 127)
    v = lut[codes] * mx[:, None]
    rec, q = affine_values(out_w, s, b, sb_dt, G)
    assert q.min() >= 0 and q.max() <= 15
    lo, hi = v.min(1), v.max(1)
    sf = load(s, sb_dt).astype(np.float64)
    st = (hi - lo) / 15
    # scale and bias: the group's own range, stored in the dtype
    assert np.allclose(sf, st, rtol={F32: 1e-6, BF16: 2 ** -8, F16: 2 ** -11}[sb_dt], atol=0)
    assert np.array_equal(load(b, sb_dt), load(store(lo, sb_dt), sb_dt))
    # the minimum sits on level 0; every code is the nearest level of the fp32 grid
    flat = hi == lo
    assert np.all(q[flat] == 0) and np.all(sf[flat] == 0)
    assert np.all(q[v == lo[:, None]] == 0)
    t = np.where(st[:, None] > 0, (v - lo[:, None]) / np.where(st > 0, st, 1)[:, None], 0)
    near = np.clip(np.floor(t + 0.5), 0, 15)
    tie = np.abs(t - np.floor(t) - 0.5) < 1e-4
    assert np.all((q == near) | tie)
    # reconstruction within half a step (plus the dtype rounding of scale and bias)
    slack = {F32: 1e-6, BF16: 2 ** -7, F16: 2 ** -10}[sb_dt]
    err = np.abs(rec - v)
    assert np.all(err <= st[:, None] * (0.5 + 16 * slack) + np.abs(lo)[:, None] * slack + 1e-30)


def test_fixed_grid_would_be_worse():
    """The per-group fit beats a fixed full-range (+-6) grid on narrow groups,
    the reason the reference fits each group (GPTOSSText.swift:1040-1052): a
    transcode that skipped the fit fails the bound above."""
    packed, e8, codes = random_groups(700, seed=3)
    lut = np.array(GOLD["mxfp4_lut"]["lut"])
    v = lut[codes] * (2.0 ** (e8.astype(np.float64) - 127))[:, None]
    out_w, s, b = orc.mxfp4_to_affine(packed, e8, F32)
    rec, _ = affine_values(out_w, s, b, F32, 700)
    mx = 2.0 ** (e8.astype(np.float64) - 127)
    fixed = np.round((v + 6 * mx[:, None]) / (12 * mx[:, None] / 15)) * (12 * mx[:, None] / 15) - 6 * mx[:, None]
    narrow = slice(2, None, 7)
    assert np.abs(fixed[narrow] - v[narrow]).max() > 4 * np.abs(rec[narrow] - v[narrow]).max()


def test_exponent_step_doubles_scale_and_bias():
    packed, e8, _ = random_groups(500, seed=5, e_range=(60, 190))
    w1, s1, b1 = orc.mxfp4_to_affine(packed, e8, F32)
    w2, s2, b2 = orc.mxfp4_to_affine(packed, e8 + 1, F32)
    assert np.array_equal(w1, w2)
    assert np.array_equal(s2, 2 * s1) and np.array_equal(b2, 2 * b1)


def test_in_place_matches():
    packed, e8, _ = random_groups(64, seed=6)
    w1, _, _ = orc.mxfp4_to_affine(packed, e8, BF16)
    same = packed.copy()
    lib = orc.lib()
    s = np.zeros(64, np.uint16)
    b = np.zeros(64, np.uint16)
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    lib.or_mxfp4_to_affine(ptr(same), ptr(e8), 64, ptr(same), ptr(s), ptr(b), BF16)
    assert np.array_equal(same, w1)


# ------------------------------------------------------------ checkpoint --

def write_mxfp4(path, base, E, N, K, seed, bias_dt="BF16", extra=None):
    from test_safetensors import write_st
    rng = np.random.default_rng(seed)
    G = E * N * (K // 32)
    packed, e8, _ = random_groups(G, seed=seed, e_range=(118, 124))
    bias = store(rng.normal(0, 0.1, (E, N)), BF16 if bias_dt == "BF16" else F16)
    t = {f"{base}.weight": packed.reshape(E, N, K // 8),
         f"{base}.scales": e8.reshape(E, N, K // 32),
         f"{base}.bias": (bias_dt, [E, N], bias.tobytes())}
    if extra:
        t.update(extra)
    write_st(path, t)
    return packed.reshape(E, N, K // 8), e8.reshape(E, N, K // 32), bias


def test_mxfp4_layout_validation(tmp_path):
    from test_safetensors import Bundle, write_st
    write_mxfp4(tmp_path / "m.safetensors", "l.experts.gate_proj", 2, 64, 128, 0)
    b = Bundle(tmp_path / "m.safetensors")
    nb, ns = C.c_size_t(), C.c_size_t()
    assert b.lib.moe_st_mxfp4_bytes(b.h, b"l.experts.gate_proj", _lib.MOE_BF16, C.byref(nb),
                                    C.byref(ns)) == _lib.MOE_OK
    a = lambda n: (n + 255) // 256 * 256  # noqa: E731
    G = 2 * 64 * 4
    assert nb.value == a(G * 16) + 2 * a(G * 2) + a(2 * 64 * 2)
    assert ns.value == a(G) + a(2 * 64 * 2)
    assert b.lib.moe_st_mxfp4_bytes(b.h, b"l.experts.up_proj", _lib.MOE_BF16, C.byref(nb),
                                    C.byref(ns)) == _lib.MOE_ERR_INVALID
    b.close()
    write_st(tmp_path / "bad.safetensors", {"x.weight": np.zeros((2, 64, 16), np.uint32),
                                             "x.scales": np.zeros((2, 64, 3), np.uint8),
                                             "x.bias": np.zeros((2, 64), np.float32)})
    b = Bundle(tmp_path / "bad.safetensors")
    assert b.lib.moe_st_mxfp4_bytes(b.h, b"x", _lib.MOE_BF16, C.byref(nb), C.byref(ns)) \
        == _lib.MOE_ERR_INVALID
    assert "shapes disagree" in _lib.last_error()
    b.close()


# --------------------------------------------------------------------- GPU --

def _torch():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.gpu
@pytest.mark.parametrize("sb_dt", [BF16, F16, F32])
@pytest.mark.parametrize("in_place", [False, True])
def test_transcode_bit_exact(sb_dt, in_place):
    torch = _torch()
    from moe_spec import to_torch
    G = 70001
    # exponents 3..254; below 3 the reference's own f32 intermediates are
    # subnormal, which the GPU flushes (test_transcode_tiny_exponents)
    packed, e8, _ = random_groups(G, seed=11 + sb_dt, e_range=(3, 255))
    ref_w, ref_s, ref_b = orc.mxfp4_to_affine(packed, e8, sb_dt)
    pt = torch.from_numpy(packed.view(np.int32)).cuda()
    et = torch.from_numpy(e8).cuda()
    ow = pt if in_place else torch.empty_like(pt)
    tdt = {BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[sb_dt]
    s = torch.empty(G, dtype=tdt, device="cuda")
    b = torch.empty(G, dtype=tdt, device="cuda")
    _lib.check(_lib.load().moe_mxfp4_to_affine(
        C.c_void_p(pt.data_ptr()), C.c_void_p(et.data_ptr()), G, C.c_void_p(ow.data_ptr()),
        C.c_void_p(s.data_ptr()), C.c_void_p(b.data_ptr()), sb_dt,
        C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    got_w = ow.cpu().numpy().view(np.uint32).reshape(G, 4)
    bad = np.nonzero(np.any(got_w != ref_w, axis=1))[0]
    assert bad.size == 0, f"{bad.size} groups differ; exponents {sorted(set(e8[bad].tolist()))[:20]}"

    bits = np.uint32 if sb_dt == F32 else np.uint16
    sv = s.view(torch.int32 if sb_dt == F32 else torch.int16).cpu().numpy().view(bits)
    bv = b.view(torch.int32 if sb_dt == F32 else torch.int16).cpu().numpy().view(bits)
    assert np.array_equal(sv, ref_s.view(bits)), "scales"
    assert np.array_equal(bv, ref_b.view(bits)), "biases"


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 5, 200])
def test_mxfp4_checkpoint_layer(tmp_path, T):
    """A GPT-OSS-shaped layer whose experts come from an MXFP4 checkpoint:
    the reader's transcode matches the oracle's bit for bit, and the layer
    on it meets the bar against the oracle layer on the oracle's transcode."""
    torch = _torch()
    from ffai_amd import layer as fl
    from ffai_amd.safetensors import SafeTensorsBundle
    from moe_spec import to_numpy_f32, to_torch
    E, H, I, k = 8, 512, 640, 4
    p = "model.layers.0.mlp.experts"
    raw = {}
    for name, (n, kk), seed in (("gate_proj", (I, H), 1), ("up_proj", (I, H), 2),
                                ("down_proj", (H, I), 3)):
        raw[name] = write_mxfp4(tmp_path / f"{name}.safetensors", f"{p}.{name}", E, n, kk, seed)
    with SafeTensorsBundle(str(tmp_path)) as b:
        prj = {n: b.mxfp4Experts(f"{p}.{n}", torch.bfloat16) for n in raw}
    qs = {}
    for n, (packed, e8, bias) in raw.items():
        w, s, bb = orc.mxfp4_to_affine(packed, e8, BF16)
        got = prj[n]
        assert got.bits == 4 and got.group_size == 32
        assert np.array_equal(got.weight.cpu().numpy().view(np.uint32), w), n
        assert np.array_equal(got.scales.view(torch.int16).cpu().numpy().view(np.uint16), s), n
        assert np.array_equal(got.biases.view(torch.int16).cpu().numpy().view(np.uint16), bb), n
        assert np.array_equal(got.out_bias.view(torch.int16).cpu().numpy().view(np.uint16), bias), n
        qs[n] = orc.QProj(w, s, bb, 4, 32, BF16, out_bias=bias)
    rng = np.random.default_rng(0)
    spec = LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), (E, H)), BF16), router_dt=BF16,
                     router_bias=store(rng.normal(0, 0.1, E), BF16), gating=orc.TOPK_THEN_SOFTMAX,
                     gate=qs["gate_proj"], up=qs["up_proj"], down=qs["down_proj"],
                     activation=orc.ACT_GPTOSS, name="mxfp4")
    layer = fl.MoELayer(router_weight=to_torch(spec.router_weight),
                        router=fl.MoERouter(E, k, fl.MoEGatingMode.topKThenSoftmax, True),
                        gate=prj["gate_proj"], up=prj["up_proj"], down=prj["down_proj"], hidden=H,
                        act_dtype=torch.bfloat16, router_bias=to_torch(spec.router_bias),
                        activation=_lib.MOE_ACT_GPTOSS, alpha=1.702, limit=7.0)
    x = spec.x(T, seed=T)
    y, tr = layer.forward(to_torch(x), trace=True)
    torch.cuda.synchronize()
    y_ref, _, idx, w = orc.moe_layer(spec, x, given_logits=to_numpy_f32(tr["logits"]))
    # both paths meet the layer bar against the fp32 oracle: the streaming
    # GEMVs keep the dequantised weights in f32, the matrix-core GEMM rounds
    # each one once to f16 (the transcoded grids' scales, span / 15, are not
    # dyadic, so bf16 operands moved this layer by about 4e-3 mean relative)
    check_close(to_numpy_f32(y), load(y_ref, BF16), BF16, f"mxfp4 layer T={T}")
    if T * k >= 32 * E:
        # and an independent float64 composition of the dequantised experts
        ref64 = gptoss_composition(spec, x, idx, w)
        check_close(to_numpy_f32(y), ref64, BF16, f"mxfp4 layer T={T} vs float64 composition")


def gptoss_composition(spec, x, idx, w):
    """float64 GPT-OSS layer from independently dequantised experts
    (projection biases and the clamped activation as GPTOSSText.swift:
    1399-1441 apply them)."""
    from test_oracle_golden import _dense
    T, H, I = x.shape[0], spec.hidden, spec.intermediate
    xf = load(x, BF16).astype(np.float64)
    rd = lambda a: load(store(a, BF16), BF16).astype(np.float64)  # noqa: E731

    def dense(q, e, n, kk):
        return _dense(q.weight[e], load(q.scales[e], q.sb_dt), load(q.biases[e], q.sb_dt), q.bits,
                      q.gs, n, kk)

    ob = lambda q, e: load(q.out_bias[e], BF16).astype(np.float64)  # noqa: E731
    out = np.zeros((T, H))
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(spec.top_k):
            e = idx[t, s]
            g = rd(rd(dense(spec.gate, e, I, H) @ xf[t]) + ob(spec.gate, e))
            u = rd(rd(dense(spec.up, e, I, H) @ xf[t]) + ob(spec.up, e))
            gc, uc = np.minimum(g, spec.limit), np.clip(u, -spec.limit, spec.limit)
            a = rd(gc / (1 + np.exp(-spec.alpha * gc)) * (uc + 1))
            yv = rd(rd(dense(spec.down, e, H, I) @ a) + ob(spec.down, e))
            acc = acc + np.float32(rd(np.float32(w[t, s]))) * yv.astype(np.float32)
        out[t] = rd(acc)
    return out


def test_gptoss_composition_matches_oracle():
    """The composition above agrees with the oracle layer, so it is a fair
    second reference for the matrix-core path."""
    rng = np.random.default_rng(1)
    E, H, I, k = 4, 128, 96, 2
    qs = {}
    for n, (nn, kk) in (("g", (I, H)), ("u", (I, H)), ("d", (H, I))):
        packed, e8, _ = random_groups(E * nn * kk // 32, seed=len(n) + nn, e_range=(118, 124))
        w_, s_, b_ = orc.mxfp4_to_affine(packed.reshape(E, nn, kk // 8), e8.reshape(E, nn, kk // 32), BF16)
        qs[n] = orc.QProj(w_, s_, b_, 4, 32, BF16, out_bias=store(rng.normal(0, 0.1, (E, nn)), BF16))
    spec = LayerSpec(H, E, k, I, BF16, router_weight=store(rng.normal(0, 0.1, (E, H)), BF16),
                     router_dt=BF16, gating=orc.TOPK_THEN_SOFTMAX, gate=qs["g"], up=qs["u"],
                     down=qs["d"], activation=orc.ACT_GPTOSS)
    x = spec.x(6)
    y, _, idx, w = orc.moe_layer(spec, x)
    check_close(load(y, BF16), gptoss_composition(spec, x, idx, w), BF16, "composition")


@pytest.mark.gpu
def test_transcode_tiny_exponents():
    """e8m0 0..2 (magnitudes below 2^-124): finite scales and biases, codes
    in range; bit-exactness is not claimed there."""
    torch = _torch()
    G = 3000
    packed, e8, _ = random_groups(G, seed=21, e_range=(0, 3))
    pt = torch.from_numpy(packed.view(np.int32)).cuda()
    et = torch.from_numpy(e8).cuda()
    ow = torch.empty_like(pt)
    s = torch.empty(G, dtype=torch.float32, device="cuda")
    b = torch.empty(G, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().moe_mxfp4_to_affine(
        C.c_void_p(pt.data_ptr()), C.c_void_p(et.data_ptr()), G, C.c_void_p(ow.data_ptr()),
        C.c_void_p(s.data_ptr()), C.c_void_p(b.data_ptr()), F32,
        C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert torch.isfinite(s).all() and torch.isfinite(b).all()
    assert (s.abs() < 1e-36).all() and (b.abs() < 1e-36).all()

