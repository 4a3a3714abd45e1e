"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the
checker: the reference's own known-answer vectors (tests/golden/
reference_kats.json), independent formulations of the formats, brute force
and closed forms. CPU only."""
import json
import math
import os

import numpy as np
import pytest

import oracle as orc
from moe_spec import check_close

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


# ------------------------------------------------------------ conversions --

def _bf16_nearest(x: np.ndarray) -> np.ndarray:
    """bf16 RNE by explicit nearest-neighbour search in float64 (independent
    of the bit-bias trick)."""
    x = x.astype(np.float32)
    bits = x.view(np.uint32)
    lo = (bits & 0xFFFF0000).view(np.float32).astype(np.float64)
    step_bits = ((bits & 0xFFFF0000) + 0x10000).astype(np.uint32)
    hi = step_bits.view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dhi = np.abs(xd - lo), np.abs(hi - xd)
    lsb_even = ((bits >> 16) & 1) == 0
    pick_lo = (dlo < dhi) | ((dlo == dhi) & lsb_even)
    out = np.where(pick_lo, bits >> 16, step_bits >> 16).astype(np.uint16)
    return out


def test_bf16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 10, 200000), rng.uniform(-1e-30, 1e-30, 1000)]).astype(np.float32)
    # exact ties: low half 0x8000
    ties = ((rng.integers(0, 128, 1000).astype(np.uint32) << 16) | 0x3F800000 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties])
    got = orc.from_f32(x, orc.BF16)
    assert np.array_equal(got, _bf16_nearest(x))
    # every finite bf16 value round-trips
    allb = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    f = orc.to_f32(allb, orc.BF16)
    finite = np.isfinite(f)
    assert np.array_equal(orc.from_f32(f[finite], orc.BF16), allb[finite])


def test_f16_matches_ieee_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 100, 200000), rng.normal(0, 1e-5, 50000),
                        [65504, 65519.9, 65520, 1e6, -1e6, 6e-8, 2.98e-8, 0.0, -0.0]]).astype(np.float32)
    np.seterr(over="ignore")
    got = orc.from_f32(x, orc.F16)
    assert np.array_equal(got.view(np.uint16), x.astype(np.float16).view(np.uint16))
    allh = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = orc.to_f32(allh, orc.F16)
    assert np.array_equal(f[np.isfinite(f)], allh.astype(np.float32)[np.isfinite(f)])


def test_expf_within_two_ulp():
    xs = np.concatenate([np.linspace(-87, 88, 20001), np.linspace(-1, 1, 5001)]).astype(np.float32)
    for x in xs[::7]:
        got = orc.expf(float(x))
        ref = math.exp(float(x))
        ulp = math.ulp(np.float32(ref)) if ref > 0 else 1e-45
        ulp32 = float(np.spacing(np.float32(ref)))
        assert abs(got - ref) <= 2 * ulp32, (x, got, ref, ulp)
    assert orc.expf(-100.0) == 0.0


# ------------------------------------------------------------- bit stream --

def _np_unpack(words, bits, n):
    """Little-endian bit stream read through numpy's unpackbits."""
    b = np.unpackbits(np.ascontiguousarray(words, dtype="<u4").view(np.uint8), bitorder="little")
    b = b[: n * bits].reshape(n, bits).astype(np.uint32)
    return (b << np.arange(bits, dtype=np.uint32)).sum(1)


def _bytes_to_words(bs):
    bs = np.asarray(bs, dtype=np.uint8)
    return bs.view("<u4").astype(np.uint32)


# Byte layouts of the reference's test packers
# (Tests/FFAITests/Ops/QuantizedOpsTests.swift:33-121), as vectors of bytes.
def _pack_ref(q, bits):
    q = [int(v) for v in q]
    out = []
    if bits == 4:
        for i in range(0, len(q), 8):
            w = 0
            for j in range(8):
                w |= (q[i + j] & 0xF) << (4 * j)
            out += list(int(w).to_bytes(4, "little"))
    elif bits == 8:
        for i in range(0, len(q), 4):
            out += [q[i + j] & 0xFF for j in range(4)]
    elif bits == 2:
        for i in range(0, len(q), 16):
            w = 0
            for j in range(16):
                w |= (q[i + j] & 3) << (2 * j)
            out += list(int(w).to_bytes(4, "little"))
    elif bits == 6:
        for p in range(0, len(q), 4):
            v0, v1, v2, v3 = (q[p + j] & 0x3F for j in range(4))
            out += [(v0 | ((v1 & 3) << 6)) & 0xFF, (((v1 >> 2) & 15) | ((v2 & 15) << 4)) & 0xFF,
                    (((v2 >> 4) & 3) | (v3 << 2)) & 0xFF]
    elif bits == 3:
        for c in range(0, len(q), 8):
            v = [q[c + j] & 7 for j in range(8)]
            out += [(v[0] | (v[1] << 3) | ((v[2] & 3) << 6)) & 0xFF,
                    (((v[2] >> 2) & 1) | (v[3] << 1) | (v[4] << 4) | ((v[5] & 1) << 7)) & 0xFF,
                    (((v[5] >> 1) & 3) | (v[6] << 2) | (v[7] << 5)) & 0xFF]
    elif bits == 5:
        for c in range(0, len(q), 8):
            v = [q[c + j] & 31 for j in range(8)]
            out += [(v[0] | ((v[1] & 7) << 5)) & 0xFF,
                    (((v[1] >> 3) & 3) | (v[2] << 2) | ((v[3] & 1) << 7)) & 0xFF,
                    (((v[3] >> 1) & 15) | ((v[4] & 15) << 4)) & 0xFF,
                    (((v[4] >> 4) & 1) | (v[5] << 1) | ((v[6] & 3) << 6)) & 0xFF,
                    (((v[6] >> 2) & 7) | (v[7] << 3)) & 0xFF]
    return _bytes_to_words(out)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_pack_matches_reference_packers(bits):
    rng = np.random.default_rng(bits)
    n = 64 * 5
    q = rng.integers(0, 1 << bits, n).astype(np.uint8)
    ref = _pack_ref(q, bits)
    got = orc.pack_codes(q, bits)
    assert np.array_equal(got, ref)
    assert np.array_equal(orc.unpack_codes(ref, bits, n), q)
    assert np.array_equal(_np_unpack(ref, bits, n), q)
    # every code value in every position
    q2 = (np.arange(n) % (1 << bits)).astype(np.uint8)
    assert np.array_equal(orc.unpack_codes(_pack_ref(q2, bits), bits, n), q2)


def test_dequant_int2_kat():
    g = GOLD["dequant_int2"]
    codes = np.array([i % 4 for i in range(16)], dtype=np.uint8)
    w = orc.pack_codes(codes, 2)
    out = orc.dequantize_affine(w, np.array([g["scale"]], np.float32), np.array([g["bias"]], np.float32),
                                orc.F32, 2, g["group_size"], 16)
    assert np.allclose(out, [0.5 * (i % 4) - 1 for i in range(16)], atol=g["tol"])


def test_dequant_validation_rules():
    w = np.zeros(16, np.uint32)
    s = np.ones(8, np.float32)
    with pytest.raises(ValueError):  # gs not a multiple of pack factor for 4-bit
        orc.dequantize_affine(w, s, s, orc.F32, 4, 4, 64)
    with pytest.raises(ValueError):  # 3-bit needs gs*bits % 32 == 0
        orc.dequantize_affine(w, s, s, orc.F32, 3, 16, 64)
    with pytest.raises(ValueError):
        orc.dequantize_affine(w, s, s, orc.F32, 7, 64, 64)
    assert orc.packed_u32_count(64, 3) == 6
    assert orc.packed_u32_count(10, 3) == -1


def test_derive_bits_kat():
    g = GOLD["derive_bits"]
    for in_f, bits in g["cases"]:
        assert orc.derive_bits(in_f * bits // 32, in_f // g["group_size"], g["group_size"]) == bits
    assert orc.derive_bits(7, 1, 64) == -1


# ----------------------------------------------------------------- router --

_GATING = {"softmaxThenTopK": orc.SOFTMAX_THEN_TOPK, "topKThenSoftmax": orc.TOPK_THEN_SOFTMAX}


@pytest.mark.parametrize("case", GOLD["router"], ids=lambda c: c["src"].split("/")[-1])
def test_router_kats(case):
    idx, w = orc.route(np.array(case["logits"], np.float32), case["k"], _GATING[case["gating"]],
                       case["norm"])
    idx, w = idx[0].tolist(), w[0]
    if "idx" in case:
        assert idx == case["idx"]
    if "idx_set" in case:
        assert set(idx) == set(case["idx_set"])
    if "w" in case:
        assert np.allclose(w, case["w"], atol=case["tol"])
    if case.get("sum_to_one"):
        assert abs(w.sum() - 1) < 1e-5
    if "sum_below" in case:
        assert w.sum() < case["sum_below"]
    if "w_of_1_above" in case:
        assert w[idx.index(1)] > case["w_of_1_above"]


def _brute_topk(v, k):
    order = sorted(range(len(v)), key=lambda i: (-float(v[i]), i))
    return order[:k]


@pytest.mark.parametrize("E,k", [(8, 2), (32, 4), (128, 8), (256, 8), (7, 7)])
def test_router_matches_brute_force(E, k):
    rng = np.random.default_rng(E * 31 + k)
    T = 64
    # small-integer logits make ties common
    logits = rng.integers(-3, 4, size=(T, E)).astype(np.float32)
    logits[::2] = orc.round_dt(rng.normal(0, 1, size=(T // 2, E)), orc.BF16)
    bias = rng.normal(0, 0.01, size=E).astype(np.float32)
    for gating, norm, eb in [(orc.SOFTMAX_THEN_TOPK, True, None), (orc.TOPK_THEN_SOFTMAX, True, None),
                             (orc.SOFTMAX_THEN_TOPK, False, None), (orc.SOFTMAX_THEN_TOPK, True, bias)]:
        idx, w = orc.route(logits, k, gating, norm, eb)
        for t in range(T):
            l = logits[t]
            if gating == orc.TOPK_THEN_SOFTMAX or (norm and eb is None):
                sel = _brute_topk(l, k)
                p = np.exp(l[sel].astype(np.float64) - l[sel].max())
                ref = p / p.sum()
            else:
                p = np.exp(l.astype(np.float64) - l.max())
                p = (p / p.sum()).astype(np.float32)
                gp = orc.softmax(l)
                assert np.allclose(gp, p, rtol=2e-5, atol=1e-9)
                if eb is not None:
                    gp = gp + eb
                sel = _brute_topk(gp, k)
                ref = gp[sel].astype(np.float64)
                if norm:
                    ref = ref / ref.sum()
            assert idx[t].tolist() == sel
            assert np.allclose(w[t], ref, rtol=2e-5, atol=1e-9)


def _np_sigmoid_route(l, k, norm, eb, rs):
    """NemotronHText.swift:844-867 restated with a full stable sort; the
    sigmoid uses the pinned exp (or_expf, within 2 ulp of exp)."""
    raw = np.array([np.float32(1.0) / (np.float32(1.0) + np.float32(orc.expf(-float(v))))
                    for v in l], np.float32)
    score = raw + eb if eb is not None else raw
    sel = _brute_topk(score, k)
    fw = raw[sel].astype(np.float32)
    if k > 1 and norm:
        s = np.float32(0)
        for v in fw:
            s = np.float32(s + v)
        fw = fw / np.float32(s + np.float32(1e-20))
    return sel, (fw * np.float32(rs)).astype(np.float32), raw


@pytest.mark.parametrize("E,k", [(8, 1), (32, 4), (64, 6), (128, 8), (256, 8)])
@pytest.mark.parametrize("norm,bias,rs", [(True, True, 2.5), (True, False, 1.0), (False, True, 1.0)])
def test_sigmoid_router_matches_brute_force(E, k, norm, bias, rs):
    rng = np.random.default_rng(E * 7 + k)
    T = 48
    logits = rng.integers(-3, 4, size=(T, E)).astype(np.float32)
    logits[::2] = orc.round_dt(rng.normal(0, 1.5, size=(T // 2, E)), orc.BF16)
    eb = rng.uniform(-0.05, 0.05, size=E).astype(np.float32) if bias else None
    idx, w = orc.route(logits, k, orc.SIGMOID_TOPK, norm, eb, routed_scale=rs)
    for t in range(T):
        sel, ref, raw = _np_sigmoid_route(logits[t], k, norm, eb, rs)
        assert idx[t].tolist() == sel
        assert np.array_equal(w[t], ref)
        # invariants the reference fixes: the weights follow the unbiased
        # sigmoid of the picked logits; renormalised ones sum to the routed
        # scale; a single pick is never renormalised
        p = 1.0 / (1.0 + np.exp(-logits[t, sel].astype(np.float64)))
        if k > 1 and norm:
            assert abs(float(w[t].astype(np.float64).sum()) - rs) < 1e-5 * rs
            assert np.allclose(w[t], rs * p / p.sum(), rtol=1e-5)
        else:
            assert np.allclose(w[t], rs * p, rtol=1e-5)
    if bias:
        # the correction bias steers the selection but never the weights: a
        # router that weighted by the biased score would differ here
        biased = np.array([[(1 / (1 + math.exp(-float(logits[t, e])))) + eb[e] for e in idx[t]]
                           for t in range(T)])
        assert not np.allclose(w / rs, biased / (biased.sum(1, keepdims=True) if norm and k > 1 else 1),
                               rtol=1e-3)


def test_logit_and_expert_scales():
    """Gemma 4 routing (Gemma4Text.swift:938-950): top-k of hidden^-0.5-scaled
    logits, softmax over the k, times per_expert_scale[e]."""
    rng = np.random.default_rng(11)
    T, E, k = 32, 64, 8
    logits = orc.round_dt(rng.normal(0, 20, size=(T, E)), orc.BF16)
    ls = float(np.float32(2816 ** -0.5))
    es = rng.uniform(0.5, 1.5, size=E).astype(np.float32)
    idx, w = orc.route(logits, k, orc.TOPK_THEN_SOFTMAX, True, logit_scale=ls, expert_scale=es)
    idx0, w0 = orc.route(logits, k, orc.TOPK_THEN_SOFTMAX, True, logit_scale=ls)
    assert np.array_equal(idx, idx0)
    assert np.array_equal(w, (w0 * es[idx]).astype(np.float32))
    for t in range(T):
        sel = _brute_topk(logits[t], k)  # a positive scale keeps the order
        z = logits[t, sel].astype(np.float64) * ls
        p = np.exp(z - z.max())
        assert idx[t].tolist() == sel
        assert np.allclose(w0[t], p / p.sum(), rtol=2e-5)
        # the scale sets the temperature: unscaled logits give other weights
        q = np.exp(logits[t, sel].astype(np.float64) - logits[t, sel].max())
        assert not np.allclose(w0[t], q / q.sum(), rtol=1e-2)
    # the per-expert scale applies after the softmax: the scaled weights no
    # longer sum to one
    assert not np.allclose(w.sum(1), 1.0, atol=1e-3)


def test_softmax_degenerate_is_uniform():
    out = orc.softmax(np.full(5, -np.inf, np.float32))
    assert np.allclose(out, 0.2)


# ------------------------------------------------------------------- plan --

@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (16, 2, 8), (64, 8, 128), (300, 8, 256), (5, 4, 4)])
def test_dispatch_plan_brute_force(T, k, E):
    rng = np.random.default_rng(T + k + E)
    idx = rng.integers(0, E, size=(T, k)).astype(np.uint32)
    counts, offsets, perm, inv = orc.dispatch_plan(idx, E)
    flat = idx.ravel()
    ref_perm = sorted(range(T * k), key=lambda m: (int(flat[m]), m))
    assert perm.tolist() == ref_perm
    assert np.array_equal(inv[perm], np.arange(T * k))
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets.astype(np.int64)), counts)


# ------------------------------------------------------------ grouped GEMM --

def _dense(words, scales, biases, bits, gs, N, K):
    codes = _np_unpack(words.ravel(), bits, N * K).reshape(N, K).astype(np.float32)
    s = np.repeat(scales.reshape(N, K // gs), gs, axis=1).astype(np.float32)
    b = np.repeat(biases.reshape(N, K // gs), gs, axis=1).astype(np.float32)
    return (s * codes + b).astype(np.float64)


@pytest.mark.parametrize("cell", GOLD["bgemm_cells"], ids=lambda c: c["src"].split(":")[-1])
def test_qgemm_reference_generator_cells(cell):
    """MoEBgemmBm64MppTests.swift:159-271 generator; the oracle's grouped
    product against a float64 matmul of the independently dequantised
    weights (cos >= 0.99 is the reference bar; this asserts 1e-5)."""
    E, M, N, K, gs = cell["E"], cell["M"], cell["N"], cell["K"], cell["gs"]
    sW, sS, sB, sX = cell["seeds"]
    if cell["sparse"]:
        ind = np.sort([(r * (E // max(M, 1))) % E for r in range(M)]).astype(np.uint32)
    else:
        ind = np.array([r // (M // E) for r in range(M)], dtype=np.uint32)
    i = np.arange(E * N * K, dtype=np.int64)
    codes = ((i * sW + 3) & 0xF).astype(np.uint8).reshape(E, N, K)
    g = np.arange(E * N * (K // gs), dtype=np.int64)
    scales = (0.005 + 0.001 * ((g * sS) % 137) / 137.0).astype(np.float32).reshape(E, N, K // gs)
    biases = (-0.02 + 0.005 * ((g * sB) % 149) / 149.0).astype(np.float32).reshape(E, N, K // gs)
    x = (0.05 * ((np.arange(M * K) * sX) % 223) / 223.0 - 0.025).astype(np.float32).reshape(M, K)
    w = orc.pack_codes(codes.reshape(E * N, K), 4).reshape(E, N, K // 8)
    p = orc.QProj(w, scales, biases, 4, gs, orc.F32)
    got = orc.qgemm_rows(p, x, ind)
    ref = np.zeros((M, N))
    for e in np.unique(ind):
        rows = ind == e
        ref[rows] = x[rows].astype(np.float64) @ _dense(w[e], scales[e], biases[e], 4, gs, N, K).T
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)
    cos = float((got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    assert cos >= cell["cos_min"]


def _bf_trunc(a):
    return (np.asarray(a, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)


def _expr(e, **v):
    return eval(e, {"__builtins__": {}}, v)


@pytest.mark.parametrize("cell", GOLD["gemv_cells"], ids=lambda c: f"bits{c['bits']}")
def test_gemv_reference_cells(cell):
    """QuantizedOpsTests.swift:126-438: per-bit dequant GEMV cells."""
    bits, OUT, IN, gs = cell["bits"], cell["out"], cell["in"], cell["gs"]
    q = np.array([[_expr(cell["q"], j=j, r=r) for j in range(IN)] for r in range(OUT)], np.uint8)
    ng = IN // gs
    per_group = "i" in cell["scale"]
    n_sb = OUT * ng if per_group else OUT
    sc = np.array([_expr(cell["scale"], i=i, r=i) for i in range(n_sb)], np.float32)
    bi = np.array([_expr(cell["bias"], i=i, r=i) for i in range(n_sb)], np.float32)
    x = np.array([_expr(cell["x"], j=j) for j in range(IN)], np.float32)
    if cell["sb"] == "bf16_trunc":
        sc, bi, x = _bf_trunc(sc), _bf_trunc(bi), _bf_trunc(x)
        sb_store = (sc.view(np.uint32) >> 16).astype(np.uint16)
        bb_store = (bi.view(np.uint32) >> 16).astype(np.uint16)
        sb_dt = orc.BF16
    else:
        sb_store, bb_store, sb_dt = sc, bi, orc.F32
    sc2, bi2 = sc.reshape(OUT, -1), bi.reshape(OUT, -1)
    if sc2.shape[1] == 1 and ng > 1:
        sc2, bi2 = np.repeat(sc2, ng, 1), np.repeat(bi2, ng, 1)
        sb_store = np.repeat(sb_store.reshape(OUT, 1), ng, 1)
        bb_store = np.repeat(bb_store.reshape(OUT, 1), ng, 1)
    w = orc.pack_codes(q, bits).reshape(1, OUT, IN * bits // 32)
    p = orc.QProj(w, np.asarray(sb_store).reshape(1, OUT, ng), np.asarray(bb_store).reshape(1, OUT, ng),
                  bits, gs, sb_dt)
    got = orc.qgemm_rows(p, x.reshape(1, IN), np.zeros(1, np.uint32))[0]
    ref = np.array([sum((float(q[r, j]) * float(sc2[r, j // gs]) + float(bi2[r, j // gs])) * float(x[j])
                        for j in range(IN)) for r in range(OUT)])
    tol = cell["tol"]
    for r in range(OUT):
        t = tol if isinstance(tol, float) else max(abs(ref[r]) * 0.05, 1.0)
        assert abs(got[r] - ref[r]) < t
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("cell", GOLD["gemv_cells"], ids=lambda c: f"bits{c['bits']}")
def test_router_logits_q_reference_cells(cell):
    """The quantised router (QuantizedLinear, Layers.swift:371-400) on the
    reference's per-bit GEMV cells (QuantizedOpsTests.swift:126-438): same
    products as or_qgemm_rows, one row per expert, f32 rows so nothing rounds
    after the dot product."""
    bits, OUT, IN, gs = cell["bits"], cell["out"], cell["in"], cell["gs"]
    q = np.array([[_expr(cell["q"], j=j, r=r) for j in range(IN)] for r in range(OUT)], np.uint8)
    ng = IN // gs
    n_sb = OUT * ng if "i" in cell["scale"] else OUT
    sc = np.array([_expr(cell["scale"], i=i, r=i) for i in range(n_sb)], np.float32)
    bi = np.array([_expr(cell["bias"], i=i, r=i) for i in range(n_sb)], np.float32)
    x = np.array([_expr(cell["x"], j=j) for j in range(IN)], np.float32)
    if cell["sb"] == "bf16_trunc":
        sc, bi, x = _bf_trunc(sc), _bf_trunc(bi), _bf_trunc(x)
    sc2, bi2 = sc.reshape(OUT, -1), bi.reshape(OUT, -1)
    if sc2.shape[1] == 1 and ng > 1:
        sc2, bi2 = np.repeat(sc2, ng, 1), np.repeat(bi2, ng, 1)
    w = orc.pack_codes(q, bits).reshape(1, OUT, IN * bits // 32)
    p = orc.QProj(w, np.ascontiguousarray(sc2.reshape(1, OUT, ng)),
                  np.ascontiguousarray(bi2.reshape(1, OUT, ng)), bits, gs, orc.F32)
    got = orc.router_logits_q(x.reshape(1, IN), orc.F32, p)[0]
    ref = np.array([sum((float(q[r, j]) * float(sc2[r, j // gs]) + float(bi2[r, j // gs])) * float(x[j])
                        for j in range(IN)) for r in range(OUT)])
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-4)
    assert np.array_equal(got, orc.qgemm_rows(p, x.reshape(1, IN), np.zeros(1, np.uint32))[0])


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_router_logits_q_equals_dense_restatement(bits):
    """The quantised router equals the dense router run on the stream's own
    dequantisation (or_dequantize_affine, an independent unpack of the bit
    stream) bit for bit, bias double rounding included; a router whose groups
    are read with the wrong group size does not."""
    from moe_spec import affine_quantize
    rng = np.random.default_rng(bits)
    E, H, gs = 24, 256, 64
    q = affine_quantize(rng.normal(0, 1 / 16, size=(E, H)), bits, gs, orc.BF16)
    x = orc.from_f32(rng.normal(0, 1, size=(5, H)).astype(np.float32), orc.BF16)
    b = orc.from_f32(rng.normal(0, 0.1, size=E).astype(np.float32), orc.BF16)
    dense = orc.dequantize_affine(q.weight, q.scales, q.biases, q.sb_dt, bits, gs, E * H)
    ref = orc.router_logits(x, orc.BF16, np.ascontiguousarray(dense, np.float32).reshape(E, H),
                            orc.F32, b)
    got = orc.router_logits_q(x, orc.BF16, q, b)
    assert np.array_equal(got, ref)
    wrong = orc.QProj(q.weight, q.scales.reshape(1, E, -1)[:, :, : H // 128].copy(),
                      q.biases.reshape(1, E, -1)[:, :, : H // 128].copy(), bits, 128, q.sb_dt)
    assert not np.array_equal(orc.router_logits_q(x, orc.BF16, wrong, b), ref)


# ------------------------------------------------ activations / combine ----

def test_swiglu_kat():
    g = GOLD["swiglu"]
    for gv, uv in zip(g["gate"], g["up"]):
        assert abs(orc.act(gv, uv) - uv * gv / (1 + math.exp(-gv))) < 1e-5


def test_gptoss_activation_closed_form():
    a, lim = 1.702, 7.0
    for gv, uv in [(0.5, 0.3), (9.0, 2.0), (-9.0, 2.0), (1.0, 8.0), (1.0, -8.0), (7.0, -7.0), (-0.2, 0.0)]:
        gc = min(gv, lim)  # upper clamp only on the gate
        uc = min(max(uv, -lim), lim)
        ref = gc / (1 + math.exp(-a * gc)) * (uc + 1)
        assert abs(orc.act(gv, uv, orc.ACT_GPTOSS, a, lim) - ref) < 1e-5 * max(1, abs(ref))


def test_gelu_kat():
    """The reference's GELU test (OpsTests.swift:254-302): the tanh form
    within 1e-3 at its four points, finite in bf16 over [-15, 15]."""
    g = GOLD["gelu"]
    c = math.sqrt(2.0 / math.pi)
    for v in g["x"]:
        ref = 0.5 * v * (1 + math.tanh(c * (v + 0.044715 * v ** 3)))
        assert abs(orc.gelu(v) - ref) < g["tol"]
    sw = g["bf16_finite_sweep"]
    xs = np.arange(sw["from"], sw["through"] + sw["by"] / 2, sw["by"])
    for v in orc.round_dt(xs, orc.BF16):
        out = orc.act(float(v), 1.0, orc.ACT_GEGLU, dt=orc.BF16)
        assert math.isfinite(out)
        ref = 0.5 * v * (1 + math.tanh(c * (v + 0.044715 * v ** 3)))
        assert abs(out - ref) <= 2 ** -7 * abs(ref) + 1e-6
    # the erf form differs from the tanh form by more than a bf16 ulp near
    # x = -2.5 .. -3.5: the oracle follows the tanh form
    v = -3.0
    erf_form = 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
    assert abs(orc.gelu(v) - erf_form) > 1e-4


def test_geglu_and_relu2_closed_forms():
    # GEGLU stores the GELU in the activation dtype before the product
    # (Gemma4Text.swift:965)
    for gv, uv in [(0.7, 3.0), (-1.3, 2.5), (2.2, -0.9), (9.0, 1.5)]:
        gl = float(orc.round_dt(np.array([orc.gelu(gv)], np.float32), orc.BF16)[0])
        assert orc.act(gv, uv, orc.ACT_GEGLU, dt=orc.BF16) == np.float32(gl * uv)
        assert orc.act(gv, uv, orc.ACT_GEGLU) == np.float32(np.float32(orc.gelu(gv)) * np.float32(uv))
    # squared ReLU of the up projection; no gate (NemotronHText.swift:759-760)
    for gv, uv in [(5.0, 1.5), (-5.0, 1.5), (0.0, -2.0), (1.0, 0.0), (3.0, -0.25)]:
        assert orc.act(gv, uv, orc.ACT_RELU2) == np.float32(max(uv, 0.0) ** 2)


def _add_rmsnorm_inputs(g):
    n, rows = g["n"], g["n_rows"]
    a = np.array([_expr(g["a"], i=i) for i in range(rows * n)], np.float32).reshape(rows, n)
    b = np.array([_expr(g["b"], i=i) for i in range(rows * n)], np.float32).reshape(rows, n)
    w = np.array([_expr(g["w"], d=d) for d in range(n)], np.float32)
    return a, b, w


def test_add_rmsnorm_kat():
    """The reference's addAndRmsNorm test (OpsTests.swift:1009-1060) with its
    own generators and tolerances."""
    g = GOLD["add_rmsnorm"]
    a, b, w = _add_rmsnorm_inputs(g)
    res, xn = orc.add_rmsnorm(a, b, w, g["eps"])
    s = a.astype(np.float64) + b
    rms = np.sqrt((s * s).mean(axis=1, keepdims=True) + g["eps"])
    assert np.all(np.abs(res - s) < g["tol_residual"])
    assert np.all(np.abs(xn - s / rms * w) < g["tol_normed"])
    # a norm over the sum instead of the mean, or without the weight, fails
    assert not np.all(np.abs(xn - s / np.sqrt((s * s).sum(1, keepdims=True)) * w) < g["tol_normed"])
    assert not np.all(np.abs(xn - s / rms) < g["tol_normed"])


def test_rmsnorm_kat():
    """OpsTests.swift:439-468: x = 1..128, weight 1, y = x / rms(x)."""
    g = GOLD["rmsnorm"]
    x = np.array([_expr(g["x"], i=i) for i in range(g["n"])], np.float32)
    _, xn = orc.add_rmsnorm(x, np.zeros_like(x), np.full(g["n"], g["w"], np.float32), g["eps"])
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean())
    assert np.all(np.abs(xn[0] - ref) < g["tol"])


def test_add_rmsnorm_bf16_rounding():
    """The residual and the normalised row are each stored in the dtype."""
    rng = np.random.default_rng(4)
    a = orc.round_dt(rng.normal(size=(3, 256)), orc.BF16)
    b = orc.round_dt(rng.normal(size=(3, 256)), orc.BF16)
    w = orc.round_dt(rng.uniform(0.5, 1.5, 256), orc.BF16)
    res, xn = orc.add_rmsnorm(a, b, w, 1e-6, orc.BF16)
    assert np.array_equal(res, orc.round_dt(a + b, orc.BF16))
    assert np.array_equal(xn, orc.round_dt(xn, orc.BF16))
    ref = res / np.sqrt((res.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.all(np.abs(xn - ref) <= 2 ** -8 * np.abs(ref) + 1e-30)


def test_sigmoid_fma_residual_kat():
    """OpsSpecialPathTests.swift:357-382."""
    g = GOLD["sigmoid_fma_residual"]
    gate = 1.0 / (1.0 + math.exp(-g["gate"]))
    out = orc.residual_combine(g["residual"], g["base"], g["value"], gate)
    assert np.all(np.abs(out - np.array(g["out"])) < g["tol"])
    # without the residual it is sigmoidScalarFMA; without a value the plain add
    assert np.allclose(orc.residual_combine(None, g["base"], g["value"], gate), [11, 22, 33, 44])
    assert np.allclose(orc.residual_combine(g["residual"], g["base"]), [110, 220, 330, 440])


def test_unpermute_kat():
    g = GOLD["unpermute"]
    Y = np.array(g["expert_outputs"], np.float32)
    out = orc.unpermute(Y, np.array(g["inv_perm"], np.uint32), np.array(g["weights"], np.float32),
                        g["T"], Y.shape[1], g["k"], orc.F32)
    assert np.allclose(out, g["out"], atol=g["tol"])


# ------------------------------------------------------------ whole layer --

def scalar_layer_spec(shared: bool):
    """The reference's 4-expert top-2 scalar KAT (MoELayerTests.swift:
    147-265) in mlx-affine form: hidden = intermediate = 64 with every
    weight zero except element [0,0]; that element is the scalar, encoded as
    code 1 times a group scale equal to the scalar (bias 0)."""
    from moe_spec import LayerSpec
    g = GOLD["layer_scalar"]
    H = I = 64
    E = 4

    def proj(vals, n, kk):
        E_ = len(vals)
        codes = np.zeros((E_ * n, kk), np.uint8)
        scales = np.zeros((E_, n, kk // 64), np.float32)
        for e, v in enumerate(vals):
            codes[e * n, 0] = 1
            scales[e, 0, 0] = v
        w = orc.pack_codes(codes, 4).reshape(E_, n, kk // 8)
        return orc.QProj(w, scales, np.zeros_like(scales), 4, 64, orc.F32)

    rw = np.zeros((E, H), np.float32)
    rw[:, 0] = g["gate_w"]
    sh = None
    if shared:
        sh = (proj([g["shared"]["g"]], I, H), proj([g["shared"]["u"]], I, H), proj([g["shared"]["d"]], H, I))
    return LayerSpec(H, E, 2, I, orc.F32, router_weight=rw, router_dt=orc.F32,
                     gate=proj(g["g"], I, H), up=proj(g["u"], I, H), down=proj(g["d"], H, I),
                     shared=sh, name="scalar")


def scalar_layer_expected(shared: bool):
    g = GOLD["layer_scalar"]
    x = g["x"]

    def swiglu_ref(gw, uw, dw):
        gx = gw * x
        return dw * (gx / (1 + math.exp(-gx)) * (uw * x))

    e1, e2 = g["experts"]
    out = g["w1"] * swiglu_ref(g["g"][e1], g["u"][e1], g["d"][e1]) + \
        g["w2"] * swiglu_ref(g["g"][e2], g["u"][e2], g["d"][e2])
    if shared:
        out += swiglu_ref(g["shared"]["g"], g["shared"]["u"], g["shared"]["d"])
    return out


@pytest.mark.parametrize("shared", [False, True])
def test_layer_scalar_kat(shared):
    spec = scalar_layer_spec(shared)
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = GOLD["layer_scalar"]["x"]
    y, logits, idx, w = orc.moe_layer(spec, x)
    assert idx[0].tolist() == GOLD["layer_scalar"]["experts"]
    assert np.allclose(logits[0], [1, 3, 2, 0])
    assert abs(y[0, 0] - scalar_layer_expected(shared)) < GOLD["layer_scalar"]["tol"]
    assert np.all(y[0, 1:] == 0)


def test_layer_given_logits_path_is_identical():
    from moe_spec import cfg_tiny
    spec = cfg_tiny()
    x = spec.x(16)
    y, logits, idx, w = orc.moe_layer(spec, x)
    y2, _, idx2, w2 = orc.moe_layer(spec, x, given_logits=logits)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16))
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)


def test_layer_tiny_matches_float64_composition():
    """Whole tiny layer against a float64 composition of
    independently dequantised experts with the same storage rounding points."""
    from moe_spec import cfg_tiny, load, store
    spec = cfg_tiny()
    x = spec.x(16)
    y, logits, idx, w = orc.moe_layer(spec, x)
    xf = load(x, spec.act_dt).astype(np.float64)
    rw = load(spec.router_weight, spec.router_dt).astype(np.float64)
    ref_logits = load(store(xf @ rw.T, spec.act_dt), spec.act_dt)
    assert np.array_equal(ref_logits, logits)
    H, I = spec.hidden, spec.intermediate
    rd = lambda a: load(store(a, spec.act_dt), spec.act_dt).astype(np.float64)  # noqa: E731
    ref = np.zeros((16, H))
    for t in range(16):
        acc = np.zeros(H, np.float32)
        for s in range(spec.top_k):
            e = idx[t, s]
            G = _dense(spec.gate.weight[e], load(spec.gate.scales[e], orc.F16), load(spec.gate.biases[e], orc.F16), 4, 64, I, H)
            U = _dense(spec.up.weight[e], load(spec.up.scales[e], orc.F16), load(spec.up.biases[e], orc.F16), 4, 64, I, H)
            D = _dense(spec.down.weight[e], load(spec.down.scales[e], orc.F16), load(spec.down.biases[e], orc.F16), 4, 64, H, I)
            g, u = rd(G @ xf[t]), rd(U @ xf[t])
            a = rd(g / (1 + np.exp(-g)) * u)
            yv = rd(D @ a)
            acc = acc + np.float32(rd(np.float32(w[t, s]))) * yv.astype(np.float32)
        ref[t] = rd(acc)
    check_close(load(y, spec.act_dt), ref, spec.act_dt, "tiny layer vs float64 composition")


def _composition(spec, x, idx, w, rx=None):
    """float64 composition of independently dequantised experts with the
    storage rounding points of the reference: gate/up (or the single up
    projection) rounded, the activation rounded, down rounded, the combine in
    f32 with each weight rounded, then the shared expert added."""
    from moe_spec import load, store
    T, H, I = x.shape[0], spec.hidden, spec.intermediate
    xf = load(x, spec.act_dt).astype(np.float64)
    rd = lambda a: load(store(a, spec.act_dt), spec.act_dt).astype(np.float64)  # noqa: E731

    def dense(q, e, n, kk):
        return _dense(q.weight[e], load(q.scales[e], q.sb_dt), load(q.biases[e], q.sb_dt), q.bits,
                      q.gs, n, kk)

    def expert(gq, uq, dq, e, xv, n):
        u = rd(dense(uq, e, n, spec.hidden) @ xv)
        if spec.activation == orc.ACT_RELU2:
            a = rd(np.maximum(u, 0.0) ** 2)
        elif spec.activation == orc.ACT_GEGLU:
            g = rd(dense(gq, e, n, spec.hidden) @ xv)
            c = math.sqrt(2.0 / math.pi)
            a = rd(rd(0.5 * g * (1 + np.tanh(c * (g + 0.044715 * g ** 3)))) * u)
        else:
            g = rd(dense(gq, e, n, spec.hidden) @ xv)
            a = rd(g / (1 + np.exp(-g)) * u)
        return rd(dense(dq, e, spec.hidden, n) @ a)

    ref = np.zeros((T, H))
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(spec.top_k):
            e = idx[t, s]
            yv = expert(spec.gate, spec.up, spec.down, e, xf[t], I)
            acc = acc + np.float32(rd(np.float32(w[t, s]))) * yv.astype(np.float32)
        out = rd(acc)
        if spec.shared is not None:
            sg, su, sd = spec.shared
            out = rd(out + expert(sg, su, sd, 0, xf[t], su.n))
        ref[t] = out
    return ref


@pytest.mark.parametrize("family", ["nemotron", "gemma4"])
def test_layer_family_matches_float64_composition(family):
    """NemotronH (sigmoid router, squared-ReLU experts without a gate,
    squared-ReLU shared expert, routed scale) and Gemma 4 (scaled logits,
    per-expert scale, GELU-gated experts, a router input of its own) layers
    against the float64 composition, with routing from the numpy
    restatements above."""
    from moe_spec import cfg_gemma4, cfg_nemotron, load
    spec = (cfg_nemotron(hidden=256, inter=128, shared_inter=192, n_experts=16, top_k=4)
            if family == "nemotron" else cfg_gemma4(hidden=256, inter=128, n_experts=16, top_k=4))
    T = 6
    x = spec.x(T)
    rx = spec.router_x(T)
    y, logits, idx, w = orc.moe_layer(spec, x, router_x=rx)
    lx = x if rx is None else rx
    ref_logits = orc.router_logits(lx, spec.act_dt, spec.router_weight, spec.router_dt)
    assert np.array_equal(ref_logits, logits)
    for t in range(T):
        if family == "nemotron":
            sel, ref_w, _ = _np_sigmoid_route(logits[t], spec.top_k, True, spec.expert_bias,
                                              spec.routed_scale)
        else:
            sel = _brute_topk(logits[t], spec.top_k)
            z = logits[t, sel].astype(np.float64) * spec.logit_scale
            p = np.exp(z - z.max())
            ref_w = (p / p.sum()) * spec.expert_scale[sel]
        assert idx[t].tolist() == sel
        assert np.allclose(w[t], ref_w, rtol=2e-5)
    ref = _composition(spec, x, idx, w)
    check_close(load(y, spec.act_dt), ref, spec.act_dt, f"{family} layer vs float64 composition")
    if family == "gemma4":
        # routing on the expert input instead of the router's rows is caught
        y_same = orc.moe_layer(spec, x)[0]
        assert not np.array_equal(y_same.view(np.uint16), y.view(np.uint16))


@pytest.mark.parametrize("shared", [False, True])
def test_layer_residual_composes(shared):
    """The block between the decoder steps: residual and normalised rows from
    the pinned add + RMSNorm, the block on the normalised rows, and (without
    a shared expert) y = round(residual + block output) exactly."""
    from moe_spec import cfg_tiny, load, store
    import copy
    spec = cfg_tiny()
    if shared:
        spec = copy.copy(spec)
        spec.shared = (spec.gate, spec.up, spec.down)
        spec.shared = tuple(orc.QProj(q.weight[:1], q.scales[:1], q.biases[:1], q.bits, q.gs, q.sb_dt)
                            for q in spec.shared)
    rng = np.random.default_rng(9)
    T, H = 5, spec.hidden
    h = spec.x(T, seed=1)
    m = store(rng.normal(0, 0.5, size=(T, H)), spec.act_dt)
    nw = load(store(rng.uniform(0.5, 1.5, H), spec.act_dt), spec.act_dt)
    y, xn, res, logits, idx, w = orc.moe_layer_residual(spec, h, m, nw, 1e-6)
    r2, xn2 = orc.add_rmsnorm(load(h, spec.act_dt), load(m, spec.act_dt), nw, 1e-6, spec.act_dt)
    assert np.array_equal(res, r2) and np.array_equal(xn, xn2)
    y_plain, logits2, idx2, w2 = orc.moe_layer(spec, store(xn, spec.act_dt))
    assert np.array_equal(logits, logits2) and np.array_equal(idx, idx2)
    if not shared:
        assert np.array_equal(load(y, spec.act_dt),
                              orc.round_dt(res + load(y_plain, spec.act_dt), spec.act_dt))
    else:
        # the residual joins the shared add's rounding, so only tolerance-close
        check_close(load(y, spec.act_dt), load(y_plain, spec.act_dt) + res, spec.act_dt,
                    "residual with shared expert")


def test_float_bar_catches_planted_mistakes():
    """The layer tolerance passes storage-ulp rounding flips but fails a
    wrong expert and a dropped expert term (mistakes planted in oracle
    outputs on the CPU)."""
    import copy
    from moe_spec import cfg_tiny, load
    spec = cfg_tiny()
    x = spec.x(16)
    y, logits, idx, w = orc.moe_layer(spec, x)
    ref = load(y, spec.act_dt)
    # one-ulp flips on 5% of the elements pass
    rng = np.random.default_rng(3)
    flip = y.copy().view(np.uint16)
    sel = rng.random(flip.shape) < 0.05
    flip[sel] = flip[sel] + np.uint16(1)  # one ulp away from zero, either sign
    check_close(load(flip.view(y.dtype), spec.act_dt), ref, spec.act_dt, "ulp flips")
    # token 0 routed to an expert it did not select
    bad = logits.copy()
    top, other = int(idx[0, 0]), int(next(e for e in range(spec.n_experts) if e not in idx[0]))
    bad[0, top], bad[0, other] = logits[0, other], logits[0, top]
    y_wrong = orc.moe_layer(spec, x, given_logits=bad)[0]
    with pytest.raises(AssertionError):
        check_close(load(y_wrong, spec.act_dt), ref, spec.act_dt, "wrong expert")
    # one expert's down projection dropped (scales and biases zero)
    drop = copy.copy(spec)
    drop.down = copy.copy(spec.down)
    e0 = int(idx[0, 1])
    s, b = spec.down.scales.copy(), spec.down.biases.copy()
    s[e0] = 0
    b[e0] = 0
    drop.down = orc.QProj(spec.down.weight, s, b, spec.down.bits, spec.down.gs, spec.down.sb_dt)
    y_drop = orc.moe_layer(drop, x, given_logits=logits)[0]
    with pytest.raises(AssertionError):
        check_close(load(y_drop, spec.act_dt), ref, spec.act_dt, "dropped expert")
