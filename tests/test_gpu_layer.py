"""GPU parity tests: libmoehip.so through its C ABI against the CPU oracle.

Integer outputs (expert ids, dispatch permutations, unpacked codes) must be
bit-exact; float outputs meet moe_spec.check_close (bf16/f16: max-abs 2e-2 on
the output's RMS scale and 1e-3 mean relative; f32: 1e-3).
Routing is compared at the router input: the oracle routes from the logits
the GPU produced, so ids and weights must match exactly, and the GPU logits
themselves must be within one storage ulp of the oracle's."""
import ctypes as C

import numpy as np
import pytest

import oracle as orc
from moe_spec import (BF16, F16, F32, affine_quantize, cfg_bits, cfg_gemma4, cfg_gptoss, cfg_mixed,
                      cfg_nemotron, cfg_qwen3, cfg_tiny, check_close, gen_qproj, load, store,
                      to_numpy_f32, to_torch, with_quantised_router, zipf_router_bias)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from ffai_amd import _lib  # noqa: E402
from ffai_amd._lib import check  # noqa: E402


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return C.c_void_p(t.data_ptr())


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    _lib.load()
    yield
    torch.cuda.synchronize()


# ------------------------------------------------------------ bit stream --

@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequantize_codes_bit_exact(bits):
    rng = np.random.default_rng(bits)
    n = 64 * 97
    words = rng.integers(0, 2**32, n * bits // 32, dtype=np.uint64).astype(np.uint32)
    ones = np.ones(n // 64, np.float32)
    zeros = np.zeros(n // 64, np.float32)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    # device copies are held in locals: a temporary's memory could be reused
    # by the next allocation before the kernel runs
    wt, onest, zerost = to_torch(words.view(np.int32)), to_torch(ones), to_torch(zeros)
    check(_lib.load().moe_dequantize_affine(_p(wt), _p(onest), _p(zerost), F32, bits, 64, n,
                                            _p(out), F32, _stream()))
    torch.cuda.synchronize()
    codes = orc.unpack_codes(words, bits, n)
    assert np.array_equal(out.cpu().numpy(), codes.astype(np.float32))
    # bf16 scales/biases, bf16 output: the oracle's dequant rounded once
    s = store(rng.uniform(0.005, 0.02, n // 64), BF16)
    b = store(rng.uniform(-0.1, 0.1, n // 64), BF16)
    out2 = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    st, bt = to_torch(s), to_torch(b)
    check(_lib.load().moe_dequantize_affine(_p(wt), _p(st), _p(bt), BF16, bits, 64, n, _p(out2),
                                            BF16, _stream()))
    torch.cuda.synchronize()
    ref = orc.round_dt(orc.dequantize_affine(words, s, b, BF16, bits, 64, n), BF16)
    got = out2.float().cpu().numpy()
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------- router --

@pytest.mark.parametrize("E,k", [(8, 2), (32, 4), (128, 8), (256, 8), (512, 16)])
@pytest.mark.parametrize("mode", ["renorm", "topk_softmax", "no_renorm", "bias"])
def test_router_topk_bit_exact(E, k, mode):
    rng = np.random.default_rng(E + k)
    T = 96
    logits = np.concatenate([rng.integers(-3, 4, size=(T // 2, E)).astype(np.float32),
                             rng.normal(0, 1, size=(T // 2, E)).astype(np.float32)])
    lb = store(logits, BF16)
    lf = load(lb, BF16)
    gating, norm, eb = {"renorm": (0, True, None), "topk_softmax": (1, True, None),
                        "no_renorm": (0, False, None),
                        "bias": (0, True, rng.normal(0, 0.01, E).astype(np.float32))}[mode]
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(T, k, dtype=torch.float32, device="cuda")
    ebt = None if eb is None else to_torch(eb)
    lt = to_torch(lb)
    check(_lib.load().moe_router_topk(_p(lt), BF16, T, E, k, gating, int(norm),
                                      None if ebt is None else _p(ebt), _p(idx), _p(w), _stream()))
    torch.cuda.synchronize()
    ref_idx, ref_w = orc.route(lf, k, gating, norm, eb)
    assert np.array_equal(_u32(idx), ref_idx)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), ref_w.view(np.uint32))


@pytest.mark.parametrize("T", [19, 77])
@pytest.mark.parametrize("dt,wdt,E,H", [(BF16, BF16, 128, 2048), (F16, F16, 8, 256), (BF16, BF16, 32, 2880),
                                         (F32, F32, 4, 64), (F16, F16, 64, 128), (BF16, BF16, 1, 768)])
def test_router_logits_within_one_ulp(dt, wdt, E, H, T):
    """T >= 32 with one 16-bit type and H % 64 == 0 runs on the matrix cores
    (a partial last token tile at T = 77; H = 128 leaves half of the K-split
    waves without a group; H = 2880 splits 45 groups unevenly and ends in a
    partial 256-value chunk; H = 768 is an odd count of chunks; E = 1, a
    shared gate, repeats its one row over the expert tile)."""
    rng = np.random.default_rng(H + T)
    x = store(rng.normal(0, 1, (T, H)), dt)
    W = store(rng.normal(0, 1 / np.sqrt(H), (E, H)), wdt)
    bias = store(rng.normal(0, 0.1, E), dt)
    out = torch.empty(T, E, dtype={BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[dt],
                      device="cuda")
    xt, Wt, bt = to_torch(x), to_torch(W), to_torch(bias)
    check(_lib.load().moe_router_logits(_p(xt), dt, T, H, _p(Wt), wdt, _p(bt), E, _p(out),
                                        _stream()))
    torch.cuda.synchronize()
    ref = orc.router_logits(x, dt, W, wdt, bias)
    got = to_numpy_f32(out)
    ulp = np.abs(ref) * (2.0 ** -7 if dt == BF16 else 2.0 ** -10 if dt == F16 else 2.0 ** -22) + 1e-6
    # the bias add rounds a second time: two storage ulps at most
    assert np.all(np.abs(got - ref) <= 2.02 * ulp)


# ------------------------------------------------------------------- plan --

@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("T,E,H,gs,dt,bias", [
    (1, 32, 2880, 64, BF16, True),     # one token: one wave per expert
    (7, 40, 1024, 32, F16, False),     # a few tokens, E not a multiple of 32
    (64, 128, 2048, 64, BF16, False),  # many tokens: the matrix-core kernel
    (96, 64, 768, 128, F16, True),
    (40, 40, 512, 64, BF16, True),     # many tokens, E % 32 != 0: the row kernel
])
def test_router_logits_q(bits, T, E, H, gs, dt, bias):
    """moe_router_logits_q (an mlx QuantizedLinear router) against the oracle's
    quantised router: codes exact, per-group scale and bias in fp32."""
    rng = np.random.default_rng(bits * 1000 + T)
    sb = BF16 if dt == F16 else F16
    q = affine_quantize(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), bits, gs, sb)
    x = store(rng.normal(0, 1, size=(T, H)), dt)
    b = store(rng.normal(0, 0.1, size=E), dt) if bias else None
    ref = orc.router_logits_q(x, dt, q, b)
    P = lambda a: to_torch(a) if a.dtype != np.uint32 else torch.from_numpy(a.view(np.int32)).cuda()  # noqa: E731
    w, sc, bi = P(q.weight), to_torch(q.scales), to_torch(q.biases)
    qp = _lib.QProj(w.data_ptr(), sc.data_ptr(), bi.data_ptr(), None, bits, gs, sb, E, H, 1)
    xt = to_torch(x)
    bt = None if b is None else to_torch(b)
    out = torch.empty(T, E, dtype=xt.dtype, device="cuda")
    check(_lib.load().moe_router_logits_q(_p(xt), dt, T, H, C.byref(qp),
                                          None if bt is None else _p(bt), E, _p(out), _stream()))
    torch.cuda.synchronize()
    got = to_numpy_f32(out)
    ulp = np.abs(ref) * (2.0 ** -7 if dt == BF16 else 2.0 ** -10) + 1e-6
    tol = 2.02 * ulp + 1e-4 * (1.0 + np.abs(ref).max(axis=1, keepdims=True))
    assert np.all(np.abs(got - ref) <= tol), float(np.abs(got - ref).max())
    # most logits round to the oracle's value exactly (f16 rows carry three
    # more mantissa bits, and its magic offset 1024 cancels more than bf16's
    # 128, so fewer of them do)
    assert np.mean(got == ref) > (0.9 if dt == BF16 else 0.6)


@pytest.mark.parametrize("T", [1, 64, 256])
def test_layer_quantised_router_qwen3(T):
    """A 4-bit mlx router on the Qwen3 shape: one token (row kernel), 64 rows
    (matrix-core GEMV experts) and 256 rows (grouped GEMM experts)."""
    run_layer(with_quantised_router(cfg_qwen3(), bits=4), T, seed=T)


@pytest.mark.parametrize("T", [1, 48])
def test_layer_quantised_router_gptoss(gptoss, T):
    """An 8-bit router with GPT-OSS's bias (double rounding after the
    quantised product)."""
    run_layer(with_quantised_router(gptoss, bits=8), T, seed=T)


@pytest.mark.parametrize("T", [1, 64])
def test_layer_quantised_shared_gate(mixed, T):
    """A 4-bit router and a 4-bit shared_expert_gate (Qwen3xText.swift:660-661,
    947-951) on the mixed-bit layer."""
    run_layer(with_quantised_router(mixed, bits=4, shared_gate_bits=4), T, seed=T + 1)


@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (1, 4, 32), (16, 2, 8), (64, 8, 128), (512, 8, 128),
                                   (4096, 8, 128), (2048, 8, 256), (777, 3, 1000)])
def test_dispatch_plan_bit_exact(T, k, E):
    rng = np.random.default_rng(T * 7 + E)
    if T >= 2048:  # skewed load as in the Zipf prefill config
        p = (np.arange(E) + 1.0) ** -1.1
        idx = rng.choice(E, size=(T, k), p=p / p.sum()).astype(np.uint32)
    else:
        idx = rng.integers(0, E, (T, k)).astype(np.uint32)
    M = T * k
    lib = _lib.load()
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(M, dtype=torch.int32, device="cuda")
    inv = torch.empty(M, dtype=torch.int32, device="cuda")
    wsb = lib.moe_dispatch_workspace_bytes(T, k, E)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    idxt = to_torch(idx.view(np.int32))
    check(lib.moe_dispatch_plan(_p(idxt), T, k, E, _p(counts), _p(offsets),
                                _p(perm), _p(inv), _p(ws), wsb, _stream()))
    torch.cuda.synchronize()
    rc, ro, rp, ri = orc.dispatch_plan(idx, E)
    assert np.array_equal(_u32(counts), rc)
    assert np.array_equal(_u32(offsets), ro)
    assert np.array_equal(_u32(perm), rp)
    assert np.array_equal(_u32(inv), ri)


# ------------------------------------------------------- grouped products --

@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("dt,sb", [(BF16, BF16), (BF16, F16), (F16, F16), (F32, F32)])
def test_expert_matmul_all_widths(bits, dt, sb):
    rng = np.random.default_rng(bits * 10 + dt)
    E, N, K, M = 6, 96, 320, 23
    from moe_spec import gen_qproj
    p = gen_qproj(rng, E, N, K, bits, 64, sb)
    rows = np.sort(rng.integers(0, E, M)).astype(np.uint32)
    offsets = np.searchsorted(rows, np.arange(E + 1)).astype(np.uint32)
    a = store(rng.normal(0, 1, (M, K)), dt)
    lib = _lib.load()
    q = _lib.QProj(0, 0, 0, None, bits, 64, sb, N, K, E)
    wt, st, bt = to_torch(p.weight.view(np.int32)), to_torch(p.scales), to_torch(p.biases)
    q.weight, q.scales, q.biases = wt.data_ptr(), st.data_ptr(), bt.data_ptr()
    at = to_torch(a)
    out = torch.empty(M, N, dtype=at.dtype, device="cuda")
    wsb = lib.moe_expert_matmul_workspace_bytes(C.byref(q), dt, M)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    offt = to_torch(offsets.view(np.int32))
    check(lib.moe_expert_matmul(C.byref(q), _p(at), dt, None, 1, M, _p(offt), _p(out), _p(ws), wsb,
                                _stream()))
    torch.cuda.synchronize()
    ref = orc.round_dt(orc.qgemm_rows(p, load(a, dt), rows), dt)
    check_close(to_numpy_f32(out), ref, dt, f"expert_matmul bits={bits}")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("dt,sb,gs", [(BF16, BF16, 64), (BF16, F16, 128), (F16, F16, 32),
                                      (F16, BF16, 64)])
@pytest.mark.parametrize("gather", [False, True])
def test_expert_matmul_mfma(bits, dt, sb, gs, gather):
    """The matrix-core path (enough rows per expert): uneven experts, an
    empty expert, partial row tiles, a partial column block, and the
    activation gather through a permutation."""
    rng = np.random.default_rng(bits * 100 + dt * 10 + gs + gather)
    from moe_spec import gen_qproj
    E, N, K, topk = 5, 200, 384, 4
    counts = np.array([300, 0, 131, 57, 212])  # M = 700 = 175 tokens x 4
    M = int(counts.sum())
    f = 15.0 / (2 ** bits - 1)
    p = gen_qproj(rng, E, N, K, bits, gs, sb, s_range=(0.005 * f, 0.02 * f))
    experts = np.repeat(np.arange(E), counts).astype(np.uint32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    if gather:
        T = M // topk
        a = store(rng.normal(0, 1, (T, K)), dt)
        perm = rng.permutation(M).astype(np.uint32)  # sorted position -> t*topk + s
        src = load(a, dt)[perm // topk]
    else:
        a = store(rng.normal(0, 1, (M, K)), dt)
        perm = None
        src = load(a, dt)
    lib = _lib.load()
    q = _lib.QProj(0, 0, 0, None, bits, gs, sb, N, K, E)
    wt, st, bt = to_torch(p.weight.view(np.int32)), to_torch(p.scales), to_torch(p.biases)
    q.weight, q.scales, q.biases = wt.data_ptr(), st.data_ptr(), bt.data_ptr()
    at = to_torch(a)
    out = torch.empty(M, N, dtype=at.dtype, device="cuda")
    wsb = lib.moe_expert_matmul_workspace_bytes(C.byref(q), dt, M)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    offt = to_torch(offsets.view(np.int32))
    pt = to_torch(perm.view(np.int32)) if gather else None
    check(lib.moe_expert_matmul(C.byref(q), _p(at), dt, _p(pt) if gather else None, topk, M, _p(offt),
                                _p(out), _p(ws), wsb, _stream()))
    torch.cuda.synchronize()
    ref = orc.round_dt(orc.qgemm_rows(p, src, experts), dt)
    # The matrix-core path rounds every dequantised weight once to f16 (2^-12
    # relative) and scales bf16 activations exactly into f16 range, so a single
    # product meets the layer bar (the reference tests its simdgroup-matrix
    # kernels, which round weights to the input dtype, at cosine >= 0.99:
    # MoEBgemmBm64MppTests.swift:82-114).
    check_close(to_numpy_f32(out), ref, dt, f"mfma expert_matmul bits={bits} gs={gs}")


def test_gemm_operand_range_bf16():
    """The matrix-core path feeds a bf16 input to the matrix cores as f16
    values x 2^-8, converted to nearest: a row element at 2^25 (beyond
    65504 * 2^8) saturates to 65504 * 2^8, and one at 2^-20 (an f16
    subnormal after the scale) rounds to the nearest subnormal. The product
    equals the fp32 oracle's on the input converted that way, and differs
    from the unconverted input's where the value saturated."""
    rng = np.random.default_rng(77)
    from moe_spec import gen_qproj
    E, N, K, bits, gs, dt, sb = 2, 128, 256, 4, 64, BF16, BF16
    counts = np.array([40, 24])
    M = int(counts.sum())
    p = gen_qproj(rng, E, N, K, bits, gs, sb)
    experts = np.repeat(np.arange(E), counts).astype(np.uint32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    xf = rng.normal(0, 1, (M, K))
    xf[3, 17] = 2.0 ** 25
    xf[5, 9] = -(2.0 ** 25)
    xf[7, 100] = 2.0 ** -20 * 1.37
    a = store(xf, dt)
    src = load(a, dt)
    # the operand conversion, restated: scale, saturate, f16 to nearest
    v = np.clip(src.astype(np.float32) * np.float32(2.0 ** -8), -65504, 65504)
    conv = v.astype(np.float16).astype(np.float32) * np.float32(2.0 ** 8)
    assert conv[3, 17] == 65504.0 * 256 and conv[5, 9] == -65504.0 * 256
    lib = _lib.load()
    q = _lib.QProj(0, 0, 0, None, bits, gs, sb, N, K, E)
    wt, st, bt = to_torch(p.weight.view(np.int32)), to_torch(p.scales), to_torch(p.biases)
    q.weight, q.scales, q.biases = wt.data_ptr(), st.data_ptr(), bt.data_ptr()
    at = to_torch(a)
    out = torch.empty(M, N, dtype=at.dtype, device="cuda")
    wsb = lib.moe_expert_matmul_workspace_bytes(C.byref(q), dt, M)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    offt = to_torch(offsets.view(np.int32))
    check(lib.moe_expert_matmul(C.byref(q), _p(at), dt, None, 1, M, _p(offt), _p(out), _p(ws), wsb,
                                _stream()))
    torch.cuda.synchronize()
    got = to_numpy_f32(out)
    ref = orc.round_dt(orc.qgemm_rows(p, conv, experts), dt)
    check_close(got, ref, dt, "bf16 operand range on the matrix-core path")
    raw = orc.round_dt(orc.qgemm_rows(p, src, experts), dt)
    assert np.abs(got[3] - raw[3]).max() > 1e3, "the 2^25 element should saturate"


# ------------------------------------------------------------ whole layer --

@pytest.mark.parametrize("E,k", [(8, 1), (32, 4), (64, 6), (128, 8), (512, 16)])
@pytest.mark.parametrize("mode", ["sigmoid_bias_scaled", "sigmoid_plain", "sigmoid_no_renorm",
                                  "gemma_scales"])
def test_router_topk_scaled_bit_exact(E, k, mode):
    """NemotronH sigmoid routing and Gemma 4 scaled routing through
    moe_router_topk_scaled: ids and f32 weights bit-exact."""
    rng = np.random.default_rng(E * 3 + k)
    T = 96
    logits = np.concatenate([rng.integers(-3, 4, size=(T // 2, E)).astype(np.float32),
                             rng.normal(0, 1.5, size=(T // 2, E)).astype(np.float32)])
    lb = store(logits, BF16)
    lf = load(lb, BF16)
    eb = es = None
    ls, rs = 1.0, 1.0
    if mode.startswith("sigmoid"):
        gating, norm = orc.SIGMOID_TOPK, mode != "sigmoid_no_renorm"
        if mode == "sigmoid_bias_scaled":
            eb = rng.uniform(-0.05, 0.05, E).astype(np.float32)
            rs = 2.5
    else:
        gating, norm = orc.TOPK_THEN_SOFTMAX, True
        ls = float(np.float32(2816 ** -0.5))
        es = rng.uniform(0.5, 1.5, E).astype(np.float32)
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(T, k, dtype=torch.float32, device="cuda")
    ebt = None if eb is None else to_torch(eb)
    est = None if es is None else to_torch(es)
    lt = to_torch(lb)
    check(_lib.load().moe_router_topk_scaled(_p(lt), BF16, T, E, k, gating, int(norm),
                                             None if ebt is None else _p(ebt), ls, rs,
                                             None if est is None else _p(est), _p(idx), _p(w),
                                             _stream()))
    torch.cuda.synchronize()
    ref_idx, ref_w = orc.route(lf, k, gating, norm, eb, logit_scale=ls, routed_scale=rs,
                               expert_scale=es)
    assert np.array_equal(_u32(idx), ref_idx)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), ref_w.view(np.uint32))


@pytest.mark.parametrize("act", [orc.ACT_GEGLU, orc.ACT_RELU2])
def test_activation_apply_new_kinds(act):
    """GELU-gated and squared-ReLU elementwise activations; the bf16 GELU
    stays finite over the reference's [-15, 15] sweep (OpsTests.swift:
    275-302). ReLU^2 is called without a gate buffer."""
    xs = np.arange(-15.0, 15.0 + 0.125, 0.25)
    rng = np.random.default_rng(act)
    g = store(np.concatenate([xs, rng.normal(0, 3, 4096 - xs.size)]), BF16)
    u = store(rng.normal(0, 2, g.size), BF16)
    gt, ut = to_torch(g), to_torch(u)
    out = torch.empty_like(ut)
    check(_lib.load().moe_activation_apply(None if act == orc.ACT_RELU2 else _p(gt), _p(ut), _p(out),
                                           g.size, BF16, act, 0.0, 0.0, _stream()))
    torch.cuda.synchronize()
    got = to_numpy_f32(out)
    gf, uf = load(g, BF16), load(u, BF16)
    ref = np.array([orc.act(float(a), float(b), act, dt=BF16) for a, b in zip(gf, uf)], np.float32)
    ref = load(store(ref, BF16), BF16)
    assert np.all(np.isfinite(got))
    if act == orc.ACT_RELU2:
        assert np.array_equal(got, ref)
    else:
        # tanh from exp and the hardware reciprocal: within one bf16 ulp of the
        # libm-tanh oracle, after the GELU's own bf16 rounding
        assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) * 2.01 + 1e-6)


def run_layer(spec, T, seed=0):
    dev = spec.device()
    x = spec.x(T, seed)
    rx = spec.router_x(T, seed)  # None unless the router reads its own rows
    y, tr = dev.forward(to_torch(x), trace=True, router_x=None if rx is None else to_torch(rx))
    torch.cuda.synchronize()
    logits_gpu = to_numpy_f32(tr["logits"])
    logits_cpu = spec.oracle_logits(x if rx is None else rx)
    assert np.all(np.abs(logits_gpu - logits_cpu) <= spec.logits_tolerance(logits_cpu)), \
        "router logits"
    y_ref, _, idx_ref, w_ref = orc.moe_layer(spec, x, given_logits=logits_gpu, router_x=rx)
    assert np.array_equal(_u32(tr["topk_idx"]), idx_ref), "expert ids"
    assert np.array_equal(tr["topk_weight"].cpu().numpy().view(np.uint32), w_ref.view(np.uint32)), \
        "combine weights"
    _, _, rp, _ = orc.dispatch_plan(idx_ref, spec.n_experts)
    assert np.array_equal(_u32(tr["perm"]), rp), "dispatch permutation"
    stats = check_close(to_numpy_f32(y), load(y_ref, spec.act_dt), spec.act_dt, f"{spec.name} T={T}")
    print(f"{spec.name} T={T}: max|d|/rms={stats[0]:.3e} mean_rel={stats[1]:.3e}")
    return dev, x, y


@pytest.mark.parametrize("shared", [False, True])
def test_layer_scalar_kat(shared):
    """The reference's own MoELayer KAT (MoELayerTests.swift:147-265)."""
    from test_oracle_golden import scalar_layer_expected, scalar_layer_spec
    spec = scalar_layer_spec(shared)
    dev = spec.device()
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = 2.0
    y = dev.forward(to_torch(x)).cpu().numpy()
    assert abs(y[0, 0] - scalar_layer_expected(shared)) < 1e-3
    assert np.all(y[0, 1:] == 0)


@pytest.fixture(scope="module")
def tiny():
    return cfg_tiny()


@pytest.mark.parametrize("T", [1, 2, 16])
def test_layer_tiny(tiny, T):
    run_layer(tiny, T)


@pytest.fixture(scope="module")
def gptoss():
    return cfg_gptoss()


@pytest.mark.parametrize("T", [1, 3, 64])
def test_layer_gptoss(gptoss, T):
    run_layer(gptoss, T, seed=T)


def test_layer_gptoss_expert_bias():
    run_layer(cfg_gptoss(seed=3, n_experts=8, hidden=512, inter=640, expert_bias=True), 1)
    run_layer(cfg_gptoss(seed=3, n_experts=8, hidden=512, inter=640, expert_bias=True), 5)


@pytest.mark.parametrize("dt", [BF16, F16, F32])
@pytest.mark.parametrize("T,H", [(1, 128), (3, 2880), (2, 4096), (1, 8192)])
def test_add_rmsnorm_op(dt, T, H):
    """moe_add_rmsnorm: the residual bit-exact, the normalised row within one
    storage ulp (the sum of squares is reduced in another order)."""
    rng = np.random.default_rng(T * 7 + H)
    a = store(rng.normal(0, 1, (T, H)), dt)
    b = store(rng.normal(0, 0.5, (T, H)), dt)
    wv = store(rng.uniform(0.5, 1.5, H), dt)
    at, bt, wt = to_torch(a), to_torch(b), to_torch(wv)
    res, xn = torch.empty_like(at), torch.empty_like(at)
    check(_lib.load().moe_add_rmsnorm(_p(at), _p(bt), _p(wt), 1e-6, T, H, dt, _p(res), _p(xn),
                                      _stream()))
    torch.cuda.synchronize()
    r_ref, x_ref = orc.add_rmsnorm(load(a, dt), load(b, dt), load(wv, dt), 1e-6, dt)
    assert np.array_equal(to_numpy_f32(res), r_ref)
    # one storage ulp for 16-bit rows (the rounding of a value that moved by a
    # few f32 ulps); f32 itself: 1e-5 relative, the drift of a sequential f32
    # sum of up to 8192 squares against a tree-ordered one (the reference's
    # own bar is 1e-2, OpsTests.swift:1052-1058)
    tol = {BF16: 2.0 ** -7, F16: 2.0 ** -10, F32: 1e-5}[dt]
    assert np.all(np.abs(to_numpy_f32(xn) - x_ref) <= 1.01 * tol * np.abs(x_ref) + 1e-30)


def run_layer_residual(spec, T, seed=0):
    """moe_layer_forward_residual against the oracle's block between the
    decoder steps: the residual bit-exact, routing from the GPU's logits
    bit-exact, the output to the float bar."""
    dev = spec.device()
    rng = np.random.default_rng(seed + 77)
    H = spec.hidden
    h = spec.x(T, seed)
    m = store(rng.normal(0, 0.5, (T, H)), spec.act_dt)
    nw = store(rng.uniform(0.5, 1.5, H), spec.act_dt)
    ht, mt, nwt = to_torch(h), to_torch(m), to_torch(nw)
    y = torch.empty_like(ht)
    res = torch.empty_like(ht)
    E, k = spec.n_experts, spec.top_k
    tr_t = dict(logits=torch.empty(T, E, dtype=ht.dtype, device="cuda"),
                topk_idx=torch.empty(T, k, dtype=torch.int32, device="cuda"),
                topk_weight=torch.empty(T, k, dtype=torch.float32, device="cuda"))
    tr = _lib.LayerTrace(tr_t["logits"].data_ptr(), tr_t["topk_idx"].data_ptr(),
                         tr_t["topk_weight"].data_ptr(), None, None)
    ws = dev.workspace(T)
    check(_lib.load().moe_layer_forward_residual(C.byref(dev.desc), _p(ht), _p(mt), _p(nwt), 1e-6, T,
                                                 _p(y), _p(res), _p(ws), ws.numel(), C.byref(tr),
                                                 _stream()))
    torch.cuda.synchronize()
    lg = to_numpy_f32(tr_t["logits"])
    y_ref, xn_ref, r_ref, l_ref, idx_ref, w_ref = orc.moe_layer_residual(
        spec, h, m, load(nw, spec.act_dt), 1e-6, given_logits=lg)
    assert np.array_equal(to_numpy_f32(res), r_ref), "residual"
    # logits of a normalised row that may differ from the oracle's by an ulp
    # in a few elements: a few storage ulps
    ulp = 2.0 ** -7 if spec.act_dt == BF16 else 2.0 ** -10 if spec.act_dt == F16 else 2.0 ** -20
    l_cpu = orc.router_logits(store(xn_ref, spec.act_dt), spec.act_dt, spec.router_weight,
                              spec.router_dt, spec.router_bias)
    assert np.all(np.abs(lg - l_cpu) <= 4.02 * ulp * np.abs(l_cpu) + 4 * ulp), "router logits"
    assert np.array_equal(_u32(tr_t["topk_idx"]), idx_ref), "expert ids"
    assert np.array_equal(tr_t["topk_weight"].cpu().numpy().view(np.uint32), w_ref.view(np.uint32))
    stats = check_close(to_numpy_f32(y), load(y_ref, spec.act_dt), spec.act_dt,
                        f"{spec.name} residual T={T}")
    print(f"{spec.name} residual T={T}: max|d|/rms={stats[0]:.3e} mean_rel={stats[1]:.3e}")


@pytest.mark.parametrize("cfg,T", [("gptoss", 1), ("gptoss", 4), ("qwen3", 1), ("qwen3", 64),
                                   ("mixed", 1), ("mixed", 40), ("tiny_f32", 2)])
def test_layer_residual(cfg, T):
    """The block with the decoder steps folded in: one token runs the add and
    norm inside the router launch (16-bit, hidden <= 4096), other calls the
    standalone add + RMSNorm; the residual joins the last store (down + combine,
    the shared add, or the unpermute)."""
    spec = {"gptoss": lambda: cfg_gptoss(),
            "qwen3": lambda: cfg_qwen3(),
            "mixed": lambda: cfg_mixed(n_experts=64),
            "tiny_f32": lambda: cfg_tiny(act_dt=F32)}[cfg]()
    if cfg == "tiny_f32":
        spec.gate, spec.up, spec.down = (
            orc.QProj(q.weight, load(q.scales, F16), load(q.biases, F16), q.bits, q.gs, F32)
            for q in (spec.gate, spec.up, spec.down))
        spec.router_weight, spec.router_dt = load(spec.router_weight, F16), F32
    run_layer_residual(spec, T, seed=T)


@pytest.fixture(scope="module")
def nemotron():
    return cfg_nemotron()


@pytest.mark.parametrize("T", [1, 5, 48, 400])
def test_layer_nemotron(nemotron, T):
    """Sigmoid router + correction bias + routed scale, squared-ReLU experts
    without a gate projection, squared-ReLU shared expert; T=400 takes the
    matrix-core path for the routed and shared experts."""
    run_layer(nemotron, T, seed=T)


@pytest.fixture(scope="module")
def gemma4():
    return cfg_gemma4()


@pytest.mark.parametrize("T", [1, 5, 40, 300])
def test_layer_gemma4(gemma4, T):
    """Scaled logits, per-expert scale, GELU-gated experts and a router
    input of its own; T=1 runs the one-token kernels, T=300 the matrix
    cores."""
    run_layer(gemma4, T, seed=T)


@pytest.fixture(scope="module")
def qwen3():
    return cfg_qwen3()


@pytest.mark.parametrize("B", [1, 4, 16, 64])
def test_layer_qwen3_decode(qwen3, B):
    run_layer(qwen3, B, seed=B)


def test_layer_qwen3_prefill_zipf():
    """256 tokens on the Qwen3 shape: 16 rows per expert on average, the
    fewest with which a layer of 64 or more experts takes the grouped GEMM,
    with Zipf-skewed expert loads (many experts of a few rows, a few large)."""
    spec = cfg_qwen3(seed=5, router_bias=zipf_router_bias(128, 1.1, beta=1.0))
    run_layer(spec, 256)


@pytest.fixture(scope="module")
def mixed():
    return cfg_mixed()


@pytest.mark.parametrize("T", [1, 24, 64])
def test_layer_mixed_bits_shared(mixed, T):
    run_layer(mixed, T)


def _shared_variant(kind):
    """One-token shared-expert layers on either side of the limits of the
    fused path (the shared expert inside the two one-token launches)."""
    if kind == "m2":        # SI = 2 I: two column slices per down block
        return cfg_mixed(n_experts=64, shared_inter=1024)
    if kind == "m5":        # k + m = 13 waves: more than a down block takes
        return cfg_mixed(n_experts=64, shared_inter=2560)
    spec = cfg_mixed(n_experts=64)
    rng = np.random.default_rng(11)
    H, SI = spec.hidden, 512
    if kind == "other_bits":  # shared gate/up 4-bit against routed 3-bit
        spec.shared = (gen_qproj(rng, 1, SI, H, 4, 64, BF16), gen_qproj(rng, 1, SI, H, 4, 64, BF16),
                       spec.shared[2])
    elif kind == "f32_gate":  # router and shared gate rows in f32: the gate's own launch
        spec.router_weight = load(spec.router_weight, BF16)
        spec.shared_gate_weight = load(spec.shared_gate_weight, BF16)
        spec.router_dt = F32
    elif kind == "out_bias":  # output biases on every shared projection
        spec.shared = (gen_qproj(rng, 1, SI, H, 3, 64, BF16, out_bias_dt=BF16),
                       gen_qproj(rng, 1, SI, H, 3, 64, BF16, out_bias_dt=BF16),
                       gen_qproj(rng, 1, H, SI, 6, 64, BF16, out_bias_dt=BF16))
    return spec


@pytest.mark.parametrize("kind,fused", [("m1", True), ("m2", True), ("m5", False),
                                        ("other_bits", False), ("f32_gate", True),
                                        ("out_bias", True)])
def test_one_token_shared_expert(kind, fused):
    """At one token a shared expert whose projections have the routed ones'
    formats runs inside gateup1_kernel / down1_kernel (moe_layer_path reports
    decode1 for its stages), otherwise on its own launches; both match the
    oracle."""
    spec = cfg_mixed(n_experts=64) if kind == "m1" else _shared_variant(kind)
    p = _lib.LayerPaths()
    check(_lib.load().moe_layer_path(C.byref(spec.device().desc), 1, C.byref(p)))
    names = p.names()
    assert names["gate_up"] == names["down"] == "decode1"
    want = "decode1" if fused else "gemv"
    assert names["shared_gate_up"] == names["shared_down"] == want, names
    run_layer(spec, 1, seed=3)


@pytest.mark.parametrize("cfg,T,dec1", [("qwen3", 2, True), ("qwen3", 8, True), ("gptoss", 5, True),
                                        ("gptoss", 6, False), ("mixed", 3, True),
                                        ("nemotron", 4, True)])
def test_few_token_decode(cfg, T, dec1):
    """Calls of a few tokens run the one-token kernels with one block row per
    token (each block routes its token itself; a shared expert and the
    trace's dispatch plan take their own launches) while the T k expert
    slices they stream stay within 1.35 per distinct expert expected under
    uniform routing: Qwen3 (128 experts, top-8) up to 8 tokens, GPT-OSS (32,
    top-4) up to 5 (6 tokens: 24 slices over 19.7 expected experts), the
    mixed-bit and NemotronH shapes. Both paths match the oracle, residual
    included."""
    spec = {"qwen3": lambda: cfg_qwen3(),
            "gptoss": lambda: cfg_gptoss(),
            "mixed": lambda: cfg_mixed(n_experts=64),
            "nemotron": lambda: cfg_nemotron()}[cfg]()
    p = _lib.LayerPaths()
    check(_lib.load().moe_layer_path(C.byref(spec.device().desc), T, C.byref(p)))
    names = p.names()
    if dec1:
        assert names["gate_up"] == names["down"] == "decode1", names
    else:
        assert names["gate_up"] != "decode1" and names["down"] != "decode1", names
    if spec.shared is not None:
        assert names["shared_gate_up"] != "decode1", names
    run_layer(spec, T, seed=T)
    run_layer_residual(spec, T, seed=T + 1)


BITS_CASES = [(2, 8, 64, F16, BF16), (5, 2, 32, BF16, F16), (8, 5, 128, F16, F16),
              (6, 3, 64, BF16, BF16), (3, 4, 128, BF16, BF16), (8, 8, 64, BF16, BF16)]


@pytest.mark.parametrize("case", BITS_CASES, ids=lambda c: f"gu{c[0]}-d{c[1]}-gs{c[2]}-sb{c[3]}-x{c[4]}")
@pytest.mark.parametrize("T", [1, 5])
def test_layer_bit_widths(case, T):
    """Decode (T=1) and batched paths over every packed width and group size."""
    run_layer(cfg_bits(*case), T)


@pytest.mark.parametrize("case", [(4, 4, 64, BF16, BF16), (3, 6, 64, BF16, BF16),
                                  (5, 8, 128, F16, F16), (2, 4, 32, F16, BF16),
                                  (6, 3, 32, BF16, F16), (8, 2, 64, F16, F16)],
                         ids=lambda c: f"gu{c[0]}-d{c[1]}-gs{c[2]}-sb{c[3]}-x{c[4]}")
def test_layer_mfma_path(case):
    """Whole layers with enough rows per expert for the matrix-core GEMMs."""
    run_layer(cfg_bits(*case, n_experts=4, top_k=2), 160)


@pytest.mark.parametrize("case", [(4, 4, 32, BF16, BF16), (4, 4, 32, F16, F16), (4, 4, 128, BF16, F16),
                                  (3, 6, 64, BF16, BF16), (2, 5, 32, F16, BF16), (6, 3, 128, F16, F16),
                                  (5, 2, 64, BF16, F16)],
                         ids=lambda c: f"gu{c[0]}-d{c[1]}-gs{c[2]}-sb{c[3]}-x{c[4]}")
def test_layer_batched_mma_path(case):
    """Up to 23 rows per used expert on average with 2- to 6-bit weights (24
    and more take the grouped GEMM): the batched GEMV on
    the matrix cores (codes of 3, 5 and 6 bits straddle words inside a lane's
    8-value block), with a partial last block of down rows (hidden 544 is 8.5
    blocks of 64) and passes of 16 activation rows (up to 30 rows for one
    expert at T = 40, 8 experts, top-3)."""
    gs = case[2]
    hidden = 544 if gs == 32 else 640
    run_layer(cfg_bits(*case, hidden=hidden, inter=384, n_experts=8, top_k=3), 40)


def test_layer_qwen3_mfma_zipf():
    """Qwen3-MoE shape (16 experts) on the matrix-core path, Zipf routing."""
    spec = cfg_qwen3(seed=11, n_experts=16, router_bias=zipf_router_bias(16, 1.1, beta=1.0))
    run_layer(spec, 96)


def test_layer_is_deterministic(qwen3):
    dev = qwen3.device()
    x = to_torch(qwen3.x(64, seed=9))
    y1 = dev.forward(x).clone()
    y2 = dev.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_layer_handle_matches_forward(tiny):
    """moe_layer_create / decode / decode_many (the MoELayer instance API).
    The first call reserves scratch for one row; the 16-row call on another
    stream grows it (the old scratch freed in the first stream's order, the
    new one allocated in the second's), and a later one-row call reuses it."""
    dev = tiny.device()
    lib = _lib.load()
    h = C.c_void_p()
    check(lib.moe_layer_create(C.byref(dev.desc), C.byref(h)))
    try:
        x = to_torch(tiny.x(16))
        x1 = x[:1].contiguous()
        ref = dev.forward(x)
        ref1 = dev.forward(x1)
        torch.cuda.synchronize()
        one = torch.empty_like(x1)
        check(lib.moe_layer_decode(h, _p(x1), _p(one), _stream()))
        out = torch.empty_like(x)
        s2 = torch.cuda.Stream()
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s2):
            check(lib.moe_layer_decode_many(h, _p(x), 16, _p(out), _stream()))
        torch.cuda.current_stream().wait_stream(s2)
        again = torch.empty_like(x1)
        check(lib.moe_layer_decode(h, _p(x1), _p(again), _stream()))
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(one.view(torch.int16), ref1.view(torch.int16))
        assert torch.equal(again.view(torch.int16), ref1.view(torch.int16))
    finally:
        lib.moe_layer_destroy(h)


# ------------------------------------------------ one token: repeated use --

def test_decode_back_to_back(gptoss):
    """One-token calls queued without a host sync: every output matches the
    call made alone."""
    dev = gptoss.device()
    xs = [to_torch(gptoss.x(1, seed=s)) for s in range(4)]
    ref = [dev.forward(x).clone() for x in xs]
    torch.cuda.synchronize()
    outs = [dev.forward(xs[i % 4]).clone() for i in range(64)]
    torch.cuda.synchronize()
    for i, y in enumerate(outs):
        assert torch.equal(y.view(torch.int16), ref[i % 4].view(torch.int16)), f"call {i}"


@pytest.mark.parametrize("cfg,T", [("gptoss", 1), ("gptoss", 64), ("mixed", 1), ("mixed", 64),
                                   ("nemotron", 5), ("nemotron", 40)])
def test_layer_graph_replay(request, cfg, T):
    """A layer call captured in a HIP graph: every replay, with eager work
    between replays, matches the eager result. The shared-expert layers
    (mixed, nemotron) fork their shared expert onto a side stream and join
    it back, which the capture records as graph edges."""
    spec = request.getfixturevalue(cfg)
    dev = spec.device()
    x = to_torch(spec.x(T, seed=2))
    y_eager = dev.forward(x).clone()
    dev.workspace(T)
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dev.forward(x, out=out, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dev.forward(x, out=out, stream=torch.cuda.current_stream())
    for r in range(5):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), y_eager.view(torch.int16)), f"replay {r}"
        dev.forward(x)  # eager work between replays
        torch.cuda.synchronize()


_CAPTURE_FIRST = r"""
import sys, torch
sys.path.insert(0, "tests")
from moe_spec import cfg_mixed, to_torch
spec = cfg_mixed()
dev = spec.device()
x = to_torch(spec.x(64, seed=3))
dev.workspace(64)
out = torch.empty_like(x)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):  # the process's first shared-expert call
    dev.forward(x, out=out, stream=torch.cuda.current_stream())
y_eager = dev.forward(x).clone()
torch.cuda.synchronize()
for r in range(3):
    out.fill_(0)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), y_eager.view(torch.int16)), r
print("ok")
"""


def test_shared_expert_first_call_captured():
    """The first call of a shared-expert layer in a process, made inside a
    stream capture, creates no side stream there: the graph replays match
    the eager result computed afterwards (which forks the side stream)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST], cwd=root, capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:] + r.stderr[-2000:]

