#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Default workload: BASELINE.json configs[1], a GPT-OSS-20B-shaped MoE decode
layer (hidden = intermediate = 2880, 32 experts, top-4 on logits then softmax,
clamped SwiGLU, mlx affine 4-bit gs64 with bf16 scales/biases, biased bf16
router) on one token. 24 independent layers' weights stay resident in HBM
(10.7 GB, beyond the 256 MB Infinity Cache) and successive calls rotate
through them: call c (warm-up calls included) runs layer c % 24, so a layer's
weights come back only after 23 other layers (1.3 GB) have streamed. One
step = one layer call on one token; the timed calls are 5 HIP-graph replays,
each of the next stretch of the rotation.

Prints one JSON line:
  value       MoE-layer tokens/s (1 token per step / time per step)
  roofline    the dominant kernel (routed gate/up grouped GEMV), HBM bound:
              algorithmic bytes per launch / its average duration, timed with
              hipEvents on the launch stream; `rocprof` beside it divides the
              same bytes by the committed rocprofv3 average of that kernel
  cpu_baseline the C oracle (oracle/) on layer 0, one token at a time
The default line also carries configs[3] (`prefill`), configs[4] (`mixed`),
configs[4]'s layer at one token (`mixed1`) and the configs[2] sweep
(`qwen3_decode`, 1 / 4 / 16 / 64 tokens).
Other configs: --config qwen3 (configs[2], --batch B), prefill,
mixed; --config ckpt_load times the checkpoint reader loading
stacked mlx-affine experts from the page cache into HBM.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    # name: hidden, experts, top_k, inter, gate/up bits, down bits, sb dtype, activation,
    #       gating, router bias, tokens, shared inter
    "gptoss": dict(H=2880, E=32, k=4, I=2880, bits_gu=4, bits_d=4, sb="bf16", act="gptoss",
                   gating="topk_softmax", router_bias=True, T=1, SI=0,
                   workload="gptoss20b_moe_decode_b1"),
    "qwen3": dict(H=2048, E=128, k=8, I=768, bits_gu=4, bits_d=4, sb="f16", act="swiglu",
                  gating="softmax_topk", router_bias=False, T=1, SI=0,
                  workload="qwen3moe_decode"),
    "prefill": dict(H=2048, E=128, k=8, I=768, bits_gu=4, bits_d=4, sb="f16", act="swiglu",
                    gating="softmax_topk", router_bias="zipf", beta=0.33, T=4096, SI=0,
                    workload="qwen3moe_prefill_4096_zipf1.1_maxmed10"),
    "mixed": dict(H=2048, E=256, k=8, I=512, bits_gu=3, bits_d=6, sb="bf16", act="swiglu",
                  gating="softmax_topk", router_bias=False, T=2048, SI=512,
                  workload="mixed_3b6b_shared_prefill_2048"),
    # configs[4]'s layer at one token: the 3/6-bit one-token kernels
    "mixed1": dict(H=2048, E=256, k=8, I=512, bits_gu=3, bits_d=6, sb="bf16", act="swiglu",
                   gating="softmax_topk", router_bias=False, T=1, SI=512,
                   workload="mixed_3b6b_shared_decode_b1"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------ hip events --
class HipEvents:
    """hipEvent handles straight from libamdhip64 (recorded by libmoehip)."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self):
        e = C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        assert self.hip.hipEventSynchronize(b) == 0
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, e):
        self.hip.hipEventDestroy(e)


# ------------------------------------------------------------- the layer --
def make_layer(cfg, seed, torch, fl, lib):
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    H, E, I = cfg["H"], cfg["E"], cfg["I"]
    sb = {"bf16": torch.bfloat16, "f16": torch.float16}[cfg["sb"]]

    def proj(E_, N, K, bits):
        words = K * bits // 32
        w = torch.randint(0, 256, (E_, N, words * 4), dtype=torch.uint8, device=dev, generator=g)
        s = torch.empty(E_, N, K // 64, dtype=sb, device=dev).uniform_(0.005, 0.02, generator=g)
        b = torch.empty(E_, N, K // 64, dtype=sb, device=dev).uniform_(-0.1, 0.1, generator=g)
        return fl.StackedExperts(w.view(torch.int32), s, b, bits, 64)

    rw = (torch.randn(E, H, device=dev, generator=g) / math.sqrt(H)).to(torch.bfloat16)
    rb = None
    if cfg["router_bias"] is True:
        rb = (torch.randn(E, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    elif cfg["router_bias"] == "zipf":
        rb = zipf_bias(E, cfg["beta"], seed, torch).to(dev)
    gating = fl.MoEGatingMode.topKThenSoftmax if cfg["gating"] == "topk_softmax" else \
        fl.MoEGatingMode.softmaxThenTopK
    router = fl.MoERouter(E, cfg["k"], gating, True)
    shared = None
    sgw = None
    if cfg["SI"]:
        shared = (proj(1, cfg["SI"], H, cfg["bits_gu"]), proj(1, cfg["SI"], H, cfg["bits_gu"]),
                  proj(1, H, cfg["SI"], cfg["bits_d"]))
        sgw = (torch.randn(1, H, device=dev, generator=g) / math.sqrt(H)).to(torch.bfloat16)
    act = lib.MOE_ACT_GPTOSS if cfg["act"] == "gptoss" else lib.MOE_ACT_SWIGLU
    return fl.MoELayer(router_weight=rw, router=router,
                       gate=proj(E, I, H, cfg["bits_gu"]), up=proj(E, I, H, cfg["bits_gu"]),
                       down=proj(E, H, I, cfg["bits_d"]), hidden=H, act_dtype=torch.bfloat16,
                       router_bias=rb, activation=act, alpha=1.702, limit=7.0, shared=shared,
                       shared_gate_weight=sgw)


def zipf_bias(E, beta, seed, torch):
    import numpy as np
    rng = np.random.default_rng(seed + 7)
    ranks = rng.permutation(E) + 1
    p = ranks.astype(np.float64) ** -1.1
    p /= p.sum()
    return torch.from_numpy((beta * np.log(p)).astype(np.float32)).to(torch.bfloat16)


def proj_bytes(p, experts):
    """Compulsory HBM bytes of `experts` experts of one stacked projection."""
    n, k = p.n, p.k
    sb = p.scales.element_size()
    return experts * (n * k * p.bits // 8 + 2 * n * (k // p.group_size) * sb)


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` (the gate/up launch) from the committed
    FETCH_SIZE / WRITE_SIZE passes (the profiles/*_traffic.json whose
    "workload" is this one), or None."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_traffic.json"))):
        with open(path) as f:
            data = json.load(f)
        if data.get("workload") == workload:
            k = data.get("kernels", {}).get(kernel)
            return None if k is None else k["hbm_bytes"]
    return None


# ------------------------------------------------------------ CPU oracle --
def cpu_threads():
    """Worker threads for the all-core baseline: the cores this process may run
    on, at most 16 (one GPU's share of the box)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_baseline(layer, cfg, torch, budget_s=10.0):
    """Times the C oracle (oracle/) on layer 0 in two modes on this host's
    cores: one thread, and one thread per core over independent token rows
    (the reference's host loop runs per token under concurrentPerform,
    MoELayer.swift:744-748). ctypes releases the GIL for each oracle call.
    Each mode runs calls of T rows (T = 1 for decode, 4 otherwise) for about
    budget_s seconds."""
    import concurrent.futures as cf

    import numpy as np
    import oracle as orc

    def host(t):
        if t is None:
            return None
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16)
        if t.dtype == torch.int32:
            return t.numpy().view(np.uint32)
        if t.dtype == torch.float16:
            return t.view(torch.int16).numpy().view(np.uint16)
        return t.numpy()

    def qp(p):
        return orc.QProj(host(p.weight), host(p.scales), host(p.biases), p.bits, p.group_size,
                         orc.BF16 if p.scales.dtype == torch.bfloat16 else orc.F16)

    keep = dict(rw=host(layer.router_weight), rb=host(layer.router_bias), gate=qp(layer.gate),
                up=qp(layer.up), down=qp(layer.down))
    L = orc.OrLayer()
    L.hidden, L.n_experts, L.top_k = cfg["H"], cfg["E"], cfg["k"]
    L.intermediate, L.act_dt = cfg["I"], orc.BF16
    L.router_weight, L.router_dt = keep["rw"].ctypes.data, orc.BF16
    L.router_bias = None if keep["rb"] is None else keep["rb"].ctypes.data
    L.gating = orc.TOPK_THEN_SOFTMAX if cfg["gating"] == "topk_softmax" else orc.SOFTMAX_THEN_TOPK
    L.norm_topk = 1
    L.gate, L.up, L.down = keep["gate"].c(), keep["up"].c(), keep["down"].c()
    L.activation = orc.ACT_GPTOSS if cfg["act"] == "gptoss" else orc.ACT_SWIGLU
    L.alpha, L.limit = 1.702, 7.0
    if layer.shared is not None:
        keep["shared"] = tuple(qp(p) for p in layer.shared)
        keep["sgw"] = host(layer.shared_gate_weight)
        L.has_shared = 1
        L.shared_gate, L.shared_up, L.shared_down = (q.c() for q in keep["shared"])
        L.shared_gate_weight = None if keep["sgw"] is None else keep["sgw"].ctypes.data
    lib = orc.lib()
    T = 1 if cfg["T"] == 1 else 4
    rng = np.random.default_rng(1)
    nx = 256
    x = orc.from_f32(rng.normal(0, 1, (nx, T, cfg["H"])).astype(np.float32), orc.BF16)

    def one(i, y):
        lib.or_moe_layer(C.byref(L), x[i % nx].ctypes.data_as(C.c_void_p), T,
                         y.ctypes.data_as(C.c_void_p), None, None, None, None)

    # single thread
    y = np.zeros((T, cfg["H"]), np.uint16)
    t0 = time.perf_counter()
    n1 = 0
    while n1 < 3 or time.perf_counter() - t0 < budget_s:
        one(n1, y)
        n1 += 1
        if n1 >= 4096:
            break
    dt1 = time.perf_counter() - t0
    # all cores: each worker runs its own token rows
    nt = cpu_threads()
    stop = time.perf_counter() + budget_s

    def worker(w):
        yw = np.zeros((T, cfg["H"]), np.uint16)
        n = 0
        while n < 2 or time.perf_counter() < stop:
            one(w + nt * n, yw)
            n += 1
        return n

    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(max_workers=nt) as ex:
        counts = list(ex.map(worker, range(nt)))
    dtn = time.perf_counter() - t0
    nall = sum(counts)
    single = n1 * T / dt1
    allc = nall * T / dtn
    return dict(value=round(allc, 2), unit="tokens/s", cores=nt, kind="port",
                single_thread=round(single, 2), all_cores=round(allc, 2),
                nproc=os.cpu_count(),
                sample=f"C oracle on layer 0, calls of {T} token row(s): {n1} calls on one "
                       f"thread in {dt1:.1f} s; {nall} calls on {nt} threads (one per core, "
                       f"independent rows) in {dtn:.1f} s")


# ------------------------------------------------------- checkpoint load --
def bench_ckpt_load(args, torch):
    """Stacked-expert checkpoint load: Qwen3-30B-A3B-shaped MoE layers (128
    experts, hidden 2048, moe_intermediate 768, 4-bit gs64, f16 scales)
    written as an mlx checkpoint, read from the page cache into HBM by
    SafeTensorsBundle.stackedExperts. Bound: the host-to-device link, whose
    rate is measured here with a pinned-buffer copy of the same size."""
    import shutil
    import tempfile

    import numpy as np
    from ffai_amd import _lib as lib
    from ffai_amd.safetensors import SafeTensorsBundle, SafeTensorsWriter

    E, H, I, gs, bits, nl = 128, 2048, 768, 64, 4, 2
    rng = np.random.default_rng(0)
    d = tempfile.mkdtemp(prefix="moe_ckpt_")
    try:
        bases = []
        w = SafeTensorsWriter(os.path.join(d, "model.safetensors"))
        for l in range(nl):
            for name, (n, k) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                base = f"model.layers.{l}.mlp.switch_mlp.{name}"
                words = k * bits // 32
                w.append(f"{base}.weight", lib.MOE_ST_U32, [E, n, words],
                         rng.integers(0, 2**32, size=(E, n, words), dtype=np.uint64).astype(np.uint32))
                sc = rng.uniform(0.005, 0.02, size=(E, n, k // gs)).astype(np.float16)
                w.append(f"{base}.scales", lib.MOE_ST_F16, sc.shape, sc)
                w.append(f"{base}.biases", lib.MOE_ST_F16, sc.shape, (-sc * 8).astype(np.float16))
                bases.append(base)
        w.finalize()
        path = os.path.join(d, "model.safetensors")
        with open(path, "rb") as f:  # into the page cache
            while f.read(64 << 20):
                pass
        total = 0
        with SafeTensorsBundle(d) as b:
            for base in bases:
                for suf in (".weight", ".scales", ".biases"):
                    total += b.info(base + suf)[2]

        def load_all():
            with SafeTensorsBundle(d) as b:
                out = b.stackedExpertsMany(bases, gs)
            torch.cuda.synchronize()
            return out

        for _ in range(max(1, args.warmup)):
            load_all()
        reps = max(1, args.steps)
        t0 = time.perf_counter()
        for _ in range(reps):
            load_all()
        dt = (time.perf_counter() - t0) / reps
        value = total / dt / 1e9

        # the link's rate: one pinned-buffer copy of the same size
        host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
        dev = torch.empty(total, dtype=torch.uint8, device="cuda")
        dev.copy_(host, non_blocking=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            dev.copy_(host, non_blocking=True)
        torch.cuda.synchronize()
        pinned = total * 3 / (time.perf_counter() - t0) / 1e9
        # a pageable copy straight out of the mapping, for comparison
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        src = torch.from_numpy(np.asarray(mm[: total]))
        t0 = time.perf_counter()
        dev.copy_(src)
        torch.cuda.synchronize()
        pageable = total / (time.perf_counter() - t0) / 1e9
        del mm, src
        # CPU baseline: the reference's load copies every tensor out of the
        # mapping into its own buffer (SafeTensors.swift:195-215)
        bufs = {}
        with SafeTensorsBundle(d) as b:
            t0 = time.perf_counter()
            for base in bases:
                for suf in (".weight", ".scales", ".biases"):
                    nb = b.info(base + suf)[2]
                    buf = bufs.setdefault(base + suf, (C.c_uint8 * nb)())
                    lib.check(lib.load().moe_st_read_host(b._h, (base + suf).encode(), buf, nb))
            cpu_dt = time.perf_counter() - t0
    finally:
        shutil.rmtree(d, ignore_errors=True)
    out = {
        "metric": "stacked-expert checkpoint load (page cache -> HBM)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": reps,
        "warmup": max(1, args.warmup), "ms_per_step": round(dt * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic mlx checkpoint (random codes, f16 scales/biases) in the page cache",
        "config": {"workload": "qwen3_30b_a3b_moe_stacks_x2_ckpt_load", "experts": E,
                   "hidden": H, "intermediate": I, "bits": bits, "group_size": gs,
                   "layers": nl, "bytes": total, "parallelism": "single-gpu"},
        "roofline": {"bound": "h2d", "achieved": round(value, 2), "peak": round(pinned, 2),
                     "unit": "GB/s", "frac": round(value / pinned, 4), "traffic": None,
                     "peak_source": "pinned host buffer -> HBM copy of the same size, measured"},
        "pageable_copy_GBps": round(pageable, 2),
        "cpu_baseline": {"value": round(total / cpu_dt / 1e9, 2), "unit": "GB/s", "cores": 1,
                         "kind": "port",
                         "sample": f"copy of every tensor out of the mapping into host buffers "
                                   f"({total / 1e9:.2f} GB, single thread)"},
    }
    print(json.dumps(out), flush=True)


# --------------------------------------------------------- decoder step --
def bench_decoder_step(args, torch, cfg):
    """The block with the decoder steps on either side (Qwen3xText.swift:
    2640-2670, 1015-1035): r = h + m, y = r + MoE(rmsnorm(r) * w). Times the
    fused entry (moe_layer_forward_residual: add + norm inside the router
    launch, the residual in the last store) against the same work as three
    calls (moe_add_rmsnorm, the block, a residual add), each captured in a
    HIP graph over the resident layers."""
    from ffai_amd import _lib as lib
    from ffai_amd import layer as fl
    T, H = cfg["T"], cfg["H"]
    L = args.layers if T <= 64 else min(args.layers, 4)
    log(f"building {L} resident layers of {args.config} (decoder step) ...")
    layers = [make_layer(cfg, seed=100 + l, torch=torch, fl=fl, lib=lib) for l in range(L)]
    bf = torch.bfloat16
    hs = [torch.randn(T, H, device="cuda").to(bf) for _ in range(L)]
    ms = [(0.5 * torch.randn(T, H, device="cuda")).to(bf) for _ in range(L)]
    nws = [torch.empty(H, device="cuda").uniform_(0.5, 1.5).to(bf) for _ in range(L)]
    ys = [torch.empty_like(h) for h in hs]
    rs = [torch.empty_like(h) for h in hs]
    xn = [torch.empty_like(h) for h in hs]
    tmp = [torch.empty_like(h) for h in hs]
    stream = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    for l in range(L):
        layers[l].workspace(T)

    def fused(l):
        layers[l].forward_residual(hs[l], ms[l], nws[l], 1e-6, out=ys[l])

    def unfused(l):
        lib.check(lib.load().moe_add_rmsnorm(
            C.c_void_p(hs[l].data_ptr()), C.c_void_p(ms[l].data_ptr()),
            C.c_void_p(nws[l].data_ptr()), 1e-6, T, H, lib.MOE_BF16, C.c_void_p(rs[l].data_ptr()),
            C.c_void_p(xn[l].data_ptr()), stream()))
        layers[l].forward(xn[l], out=tmp[l])
        torch.add(rs[l], tmp[l], out=ys[l])

    steps = max(L, (args.steps // L) * L)
    warm = max(L, (args.warmup // L) * L)
    res = {}
    for name, fn in (("fused", fused), ("unfused", unfused)):
        for i in range(warm):
            fn(i % L)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for l in range(L):
                fn(l)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps // L):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / steps
        log(f"{name}: {res[name] * 1e3:.2f} us/step")
    # the fused result equals the three-call result (same kernels downstream
    # of the normalised rows; the fused norm is reduced in another order, so
    # a few elements may differ by an ulp)
    fused(0)
    ref = ys[0].clone()
    unfused(0)
    torch.cuda.synchronize()
    diff = (ref.float() - ys[0].float()).abs().max().item()
    out = {
        "metric": "MoE block with decoder steps, tokens/s",
        "value": round(T * 1000.0 / res["fused"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": warm, "ms_per_step": round(res["fused"], 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random packed codes, U-distributed scales/biases, N(0,1) rows)",
        "config": {"workload": cfg["workload"] + "+decoder_step", "hidden": H,
                   "experts": cfg["E"], "top_k": cfg["k"], "tokens_per_step": T,
                   "resident_layers": L, "parallelism": "single-gpu"},
        "fused_us": round(res["fused"] * 1e3, 3), "unfused_us": round(res["unfused"] * 1e3, 3),
        "saved_us": round((res["unfused"] - res["fused"]) * 1e3, 3),
        "max_abs_diff_vs_unfused": diff,
    }
    print(json.dumps(out), flush=True)


# ------------------------------------------------------- MXFP4 transcode --
def bench_mxfp4(args, torch):
    """GPT-OSS-20B's expert stacks (32 experts x gate/up/down of 2880 x 2880,
    MXFP4) transcoded in HBM to affine 4-bit with bf16 scales and biases
    (moe_mxfp4_to_affine, in place). Algorithmic bytes per 32-code group: 16
    packed + 1 exponent read, 16 codes + 2 + 2 scale/bias written = 37."""
    import numpy as np
    from ffai_amd import _lib as lib
    E, H, I = 32, 2880, 2880
    groups = E * (2 * I * H + H * I) // 32
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    packed = torch.randint(-2**31, 2**31 - 1, (groups * 4,), dtype=torch.int32, device="cuda",
                           generator=g)
    e8 = torch.randint(118, 125, (groups,), dtype=torch.uint8, device="cuda", generator=g)
    s = torch.empty(groups, dtype=torch.bfloat16, device="cuda")
    b = torch.empty(groups, dtype=torch.bfloat16, device="cuda")
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731

    def run():
        # out of place into `out` keeps every repetition on the same input
        lib.check(lib.load().moe_mxfp4_to_affine(P(packed), P(e8), groups, P(out), P(s), P(b),
                                                 lib.MOE_BF16, st))

    out = torch.empty_like(packed)
    for _ in range(max(1, args.warmup)):
        run()
    reps = max(1, args.steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = groups * 37
    gbs = nbytes / (ms * 1e-3) / 1e9
    # CPU baseline: the oracle's restatement of the reference loop, one thread
    import oracle as orc
    ns = 200000
    pk = packed[: ns * 4].cpu().numpy().view(np.uint32)
    ee = e8[:ns].cpu().numpy()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < 10.0:
        orc.mxfp4_to_affine(pk, ee, orc.BF16)
        n += 1
    cdt = time.perf_counter() - t0
    out_line = {
        "metric": "MXFP4 -> affine 4-bit transcode (GPT-OSS-20B layer experts)",
        "value": round(groups * 32 / (ms * 1e-3) / 1e9, 2), "unit": "Gweights/s", "n_gpus": 1,
        "steps": reps, "warmup": max(1, args.warmup), "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (random fp4 codes, e8m0 118..124)",
        "config": {"workload": "gptoss20b_layer_experts_mxfp4_transcode", "experts": E,
                   "hidden": H, "intermediate": I, "groups": groups, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": nbytes, "kernel": "mxfp4_affine_kernel<bf16>"},
        "cpu_baseline": {"value": round(n * ns * 32 / cdt / 1e9, 4), "unit": "Gweights/s",
                         "cores": 1, "kind": "port",
                         "sample": f"{n} oracle transcodes of {ns} groups ({cdt:.1f} s)"},
    }
    print(json.dumps(out_line), flush=True)


# ------------------------------------------------------------------ main --
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400,
                    help="timed layer calls (up to 5 repeats of at least one layer rotation each, median reported)")
    ap.add_argument("--warmup", type=int, default=240, help="untimed eager layer calls first")
    ap.add_argument("--config", default="gptoss",
                    choices=sorted(CONFIGS) + ["ckpt_load", "mxfp4"])
    ap.add_argument("--batch", type=int, default=None, help="tokens per step (overrides config)")
    ap.add_argument("--layers", type=int, default=24, help="resident layers rotated per step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="default config only: skip the prefill and mixed-bit lines")
    ap.add_argument("--decoder-step", action="store_true",
                    help="time the block with the residual add + RMSNorm before it and the "
                         "residual add after it, fused against three calls")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 10 plain device copies of BYTES each (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    ap.add_argument("--summarize-rocprof", metavar="CSV",
                    help="write --out (profiles/<name>_kernel_stats.json) from a rocprofv3 "
                         "kernel_trace.csv of --workload made by --command, then exit")
    ap.add_argument("--summarize-traffic", action="store_true",
                    help="write --out (profiles/<name>_traffic.json) from the FETCH_SIZE / "
                         "WRITE_SIZE counter CSVs of --workload and of a --copy-probe run")
    ap.add_argument("--summarize-counters", nargs="+", metavar="CSV",
                    help="write --out (profiles/<name>_counters.json) from rocprofv3 --pmc "
                         "counter CSVs of --workload made by --command, then exit")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-bytes", type=int, default=268435456)
    ap.add_argument("--workload")
    ap.add_argument("--command")
    ap.add_argument("--out")
    args = ap.parse_args()
    if args.summarize_rocprof:
        summarize_rocprof(args)
        return
    if args.summarize_traffic:
        summarize_traffic(args)
        return
    if args.summarize_counters:
        summarize_counters(args)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py: this build measures one GPU only (single-GPU MoE layer; no multi-GPU "
              "path is built). Run with --gpus 1.", flush=True)
        sys.exit(2)

    import torch
    if args.copy_probe:
        n = args.copy_probe // 4
        src = torch.ones(n, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 10 copies of {n * 4} bytes")
        return
    if args.config == "ckpt_load":
        bench_ckpt_load(args, torch)
        return
    if args.config == "mxfp4":
        bench_mxfp4(args, torch)
        return
    from ffai_amd import _lib as lib
    from ffai_amd import layer as fl

    cfg = dict(CONFIGS[args.config])
    if args.batch:
        cfg["T"] = args.batch
    if args.config == "qwen3":
        cfg["workload"] = f"qwen3moe_decode_b{cfg['T']}"
    if args.decoder_step:
        bench_decoder_step(args, torch, cfg)
        return
    torch.manual_seed(0)
    L = args.layers if cfg["T"] <= 64 else min(args.layers, 4)
    res, layer0 = run_config(cfg, torch, fl, lib, steps=args.steps, warmup=args.warmup, L=L)
    out = {
        "metric": "MoE-layer tokens/s",
        "value": res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random packed codes, U-distributed scales/biases, N(0,1) activations)",
        "config": res["config"],
        "timing": res["timing"],
        "roofline": res["roofline"],
        "expert_stream": res["expert_stream"],
    }
    if args.config == "gptoss" and not args.batch and not args.no_extra:
        # the metric's other two parts, on the prefill configs (configs[3],
        # configs[4]): fixed counts, independent of --steps / --warmup
        # plus the one-token 3/6-bit row (configs[4]'s layer at T = 1)
        for name, st2, wu2, L2 in (("prefill", 60, 6, 4), ("mixed", 60, 6, 4), ("mixed1", 480, 48, 24)):
            c2 = dict(CONFIGS[name])
            r2, _ = run_config(c2, torch, fl, lib, steps=st2, warmup=wu2, L=L2)
            out[name] = {"workload": c2["workload"], "tokens_per_s": r2["tokens_per_s"],
                         "ms_per_step": r2["ms_per_step"], "steps": st2, "warmup": wu2,
                         "timing": r2["timing"], "roofline": r2["roofline"],
                         "layer_roofline": r2["layer_roofline"], "paths": r2["config"]["paths"],
                         "resident_layers": r2["config"]["resident_layers"],
                         "timed_layers": r2["config"]["timed_layers"]}
            if "zipf" in r2["config"]:
                out[name]["zipf"] = r2["config"]["zipf"]
        # the Qwen3-MoE-shaped decode sweep over batch sizes, on
        # one set of 24 resident layers (8.2 GB)
        qcfg = dict(CONFIGS["qwen3"])
        qlayers = build_layers(qcfg, args.layers, torch, fl, lib)
        sweep = {}
        for B in (1, 4, 16, 64):
            c2 = dict(qcfg, T=B, workload=f"qwen3moe_decode_b{B}")
            r2, _ = run_config(c2, torch, fl, lib, steps=240, warmup=24, L=len(qlayers),
                               layers=qlayers)
            sweep[f"b{B}"] = {"workload": c2["workload"], "tokens_per_s": r2["tokens_per_s"],
                              "ms_per_step": r2["ms_per_step"], "steps": 240, "warmup": 24,
                              "distinct_experts": r2["expert_stream"]["distinct_experts"],
                              "layer_roofline": r2["layer_roofline"], "roofline": r2["roofline"],
                              "timing": r2["timing"], "paths": r2["config"]["paths"],
                              "resident_layers": r2["config"]["resident_layers"],
                              "timed_layers": r2["config"]["timed_layers"]}
        del qlayers
        out["qwen3_decode"] = sweep
    copy = copy_bandwidth(torch)
    out["hbm_copy"] = {"GBps": copy, "method": "1 GiB device-to-device copy x 10, read + write "
                       "bytes over the event time"}
    roofs = [out["roofline"]] + [out[n]["roofline"] for n in ("prefill", "mixed", "mixed1")
                                 if n in out]
    roofs += [v[key] for v in out.get("qwen3_decode", {}).values()
              for key in ("roofline", "layer_roofline")]
    for r in roofs:
        if r["bound"] == "hbm":
            r["frac_of_copy"] = round(r["achieved"] / copy, 4)
    log(f"device copy {copy:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle ...")
        cpu = cpu_baseline(layer0, cfg, torch)
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


def copy_bandwidth(torch, nbytes=1 << 30, reps=10):
    """Measured device-copy bandwidth (bytes read + bytes written per second)
    of a plain 1 GiB device-to-device copy, timed with events: the practical
    HBM ceiling next to the 8 TB/s vendor peak."""
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    b.synchronize()
    gbps = 2.0 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst
    return round(gbps, 1)


def build_layers(cfg, L, torch, fl, lib):
    log(f"building {L} resident layers of {cfg['workload']} ...")
    return [make_layer(cfg, seed=100 + l, torch=torch, fl=fl, lib=lib) for l in range(L)]


def graph_upload(g, torch):
    """hipGraphUpload of a captured graph's executable, so that its first
    replay does not also pay for moving the graph to the device. Best effort:
    a torch build without the raw handle skips it."""
    try:
        hip = C.CDLL("libamdhip64.so")
        hip.hipGraphUpload.argtypes = [C.c_void_p, C.c_void_p]
        ex = g.raw_cuda_graph_exec()
        ex = ex if isinstance(ex, int) else int(ex)
        return hip.hipGraphUpload(C.c_void_p(ex),
                                  C.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    except Exception:  # noqa: BLE001
        return False


def rocprof_avg_us(workload, kernel):
    """Average duration (us) of `kernel` (its short name) in the committed
    rocprofv3 --kernel-trace --stats summary of `workload`
    (profiles/*_kernel_stats.json, written by --summarize-rocprof), with the
    summary's file name; (None, None) when no summary covers it."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_kernel_stats.json"))):
        with open(path) as f:
            data = json.load(f)
        if data.get("workload") != workload:
            continue
        k = data.get("kernels", {}).get(kernel)
        if k is not None:
            return k["avg_us"], os.path.relpath(path, ROOT)
    return None, None


def run_config(cfg, torch, fl, lib, steps, warmup, L, layers=None):
    """Times `steps` layer calls (one step = one call of the layer on cfg["T"]
    token rows) after `warmup` untimed eager calls. Calls rotate through L
    resident layers: call c (warm-up calls first) runs layer c % L, so the
    timed calls continue the rotation where the warm-up stopped and every
    layer is used again only after the L - 1 others; before them, each
    layer is called once as set-up (starting at the first timed layer). The graphs of the timed
    calls are captured, uploaded and launched once (untimed: a graph's first
    launch carries a one-time runtime cost), and the warm-up calls run right
    before the timed ones, so that the timed calls start on the clocks of a
    running loop. The timed steps run as min(5, steps // L) repeats, at least
    one (steps // repeats calls each, the remainder spread over the first
    repeats), each one HIP-graph replay of its own stretch of the rotation,
    bracketed by events on the launch stream; ms_per_step is the median over
    the repeats of (repeat time / its calls). Every call, untimed ones
    included, advances one clock; a timed call's reuse distance is the
    number of calls since its layer's previous call."""
    T = cfg["T"]
    if layers is None:
        layers = build_layers(cfg, L, torch, fl, lib)
    L = len(layers)
    log(f"{cfg['workload']}: T={T}, {L} resident layers")
    xs = [torch.randn(T, cfg["H"], device="cuda").to(torch.bfloat16) for _ in range(L)]
    ys = [torch.empty_like(x) for x in xs]
    for l in range(L):
        layers[l].workspace(T)
    # set-up: every resident layer is called once, as a decode loop has used
    # every layer before any given step (a layer's first call after a long
    # idle stretch reads 1.5-2 us slower on GPT-OSS). The pass starts at the
    # first timed layer, so between a timed layer's set-up call and its timed
    # call come at least L + warmup other calls (GPT-OSS: 24 x 56 MB), far
    # more than the 256 MB memory-side cache holds.
    clock = 0          # calls so far, in the order the device runs them
    last_use = {}      # layer -> clock of its latest call
    for i in range(L):
        l = (warmup + i) % L
        layers[l].forward(xs[l], out=ys[l])
        last_use[l] = clock
        clock += 1
    torch.cuda.synchronize()
    paths = layers[0].paths(T)

    # the timed steps: up to 5 repeats, each one HIP-graph replay of the next
    # stretch of the rotation and each at least one full rotation long (a
    # repeat of a few calls would mostly time the replay's own start and end)
    nrep = max(1, min(5, steps // L))
    sizes = [steps // nrep + (1 if r < steps % nrep else 0) for r in range(nrep)]
    graphs = []
    timed_seq = []     # layer of each timed call, in order
    c = warmup
    for n in sizes:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(n):
                l = c % L
                layers[l].forward(xs[l], out=ys[l])
                timed_seq.append(l)
                c += 1
        graphs.append(g)
    uploaded = all([graph_upload(g, torch) for g in graphs])
    torch.cuda.synchronize()
    # each graph launched once, untimed: after hipGraphUpload the first
    # launch of an executable graph still stalls once for about 30 us on
    # this runtime (one gap inside the replay, none in later replays:
    # GPT-OSS 20-call replay 22.6-23.0 us per call first, 21.5-21.6 after)
    for g in graphs:
        g.replay()
    for l in timed_seq:
        last_use[l] = clock
        clock += 1
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(nrep)]
    # warm-up: exactly `warmup` eager calls, right before the timed replays
    # (capture and upload leave the device idle for milliseconds; run before
    # them, the warm-up left the first timed calls on idle clocks)
    for c in range(warmup):
        layers[c % L].forward(xs[c % L], out=ys[c % L])
        last_use[c % L] = clock
        clock += 1
    torch.cuda.synchronize()
    reuse = []
    for l in timed_seq:
        reuse.append(clock - last_use[l])
        last_use[l] = clock
        clock += 1
    timed_layers = set(timed_seq)
    w0 = time.perf_counter()
    for r in range(nrep):
        evs[r][0].record()
        graphs[r].replay()
        evs[r][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    each = [evs[r][0].elapsed_time(evs[r][1]) / n for r, n in enumerate(sizes)]
    span = evs[0][0].elapsed_time(evs[-1][1]) / steps
    per_step = sorted(each)
    ms_per_step = per_step[len(per_step) // 2]
    value = T * 1000.0 / ms_per_step
    min_reuse = min(reuse) if reuse else None
    log(f"{steps} steps in {nrep} repeats {sizes}: {ms_per_step * 1e3:.2f} us/step (median), "
        f"repeats {[round(v * 1e3, 2) for v in each]} us/step, all {span * 1e3:.2f}; "
        f"{len(timed_layers)} layers timed, min reuse distance {min_reuse}; "
        f"wall {wall * 1e3:.1f} ms")
    del graphs

    # kernel-level timing of the routed expert kernels: start/end events
    # recorded by the kernels' own dispatch on the launch stream
    ev = HipEvents()
    reps = max(1, min(20, 480 // L)) if T <= 64 else 4
    marks = [[[ev.create() for _ in range(4)] for _ in range(L)] for _ in range(reps)]
    trace = []
    for r in range(reps):
        for l in range(L):
            t = lib.LayerTrace()
            for i in range(4):
                t.events[i] = marks[r][l][i].value
            trace.append(t)
    j = 0
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for r in range(reps):
        for l in range(L):
            lay = layers[l]
            lib.check(lib.load().moe_layer_forward(
                C.byref(lay.desc), C.c_void_p(xs[l].data_ptr()), T, C.c_void_p(ys[l].data_ptr()),
                C.c_void_p(lay._ws.data_ptr()), lay._ws.numel(), C.byref(trace[j]), stream))
            j += 1
    torch.cuda.synchronize()
    gu = [ev.elapsed_ms(marks[r][l][0], marks[r][l][1]) for r in range(reps) for l in range(L)]
    dn = [ev.elapsed_ms(marks[r][l][2], marks[r][l][3]) for r in range(reps) for l in range(L)]
    for row in marks:
        for m in row:
            for e in m:
                ev.destroy(e)
    gu_us = 1e3 * sum(gu) / len(gu)
    dn_us = 1e3 * sum(dn) / len(dn)

    # algorithmic bytes: distinct experts actually routed (GEMV paths) or FLOPs (GEMM)
    lay0 = layers[0]
    _, tr = lay0.forward(xs[0], trace=True)
    torch.cuda.synchronize()
    U = int(torch.unique(tr["topk_idx"]).numel())
    H, I, k = cfg["H"], cfg["I"], cfg["k"]
    gu_bytes = proj_bytes(lay0.gate, U) + proj_bytes(lay0.up, U) + T * H * 2 + T * k * I * 2
    dn_bytes = proj_bytes(lay0.down, U) + T * k * I * 2 + T * H * 2
    sh_gu_bytes = sh_dn_bytes = 0
    if lay0.shared is not None:
        sg, su, sd = lay0.shared
        sh_gu_bytes = (0 if sg is None else proj_bytes(sg, 1)) + proj_bytes(su, 1)
        sh_dn_bytes = proj_bytes(sd, 1)
    if paths["shared_gate_up"] == "decode1":
        # the one-token launches also stream the shared expert
        gu_bytes += sh_gu_bytes + T * su.n * 2
        dn_bytes += sh_dn_bytes + T * su.n * 2
        # its activation row is written and read inside the layer: not layer traffic
        sh_gu_bytes, sh_dn_bytes = -T * su.n * 4, 0
    M = T * k
    gu_flops = 2.0 * M * 2 * H * I
    dn_flops = 2.0 * M * H * I
    sh_flops = 0.0
    if cfg["SI"]:
        sh_flops = 2.0 * T * 3 * H * cfg["SI"]
    router_bytes = cfg["E"] * H * 2
    layer_bytes = gu_bytes + dn_bytes - T * k * I * 4 + router_bytes + sh_gu_bytes + sh_dn_bytes
    kname = {"decode1": "gateup1_kernel",
             "gemm": "gemm_grouped_gateup", "gemv_mma": "gemv_mma_gateup",
             "gemv": "gemv_multi_gateup"}[paths["gate_up"]]
    if paths["gate_up"] == "gemm":
        roof = dict(bound="mfma", achieved=round(gu_flops / (gu_us * 1e-6) / 1e12, 2),
                    peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s")
        layer_flops = gu_flops + dn_flops + sh_flops
        layer_roof = dict(bound="mfma", flops=layer_flops,
                          achieved=round(layer_flops / (ms_per_step * 1e-3) / 1e12, 2),
                          peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s")
    else:
        # the GEMV paths stream each routed expert's weights once: HBM roofline
        roof = dict(bound="hbm", achieved=round(gu_bytes / (gu_us * 1e-6) / 1e9, 1),
                    peak=HBM_PEAK_GBS, unit="GB/s")
        layer_roof = dict(bound="hbm", bytes=layer_bytes,
                          achieved=round(layer_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                          peak=HBM_PEAK_GBS, unit="GB/s")
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    layer_roof["frac"] = round(layer_roof["achieved"] / layer_roof["peak"], 4)
    roof["traffic"] = measured_traffic(cfg["workload"], kname)
    roof["kernel"] = {"decode1": "gateup1_kernel (one-token gate/up with routing)",
                      "gemm": "gemm_grouped_kernel (MFMA gate/up over the expert row tiles)",
                      "gemv_mma": "gemv_mma_kernel (MFMA gate/up over the dispatch plan)",
                      "gemv": "gemv_multi_kernel (routed gate/up over the dispatch plan)"}[
                          paths["gate_up"]]
    roof["avg_us"] = round(gu_us, 3)
    work = gu_bytes if roof["bound"] == "hbm" else gu_flops
    if roof["bound"] == "hbm":
        roof["algorithmic_bytes"] = gu_bytes
    else:
        roof["algorithmic_flops"] = gu_flops
    roof["avg_us_method"] = ("start/stop events recorded by the kernel's own dispatch "
                             "(dispatch included), eager pass")
    # the same work over the committed rocprofv3 average of this kernel
    rp_us, rp_file = rocprof_avg_us(cfg["workload"], kname)
    if rp_us:
        scale = 1e9 if roof["bound"] == "hbm" else 1e12
        ach = work / (rp_us * 1e-6) / scale
        roof["rocprof"] = {"avg_us": rp_us, "achieved": round(ach, 2),
                           "frac": round(ach / roof["peak"], 4), "summary": rp_file}
    log(f"gate/up kernel {gu_us:.2f} us ({gu_bytes / 1e6:.2f} MB, {gu_flops / 1e9:.1f} GFLOP); "
        f"down {dn_us:.2f} us; U={U}; paths {paths}")
    config = {"workload": cfg["workload"], "hidden": H, "experts": cfg["E"], "top_k": k,
              "intermediate": I, "tokens_per_step": T, "bits": [cfg["bits_gu"], cfg["bits_d"]],
              "group_size": 64, "resident_layers": L, "timed_layers": len(timed_layers),
              "min_reuse_distance_calls": min_reuse, "setup_calls": L,
              "parallelism": "single-gpu",
              "paths": paths}
    if cfg["SI"]:
        config["shared_intermediate"] = cfg["SI"]
    if cfg["router_bias"] == "zipf":
        counts = torch.bincount(tr["topk_idx"].flatten().long(), minlength=cfg["E"]).float()
        config["zipf"] = {"s": 1.1, "beta": cfg["beta"],
                          "max_over_median": round(float(counts.max() / counts.median()), 2)}
    res = {
        "tokens_per_s": round(value, 1),
        "ms_per_step": round(ms_per_step, 6),
        "timing": {"repeats": nrep, "calls_per_repeat": sizes,
                   "ms_per_step_each": [round(v, 6) for v in each],
                   "ms_per_step_all": round(span, 6), "graphs_uploaded": uploaded,
                   "warmup_after_capture": True, "graphs_launched_before_timing": True,
                   "method": "graphs captured, uploaded and launched once (untimed), then the "
                             "warm-up calls, then one HIP-graph replay per repeat (each its own "
                             "stretch of the layer rotation), events on the launch stream, median"},
        "config": config,
        "roofline": roof,
        "layer_roofline": layer_roof,
        "expert_stream": {"gate_up_us": round(gu_us, 3), "down_us": round(dn_us, 3),
                          "bytes": gu_bytes + dn_bytes, "distinct_experts": U,
                          "GBps": round((gu_bytes + dn_bytes) / ((gu_us + dn_us) * 1e-6) / 1e9, 1)},
    }
    out_layer = layers[0]
    del layers, xs, ys
    torch.cuda.synchronize()
    return res, out_layer


def short_kernel_name(name):
    """A kernel's function name from its mangled name (_ZN3moe14gateup1_kernelI...
    -> gateup1_kernel). The grouped GEMM and the grouped GEMVs, which serve
    both a gate/up pair and a single projection, are named after their first
    template flag: gemm_grouped_gateup / gemm_grouped_single,
    gemv_mma_gateup, gemv_multi_single, ..."""
    import re
    m = re.match(r"_ZN\d*moe(\d+)(\w+)", name)
    if not m:
        return name
    short = m.group(2)[:int(m.group(1))]
    if short in ("gemm_grouped_kernel", "gemv_mma_kernel", "gemv_multi_kernel"):
        flag = re.search(r"Lb([01])E", name)
        short = short[: -len("_kernel")] + ("_gateup" if flag and flag.group(1) == "1" else "_single")
    return short


def grid_keys(groups):
    """Names for (short kernel name, grid size) groups: one kernel launched at
    several grid sizes (the grouped GEMM runs the routed experts and, on a
    side stream, the shared expert) keeps its plain name for the grid with the
    largest total and gets name@<grid threads> for the others."""
    by_name = {}
    for (name, grid), total in groups.items():
        by_name.setdefault(name, []).append((total, grid))
    keys = {}
    for name, lst in by_name.items():
        lst.sort(reverse=True)
        for i, (_, grid) in enumerate(lst):
            keys[(name, grid)] = name if i == 0 else f"{name}@{grid}"
    return keys


def summarize_rocprof(args):
    """Writes profiles/<name>_kernel_stats.json from a rocprofv3
    kernel_trace.csv (--kernel-trace, one row per dispatch): per kernel
    (mangled names shortened to the function name, split by grid size as
    grid_keys names them) calls and average / median / min / max duration in
    us and the share of the run's GPU time, with the workload and the command
    that produced the CSV. Kernels outside the library (torch's set-up fills
    and copies, the bench's device spin) are one line in total. bench.py
    reads these summaries for the rocprof side of its rooflines."""
    import csv
    import statistics
    durs, mangled = {}, {}
    other = {"calls": 0, "total_us": 0.0}
    total_all = 0.0
    with open(args.summarize_rocprof) as f:
        for r in csv.DictReader(f):
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            total_all += us
            name = r["Kernel_Name"]
            if not name.startswith("_ZN3moe"):
                other["calls"] += 1
                other["total_us"] += us
                continue
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            key = (short_kernel_name(name), grid)
            durs.setdefault(key, []).append(us)
            mangled[key] = name
    keys = grid_keys({k: sum(v) for k, v in durs.items()})
    kernels = {}
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        kernels[keys[k]] = {"calls": len(v), "grid_threads": k[1],
                            "avg_us": round(sum(v) / len(v), 3),
                            "median_us": round(statistics.median(v), 3),
                            "min_us": round(min(v), 3), "max_us": round(max(v), 3),
                            "share_pct": round(100.0 * sum(v) / total_all, 2),
                            "mangled": mangled[k]}
    other["total_us"] = round(other["total_us"], 1)
    other["share_pct"] = round(100.0 * other["total_us"] / total_all, 2)
    out = {"workload": args.workload, "command": args.command, "kernels": kernels,
           "other_kernels": other}
    with open(args.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {args.out}: {len(kernels)} kernels")


def counter_means(path):
    """Mean value per (kernel, counter) of a rocprofv3 --pmc counter CSV
    (one row per dispatch and counter). Kernels are keyed by their short
    name, split by grid size as grid_keys names them (the grouped GEMM's
    routed and shared-expert launches apart)."""
    import collections
    import csv
    acc = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            acc[(short_kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]),
                 r["Counter_Name"])].append(float(r["Counter_Value"]))
    totals = collections.defaultdict(float)
    for (k, g, c), v in acc.items():
        totals[(k, g)] += sum(v)
    keys = grid_keys(totals)
    return {(keys[(k, g)], c): sum(v) / len(v) for (k, g, c), v in acc.items()}


def summarize_traffic(args):
    """Writes profiles/<name>_traffic.json from four rocprofv3 --pmc runs:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over `--copy-probe BYTES`
    (a plain device copy of known size, which calibrates the counters) and
    over the workload. hbm_bytes per kernel = FETCH_SIZE x 1024 x fetch_factor
    + WRITE_SIZE x 1024 x write_factor, the factors being the copy's bytes
    over what the counters read for it."""
    cf, cw = counter_means(args.copy_fetch), counter_means(args.copy_write)
    copy_f = max(v for (k, c), v in cf.items() if c == "FETCH_SIZE")
    copy_w = max(v for (k, c), v in cw.items() if c == "WRITE_SIZE")
    ff = args.copy_bytes / (copy_f * 1024.0)
    fw = args.copy_bytes / (copy_w * 1024.0)
    wf, ww = counter_means(args.fetch), counter_means(args.write)
    kernels = {}
    for (k, c), v in wf.items():
        if c != "FETCH_SIZE" or not k.startswith(("gateup1", "down1", "gemm_grouped", "gemv",
                                                  "router", "unpermute")):
            continue
        w = ww.get((k, "WRITE_SIZE"))
        if w is None:
            continue
        kernels[k] = {"FETCH_SIZE_KiB": round(v, 1), "WRITE_SIZE_KiB": round(w, 1),
                      "hbm_bytes": int(round(v * 1024 * ff + w * 1024 * fw))}
    out = {"workload": args.workload, "command": args.command,
           "calibration": {"copy_bytes": args.copy_bytes, "FETCH_SIZE_KiB": round(copy_f, 1),
                           "WRITE_SIZE_KiB": round(copy_w, 1), "fetch_factor": round(ff, 4),
                           "write_factor": round(fw, 4)},
           "kernels": kernels}
    with open(args.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {args.out}: {sorted(kernels)}")

def summarize_counters(args):
    """Writes profiles/<name>_counters.json from rocprofv3 --pmc CSVs of one
    workload (each its own pass): the mean per dispatch of every counter per
    kernel of the library and, where the counters are there, MFMA busy per
    SIMD (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x
    4 SIMDs), VALU instructions per MFMA instruction (SQ_INSTS_VALU, which
    counts the MFMAs too, over SQ_INSTS_MFMA), the share of wave cycles spent
    waiting for an instruction's operands (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES)
    and LDS bank-conflict cycles per LDS-active cycle."""
    means = {}
    for path in args.summarize_counters:
        for (k, c), v in counter_means(path).items():
            if k.startswith(("gateup1", "down1", "gemm_grouped", "gemv", "router",
                             "unpermute")):
                means.setdefault(k, {})[c] = round(v, 1)
    kernels = {}
    for k, m in sorted(means.items()):
        d = {"counters": m}
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and m.get("GRBM_GUI_ACTIVE"):
            d["mfma_busy_pct"] = round(100.0 * m["SQ_VALU_MFMA_BUSY_CYCLES"]
                                       / (m["GRBM_GUI_ACTIVE"] / 8 * 256 * 4), 1)
        if m.get("SQ_INSTS_MFMA"):
            d["valu_per_mfma"] = round(m["SQ_INSTS_VALU"] / m["SQ_INSTS_MFMA"], 2)
        if m.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_ANY" in m:
            d["wait_inst_pct"] = round(100.0 * m["SQ_WAIT_INST_ANY"] / m["SQ_WAVE_CYCLES"], 1)
        if m.get("SQ_ACTIVE_INST_LDS") and "SQ_LDS_BANK_CONFLICT" in m:
            d["lds_bank_conflict_per_active"] = round(m["SQ_LDS_BANK_CONFLICT"]
                                                      / m["SQ_ACTIVE_INST_LDS"], 3)
        kernels[k] = d
    out = {"workload": args.workload, "command": args.command, "kernels": kernels}
    with open(args.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {args.out}: {sorted(kernels)}")


if __name__ == "__main__":
    main()
