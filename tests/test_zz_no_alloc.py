"""moe_layer_forward_noalloc: the layer call whose workspace is the library's
static device scratch (for callers that cannot allocate). Its outputs and
routing must equal moe_layer_forward's bit for bit (same kernels, same
inputs) on consecutive calls, the second with fewer rows, and a call whose
workspace would exceed the scratch is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

from moe_spec import cfg_gptoss, cfg_mixed, cfg_qwen3, to_torch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from ffai_amd import _lib  # noqa: E402
from ffai_amd._lib import check  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    _lib.load()
    yield
    torch.cuda.synchronize()


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _trace(dev, T):
    E, k = dev.router.nExperts, dev.router.topK
    t = dict(logits=torch.empty(T, E, dtype=dev.act_dtype, device="cuda"),
             topk_idx=torch.empty(T, k, dtype=torch.int32, device="cuda"),
             topk_weight=torch.empty(T, k, dtype=torch.float32, device="cuda"),
             perm=torch.empty(T * k, dtype=torch.int32, device="cuda"),
             offsets=torch.empty(E + 1, dtype=torch.int32, device="cuda"))
    tr = _lib.LayerTrace(*(t[n].data_ptr() for n in
                           ("logits", "topk_idx", "topk_weight", "perm", "offsets")))
    return t, tr


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("cfg,Ts", [("qwen3", (64, 8)), ("gptoss", (4, 1)), ("mixed", (48, 2, 1)),
                                    ("qwen3", (256, 16))])
def test_noalloc_matches_forward(cfg, Ts):
    spec = {"qwen3": cfg_qwen3, "gptoss": cfg_gptoss, "mixed": cfg_mixed}[cfg]()
    dev = spec.device()
    lib = _lib.load()
    if Ts[0] == 256:
        # 16 rows per expert: the grouped GEMM, with its work items and the
        # f16 operand copy of the input in the static scratch
        assert dev.paths(256)["gate_up"] == "gemm", dev.paths(256)
        assert dev.workspace_bytes(256) <= lib.moe_layer_noalloc_max_bytes()
    for T in Ts:  # the second call has fewer rows and reuses the scratch as left
        x = to_torch(spec.x(T, seed=T))
        ref, tref = dev.forward(x, trace=True)
        ref = ref.clone()
        got = torch.full_like(x, float("nan"))
        tgot, tr = _trace(dev, T)
        print(f"noalloc {cfg} T={T}", flush=True)
        check(lib.moe_layer_forward_noalloc(C.byref(dev.desc), C.c_void_p(x.data_ptr()), T,
                                            C.c_void_p(got.data_ptr()), C.byref(tr), _stream()))
        torch.cuda.synchronize()
        assert _same(got, ref), f"{cfg} T={T}: output differs from moe_layer_forward"
        for key in ("logits", "topk_idx", "topk_weight", "perm", "offsets"):
            assert _same(tgot[key], tref[key]), f"{cfg} T={T}: {key} differs"


def test_noalloc_refuses_beyond_scratch():
    spec = cfg_qwen3()
    dev = spec.device()
    lib = _lib.load()
    limit = lib.moe_layer_noalloc_max_bytes()
    T = 1
    while dev.workspace_bytes(T) <= limit:
        T *= 2
    x = torch.zeros(T, spec.hidden, dtype=torch.bfloat16, device="cuda")
    y = torch.full_like(x, 7.0)
    st = lib.moe_layer_forward_noalloc(C.byref(dev.desc), C.c_void_p(x.data_ptr()), T,
                                       C.c_void_p(y.data_ptr()), None, _stream())
    torch.cuda.synchronize()
    assert st == _lib.MOE_ERR_WORKSPACE, st
    assert "static scratch" in _lib.last_error()
    assert bool((y == 7.0).all()), "nothing may run when the call is refused"
