"""C-ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects contract violations on the host
before any launch (the reference traps in Swift preconditions instead:
MoELayer.swift:105-124,449-484; QuantizedOpsValidation.swift:64-110)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from ffai_amd import _lib
from ffai_amd._lib import LayerDesc, QProj

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(moe_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in moe_hip.h but not exported"
    assert set(_lib.EXPORTS) == set(names)


def test_version():
    assert b"gfx950" in _lib.load().moe_version()


def _aligned(nbytes):
    buf = np.zeros(nbytes + 64, np.uint8)
    off = (-buf.ctypes.data) % 64
    return buf, buf.ctypes.data + off


_KEEP = []


def qproj(E=4, n=64, k=64, bits=4, gs=64, sb=_lib.MOE_BF16):
    buf, p = _aligned(16)
    _KEEP.append(buf)
    return QProj(p, p, p, None, bits, gs, sb, n, k, E)


def layer(E=4, k=2, H=64, I=64, act=_lib.MOE_BF16):
    d = LayerDesc()
    d.hidden, d.n_experts, d.top_k, d.intermediate, d.act_dtype = H, E, k, I, act
    buf, p = _aligned(16)
    _KEEP.append(buf)
    d.router_weight, d.router_dtype = p, act
    sb = _lib.MOE_F32 if act == _lib.MOE_F32 else _lib.MOE_BF16
    d.gate, d.up = qproj(E, I, H, sb=sb), qproj(E, I, H, sb=sb)
    d.down = qproj(E, H, I, sb=sb)
    return d


def status(fn, *args):
    return fn(*args)


def test_valid_layer_accepted():
    lib = _lib.load()
    assert lib.moe_validate_layer(C.byref(layer())) == _lib.MOE_OK
    assert lib.moe_layer_workspace_bytes(C.byref(layer()), 16) > 0


@pytest.mark.parametrize("mutate,expect,needle", [
    (lambda d: setattr(d, "top_k", 0), _lib.MOE_ERR_INVALID, "topK"),
    (lambda d: setattr(d, "top_k", 5), _lib.MOE_ERR_INVALID, "topK"),
    (lambda d: setattr(d, "n_experts", 0), _lib.MOE_ERR_INVALID, "nExperts"),
    (lambda d: setattr(d.gate, "bits", 7), _lib.MOE_ERR_INVALID, "bits=7"),
    (lambda d: setattr(d.down, "n", 32), _lib.MOE_ERR_INVALID, "down"),
    (lambda d: setattr(d.up, "n_experts", 3), _lib.MOE_ERR_INVALID, "expert counts"),
    (lambda d: setattr(d.gate, "group_size", 48), _lib.MOE_ERR_INVALID, "multiple of group_size"),
    (lambda d: setattr(d.gate, "group_size", 16), _lib.MOE_ERR_UNSUPPORTED, "group_size=16"),
    (lambda d: setattr(d, "gating", 5), _lib.MOE_ERR_INVALID, "gating"),
    (lambda d: setattr(d, "router_weight", None), _lib.MOE_ERR_INVALID, "router"),
    (lambda d: setattr(d.gate, "weight", d.gate.weight + 4), _lib.MOE_ERR_INVALID, "aligned"),
    (lambda d: setattr(d, "has_shared", 1), _lib.MOE_ERR_INVALID, "shared"),
])
def test_invalid_layer_rejected_on_host(mutate, expect, needle):
    lib = _lib.load()
    d = layer()
    mutate(d)
    st = lib.moe_validate_layer(C.byref(d))
    assert st == expect
    assert needle in _lib.last_error()
    # the whole-layer entry point rejects it before touching the device
    st2 = lib.moe_layer_forward(C.byref(d), C.c_void_p(64), 1, C.c_void_p(64), C.c_void_p(64), 1 << 30,
                                None, None)
    assert st2 == expect


def relu2_layer():
    d = layer()
    d.activation = _lib.MOE_ACT_RELU2
    d.gate = QProj()
    return d


def test_router_families_accepted():
    lib = _lib.load()
    d = layer()
    d.gating, d.routed_scale = _lib.MOE_SIGMOID_TOPK, 2.5
    assert lib.moe_validate_layer(C.byref(d)) == _lib.MOE_OK
    d = layer()
    d.activation, d.logit_scale = _lib.MOE_ACT_GEGLU, 64 ** -0.5
    assert lib.moe_validate_layer(C.byref(d)) == _lib.MOE_OK
    assert lib.moe_validate_layer(C.byref(relu2_layer())) == _lib.MOE_OK
    d = relu2_layer()
    d.has_shared = 1
    d.shared_up, d.shared_down = qproj(1, 128, 64), qproj(1, 64, 128)
    assert lib.moe_validate_layer(C.byref(d)) == _lib.MOE_OK
    assert lib.moe_layer_workspace_bytes(C.byref(d), 8) > 0


@pytest.mark.parametrize("mutate,needle", [
    (lambda d: setattr(d, "gate", qproj()), "no gate"),
    (lambda d: setattr(d, "activation", 4), "activation"),
    (lambda d: setattr(d, "logit_scale", float("nan")), "finite"),
    (lambda d: setattr(d, "routed_scale", float("inf")), "finite"),
    (lambda d: setattr(d, "gating", 3), "gating"),
])
def test_router_family_violations_rejected(mutate, needle):
    lib = _lib.load()
    d = relu2_layer()
    mutate(d)
    assert lib.moe_validate_layer(C.byref(d)) == _lib.MOE_ERR_INVALID
    assert needle in _lib.last_error()
    assert lib.moe_layer_forward_routed(C.byref(d), C.c_void_p(64), None, 1, C.c_void_p(64),
                                        C.c_void_p(64), 1 << 30, None, None) == _lib.MOE_ERR_INVALID


def test_layer_forward_checks_workspace_and_tokens():
    lib = _lib.load()
    d = layer()
    assert lib.moe_layer_forward(C.byref(d), C.c_void_p(64), 4, C.c_void_p(64), None, 0, None,
                                 None) == _lib.MOE_ERR_WORKSPACE
    assert lib.moe_layer_forward(C.byref(d), C.c_void_p(64), 0, C.c_void_p(64), C.c_void_p(64),
                                 1 << 30, None, None) == _lib.MOE_ERR_INVALID


def test_unsupported_dtype_pair():
    lib = _lib.load()
    d = layer(act=_lib.MOE_F32)
    d.gate.sb_dtype = _lib.MOE_BF16
    assert lib.moe_validate_layer(C.byref(d)) == _lib.MOE_ERR_UNSUPPORTED


@pytest.mark.parametrize("E,k,H,I,bits_gu,bits_d,gs,T,gate_up,down", [
    # Qwen3-shaped; the path query counts min(E, T k) used experts
    (128, 8, 2048, 768, 4, 4, 64, 1, "decode1", "decode1"),
    (128, 8, 2048, 768, 4, 4, 64, 16, "gemv_mma", "gemv"),      # 1 row per expert
    (128, 8, 2048, 768, 4, 4, 64, 24, "gemv_mma", "gemv"),      # 1.5 rows
    (128, 8, 2048, 768, 4, 4, 64, 32, "gemv_mma", "gemv_mma"),  # 2 rows
    (128, 8, 2048, 768, 4, 4, 64, 256, "gemm", "gemm"),         # 16 rows
    # GPT-OSS-shaped: 2 rows per expert at 16 tokens
    (32, 4, 2880, 2880, 4, 4, 32, 16, "gemv_mma", "gemv_mma"),
    # 3-bit gate/up, 6-bit down: the matrix cores from 2 rows
    (128, 8, 2048, 768, 3, 6, 64, 16, "gemv", "gemv"),
    (128, 8, 2048, 768, 3, 6, 64, 32, "gemv_mma", "gemv_mma"),
])
def test_gemv_selection(E, k, H, I, bits_gu, bits_d, gs, T, gate_up, down):
    """The grouped kernel each projection takes (moe_layer_path, host only): a
    4-bit gate/up pair on the matrix-core GEMV at any row count, a 4-bit single
    projection from 1.8 rows per used expert, other widths from 2, the GEMM
    from 16 rows (64+ experts)."""
    d = layer(E=E, k=k, H=H, I=I)
    d.gate, d.up = qproj(E, I, H, bits_gu, gs), qproj(E, I, H, bits_gu, gs)
    d.down = qproj(E, H, I, bits_d, gs)
    p = _lib.LayerPaths()
    assert _lib.load().moe_layer_path(C.byref(d), T, C.byref(p)) == _lib.MOE_OK
    got = p.names()
    assert (got["gate_up"], got["down"]) == (gate_up, down), got


def test_derive_bits_cases():
    lib = _lib.load()
    out = C.c_int32()
    for in_f, bits in [(256, 4), (256, 8), (4096, 4), (4096, 8), (1024, 3), (1024, 6)]:
        assert lib.moe_derive_bits(in_f * bits // 32, in_f // 64, 64, C.byref(out)) == 0
        assert out.value == bits
    assert lib.moe_derive_bits(7, 1, 64, C.byref(out)) == _lib.MOE_ERR_INVALID


def test_kernel_entry_points_validate_before_launch():
    lib = _lib.load()
    p = C.c_void_p(256)
    assert lib.moe_router_topk(p, 2, 4, 8, 9, 0, 1, None, p, p, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_router_topk(p, 2, 0, 8, 2, 0, 1, None, p, p, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_router_topk(p, 2, 1, 600, 2, 0, 1, None, p, p, None) == _lib.MOE_ERR_UNSUPPORTED
    assert lib.moe_router_topk(p, 2, 4, 8, 2, 3, 1, None, p, p, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_router_topk_scaled(p, 2, 4, 8, 2, 2, 1, None, float("nan"), 1.0, None, p, p,
                                      None) == _lib.MOE_ERR_INVALID
    assert lib.moe_activation_apply(None, p, p, 8, 2, _lib.MOE_ACT_SWIGLU, 0.0, 0.0,
                                    None) == _lib.MOE_ERR_INVALID
    assert lib.moe_dispatch_plan(p, 4, 2, 8, p, p, p, p, None, 0, None) == _lib.MOE_ERR_WORKSPACE
    assert lib.moe_dequantize_affine(p, p, p, 2, 4, 4, 64, p, 2, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_dequantize_affine(p, p, p, 2, 3, 16, 64, p, 2, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_unpermute(p, p, p, 2, 12, 2, p, 2, None) == _lib.MOE_ERR_UNSUPPORTED
    q = qproj()
    assert lib.moe_expert_matmul(C.byref(q), p, 2, None, 1, 8, p, p, None, 0, None) == _lib.MOE_ERR_WORKSPACE


def test_no_oracle_in_product():
    """The product library and package never reference the CPU oracle."""
    pkg = os.path.join(ROOT, "ffai_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "moe_oracle" not in text and "import oracle" not in text, f


def test_swift_module_map():
    """swift/CMoEHIP: the module map names headers that resolve to include/
    and the library that ffai_amd/ holds, and the headers compile as plain C
    on their own (what a Swift clang importer reads)."""
    import subprocess
    d = os.path.join(ROOT, "swift", "CMoEHIP")
    text = open(os.path.join(d, "module.modulemap")).read()
    headers = re.findall(r'header\s+"([^"]+)"', text)
    assert set(headers) == {"moe_hip.h", "moe_safetensors.h"}
    for h in headers:
        assert os.path.realpath(os.path.join(d, h)) == os.path.join(ROOT, "include", h)
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-x", "c",
                        os.path.join(d, h)], check=True)
    (link,) = re.findall(r'link\s+"([^"]+)"', text)
    assert os.path.basename(_lib.LIB_PATH) == f"lib{link}.so"
    pkg = open(os.path.join(ROOT, "swift", "Package.swift")).read()
    assert '.systemLibrary(name: "CMoEHIP", path: "CMoEHIP")' in pkg
