"""Checkpoint reader over libmoehip.so's C ABI (include/moe_safetensors.h),
and a writer for the same format.

Mirrors FFAI's SafeTensorsBundle (Sources/FFAI/Loader/SafeTensors.swift:
237-397): a directory (sharded index, model.safetensors, or every
*.safetensors in name order) or a single file, tensor lookup by name, the
quantized-triplet test, and the stacked mlx-affine expert stacks the MoE
loaders read (Models/Text/Qwen3xText.swift:682-800, Gemma4Text.swift:
540-555), uploaded straight into HBM as ``layer.StackedExperts``. Parsing,
mapping and the host-to-device copies are native; PyTorch only owns the
device memory.

SafeTensorsWriter mirrors FFAI's SafeTensorsWriter (Sources/FFAI/Loader/
SafeTensorsWriter.swift:69-183): append named tensors, then finalize one file
with a sorted-key header; empty tensors and repeated names are errors.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
from typing import List, Tuple

import torch

from . import _lib
from ._lib import QProj, check
from .layer import StackedExperts

_TORCH = {
    _lib.MOE_ST_F32: torch.float32, _lib.MOE_ST_F16: torch.float16, _lib.MOE_ST_BF16: torch.bfloat16,
    _lib.MOE_ST_I32: torch.int32, _lib.MOE_ST_U32: torch.int32, _lib.MOE_ST_I64: torch.int64,
    _lib.MOE_ST_U64: torch.int64, _lib.MOE_ST_I8: torch.int8, _lib.MOE_ST_U8: torch.uint8,
}
_SB_TORCH = {_lib.MOE_F32: torch.float32, _lib.MOE_F16: torch.float16, _lib.MOE_BF16: torch.bfloat16}


def _stream(device: torch.device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _mx_views(q: QProj, buf: torch.Tensor, dtype: torch.dtype) -> StackedExperts:
    """StackedExperts views of an MXFP4 projection moe_st_load_mxfp4 placed in
    buf (affine 4-bit, group 32, per-row bias as out_bias)."""
    se = _views(q, buf, 32)
    ob = q.out_bias - buf.data_ptr()
    esz = torch.tensor([], dtype=dtype).element_size()
    se.out_bias = buf[ob:ob + q.n_experts * q.n * esz].view(dtype).view(q.n_experts, q.n)
    return se


def _views(q: QProj, buf: torch.Tensor, groupSize: int) -> StackedExperts:
    """StackedExperts views of a triplet that moe_st_load_stacked placed in buf."""
    E, N, K = q.n_experts, q.n, q.k
    base = buf.data_ptr()
    w_off, s_off, b_off = q.weight - base, q.scales - base, q.biases - base
    sdt = _SB_TORCH[q.sb_dtype]
    ssz = torch.tensor([], dtype=sdt).element_size()
    G = K // groupSize
    words = K * q.bits // 32
    weight = buf[w_off:w_off + E * N * words * 4].view(torch.int32).view(E, N, words)
    scales = buf[s_off:s_off + E * N * G * ssz].view(sdt).view(E, N, G)
    biases = buf[b_off:b_off + E * N * G * ssz].view(sdt).view(E, N, G)
    se = StackedExperts(weight, scales, biases, q.bits, groupSize)
    se._storage = buf  # the three views share this allocation
    return se


class SafeTensorsBundle:
    """One or more safetensors files as a single tensor namespace."""

    def __init__(self, path: str):
        lib = _lib.load()
        h = C.c_void_p()
        check(lib.moe_st_open(str(path).encode(), C.byref(h)))
        self._h = h
        self._lib = lib

    def close(self):
        if self._h:
            self._lib.moe_st_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- SafeTensorsBundle API -------------------------------------------
    @property
    def allKeys(self) -> List[str]:
        n = self._lib.moe_st_count(self._h)
        return [self._lib.moe_st_name(self._h, i).decode() for i in range(n)]

    def has(self, name: str) -> bool:
        return self._lib.moe_st_info(self._h, name.encode(), None, None, None, None) == _lib.MOE_OK

    def info(self, name: str) -> Tuple[int, Tuple[int, ...], int]:
        """(moe_st_dtype, shape, nbytes) of a tensor."""
        dt, nd = C.c_int32(), C.c_int32()
        shape = (C.c_int64 * _lib.MOE_ST_MAX_DIMS)()
        nb = C.c_size_t()
        check(self._lib.moe_st_info(self._h, name.encode(), C.byref(dt), C.byref(nd), shape,
                                    C.byref(nb)))
        return dt.value, tuple(shape[i] for i in range(nd.value)), nb.value

    def read_bytes(self, name: str) -> bytes:
        """The tensor's raw bytes in host memory."""
        _, _, nb = self.info(name)
        buf = (C.c_uint8 * max(nb, 1))()
        check(self._lib.moe_st_read_host(self._h, name.encode(), buf, nb))
        return bytes(buf)[:nb]

    def tensor(self, name: str, device="cuda") -> torch.Tensor:
        """tensor(named:) uploaded to the GPU. U32/U64 tensors come back as
        int32/int64 storage holding the same bits."""
        dt, shape, nb = self.info(name)
        dev = torch.device(device)
        out = torch.empty(shape, dtype=_TORCH[dt], device=dev)
        if nb:
            check(self._lib.moe_st_upload(self._h, name.encode(), C.c_void_p(out.data_ptr()), nb,
                                          _stream(dev)))
        return out

    def isQuantized(self, base: str) -> bool:
        return bool(self._lib.moe_st_is_quantized(self._h, base.encode()))

    def stackedExperts(self, base: str, groupSize: int, device="cuda") -> StackedExperts:
        """The stacked triplet at ``base`` (``<base>.weight/.scales/.biases``)
        in one device allocation, bits derived from the shapes."""
        return self.stackedExpertsMany([base], groupSize, device)[0]

    def mxfp4Experts(self, base: str, dtype: torch.dtype = torch.bfloat16,
                     device="cuda") -> StackedExperts:
        """A GPT-OSS MXFP4 stack (``<base>.weight/.scales/.bias``) transcoded
        on the GPU to affine 4-bit with group size 32, scales, biases and
        the per-row bias in ``dtype`` (transcodeStackedExperts,
        GPTOSSText.swift:1071-1236)."""
        adt = {torch.float32: _lib.MOE_F32, torch.float16: _lib.MOE_F16,
               torch.bfloat16: _lib.MOE_BF16}[dtype]
        nb, ns = C.c_size_t(), C.c_size_t()
        check(self._lib.moe_st_mxfp4_bytes(self._h, base.encode(), adt, C.byref(nb), C.byref(ns)))
        dev = torch.device(device)
        buf = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        scratch = torch.empty(ns.value, dtype=torch.uint8, device=dev)
        q = QProj()
        check(self._lib.moe_st_load_mxfp4(self._h, base.encode(), adt, C.c_void_p(buf.data_ptr()),
                                          nb.value, C.c_void_p(scratch.data_ptr()), ns.value,
                                          C.byref(q), _stream(dev)))
        torch.cuda.current_stream(dev).synchronize()  # the scratch is freed on return
        return _mx_views(q, buf, dtype)

    def stackedExpertsMany(self, bases: List[str], groupSize: int,
                           device="cuda") -> List[StackedExperts]:
        """Several triplets (a layer's gate, up and down, say) validated
        together and streamed through one queue of host-to-device copies."""
        n = len(bases)
        dev = torch.device(device)
        sizes = []
        for base in bases:
            nb = C.c_size_t()
            check(self._lib.moe_st_stacked_bytes(self._h, base.encode(), groupSize, C.byref(nb)))
            sizes.append(nb.value)
        bufs = [torch.empty(sz, dtype=torch.uint8, device=dev) for sz in sizes]
        names = (C.c_char_p * n)(*[b.encode() for b in bases])
        dsts = (C.c_void_p * n)(*[t.data_ptr() for t in bufs])
        nbytes = (C.c_size_t * n)(*sizes)
        qs = (QProj * n)()
        check(self._lib.moe_st_load_stacked_many(self._h, n, names, groupSize, dsts, nbytes, qs,
                                                 _stream(dev)))
        return [_views(q, buf, groupSize) for q, buf in zip(qs, bufs)]


_ST_NAME = {_lib.MOE_ST_F32: "F32", _lib.MOE_ST_F16: "F16", _lib.MOE_ST_BF16: "BF16",
            _lib.MOE_ST_I32: "I32", _lib.MOE_ST_U32: "U32", _lib.MOE_ST_I64: "I64",
            _lib.MOE_ST_U64: "U64", _lib.MOE_ST_I8: "I8", _lib.MOE_ST_U8: "U8"}


class SafeTensorsWriterError(ValueError):
    pass


class SafeTensorsWriter:
    """Accumulates (name, dtype, shape, bytes) and writes one safetensors
    file: u64 header length, a JSON header with sorted keys and a
    ``__metadata__`` block, the tensors' bytes in append order. The file is
    written under a temporary name and renamed into place."""

    def __init__(self, path: str):
        self.path = str(path)
        self._pending = []
        self._names = set()

    def append(self, name: str, dtype: int, shape, data) -> None:
        """dtype: a moe_st_dtype value; data: bytes or a buffer (numpy array)."""
        raw = data if isinstance(data, (bytes, bytearray)) else memoryview(data).cast("B")
        if len(raw) == 0:
            raise SafeTensorsWriterError(
                f'SafeTensorsWriter: tensor "{name}" has zero bytes - cannot write empty tensor')
        if name in self._names:
            raise SafeTensorsWriterError(f'SafeTensorsWriter: tensor "{name}" appended twice')
        if dtype not in _ST_NAME:
            raise SafeTensorsWriterError(f"SafeTensorsWriter: unknown dtype {dtype}")
        self._names.add(name)
        self._pending.append((name, dtype, [int(d) for d in shape], raw))

    def finalize(self) -> None:
        header = {"__metadata__": {"format": "pt", "writer": "ffai_amd"}}
        off = 0
        for name, dt, shape, raw in self._pending:
            header[name] = {"data_offsets": [off, off + len(raw)], "dtype": _ST_NAME[dt],
                            "shape": shape}
            off += len(raw)
        text = json.dumps(header, sort_keys=True, separators=(",", ":"),
                          ensure_ascii=False).encode()
        tmp = self.path + ".tmp"
        with open(tmp, "wb") as f:
            f.write(struct.pack("<Q", len(text)))
            f.write(text)
            for _, _, _, raw in self._pending:
                f.write(raw)
        os.replace(tmp, self.path)
        self._pending.clear()
        self._names.clear()
