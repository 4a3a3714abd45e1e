"""The checkpoint reader (include/moe_safetensors.h): the reference's own
SafeTensors tests (Tests/FFAITests/Loader/SafeTensorsTests.swift,
SafeTensorsErrorTests.swift) restated on files written here, the stacked
mlx-affine triplets with per-tensor bit derivation (Layers.swift:348-363),
and on the GPU, uploads bit-exact and checkpoint-loaded experts driving the
layer to the same bits as the in-memory stacks."""
import ctypes as C
import json
import struct

import numpy as np
import pytest

import oracle as orc
from ffai_amd import _lib
from ffai_amd._lib import MoeError
from moe_spec import BF16, F16, LayerSpec, gen_qproj, store

_DT = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int32): "I32",
       np.dtype(np.uint32): "U32", np.dtype(np.int64): "I64", np.dtype(np.uint64): "U64",
       np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8"}


def write_st(path, tensors, metadata=None, pad_to=8):
    """A safetensors file: {name: ndarray, or (dtype_name, shape, raw bytes)}.
    bf16 arrays are passed as ("BF16", shape, bytes)."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, t in tensors.items():
        if isinstance(t, tuple):
            dt, shape, raw = t
        else:
            t = np.ascontiguousarray(t)
            dt, shape, raw = _DT[t.dtype], list(t.shape), t.tobytes()
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % pad_to)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
    return path


def write_raw(path, payload: bytes, extra=b""):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(payload)) + payload + extra)
    return path


def bf16(a):
    a = store(np.asarray(a, np.float32), BF16)
    return ("BF16", list(a.shape), a.tobytes())


class Bundle:
    """Thin host-only view over moe_st_* (no GPU needed)."""

    def __init__(self, path):
        self.lib = _lib.load()
        self.h = C.c_void_p()
        st = self.lib.moe_st_open(str(path).encode(), C.byref(self.h))
        if st != _lib.MOE_OK:
            raise MoeError(st, _lib.last_error())

    def close(self):
        self.lib.moe_st_close(self.h)

    def keys(self):
        return [self.lib.moe_st_name(self.h, i).decode() for i in range(self.lib.moe_st_count(self.h))]

    def info(self, name):
        dt, nd, nb = C.c_int32(), C.c_int32(), C.c_size_t()
        shape = (C.c_int64 * 8)()
        _lib.check(self.lib.moe_st_info(self.h, name.encode(), C.byref(dt), C.byref(nd), shape,
                                        C.byref(nb)))
        return dt.value, tuple(shape[i] for i in range(nd.value)), nb.value

    def read(self, name):
        _, _, nb = self.info(name)
        buf = (C.c_uint8 * max(nb, 1))()
        _lib.check(self.lib.moe_st_read_host(self.h, name.encode(), buf, nb))
        return bytes(buf)[:nb]

    def stacked_bytes(self, base, gs):
        nb = C.c_size_t()
        _lib.check(self.lib.moe_st_stacked_bytes(self.h, base.encode(), gs, C.byref(nb)))
        return nb.value


def open_error(path):
    with pytest.raises(MoeError) as ei:
        Bundle(path)
    return str(ei.value)


# ------------------------------------------- SafeTensorsTests.swift cases --

def test_load_synthetic_single_tensor_file(tmp_path):
    """SafeTensorsTests.swift:48-64."""
    vals = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3)
    b = Bundle(write_st(tmp_path / "model.safetensors", {"alpha.weight": vals}))
    assert b.info("alpha.weight") == (_lib.MOE_ST_F32, (2, 3), 24)
    assert np.array_equal(np.frombuffer(b.read("alpha.weight"), np.float32).reshape(2, 3), vals)
    b.close()


def test_missing_tensor(tmp_path):
    """SafeTensorsTests.swift:93-111 / SafeTensorsErrorTests.swift:137-155."""
    b = Bundle(write_st(tmp_path / "m.safetensors", {"present": np.ones(1, np.float32)}))
    with pytest.raises(MoeError) as ei:
        b.info("absent")
    assert 'tensor "absent" not present' in str(ei.value)
    b.close()


def test_file_not_found():
    """SafeTensorsTests.swift:113-126."""
    assert "not found" in open_error("/__nope__/missing.safetensors")


def test_bundle_fallback_glob(tmp_path):
    """SafeTensorsTests.swift:128-143: a directory without model.safetensors
    or an index loads every *.safetensors."""
    write_st(tmp_path / "weights.safetensors", {"x": np.array([42, 43, 44], np.float32)})
    (tmp_path / "notes.txt").write_text("not a tensor file")
    b = Bundle(tmp_path)
    assert b.keys() == ["x"]
    assert np.array_equal(np.frombuffer(b.read("x"), np.float32), [42, 43, 44])
    b.close()


def test_bundle_sharded_index(tmp_path):
    """SafeTensorsTests.swift:145-175."""
    write_st(tmp_path / "model-00001-of-00002.safetensors", {"a": np.array([10], np.float32)})
    write_st(tmp_path / "model-00002-of-00002.safetensors", {"b": np.array([20], np.float32)})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {"total_size": 8},
         "weight_map": {"a": "model-00001-of-00002.safetensors",
                        "b": "model-00002-of-00002.safetensors"}}))
    b = Bundle(tmp_path)
    assert b.keys() == ["a", "b"]
    assert np.frombuffer(b.read("a"), np.float32)[0] == 10
    assert np.frombuffer(b.read("b"), np.float32)[0] == 20
    b.close()


def test_model_safetensors_preferred_over_glob(tmp_path):
    """SafeTensors.swift:270-276: model.safetensors alone when it exists."""
    write_st(tmp_path / "model.safetensors", {"m": np.zeros(1, np.float32)})
    write_st(tmp_path / "other.safetensors", {"o": np.zeros(1, np.float32)})
    b = Bundle(tmp_path)
    assert b.keys() == ["m"]
    b.close()


# -------------------------------------- SafeTensorsErrorTests.swift cases --

def test_header_too_small(tmp_path):
    """SafeTensorsErrorTests.swift:33-46."""
    p = tmp_path / "t.safetensors"
    p.write_bytes(bytes([1, 2, 3]))
    assert "smaller than 8 bytes" in open_error(p)


def test_malformed_json(tmp_path):
    """SafeTensorsErrorTests.swift:48-66."""
    assert "JSON header malformed" in open_error(write_raw(tmp_path / "t.safetensors", b"not json"))


def test_entry_missing_field(tmp_path):
    """SafeTensorsErrorTests.swift:68-86."""
    msg = open_error(write_raw(tmp_path / "t.safetensors", b'{"x": {"dtype": "F32"}}'))
    assert 'malformed entry for tensor "x"' in msg


def test_unsupported_dtype_skipped(tmp_path):
    """SafeTensorsErrorTests.swift:88-118: F64 is skipped at open and a
    lookup reports a missing tensor."""
    p = write_raw(tmp_path / "t.safetensors",
                  b'{"x": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}', bytes(8))
    b = Bundle(p)
    assert b.keys() == []
    with pytest.raises(MoeError) as ei:
        b.info("x")
    assert "not present" in str(ei.value)
    b.close()


@pytest.mark.parametrize("payload,extra", [
    (b'{"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}', bytes(8)),   # past the end
    (b'{"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}', bytes(16)),  # size mismatch
    (b'{"x": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}', b""),        # negative dim
    (b'{"x": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}', bytes(8)),    # reversed
    (b'{"x": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}', bytes(4)),  # non-integer
])
def test_entry_bounds_rejected(tmp_path, payload, extra):
    assert "malformed entry" in open_error(write_raw(tmp_path / "t.safetensors", payload, extra))


def test_header_length_beyond_file(tmp_path):
    p = tmp_path / "t.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    assert "malformed" in open_error(p)


@pytest.mark.parametrize("bad", [b'{"x": }', b'{"x": {"dtype": "F32",}}', b'{"x": [1, 2]', b'{"a": 1} x',
                                 b'{"\\ud800": 1}', b'{"x": "unterminated}'])
def test_malformed_json_variants(tmp_path, bad):
    assert "malformed" in open_error(write_raw(tmp_path / "t.safetensors", bad))


def test_metadata_escapes_padding_and_dtype_case(tmp_path):
    """__metadata__ is skipped, names may carry JSON escapes, headers may be
    padded with spaces, dtype names are case-insensitive (DType.swift:43)."""
    raw = np.arange(4, dtype=np.float16).tobytes()
    p = write_st(tmp_path / "t.safetensors",
                 {"aé\U0001f600.w": ("f16", [4], raw), "z": np.zeros((0, 3), np.float32)},
                 metadata={"format": "mlx", "nested": {"k": [1, 2.5, True, None]}}, pad_to=64)
    b = Bundle(p)
    assert b.keys() == ["aé\U0001f600.w", "z"]
    assert b.info("aé\U0001f600.w") == (_lib.MOE_ST_F16, (4,), 8)
    assert b.read("aé\U0001f600.w") == raw
    assert b.info("z") == (_lib.MOE_ST_F32, (0, 3), 0)
    b.close()


def test_later_shard_wins_duplicate_names(tmp_path):
    """SafeTensors.swift:284-287: the name index keeps the last file's entry."""
    write_st(tmp_path / "a.safetensors", {"dup": np.array([1], np.float32)})
    write_st(tmp_path / "b.safetensors", {"dup": np.array([2], np.float32)})
    b = Bundle(tmp_path)
    assert np.frombuffer(b.read("dup"), np.float32)[0] == 2
    b.close()


# ------------------------------------- SafeTensorsWriterTests.swift cases --

def test_writer_f16_round_trip(tmp_path):
    """SafeTensorsWriterTests.swift:32-60."""
    from ffai_amd.safetensors import SafeTensorsWriter
    vals = np.array([1.5, -2.0, 0.25, 3.0, 4.0, -0.5], np.float16)
    w = SafeTensorsWriter(tmp_path / "model.safetensors")
    w.append("layer.weight", _lib.MOE_ST_F16, [2, 3], vals)
    w.finalize()
    b = Bundle(tmp_path / "model.safetensors")
    assert b.info("layer.weight") == (_lib.MOE_ST_F16, (2, 3), 12)
    assert b.read("layer.weight") == vals.tobytes()
    b.close()


def test_writer_mixed_dtypes_offsets(tmp_path):
    """SafeTensorsWriterTests.swift:62-104: offsets follow append order and
    the header keys are sorted."""
    from ffai_amd.safetensors import SafeTensorsWriter
    a = np.arange(3, dtype=np.float32)
    bb = np.arange(5, dtype=np.uint8)
    c = np.arange(2, dtype=np.int64)
    p = tmp_path / "m.safetensors"
    w = SafeTensorsWriter(p)
    w.append("zeta", _lib.MOE_ST_F32, [3], a)
    w.append("alpha", _lib.MOE_ST_U8, [5], bb)
    w.append("mid", _lib.MOE_ST_I64, [2], c)
    w.finalize()
    raw = p.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    assert list(hdr) == sorted(hdr)
    assert hdr["zeta"]["data_offsets"] == [0, 12]
    assert hdr["alpha"]["data_offsets"] == [12, 17]
    assert hdr["mid"]["data_offsets"] == [17, 33]
    b = Bundle(p)
    assert b.read("zeta") == a.tobytes() and b.read("alpha") == bb.tobytes()
    assert b.read("mid") == c.tobytes()
    b.close()


def test_writer_file_loads_as_bundle(tmp_path):
    """SafeTensorsWriterTests.swift:106-128."""
    from ffai_amd.safetensors import SafeTensorsWriter
    w = SafeTensorsWriter(tmp_path / "model.safetensors")
    w.append("x", _lib.MOE_ST_F32, [2], np.array([7, 8], np.float32))
    w.finalize()
    b = Bundle(tmp_path)
    assert b.keys() == ["x"]
    b.close()


def test_writer_duplicate_and_empty_rejected(tmp_path):
    """SafeTensorsWriterTests.swift:130-170."""
    from ffai_amd.safetensors import SafeTensorsWriter, SafeTensorsWriterError
    w = SafeTensorsWriter(tmp_path / "m.safetensors")
    w.append("a", _lib.MOE_ST_F32, [1], np.zeros(1, np.float32))
    with pytest.raises(SafeTensorsWriterError, match="appended twice"):
        w.append("a", _lib.MOE_ST_F32, [1], np.zeros(1, np.float32))
    with pytest.raises(SafeTensorsWriterError, match="zero bytes"):
        w.append("e", _lib.MOE_ST_F32, [0], b"")


# -------------------------------------------------------- stacked triplets --

def stacked_tensors(base, E, N, K, bits, gs, sb="BF16", seed=0, two_d=False):
    rng = np.random.default_rng(seed)
    q = gen_qproj(rng, E, N, K, bits, gs, BF16 if sb == "BF16" else F16)
    w, s, b = q.weight, q.scales, q.biases
    if two_d:
        w, s, b = w[0], s[0], b[0]
    return q, {f"{base}.weight": np.ascontiguousarray(w),
               f"{base}.scales": (sb, list(s.shape), s.tobytes()),
               f"{base}.biases": (sb, list(b.shape), b.tobytes())}


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_stacked_layout_derives_bits(tmp_path, bits, gs):
    base = "model.layers.0.mlp.switch_mlp.gate_proj"
    q, t = stacked_tensors(base, 4, 48, 256, bits, gs)
    b = Bundle(write_st(tmp_path / "m.safetensors", t))
    assert b.lib.moe_st_is_quantized(b.h, base.encode()) == 1
    assert b.lib.moe_st_is_quantized(b.h, b"model.layers.0.mlp.switch_mlp.up_proj") == 0
    a = lambda n: (n + 255) // 256 * 256  # noqa: E731
    assert b.stacked_bytes(base, gs) == a(q.weight.nbytes) + a(q.scales.nbytes) + a(q.biases.nbytes)
    assert orc.derive_bits(q.weight.shape[-1], q.scales.shape[-1], gs) == bits
    b.close()


def test_stacked_2d_single_expert(tmp_path):
    base = "model.layers.0.mlp.shared_expert.down_proj"
    q, t = stacked_tensors(base, 1, 64, 128, 4, 64, two_d=True)
    b = Bundle(write_st(tmp_path / "m.safetensors", t))
    assert b.stacked_bytes(base, 64) > 0
    b.close()


@pytest.mark.parametrize("case,needle", [
    ("bits7", "unsupported quantization bit-width"),
    ("inconsistent", "deriveAffineQuantBits"),
    ("bias_dtype", "biases must match"),
    ("weight_dtype", "packed weight must be U32"),
    ("rows", "do not match weight rows"),
    ("missing", "not present"),
])
def test_stacked_layout_rejects(tmp_path, case, needle):
    base = "experts.switch_glu.up_proj"
    q, t = stacked_tensors(base, 2, 32, 256, 4, 64)
    if case == "bits7":  # 256 in-features at 7 bits = 56 words
        t[f"{base}.weight"] = np.zeros((2, 32, 56), np.uint32)
    elif case == "inconsistent":
        t[f"{base}.weight"] = np.zeros((2, 32, 33), np.uint32)
    elif case == "bias_dtype":
        t[f"{base}.biases"] = np.zeros((2, 32, 4), np.float32)
    elif case == "weight_dtype":
        t[f"{base}.weight"] = ("F32", [2, 32, 32], bytes(2 * 32 * 32 * 4))
    elif case == "rows":
        t[f"{base}.scales"] = bf16(np.zeros((2, 31, 4)))
        t[f"{base}.biases"] = bf16(np.zeros((2, 31, 4)))
    elif case == "missing":
        del t[f"{base}.biases"]
    b = Bundle(write_st(tmp_path / "m.safetensors", t))
    with pytest.raises(MoeError) as ei:
        b.stacked_bytes(base, 64)
    assert needle in str(ei.value)
    b.close()


def test_load_many_validates_every_triplet_first(tmp_path):
    """A bad triplet anywhere in the list fails the call before any copy
    (the first destination here is not device memory at all)."""
    base = "m.switch_mlp.gate_proj"
    _, t = stacked_tensors(base, 2, 32, 256, 4, 64)
    b = Bundle(write_st(tmp_path / "m.safetensors", t))
    need = b.stacked_bytes(base, 64)
    names = (C.c_char_p * 2)(base.encode(), b"m.switch_mlp.up_proj")
    dsts = (C.c_void_p * 2)(256, 512)
    sizes = (C.c_size_t * 2)(need, need)
    qs = (_lib.QProj * 2)()
    st = b.lib.moe_st_load_stacked_many(b.h, 2, names, 64, dsts, sizes, qs, None)
    assert st == _lib.MOE_ERR_INVALID and "not present" in _lib.last_error()
    sizes[1] = 0
    names[1] = base.encode()
    st = b.lib.moe_st_load_stacked_many(b.h, 2, names, 64, dsts, sizes, qs, None)
    assert st == _lib.MOE_ERR_INVALID and "device bytes" in _lib.last_error()
    b.close()


# --------------------------------------------------------------------- GPU --

def _torch():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.gpu
def test_upload_bit_exact(tmp_path):
    """Every dtype, including tensors spanning several staging buffers."""
    torch = _torch()
    from ffai_amd.safetensors import SafeTensorsBundle
    rng = np.random.default_rng(5)
    big = rng.integers(0, 2**32, size=(25 << 20) // 4 * 3 + 7, dtype=np.uint64).astype(np.uint32)
    t = {"f32": rng.normal(size=(3, 5)).astype(np.float32),
         "f16": rng.normal(size=(7,)).astype(np.float16),
         "bf16": bf16(rng.normal(size=(4, 4))),
         "i8": rng.integers(-128, 127, size=33, dtype=np.int8),
         "u64": rng.integers(0, 2**63, size=9, dtype=np.uint64),
         "big": big, "empty": np.zeros((0,), np.float32)}
    write_st(tmp_path / "model.safetensors", t)
    with SafeTensorsBundle(str(tmp_path)) as b:
        for name in t:
            got = b.tensor(name)
            torch.cuda.synchronize()
            flat = got.reshape(-1).view(torch.uint8) if got.numel() else None
            host = flat.cpu().numpy().tobytes() if got.numel() else b""
            assert host == b.read_bytes(name), name
        assert b.tensor("big").numel() == big.size


def _checkpoint_spec(seed=0):
    """A 3-bit gate/up, 6-bit down, bf16-scale layer with a shared expert:
    the per-tensor bit derivation must see each width."""
    rng = np.random.default_rng(seed)
    H, E, k, I, SI = 512, 16, 4, 256, 384
    shared = (gen_qproj(rng, 1, SI, H, 4, 64, BF16), gen_qproj(rng, 1, SI, H, 4, 64, BF16),
              gen_qproj(rng, 1, H, SI, 8, 64, BF16))
    return LayerSpec(H, E, k, I, BF16,
                     router_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(E, H)), BF16),
                     router_dt=BF16,
                     gate=gen_qproj(rng, E, I, H, 3, 64, BF16), up=gen_qproj(rng, E, I, H, 3, 64, BF16),
                     down=gen_qproj(rng, E, H, I, 6, 64, BF16), shared=shared,
                     shared_gate_weight=store(rng.normal(0, 1 / np.sqrt(H), size=(1, H)), BF16),
                     name="ckpt")


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 6, 300])
def test_checkpoint_experts_drive_the_layer(tmp_path, T):
    """Stacks written as an mlx checkpoint (two shards + index, Qwen-style
    switch_mlp names), loaded through the reader, give bit-identical layer
    outputs to the same stacks passed in memory, and meet the oracle bar."""
    torch = _torch()
    from ffai_amd import layer as fl
    from ffai_amd.safetensors import SafeTensorsBundle
    from moe_spec import check_close, load, to_numpy_f32, to_torch, with_quantised_router
    # the router (mlp.gate) and the shared expert's sigmoid gate are quantised
    # linears in an mlx checkpoint (loadLinear, Qwen3xText.swift:605-606, 660-661)
    spec = with_quantised_router(_checkpoint_spec(), bits=4, shared_gate_bits=4)
    p = "model.layers.7.mlp"

    def trip(base, q, two_d=False):
        w, s, b = (q.weight, q.scales, q.biases) if not two_d else (q.weight[0], q.scales[0], q.biases[0])
        return {f"{base}.weight": w, f"{base}.scales": ("BF16", list(s.shape), s.tobytes()),
                f"{base}.biases": ("BF16", list(b.shape), b.tobytes())}

    shard1 = {**trip(f"{p}.switch_mlp.gate_proj", spec.gate), **trip(f"{p}.switch_mlp.up_proj", spec.up)}
    shard2 = {**trip(f"{p}.switch_mlp.down_proj", spec.down),
              **trip(f"{p}.shared_expert.gate_proj", spec.shared[0], True),
              **trip(f"{p}.shared_expert.up_proj", spec.shared[1], True),
              **trip(f"{p}.shared_expert.down_proj", spec.shared[2], True),
              **trip(f"{p}.gate", spec.router_weight, True),
              **trip(f"{p}.shared_expert_gate", spec.shared_gate_weight, True)}
    write_st(tmp_path / "model-00001-of-00002.safetensors", shard1)
    write_st(tmp_path / "model-00002-of-00002.safetensors", shard2)
    wm = {n: "model-00001-of-00002.safetensors" for n in shard1}
    wm.update({n: "model-00002-of-00002.safetensors" for n in shard2})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))

    with SafeTensorsBundle(str(tmp_path)) as b:
        assert b.isQuantized(f"{p}.switch_mlp.gate_proj")
        g = b.stackedExperts(f"{p}.switch_mlp.gate_proj", 64)
        u, d = b.stackedExpertsMany([f"{p}.switch_mlp.up_proj", f"{p}.switch_mlp.down_proj"], 64)
        sh = tuple(b.stackedExpertsMany([f"{p}.shared_expert.{n}_proj" for n in ("gate", "up", "down")],
                                        64))
        assert b.isQuantized(f"{p}.gate") and b.isQuantized(f"{p}.shared_expert_gate")
        rq, sgq = b.stackedExpertsMany([f"{p}.gate", f"{p}.shared_expert_gate"], 64)
    assert (g.bits, u.bits, d.bits, sh[2].bits, rq.bits, sgq.bits) == (3, 3, 6, 8, 4, 4)
    assert g.weight.shape == (16, 256, 512 * 3 // 32) and sh[0].weight.shape == (1, 384, 64)
    assert rq.weight.shape == (1, 16, 64) and sgq.weight.shape == (1, 1, 64)
    mem = spec.device()
    router = fl.MoERouter(spec.n_experts, spec.top_k)
    ck = fl.MoELayer(router_weight=rq, router=router, gate=g, up=u, down=d,
                     hidden=spec.hidden, act_dtype=torch.bfloat16, shared=sh,
                     shared_gate_weight=sgq)
    xn = spec.x(T, seed=T)
    x = to_torch(xn)
    y_ck, tr = ck.forward(x, trace=True)
    y_mem = mem.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y_ck.view(torch.int16), y_mem.view(torch.int16))
    # the oracle routes from the GPU's logits, so a near-tie cannot fork it
    y_ref = orc.moe_layer(spec, xn, given_logits=to_numpy_f32(tr["logits"]))[0]
    check_close(to_numpy_f32(y_ck), load(y_ref, spec.act_dt), spec.act_dt, f"checkpoint T={T}")
