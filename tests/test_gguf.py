"""The native GGUF loader (wh_gguf_*, woolly_amd.gguf.GGUFLoader) against the
reference's own loader tests, restated: crates/woolly-gguf/tests/load_model.rs
(MockGGUFBuilder :15-145 and the tests :147-446), tensor_info.rs:264-304,
format.rs:129-146 and loader.rs:671-690.  Parsing is host code, so these run
without a GPU; the upload test is marked gpu."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from woolly_amd import gguf, synth
from woolly_amd.gguf import GGMLType, GGUFLoader, MetadataValue, MetadataValueType as VT

_FMT = {VT.UInt8: "<B", VT.Int8: "<b", VT.UInt16: "<H", VT.Int16: "<h", VT.UInt32: "<I",
        VT.Int32: "<i", VT.Float32: "<f", VT.UInt64: "<Q", VT.Int64: "<q", VT.Float64: "<d"}


def enc_str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def enc_value(t: VT, v) -> bytes:
    if t in _FMT:
        return struct.pack(_FMT[t], v)
    if t == VT.Bool:
        return bytes([1 if v else 0])
    if t == VT.String:
        return enc_str(v)
    et, items = v
    return struct.pack("<IQ", et, len(items)) + b"".join(enc_value(et, x) for x in items)


class MockGGUFBuilder:
    """The byte layout of load_model.rs:15-145: header (version 3), metadata,
    tensor infos with offsets packed back to back, zero padding to 32 bytes,
    tensor data."""

    def __init__(self, version: int = 3):
        self.version = version
        self.metadata: list[tuple[bytes, int, bytes]] = []
        self.tensors: list[tuple[str, list[int], int, bytes]] = []

    def add_metadata(self, key, t: VT, v, raw: bytes | None = None):
        self.metadata.append((key.encode() if isinstance(key, str) else key, int(t),
                              raw if raw is not None else enc_value(t, v)))
        return self

    def add_tensor(self, name: str, shape: list[int], t: GGMLType, data: bytes):
        self.tensors.append((name, shape, int(t), data))
        return self

    def build(self, pad_to: int = 32) -> bytes:
        out = bytearray(b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(self.metadata)))
        for key, t, raw in self.metadata:
            out += enc_str(key) + struct.pack("<I", t) + raw
        off = 0
        for name, shape, t, _ in self.tensors:
            out += enc_str(name) + struct.pack("<I", len(shape))
            out += b"".join(struct.pack("<Q", d) for d in shape)
            out += struct.pack("<IQ", t, off)
            n = int(np.prod(shape)) if shape else 1
            if t in GGMLType.__members__.values():  # (invalid ids: tests of the error)
                bs, ts, q = GGMLType(t).traits()
                off += ((n + bs - 1) // bs) * ts if q else n * ts
        out += b"\0" * ((-len(out)) % pad_to)
        for *_, data in self.tensors:
            out += data
        return bytes(out)


def load(data: bytes, tmp_path=None) -> GGUFLoader:
    if tmp_path is None:
        return GGUFLoader.from_bytes(data)
    p = tmp_path / "model.gguf"
    p.write_bytes(data)
    return GGUFLoader.from_path(p)


# ------------------------------------------------------------ load_model.rs
def test_load_empty_gguf(tmp_path):
    ld = load(MockGGUFBuilder().build(), tmp_path)
    h = ld.header()
    assert h.magic == b"GGUF" and h.version == 3
    assert h.tensor_count == 0 and h.metadata_kv_count == 0
    assert len(ld.tensors()) == 0 and len(ld.metadata().kv_pairs) == 0


def test_load_with_metadata(tmp_path):
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "test_arch")
            .add_metadata("general.name", VT.String, "Test Model")
            .add_metadata("general.quantization_version", VT.UInt32, 2)
            .add_metadata("general.alignment", VT.UInt32, 32)
            .add_metadata("test.bool_value", VT.Bool, True)
            .add_metadata("test.float_value", VT.Float32, 3.14)
            .add_metadata("test.array_value", VT.Array, (VT.UInt32, [1, 2, 3]))
            .build())
    ld = load(data, tmp_path)
    assert ld.header().metadata_kv_count == 7
    assert ld.architecture() == "test_arch"
    assert ld.model_name() == "Test Model"
    assert ld.quantization_version() == 2
    assert ld.alignment() == 32
    md = ld.metadata()
    assert md.kv_pairs["test.bool_value"] == MetadataValue(VT.Bool, True)
    v = md.kv_pairs["test.float_value"]
    assert v.type == VT.Float32 and abs(v.value - 3.14) < 0.001
    arr = md.get("test.array_value")
    assert arr.type == VT.Array and list(arr.value) == [1, 2, 3]


def test_load_with_tensors(tmp_path):
    t1 = bytes(range(16))
    t2 = bytes(range(32))
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "test")
            .add_tensor("weight1", [4, 4], GGMLType.F32, t1)
            .add_tensor("weight2", [4, 4, 2], GGMLType.F32, t2)
            .build())
    ld = load(data, tmp_path)
    assert ld.header().tensor_count == 2 and len(ld.tensors()) == 2
    names = ld.tensor_names()
    assert "weight1" in names and "weight2" in names
    i1 = ld.tensor_info("weight1")
    assert i1.name == "weight1" and i1.shape() == [4, 4] and i1.ggml_type == GGMLType.F32
    assert i1.n_elements() == 16 and i1.data_size() == 64
    i2 = ld.tensor_info("weight2")
    assert i2.shape() == [4, 4, 2] and i2.n_elements() == 32


def test_memory_mapped_tensor_access(tmp_path):
    tensor = np.arange(16, dtype="<f4").tobytes()
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "test")
            .add_tensor("test_tensor", [4, 4], GGMLType.F32, tensor)
            .build())
    ld = load(data, tmp_path)
    raw = ld.tensor_data("test_tensor")
    assert raw.nbytes == 64
    f = ld.tensor_data_as("test_tensor", np.float32)
    assert f.size == 16 and np.array_equal(f, np.arange(16, dtype=np.float32))


def test_quantized_tensor_handling(tmp_path):
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "test")
            .add_tensor("quantized_weight", [64], GGMLType.Q4_0, bytes(36))
            .build())
    ld = load(data, tmp_path)
    info = ld.tensor_info("quantized_weight")
    assert info.ggml_type == GGMLType.Q4_0 and info.ggml_type.is_quantized()
    assert info.data_size() == 36
    assert ld.tensor_data("quantized_weight").nbytes == 36
    with pytest.raises(gguf.InvalidTensorInfo):
        ld.tensor_data_as("quantized_weight", np.float32)


def test_error_handling(tmp_path):
    with pytest.raises(gguf.Io):
        GGUFLoader.from_path("/non/existent/file.gguf")
    with pytest.raises(gguf.InvalidMagic):
        load(b"BAD!" + bytes(20), tmp_path)
    with pytest.raises(gguf.UnsupportedVersion) as e:
        load(b"GGUF" + struct.pack("<I", 999) + bytes(16), tmp_path)
    assert e.value.version == 999


def test_tensor_not_found(tmp_path):
    ld = load(MockGGUFBuilder().add_metadata("general.architecture", VT.String, "test").build(), tmp_path)
    assert ld.tensor_info("non_existent") is None
    with pytest.raises(gguf.TensorNotFound):
        ld.tensor_data("non_existent")


def test_file_size_and_stats(tmp_path):
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "test")
            .add_tensor("large_tensor", [256], GGMLType.F32, bytes(1024))
            .build())
    ld = load(data, tmp_path)
    assert ld.file_size() == len(data)
    assert ld.total_tensor_size() == 1024


def test_all_metadata_types(tmp_path):
    b = MockGGUFBuilder()
    for key, t, v in [("test.u8", VT.UInt8, 255), ("test.i8", VT.Int8, -128),
                      ("test.u16", VT.UInt16, 65535), ("test.i16", VT.Int16, -32768),
                      ("test.u32", VT.UInt32, 4294967295), ("test.i32", VT.Int32, -2147483648),
                      ("test.f32", VT.Float32, 3.14159), ("test.bool_true", VT.Bool, True),
                      ("test.bool_false", VT.Bool, False), ("test.string", VT.String, "Hello, GGUF!"),
                      ("test.u64", VT.UInt64, 18446744073709551615),
                      ("test.i64", VT.Int64, -9223372036854775808), ("test.f64", VT.Float64, 2.718281828)]:
        b.add_metadata(key, t, v)
    md = load(b.build(), tmp_path).metadata()
    assert md.get("test.u8") == MetadataValue(VT.UInt8, 255)
    assert md.get("test.i8") == MetadataValue(VT.Int8, -128)
    assert md.get("test.u16") == MetadataValue(VT.UInt16, 65535)
    assert md.get("test.i16") == MetadataValue(VT.Int16, -32768)
    assert md.get_u32("test.u32") == 4294967295
    assert md.get_i32("test.i32") == -2147483648
    assert md.get_bool("test.bool_true") is True and md.get_bool("test.bool_false") is False
    assert md.get_string("test.string") == "Hello, GGUF!"
    assert md.get_u64("test.u64") == 18446744073709551615
    assert md.get("test.i64") == MetadataValue(VT.Int64, -9223372036854775808)
    assert abs(md.get_f32("test.f32") - 3.14159) < 1e-5
    v = md.get("test.f64")
    assert v.type == VT.Float64 and abs(v.value - 2.718281828) < 1e-9
    # typed getters return None for other types (metadata.rs:186-233)
    assert md.get_u32("test.i32") is None and md.get_f32("test.f64") is None


# ----------------------------------------------- tensor_info.rs / format.rs / loader.rs
def test_ggml_type_sizes():
    assert GGMLType.F32.type_size() == 4 and GGMLType.F16.type_size() == 2
    assert GGMLType.I8.type_size() == 1
    assert GGMLType.Q4_0.block_size() == 32 and GGMLType.Q4_0.type_size() == 18
    assert GGMLType.Q2_K.block_size() == 256 and GGMLType.Q2_K.type_size() == 82
    with pytest.raises(Exception):
        GGMLType(4)


def test_tensor_info_size_calculation(tmp_path):
    data = (MockGGUFBuilder()
            .add_tensor("test", [4, 8], GGMLType.F32, bytes(128))
            .add_tensor("test_q", [64, 64], GGMLType.Q4_0, bytes(2304))
            .build())
    ld = load(data, tmp_path)
    assert ld.tensor_info("test").n_elements() == 32 and ld.tensor_info("test").data_size() == 128
    q = ld.tensor_info("test_q")
    assert q.n_elements() == 4096 and q.data_size() == 2304


def test_magic_and_version():
    with pytest.raises(gguf.InvalidMagic):
        GGUFLoader.from_bytes(b"GGML" + struct.pack("<IQQ", 3, 0, 0))
    for v in (1, 2, 3):
        assert GGUFLoader.from_bytes(b"GGUF" + struct.pack("<IQQ", v, 0, 0)).header().version == v
    for v in (0, 4):
        with pytest.raises(gguf.UnsupportedVersion):
            GGUFLoader.from_bytes(b"GGUF" + struct.pack("<IQQ", v, 0, 0))


@pytest.mark.parametrize("alignment", [None, 32, 64, 4096])
def test_data_section_alignment(alignment):
    # loader.rs:148-164, 662-667: data starts at the end of the tensor table
    # rounded up to general.alignment (u32, default 32); tensor offsets are
    # relative to it.
    a = alignment or 32
    vals = np.arange(8, dtype="<f4").tobytes()
    b = MockGGUFBuilder()
    if alignment:
        b.add_metadata("general.alignment", VT.UInt32, alignment)
    b.add_tensor("a", [8], GGMLType.F32, vals)
    table_end = len(b.build(pad_to=1)) - len(vals)
    ld = GGUFLoader.from_bytes(b.build(pad_to=a))
    assert ld.alignment() == a
    assert ld.data_start_offset() == table_end + (-table_end) % a
    assert np.array_equal(ld.tensor_data_as("a", np.float32), np.arange(8, dtype=np.float32))


def test_alignment_ignored_unless_u32():
    b = MockGGUFBuilder().add_metadata("general.alignment", VT.UInt64, 64)
    assert GGUFLoader.from_bytes(b.build()).alignment() == 32


# ------------------------------------------------------------- robustness
def test_tensor_past_end_of_file():
    b = MockGGUFBuilder().add_tensor("w", [64], GGMLType.F32, bytes(256))
    data = b.build()[:-10]
    ld = GGUFLoader.from_bytes(data)
    with pytest.raises(gguf.BufferTooSmall) as e:
        ld.tensor_data("w")
    assert e.value.available == len(data) and e.value.needed == len(data) + 10


def test_every_truncation_fails_cleanly():
    b = (MockGGUFBuilder()
         .add_metadata("general.architecture", VT.String, "llama")
         .add_metadata("tokenizer.ggml.tokens", VT.Array, (VT.String, ["a", "bc", "def"]))
         .add_metadata("nested", VT.Array, (VT.Array, [(VT.UInt8, [1, 2]), (VT.Int16, [3])]))
         .add_tensor("w", [32], GGMLType.Q8_0, bytes(34)))
    data = b.build(pad_to=1)
    table_end = len(data) - 34
    ld = GGUFLoader.from_bytes(data)
    assert ld.metadata().get("tokenizer.ggml.tokens").value == ["a", "bc", "def"]
    assert ld.metadata().get("nested").value is None  # nested arrays: type only
    # every prefix that ends inside the header, metadata or tensor table is an
    # I/O error (unexpected end of file), as the reference's Cursor reads are
    for n in range(table_end):
        with pytest.raises(gguf.Io):
            GGUFLoader.from_bytes(data[:n])
    # past the table the file opens; the data is checked when it is read
    short = GGUFLoader.from_bytes(data[:table_end + 10])
    with pytest.raises(gguf.BufferTooSmall):
        short.tensor_data("w")


def test_invalid_utf8_and_types():
    with pytest.raises(gguf.InvalidMetadata):
        GGUFLoader.from_bytes(MockGGUFBuilder().add_metadata(b"bad\xff", VT.UInt8, 1).build())
    with pytest.raises(gguf.InvalidMetadata):
        GGUFLoader.from_bytes(MockGGUFBuilder().add_metadata("s", VT.String, b"\xc0\x80").build())
    with pytest.raises(gguf.InvalidMetadata):  # value type 13 does not exist
        GGUFLoader.from_bytes(MockGGUFBuilder().add_metadata("k", 13, None, raw=b"").build())
    with pytest.raises(gguf.InvalidTensorType):  # ggml type 4 does not exist
        GGUFLoader.from_bytes(MockGGUFBuilder().add_tensor("t", [32], 4, b"").build())


def test_duplicate_keys_last_wins():
    b = (MockGGUFBuilder().add_metadata("k", VT.UInt32, 1).add_metadata("k", VT.UInt32, 2)
         .add_tensor("t", [1], GGMLType.F32, struct.pack("<f", 1.0))
         .add_tensor("t", [1], GGMLType.F32, struct.pack("<f", 2.0)))
    ld = GGUFLoader.from_bytes(b.build())
    assert ld.metadata().get_u32("k") == 2
    assert ld.tensor_data_as("t", np.float32)[0] == 2.0


def test_random_bytes_never_crash():
    rng = np.random.default_rng(0)
    seen = set()
    base = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "llama")
            .add_metadata("arr", VT.Array, (VT.UInt32, list(range(20))))
            .add_tensor("w", [64, 2], GGMLType.Q4_0, bytes(72))
            .build())
    for trial in range(2000):
        d = bytearray(base)
        for _ in range(rng.integers(1, 6)):
            d[rng.integers(0, len(d))] = rng.integers(0, 256)
        try:
            ld = GGUFLoader.from_bytes(bytes(d))
            ld.metadata()
            for name in ld.tensor_names():
                try:
                    ld.tensor_data(name)
                except gguf.GgufError:
                    pass
            seen.add("ok")
        except gguf.GgufError as e:
            seen.add(type(e).__name__)
    assert "ok" in seen and len(seen) > 2


@pytest.mark.gpu
def test_upload_from_mapping_matches_host_weight(tmp_path):
    """wh_gguf_upload: the device copy of a Q4_0 tensor equals its file bytes and
    computes the same GEMV as an upload of the same bytes from host memory."""
    from woolly_amd import ops, synth
    from woolly_amd.device import DeviceBuffer

    n, k = 96, 512
    w = synth.quantized_weight(GGMLType.Q4_0, n, k, seed=11)
    norm = np.linspace(0.5, 1.5, k, dtype=np.float32)
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "llama")
            .add_tensor("blk.0.ffn_gate.weight", [k, n], GGMLType.Q4_0, w.tobytes())
            .add_tensor("blk.0.ffn_norm.weight", [k], GGMLType.F32, norm.tobytes())
            .build())
    ld = load(data, tmp_path)
    dw = ld.upload("blk.0.ffn_gate.weight")
    assert (dw.ggml_type, dw.n_rows, dw.k, dw.nbytes) == (2, n, k, w.nbytes)
    back = np.empty(w.nbytes, np.uint8)
    from woolly_amd import _lib
    _lib.check(_lib.load().wh_memcpy_d2h(back.ctypes.data, dw.ptr, w.nbytes, None))
    _lib.check(_lib.load().wh_device_synchronize())
    assert np.array_equal(back, np.frombuffer(w.tobytes(), np.uint8))
    dn = ld.upload("blk.0.ffn_norm.weight")
    nb = np.empty(k, np.float32)
    _lib.check(_lib.load().wh_memcpy_d2h(nb.ctypes.data, dn.ptr, 4 * k, None))
    _lib.check(_lib.load().wh_device_synchronize())
    assert np.array_equal(nb, norm)
    x = synth.activations(k, seed=12)
    xb, y1, y2 = DeviceBuffer.from_array(x), DeviceBuffer(4 * n), DeviceBuffer(4 * n)
    ref = ops.Weight(2, n, k, w)
    ops.quantized_matvec(2, dw.ptr, w.nbytes, xb, y1, n, k)
    ops.quantized_matvec(2, ref.ptr, w.nbytes, xb, y2, n, k)
    assert np.array_equal(y1.download(np.float32, n), y2.download(np.float32, n))


@pytest.mark.gpu
@pytest.mark.parametrize("t", [GGMLType.Q4_K, GGMLType.Q6_K])
def test_upload_kquant_tensor(tmp_path, t):
    """Q4_K / Q6_K tensors (a Q4_K_M file's types) upload from the mapping with
    their 256-element block sizes and compute the same GEMV as host uploads."""
    from woolly_amd import _lib, ops, synth
    from woolly_amd.device import DeviceBuffer

    n, k = 80, 1024
    w = synth.quantized_weight(int(t), n, k, seed=13)
    data = (MockGGUFBuilder()
            .add_metadata("general.architecture", VT.String, "llama")
            .add_tensor("blk.0.ffn_down.weight", [k, n], t, w.tobytes())
            .build())
    ld = load(data, tmp_path)
    dw = ld.upload("blk.0.ffn_down.weight")
    assert (dw.ggml_type, dw.n_rows, dw.k, dw.nbytes) == (int(t), n, k, w.nbytes)
    back = np.empty(w.nbytes, np.uint8)
    _lib.check(_lib.load().wh_memcpy_d2h(back.ctypes.data, dw.ptr, w.nbytes, None))
    _lib.check(_lib.load().wh_device_synchronize())
    assert np.array_equal(back, np.frombuffer(w.tobytes(), np.uint8))
    x = synth.activations(k, seed=14)
    xb, y1, y2 = DeviceBuffer.from_array(x), DeviceBuffer(4 * n), DeviceBuffer(4 * n)
    ref = ops.Weight(int(t), n, k, w)
    ops.quantized_matvec(int(t), dw.ptr, w.nbytes, xb, y1, n, k)
    ops.quantized_matvec(int(t), ref.ptr, w.nbytes, xb, y2, n, k)
    assert np.array_equal(y1.download(np.float32, n), y2.download(np.float32, n))


def test_llama_config_from_gguf_metadata():
    """LlamaModel.config_from_gguf reads GGUFModelLoader::extract_config's keys
    with their fallback keys and defaults (model/loader.rs:104-150); no GPU needed."""
    from woolly_amd import ops

    def cfg(extra, arch="llama", top=()):
        b = MockGGUFBuilder()
        if arch is not None:
            b.add_metadata("general.architecture", VT.String, arch)
        for key, vt, v in extra:
            b.add_metadata(f"{arch}.{key}", vt, v)
        for key, vt, v in top:
            b.add_metadata(key, vt, v)
        return ops.LlamaModel.config_from_gguf(load(b.build()))

    full = cfg([("embedding_length", VT.UInt32, 4096), ("block_count", VT.UInt32, 32),
                ("attention.head_count", VT.UInt32, 32), ("attention.head_count_kv", VT.UInt32, 8),
                ("feed_forward_length", VT.UInt32, 14336), ("context_length", VT.UInt32, 8192),
                ("vocab_size", VT.UInt32, 128256),
                ("rope.freq_base", VT.Float32, 500000.0), ("attention.layer_norm_epsilon", VT.Float32, 1e-6)])
    assert full == dict(hidden=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, n_ff=14336,
                        max_ctx=8192, vocab=128256, rope_base=500000.0, eps=float(np.float32(1e-6)))
    # defaults: n_kv = n_heads, n_ff = 4 hidden, context 2048, vocab 32000, base 10000,
    # eps 1e-5; the alternative epsilon key; another architecture name
    small = cfg([("embedding_length", VT.UInt32, 256), ("block_count", VT.UInt32, 2),
                 ("attention.head_count", VT.UInt32, 4), ("layer_norm_epsilon", VT.Float32, 2e-5)], arch="mistral")
    assert small == dict(hidden=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, n_ff=1024, max_ctx=2048,
                         vocab=32000, rope_base=10000.0, eps=float(np.float32(2e-5)))
    assert cfg([("embedding_length", VT.UInt32, 256), ("block_count", VT.UInt32, 2),
                ("attention.head_count", VT.UInt32, 4)])["eps"] == 1e-5
    # the fallback keys: embed_dim, layer_count, tokenizer.ggml.context_length,
    # attention.rope_theta, tokenizer.ggml.tokens.len
    alt = cfg([("embed_dim", VT.UInt32, 512), ("layer_count", VT.UInt32, 3), ("attention.head_count", VT.UInt32, 8),
               ("attention.rope_theta", VT.Float32, 1e6)],
              top=[("tokenizer.ggml.context_length", VT.UInt32, 4096), ("tokenizer.ggml.tokens.len", VT.UInt32, 777)])
    assert alt == dict(hidden=512, n_layers=3, n_heads=8, n_kv_heads=8, head_dim=64, n_ff=2048, max_ctx=4096,
                       vocab=777, rope_base=1e6, eps=1e-5)
    # the primary keys win over the fallbacks
    both = cfg([("embedding_length", VT.UInt32, 256), ("embed_dim", VT.UInt32, 512), ("block_count", VT.UInt32, 2),
                ("layer_count", VT.UInt32, 5), ("attention.head_count", VT.UInt32, 4),
                ("rope.freq_base", VT.Float32, 5e5), ("attention.rope_theta", VT.Float32, 1e6)])
    assert (both["hidden"], both["n_layers"], both["rope_base"]) == (256, 2, 5e5)
    # nothing but the architecture: the reference's defaults (hidden 4096, 32 layers, 32 heads)
    bare = cfg([])
    assert (bare["hidden"], bare["n_layers"], bare["n_heads"], bare["n_ff"]) == (4096, 32, 32, 16384)
    # no architecture: an error, as "No architecture specified in GGUF"
    with pytest.raises(ValueError, match="architecture"):
        cfg([], arch=None)


def _llama_gguf(hidden=256, n_heads=4, n_kv=2, n_ff=512, vocab=64, kv_meta=True, ff_meta=None, output=True,
                embd=True, embd_type=8):
    """A one-layer Q8_0 llama GGUF file's builder (no GPU needed to build it);
    token_embd.weight in Q8_0, or F16 with embd_type = 1."""
    from woolly_amd.gguf import GGMLType

    d = hidden // n_heads
    b = MockGGUFBuilder().add_metadata("general.architecture", VT.String, "llama")
    meta = [("embedding_length", hidden), ("block_count", 1), ("attention.head_count", n_heads),
            ("feed_forward_length", ff_meta or n_ff)]
    if kv_meta:
        meta.append(("attention.head_count_kv", n_kv))
    for key, v in meta:
        b.add_metadata("llama." + key, VT.UInt32, v)
    q8 = lambda n, k, s: synth.quantized_weight(8, n, k, seed=s).tobytes()
    norm = np.ones(hidden, np.float32).tobytes()
    b.add_tensor("blk.0.attn_norm.weight", [hidden], GGMLType.F32, norm)
    b.add_tensor("blk.0.ffn_norm.weight", [hidden], GGMLType.F32, norm)
    for nm, (n, k) in {"attn_q": (n_heads * d, hidden), "attn_k": (n_kv * d, hidden), "attn_v": (n_kv * d, hidden),
                       "attn_output": (hidden, n_heads * d), "ffn_gate": (n_ff, hidden), "ffn_up": (n_ff, hidden),
                       "ffn_down": (hidden, n_ff)}.items():
        b.add_tensor(f"blk.0.{nm}.weight", [k, n], GGMLType.Q8_0, q8(n, k, len(nm)))
    b.add_tensor("output_norm.weight", [hidden], GGMLType.F32, norm)
    if embd and embd_type == 1:
        table = synth.activations(vocab * hidden, seed=99).astype(np.float16).tobytes()
        b.add_tensor("token_embd.weight", [hidden, vocab], GGMLType.F16, table)
    elif embd:
        b.add_tensor("token_embd.weight", [hidden, vocab], GGMLType.Q8_0, q8(vocab, hidden, 99))
    if output:
        b.add_tensor("output.weight", [hidden, vocab], GGMLType.Q8_0, q8(vocab, hidden, 98))
    return b


def test_llama_from_gguf_rejects_tied_head_of_other_types(tmp_path):
    """Without output.weight the head is token_embd.weight (lazy_transformer.rs:1301-1316);
    an F16 table loads as an embedding but the head GEMV takes only the quantized
    block types, so from_gguf refuses it before uploading anything (no GPU is
    touched)."""
    from woolly_amd import ops

    ld = load(_llama_gguf(output=False, embd_type=1).build(), tmp_path)
    with pytest.raises(ValueError, match="output head"):
        ops.LlamaModel.from_gguf(ld, max_ctx=8)


def test_llama_from_gguf_rejects_mismatched_dims():
    """from_gguf compares every tensor's dims with the config before it uploads
    anything: a GQA file without attention.head_count_kv (n_kv then defaults to
    the head count) and a wrong feed_forward_length raise ValueError instead of
    letting the kernels read past the weights; a file with neither output.weight
    nor token_embd.weight has no head.  No GPU is touched."""
    from woolly_amd import ops

    with pytest.raises(ValueError, match="attn_k"):
        ops.LlamaModel.from_gguf(load(_llama_gguf(kv_meta=False).build()))
    with pytest.raises(ValueError, match="ffn_gate"):
        ops.LlamaModel.from_gguf(load(_llama_gguf(ff_meta=1024).build()))
    with pytest.raises(ValueError, match="neither"):
        ops.LlamaModel.from_gguf(load(_llama_gguf(output=False, embd=False).build()))
