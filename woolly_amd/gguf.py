"""Host-side mirror of woolly-gguf: the GGUF loader (parsed natively by
libwoolly_hip over a memory map) and the dequantization entry point, on the GPU.

  GGUFLoader (from_path, header, metadata, tensors, tensor_info, tensor_names,
    tensor_data, tensor_data_as, architecture, model_name, quantization_version,
    total_tensor_size, file_size, alignment)   crates/woolly-gguf/src/loader.rs:111-490
  GGUFMetadata (get, get_string, get_u32, get_u64, get_i32, get_f32, get_bool)
                                     metadata.rs:140-233
  TensorInfo (name, n_dims, dims, ggml_type, offset, n_elements, data_size)
                                     tensor_info.rs:187-258
  Error::{Io, InvalidMagic, UnsupportedVersion, InvalidMetadata, TensorNotFound,
          InvalidTensorInfo}          error.rs:11-64
  GGMLType ids                       crates/woolly-gguf/src/tensor_info.rs:15-30
  get_block_size / get_type_size     crates/woolly-gguf/src/dequantize.rs:208-242
  TensorInfo::data_size              tensor_info.rs:244-255
  dequantize(data, ggml_type, n)     dequantize.rs:189-205
  Error::{BufferTooSmall{needed, available}, InvalidTensorType}   error.rs:11-64
"""
from __future__ import annotations

import ctypes as C
import enum
import re

import numpy as np

from . import _lib


class GGMLType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30

    def traits(self) -> tuple[int, int, bool]:
        """(block_size, type_size, is_quantized), tensor_info.rs:128-183."""
        bs, ts, q = C.c_size_t(), C.c_size_t(), C.c_int()
        _lib.check(_lib.load().wh_ggml_type_traits(int(self), C.byref(bs), C.byref(ts), C.byref(q)))
        return int(bs.value), int(ts.value), bool(q.value)

    def block_size(self) -> int:
        return self.traits()[0]

    def type_size(self) -> int:
        return self.traits()[1]

    def is_quantized(self) -> bool:
        return self.traits()[2]


class GgufError(Exception):
    pass


class BufferTooSmall(GgufError):
    def __init__(self, needed: int, available: int):
        self.needed, self.available = needed, available
        super().__init__(f"Buffer too small: needed {needed}, available {available}")


class InvalidTensorType(GgufError):
    def __init__(self, type_id: int):
        self.type_id = type_id
        super().__init__(f"Invalid tensor type: {type_id}")


class Io(GgufError):
    pass


class InvalidMagic(GgufError):
    pass


class UnsupportedVersion(GgufError):
    def __init__(self, version: int, message: str = ""):
        self.version = version
        super().__init__(message or f"Unsupported GGUF version: {version}")


class InvalidMetadata(GgufError):
    pass


class TensorNotFound(GgufError):
    pass


class InvalidTensorInfo(GgufError):
    pass


def get_block_size(t: GGMLType) -> int:
    return int(_lib.load().wh_block_size(int(t)))


def get_type_size(t: GGMLType) -> int:
    return int(_lib.load().wh_type_size(int(t)))


def data_size(t: GGMLType, n_elements: int) -> int:
    out = C.c_uint64()
    _lib.check(_lib.load().wh_tensor_nbytes(int(t), n_elements, C.byref(out)))
    return int(out.value)


def dequantize(data, ggml_type: GGMLType, nelements: int) -> np.ndarray:
    """woolly_gguf::dequantize (dequantize.rs:189-205) on the GPU.  Q5_0 / Q5_1
    decode as woolly-tensor's dequantize_q5_0 / _q5_1 (quantization.rs:515-575):
    the reference's gguf-level versions (dequantize.rs:538-550) are stubs that
    return zeros, which this drop-in does not reproduce."""
    buf = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8)
                               if not isinstance(data, np.ndarray) else data.view(np.uint8))
    out = np.empty(nelements, dtype=np.float32)
    st = _lib.load().wh_dequantize_host(int(ggml_type), buf.ctypes.data if buf.size else None,
                                        buf.nbytes, nelements, out.ctypes.data if nelements else None)
    if st == _lib.WH_ERR_BUFFER_TOO_SMALL:
        m = re.search(r"needed (\d+) bytes, available (\d+)", _lib.last_error())
        raise BufferTooSmall(int(m.group(1)), int(m.group(2))) if m else GgufError(_lib.last_error())
    if st == _lib.WH_ERR_UNSUPPORTED_TYPE:
        raise InvalidTensorType(int(ggml_type))
    if st == _lib.WH_ERR_INVALID_METADATA:  # short K-quant data (dequantize.rs:416-418, 472-474)
        raise InvalidTensorInfo(_lib.last_error())
    _lib.check(st)
    return out


# ------------------------------------------------------------------ loader
class MetadataValueType(enum.IntEnum):
    """metadata.rs:13-42"""
    UInt8 = 0
    Int8 = 1
    UInt16 = 2
    Int16 = 3
    UInt32 = 4
    Int32 = 5
    Float32 = 6
    Bool = 7
    String = 8
    Array = 9
    UInt64 = 10
    Int64 = 11
    Float64 = 12


_SCALAR_NP = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
              6: np.float32, 10: np.uint64, 11: np.int64, 12: np.float64}


class MetadataValue:
    """A typed metadata value (metadata.rs:68-82): `type` and the Python value
    (int, float, bool, str, or a list / numpy array for arrays)."""

    __slots__ = ("type", "value")

    def __init__(self, vtype: int, value):
        self.type = MetadataValueType(vtype)
        self.value = value

    def __eq__(self, other):
        if isinstance(other, MetadataValue):
            return self.type == other.type and _eq(self.value, other.value)
        return _eq(self.value, other)

    def __repr__(self):
        return f"MetadataValue.{self.type.name}({self.value!r})"


def _eq(a, b) -> bool:
    if isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
        return np.array_equal(np.asarray(a), np.asarray(b))
    return a == b


class GGUFMetadata:
    """GGUFMetadata (metadata.rs:140-233): kv_pairs maps key -> MetadataValue."""

    def __init__(self, kv_pairs: dict):
        self.kv_pairs = kv_pairs

    def get(self, key: str):
        return self.kv_pairs.get(key)

    def _typed(self, key: str, t: MetadataValueType):
        v = self.kv_pairs.get(key)
        return v.value if v is not None and v.type == t else None

    def get_string(self, key):
        return self._typed(key, MetadataValueType.String)

    def get_u32(self, key):
        return self._typed(key, MetadataValueType.UInt32)

    def get_u64(self, key):
        return self._typed(key, MetadataValueType.UInt64)

    def get_i32(self, key):
        return self._typed(key, MetadataValueType.Int32)

    def get_f32(self, key):
        return self._typed(key, MetadataValueType.Float32)

    def get_bool(self, key):
        return self._typed(key, MetadataValueType.Bool)


class GGUFHeader:
    """GGUFHeader (format.rs:59-72)."""

    def __init__(self, h):
        self.magic = b"GGUF"
        self.version = int(h.version)
        self.tensor_count = int(h.tensor_count)
        self.metadata_kv_count = int(h.metadata_kv_count)


class TensorInfo:
    """TensorInfo (tensor_info.rs:187-258)."""

    def __init__(self, t, index: int):
        self.name = t.name.decode()
        self.n_dims = int(t.n_dims)
        self.dims = [int(t.dims[i]) for i in range(self.n_dims)]
        self.ggml_type = GGMLType(t.ggml_type)
        self.offset = int(t.offset)
        self._n_elements = int(t.n_elements)
        self._data_size = int(t.data_size)
        self.index = index

    def shape(self) -> list[int]:
        return self.dims

    def n_elements(self) -> int:
        return self._n_elements

    def data_size(self) -> int:
        return self._data_size


def _raise(st: int, what: str = "") -> None:
    msg = _lib.last_error()
    if st == _lib.WH_ERR_IO:
        raise Io(msg)
    if st == _lib.WH_ERR_INVALID_MAGIC:
        raise InvalidMagic(msg)
    if st == _lib.WH_ERR_UNSUPPORTED_VERSION:
        m = re.search(r"version (\d+)", msg)
        raise UnsupportedVersion(int(m.group(1)) if m else -1, msg)
    if st == _lib.WH_ERR_INVALID_METADATA:
        raise InvalidMetadata(msg)
    if st == _lib.WH_ERR_NOT_FOUND:
        raise TensorNotFound(what or msg)
    if st == _lib.WH_ERR_UNSUPPORTED_TYPE:
        m = re.search(r"type (\d+)", msg)
        raise InvalidTensorType(int(m.group(1)) if m else -1)
    if st == _lib.WH_ERR_BUFFER_TOO_SMALL:
        m = re.search(r"needed (\d+) bytes, available (\d+)", msg)
        raise BufferTooSmall(int(m.group(1)), int(m.group(2))) if m else GgufError(msg)
    _lib.check(st)


def _chk(st: int, what: str = "") -> None:
    if st != _lib.WH_OK:
        _raise(st, what)


class GGUFLoader:
    """GGUFLoader (loader.rs:111-490) over libwoolly_hip's native parser.  The
    file stays memory-mapped; tensor_data returns zero-copy views of it and
    upload() moves a tensor to the GPU straight from the mapping."""

    def __init__(self, handle: int, keepalive=None):
        self._h = handle
        self._keep = keepalive
        lib = _lib.load()
        hdr = _lib.wh_gguf_header()
        _chk(lib.wh_gguf_get_header(handle, C.byref(hdr)))
        self._hdr = hdr
        self._header = GGUFHeader(hdr)
        self._metadata = None
        self._tensors = None

    @classmethod
    def from_path(cls, path) -> "GGUFLoader":
        h = C.c_void_p()
        _chk(_lib.load().wh_gguf_open(str(path).encode(), C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_bytes(cls, data) -> "GGUFLoader":
        """from_mmap over an in-memory buffer (kept alive by the loader)."""
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        h = C.c_void_p()
        _chk(_lib.load().wh_gguf_open_buffer(buf.ctypes.data if buf.size else None, buf.size,
                                             C.byref(h)))
        return cls(h.value, keepalive=buf)

    def close(self) -> None:
        if self._h:
            _lib.load().wh_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- header / file
    def header(self) -> GGUFHeader:
        return self._header

    def alignment(self) -> int:
        return int(self._hdr.alignment)

    def data_start_offset(self) -> int:
        return int(self._hdr.data_offset)

    def file_size(self) -> int:
        return int(self._hdr.file_size)

    def total_tensor_size(self) -> int:
        return int(self._hdr.total_tensor_size)

    # --- metadata
    def _kv_value(self, i: int, vtype: int):
        lib = _lib.load()
        if vtype == MetadataValueType.String:
            p, n = C.c_void_p(), C.c_size_t()
            _chk(lib.wh_gguf_kv_string(self._h, i, C.byref(p), C.byref(n)))
            return C.string_at(p.value, n.value).decode() if n.value else ""
        if vtype == MetadataValueType.Array:
            et, cnt, p = C.c_int(), C.c_uint64(), C.c_void_p()
            _chk(lib.wh_gguf_kv_array(self._h, i, C.byref(et), C.byref(cnt), C.byref(p)))
            et, cnt = et.value, cnt.value
            if et in _SCALAR_NP:
                dt = np.dtype(_SCALAR_NP[et]).newbyteorder("<")
                raw = C.string_at(p.value, cnt * dt.itemsize) if cnt else b""
                return np.frombuffer(raw, dtype=dt).copy()
            if et == MetadataValueType.Bool:
                raw = C.string_at(p.value, cnt) if cnt else b""
                return [b != 0 for b in raw]
            if et == MetadataValueType.String:
                out = []
                for j in range(cnt):
                    sp, sn = C.c_void_p(), C.c_size_t()
                    _chk(lib.wh_gguf_kv_array_string(self._h, i, j, C.byref(sp), C.byref(sn)))
                    out.append(C.string_at(sp.value, sn.value).decode() if sn.value else "")
                return out
            return None  # nested arrays: type and count only
        vt, raw = C.c_int(), (C.c_uint8 * 8)()
        _chk(lib.wh_gguf_kv_scalar(self._h, i, C.byref(vt), raw))
        if vtype == MetadataValueType.Bool:
            return bool(raw[0])
        dt = np.dtype(_SCALAR_NP[vtype]).newbyteorder("<")
        v = np.frombuffer(bytes(raw)[:dt.itemsize], dtype=dt)[0]
        return float(v) if dt.kind == "f" else int(v)

    def metadata(self) -> GGUFMetadata:
        if self._metadata is None:
            lib = _lib.load()
            kv = {}
            for i in range(int(self._hdr.metadata_kv_count)):
                key, vt = C.c_char_p(), C.c_int()
                _chk(lib.wh_gguf_kv_at(self._h, i, C.byref(key), C.byref(vt)))
                kv[key.value.decode()] = MetadataValue(vt.value, self._kv_value(i, vt.value))
            self._metadata = GGUFMetadata(kv)
        return self._metadata

    def architecture(self):
        return self.metadata().get_string("general.architecture")

    def model_name(self):
        return self.metadata().get_string("general.name")

    def quantization_version(self):
        return self.metadata().get_u32("general.quantization_version")

    # --- tensors
    def tensors(self) -> dict:
        if self._tensors is None:
            lib = _lib.load()
            out = {}
            for i in range(int(self._hdr.tensor_count)):
                t = _lib.wh_gguf_tensor()
                _chk(lib.wh_gguf_tensor_at(self._h, i, C.byref(t)))
                info = TensorInfo(t, i)
                out[info.name] = info
            self._tensors = out
        return self._tensors

    def tensor_info(self, name: str):
        return self.tensors().get(name)

    def has_tensor(self, name: str) -> bool:
        """Whether the file holds a tensor of this name (loader.has_tensor, used by
        load_model_weights for the optional output.weight, loader.rs:384)."""
        return name in self.tensors()

    def tensor_names(self) -> list[str]:
        return list(self.tensors())

    def _index(self, name: str) -> int:
        idx = C.c_uint64()
        _chk(_lib.load().wh_gguf_find_tensor(self._h, name.encode(), C.byref(idx)), name)
        return int(idx.value)

    def tensor_data(self, name: str) -> np.ndarray:
        """Zero-copy uint8 view of the tensor's bytes in the mapping (valid while
        the loader is open)."""
        i = self._index(name)
        p, n = C.c_void_p(), C.c_size_t()
        _chk(_lib.load().wh_gguf_tensor_data(self._h, i, C.byref(p), C.byref(n)), name)
        if n.value == 0:
            return np.zeros(0, dtype=np.uint8)
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value))

    def tensor_data_as(self, name: str, dtype) -> np.ndarray:
        """loader.rs:427-455: typed view of a non-quantized tensor."""
        info = self.tensor_info(name)
        if info is None:
            raise TensorNotFound(name)
        if info.ggml_type.is_quantized():
            raise InvalidTensorInfo(f"Cannot get typed view of quantized tensor '{name}'")
        dt = np.dtype(dtype)
        if dt.itemsize != info.ggml_type.type_size():
            raise InvalidTensorInfo(f"Type size mismatch: expected {dt.itemsize} bytes, tensor has "
                                    f"{info.ggml_type.type_size()} bytes per element")
        return self.tensor_data(name).view(dt)

    def upload(self, name: str):
        """Device weight handle (woolly_amd.ops.Weight) straight from the mapping."""
        from .ops import Weight
        i = self._index(name)
        h = C.c_void_p()
        _chk(_lib.load().wh_gguf_upload(self._h, i, C.byref(h)), name)
        return Weight.from_handle(h.value)
