"""Host-side mirror of woolly-gguf's dequantization entry point, on the GPU.

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


def get_block_size(t: GGMLType) -> int:
    return int(_lib.load().wh_block_size(int(t)))


def get_type_size(t: GGMLType) -> int:
    return int(_lib.load().wh_type_size(int(t)))


def data_size(t: GGMLType, n_elements: int) -> int:
    out = C.c_uint64()
    _lib.check(_lib.load().wh_tensor_nbytes(int(t), n_elements, C.byref(out)))
    return int(out.value)


def dequantize(data, ggml_type: GGMLType, nelements: int) -> np.ndarray:
    """woolly_gguf::dequantize (dequantize.rs:189-205) on the GPU."""
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
    _lib.check(st)
    return out
