"""Host-side mirror of woolly-tensor's quantization API, executed on the GPU.

Names, argument meaning and errors follow
crates/woolly-tensor/src/quantization.rs so that tests read like the
reference's own:

  BlockQ4_0 / BlockQ4_1 / BlockQ5_0 / BlockQ5_1 / BlockQ8_0   quantization.rs:98-151
  QuantizationError.{UnsupportedScheme, InvalidParameters}   :8-26
  QuantizedStorage.{Q4_0, Q4_1, Q5_0, Q5_1, Q8_0}           :154-170
  dequantize_q4_0 / _q4_1 / _q5_0 / _q5_1 / _q8_0  :466, 490, 515, 545, 576
  simd.quantized_matvec(weights, input, output, m, k)       :869-909
  optimized.dequantize_blocks(storage)          :1171-1210

Every function runs the HIP kernels through libwoolly_hip's synchronous host
entry points; there is no CPU implementation here.
"""
from __future__ import annotations

import enum

import numpy as np

from . import _lib

BlockQ4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
BlockQ4_1 = np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", (16,))])
BlockQ5_0 = np.dtype([("d", "<u2"), ("qh", "u1", (4,)), ("qs", "u1", (16,))])
BlockQ5_1 = np.dtype([("d", "<u2"), ("m", "<u2"), ("qh", "u1", (4,)), ("qs", "u1", (16,))])
BlockQ8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
assert BlockQ4_0.itemsize == 18 and BlockQ4_1.itemsize == 20 and BlockQ8_0.itemsize == 34
assert BlockQ5_0.itemsize == 22 and BlockQ5_1.itemsize == 24

QK = 32


class QuantizationScheme(enum.Enum):
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 8
    Q5_0 = 6
    Q5_1 = 7


_DTYPE = {QuantizationScheme.Q4_0: BlockQ4_0, QuantizationScheme.Q4_1: BlockQ4_1,
          QuantizationScheme.Q5_0: BlockQ5_0, QuantizationScheme.Q5_1: BlockQ5_1,
          QuantizationScheme.Q8_0: BlockQ8_0}
# the schemes simd::quantized_matvec takes (Q4_0 and Q8_0 in the reference,
# quantization.rs:869-909, plus Q4_1 here); Q5 storage is dequantization only
_MATVEC = (QuantizationScheme.Q4_0, QuantizationScheme.Q4_1, QuantizationScheme.Q8_0)


class QuantizationError(Exception):
    """QuantizationError (quantization.rs:8-26)."""

    class UnsupportedScheme(Exception):
        pass

    class InvalidParameters(Exception):
        pass


def _raise(status: int) -> None:
    if status == _lib.WH_OK:
        return
    msg = _lib.last_error()
    if status == _lib.WH_ERR_UNSUPPORTED_TYPE:
        raise QuantizationError.UnsupportedScheme(msg)
    if status in (_lib.WH_ERR_INVALID_SHAPE, _lib.WH_ERR_BUFFER_TOO_SMALL,
                  _lib.WH_ERR_INVALID_ARGUMENT):
        raise QuantizationError.InvalidParameters(msg)
    raise _lib.WoollyHipError(status, msg)


class QuantizedStorage:
    """QuantizedStorage::{Q4_0, Q4_1, Q5_0, Q5_1, Q8_0}(Vec<Block>) (quantization.rs:154-170)."""

    def __init__(self, scheme: QuantizationScheme, blocks: np.ndarray):
        self.scheme = scheme
        dt = _DTYPE.get(scheme)
        if dt is not None:
            blocks = np.ascontiguousarray(blocks).view(dt).reshape(-1)
        self.blocks = blocks

    @classmethod
    def Q4_0(cls, blocks):
        return cls(QuantizationScheme.Q4_0, blocks)

    @classmethod
    def Q4_1(cls, blocks):
        return cls(QuantizationScheme.Q4_1, blocks)

    @classmethod
    def Q5_0(cls, blocks):
        return cls(QuantizationScheme.Q5_0, blocks)

    @classmethod
    def Q5_1(cls, blocks):
        return cls(QuantizationScheme.Q5_1, blocks)

    @classmethod
    def Q8_0(cls, blocks):
        return cls(QuantizationScheme.Q8_0, blocks)


def _dequantize(scheme: QuantizationScheme, blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    n = blocks.shape[0] * QK if blocks.ndim else 0
    out = np.empty(n, dtype=np.float32)
    if n == 0:
        return out
    _raise(_lib.load().wh_dequantize_host(scheme.value, blocks.ctypes.data, blocks.nbytes, n,
                                          out.ctypes.data))
    return out


def dequantize_q4_0(blocks: np.ndarray) -> np.ndarray:
    """dequantize_q4_0(&[BlockQ4_0]) -> Vec<f32> (quantization.rs:466-486)."""
    return _dequantize(QuantizationScheme.Q4_0, np.asarray(blocks, dtype=BlockQ4_0))


def dequantize_q4_1(blocks: np.ndarray) -> np.ndarray:
    """dequantize_q4_1(&[BlockQ4_1]) -> Vec<f32> (quantization.rs:490-511)."""
    return _dequantize(QuantizationScheme.Q4_1, np.asarray(blocks, dtype=BlockQ4_1))


def dequantize_q5_0(blocks: np.ndarray) -> np.ndarray:
    """dequantize_q5_0(&[BlockQ5_0]) -> Vec<f32> (quantization.rs:515-541)."""
    return _dequantize(QuantizationScheme.Q5_0, np.asarray(blocks, dtype=BlockQ5_0))


def dequantize_q5_1(blocks: np.ndarray) -> np.ndarray:
    """dequantize_q5_1(&[BlockQ5_1]) -> Vec<f32> (quantization.rs:545-573)."""
    return _dequantize(QuantizationScheme.Q5_1, np.asarray(blocks, dtype=BlockQ5_1))


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    """dequantize_q8_0(&[BlockQ8_0]) -> Vec<f32> (quantization.rs:576-590)."""
    return _dequantize(QuantizationScheme.Q8_0, np.asarray(blocks, dtype=BlockQ8_0))


class simd:  # noqa: N801 -- mirrors the reference's `quantization::simd` module
    @staticmethod
    def quantized_matvec(weights: QuantizedStorage, input: np.ndarray, output: np.ndarray,
                         m: int, k: int) -> None:
        """simd::quantized_matvec (quantization.rs:869-909), plus Q4_1.

        output[r] = sum_k W[r, k] * input[k] for r < m.  Errors: UnsupportedScheme
        for other storage, InvalidParameters for k % 32 != 0 (the reference's
        assert_eq! panic) or too few blocks."""
        if weights.scheme not in _MATVEC:
            raise QuantizationError.UnsupportedScheme(
                "Quantized matvec not implemented for this scheme")
        x = np.ascontiguousarray(input, dtype=np.float32)
        if output.dtype != np.float32 or not output.flags.c_contiguous:
            raise QuantizationError.InvalidParameters("output must be contiguous f32")
        if len(x) < k or len(output) < m:
            raise QuantizationError.InvalidParameters("input/output shorter than k/m")
        blocks = weights.blocks
        _raise(_lib.load().wh_quantized_matvec_host(weights.scheme.value, blocks.ctypes.data,
                                                    blocks.nbytes, x.ctypes.data,
                                                    output.ctypes.data, m, k))

    dequantize_q4_0_simd = staticmethod(dequantize_q4_0)
    dequantize_q4_1_simd = staticmethod(dequantize_q4_1)
    dequantize_q8_0_simd = staticmethod(dequantize_q8_0)
    dequantize_q4_0_batch = staticmethod(dequantize_q4_0)
    dequantize_q4_1_batch = staticmethod(dequantize_q4_1)
    dequantize_q5_0_batch = staticmethod(dequantize_q5_0)
    dequantize_q5_1_batch = staticmethod(dequantize_q5_1)
    dequantize_q8_0_batch = staticmethod(dequantize_q8_0)


class optimized:  # noqa: N801 -- mirrors `quantization::optimized`
    @staticmethod
    def dequantize_blocks(storage: QuantizedStorage) -> np.ndarray:
        """optimized::dequantize_blocks (quantization.rs:1171-1210)."""
        if storage.scheme not in _DTYPE:
            raise QuantizationError.UnsupportedScheme("Unsupported storage type")
        return _dequantize(storage.scheme, storage.blocks)


class device_cache:  # noqa: N801 -- the device copies behind the host-memory entry points
    """Device copies of host weights behind simd.quantized_matvec and the
    dequantize functions (wh_host_cache_*): the device-side counterpart of
    DequantizationCache::get_or_dequantize
    (crates/woolly-core/src/model/dequantization_cache.rs:121-165).  Off by
    default; with a budget, a weight array is uploaded once per host address
    and size and reused until evicted.  Cached arrays must not change."""

    @staticmethod
    def configure(max_bytes: int) -> None:
        """Sets the byte budget; 0 turns the cache off and frees everything."""
        _lib.check(_lib.load().wh_host_cache_configure(int(max_bytes)))

    @staticmethod
    def evict(array: np.ndarray) -> int:
        """Drops every entry overlapping the array's bytes; returns how many."""
        n = _lib.C.c_size_t(0)
        _lib.check(_lib.load().wh_host_cache_evict(array.ctypes.data, array.nbytes, _lib.C.byref(n)))
        return int(n.value)

    @staticmethod
    def clear() -> None:
        _lib.check(_lib.load().wh_host_cache_clear())

    @staticmethod
    def stats() -> dict:
        st = _lib.wh_host_cache_stats()
        _lib.check(_lib.load().wh_host_cache_get_stats(_lib.C.byref(st)))
        return {name: int(getattr(st, name)) for name, _ in st._fields_}
