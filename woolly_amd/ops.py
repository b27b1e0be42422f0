"""Device-level entry points (DeviceBuffer in, DeviceBuffer out, stream-ordered).

Thin wrappers over the C ABI: each call validates nothing itself; the library
returns the reference's error semantics (see include/woolly_hip.h), raised here
as WoollyHipError.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .device import DeviceBuffer, Stream

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0 = 0, 1, 2, 3, 8


def _s(stream: Stream | None):
    return stream.handle if stream else None


def _p(buf) -> int:
    if buf is None:
        return 0
    return buf.ptr if isinstance(buf, DeviceBuffer) else int(buf)


def type_size(ggml_type: int) -> int:
    return int(_lib.load().wh_type_size(ggml_type))


def block_size(ggml_type: int) -> int:
    return int(_lib.load().wh_block_size(ggml_type))


def tensor_nbytes(ggml_type: int, nelements: int) -> int:
    out = C.c_uint64()
    _lib.check(_lib.load().wh_tensor_nbytes(ggml_type, nelements, C.byref(out)))
    return int(out.value)


def dequantize(ggml_type: int, data, nbytes: int, nelements: int, out,
               stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_dequantize(ggml_type, _p(data), nbytes, nelements, _p(out),
                                         _s(stream)))


def quantized_matvec(ggml_type: int, weights, weight_nbytes: int, x, y, m: int, k: int,
                     stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_quantized_matvec(ggml_type, _p(weights), weight_nbytes, _p(x),
                                               _p(y), m, k, _s(stream)))


def matmul_workspace_bytes(ggml_type: int, n_rows: int, k: int, n_tokens: int) -> int:
    return int(_lib.load().wh_quantized_matmul_workspace_bytes(ggml_type, n_rows, k, n_tokens))


def quantized_matmul(ggml_type: int, weights, weight_nbytes: int, n_rows: int, k: int, x,
                     n_tokens: int, y, workspace=None, workspace_bytes: int = 0,
                     stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_quantized_matmul(ggml_type, _p(weights), weight_nbytes, n_rows, k,
                                               _p(x), n_tokens, _p(y), _p(workspace) or None,
                                               workspace_bytes, _s(stream)))


def rms_norm(x, weight, eps: float, tokens: int, hidden: int, out,
             stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_rms_norm(_p(x), _p(weight), eps, tokens, hidden, _p(out),
                                       _s(stream)))


def swiglu(gate, up, n: int, out, stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_swiglu(_p(gate), _p(up), n, _p(out), _s(stream)))


def ffn_workspace_bytes(hidden: int, n_ff: int, m: int) -> int:
    return int(_lib.load().wh_ffn_workspace_bytes(hidden, n_ff, m))


def ffn_swiglu(ggml_type: int, gate, up, down, hidden: int, n_ff: int, gamma, eps: float, x,
               m: int, out, workspace, workspace_bytes: int,
               stream: Stream | None = None) -> None:
    w = _lib.wh_ffn_weights(ggml_type, _p(gate), _p(up), _p(down), hidden, n_ff)
    _lib.check(_lib.load().wh_ffn_swiglu(C.byref(w), _p(gamma), eps, _p(x), m, _p(out),
                                         _p(workspace), workspace_bytes, _s(stream)))


class Weight:
    """A device-resident quantized tensor (wh_weight_upload / wh_weight_free)."""

    def __init__(self, ggml_type: int, n_rows: int, k: int, host_bytes) -> None:
        import numpy as np

        arr = np.ascontiguousarray(np.frombuffer(host_bytes, dtype=np.uint8)
                                   if not isinstance(host_bytes, np.ndarray) else host_bytes)
        h = C.c_void_p()
        _lib.check(_lib.load().wh_weight_upload(ggml_type, n_rows, k, arr.ctypes.data, arr.nbytes,
                                                C.byref(h)))
        self.handle = h.value
        self.ggml_type, self.n_rows, self.k = ggml_type, n_rows, k

    @classmethod
    def from_handle(cls, handle: int) -> "Weight":
        """Wraps a wh_weight* made by another entry point (wh_gguf_upload)."""
        w = cls.__new__(cls)
        w.handle = handle
        t, n, k = C.c_int(), C.c_size_t(), C.c_size_t()
        _lib.check(_lib.load().wh_weight_info(handle, C.byref(t), C.byref(n), C.byref(k), None))
        w.ggml_type, w.n_rows, w.k = t.value, n.value, k.value
        return w

    @property
    def ptr(self) -> int:
        return int(_lib.load().wh_weight_data(self.handle) or 0)

    @property
    def nbytes(self) -> int:
        nb = C.c_size_t()
        _lib.check(_lib.load().wh_weight_info(self.handle, None, None, None, C.byref(nb)))
        return int(nb.value)

    def free(self) -> None:
        if self.handle:
            _lib.check(_lib.load().wh_weight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                _lib.load().wh_weight_free(self.handle)
                self.handle = None
        except Exception:
            pass
