"""Small helpers for the GPU parity tests (device round trips through the C ABI)."""
from __future__ import annotations

import numpy as np

from woolly_amd import ops
from woolly_amd.device import DeviceBuffer, synchronize


def up(arr: np.ndarray, pad: int = 0, offset: int = 0) -> tuple[DeviceBuffer, int]:
    """Uploads arr at byte `offset` inside a buffer; returns (buffer, device address)."""
    arr = np.ascontiguousarray(arr)
    buf = DeviceBuffer(max(arr.nbytes + offset + pad, 1))
    if arr.nbytes:
        buf.upload(arr, offset=offset)
    return buf, buf.ptr + offset


def down(buf: DeviceBuffer, dtype, count: int, offset: int = 0) -> np.ndarray:
    synchronize()
    return buf.download(dtype, count, offset)


def gemv(t, w, x, m, k, w_offset=0):
    wb, wp = up(w, offset=w_offset)
    xb, xp = up(x)
    yb = DeviceBuffer(max(4 * m, 4))
    ops.quantized_matvec(t, wp, w.nbytes, xp, yb.ptr, m, k)
    return down(yb, np.float32, m)
