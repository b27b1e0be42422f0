"""Small helpers for the GPU parity tests (device round trips through the C ABI)."""
from __future__ import annotations

import json
import os

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


def report(tag: str, rel: float, mx: float, ref=None, **extra) -> None:
    """Prints the achieved errors of a parity check and, when the environment
    variable WH_PARITY_LOG names a file, appends them to it as one JSON line
    (tag, rel_l2, max_abs, the reference's RMS and max-abs / RMS)."""
    rec = {"tag": tag, "rel_l2": float(rel), "max_abs": float(mx)}
    if ref is not None:
        rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
        rec["ref_rms"] = rms
        rec["max_abs_over_rms"] = float(mx) / rms if rms > 0 else None
    rec.update(extra)
    print("[result] " + " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}" for k, v in rec.items()),
          flush=True)
    path = os.environ.get("WH_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
