"""wh_read_probe (the benchmark's read floor): every byte of every row is read,
in the GEMV's workgroup geometry (modes 0 and 1: workgroup b's checksum is the
xor of all 32-bit words of its rows) or as one flat byte range split into one
contiguous piece per workgroup (mode 2: the xor of the words of its piece)."""
import re

import numpy as np
import pytest

from tests._gpu import down, up
from woolly_amd import _lib, device
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("n_rows,row_bytes", [(300, 2304), (14336, 2304), (1000, 4096), (17, 1024), (4096, 576)])
def test_read_probe_checksums(gpu, mode, n_rows, row_bytes):
    print(f"[case] read_probe mode={mode} {n_rows}x{row_bytes}", flush=True)
    rng = np.random.default_rng(n_rows + row_bytes)
    m = rng.integers(0, 2**32, (n_rows, row_bytes // 4), dtype=np.uint64).astype(np.uint32)
    mb = up(m)[0]
    groups = (n_rows + 15) // 16
    cus = int(re.search(r"(\d+) CUs", device.device_name()).group(1))
    grid0 = min(groups, cus)
    rows_per_wg = -(-groups // grid0) * 16
    grid = -(-n_rows // rows_per_wg)
    out = DeviceBuffer(4 * (n_rows // 16 + 1))
    lib = _lib.load()
    _lib.check(lib.wh_read_probe(mb.ptr, row_bytes, n_rows, mode, out.ptr, None))
    got = down(out, np.uint32, grid)
    want = np.array([np.bitwise_xor.reduce(m[b * rows_per_wg:(b + 1) * rows_per_wg].reshape(-1))
                     for b in range(grid)], np.uint32)
    assert np.array_equal(got, want)


def test_read_probe_rejects_bad_arguments(gpu):
    lib = _lib.load()
    buf = DeviceBuffer(4096)
    assert lib.wh_read_probe(buf.ptr, 4097, 1, 0, buf.ptr, None) == _lib.WH_ERR_INVALID_ARGUMENT
    assert lib.wh_read_probe(buf.ptr, 64, 1, 3, buf.ptr, None) == _lib.WH_ERR_INVALID_ARGUMENT
    assert lib.wh_read_probe(buf.ptr, 64, 1, -1, buf.ptr, None) == _lib.WH_ERR_INVALID_ARGUMENT
    assert lib.wh_read_probe(None, 64, 1, 0, buf.ptr, None) == _lib.WH_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("n_rows,row_bytes", [(14336, 2304), (300, 2304), (17, 1024), (4096, 4096)])
def test_read_probe_flat_checksums(gpu, n_rows, row_bytes):
    print(f"[case] read_probe mode=2 {n_rows}x{row_bytes}", flush=True)
    rng = np.random.default_rng(n_rows * 3 + row_bytes)
    m = rng.integers(0, 2**32, n_rows * row_bytes // 4, dtype=np.uint64).astype(np.uint32)
    mb = up(m)[0]
    total = n_rows * row_bytes
    cus = int(re.search(r"(\d+) CUs", device.device_name()).group(1))
    per_wg_max = 16 * 64 * 16 * 16
    grid = cus if cus * per_wg_max >= total else -(-total // per_wg_max)
    grid = min(grid, (n_rows + 15) // 16)
    per_wg = -(-total // grid)
    per_wg = -(-per_wg // 16) * 16
    out = DeviceBuffer(4 * (n_rows // 16 + 1))
    lib = _lib.load()
    _lib.check(lib.wh_read_probe(mb.ptr, row_bytes, n_rows, 2, out.ptr, None))
    got = down(out, np.uint32, grid)
    w = per_wg // 4
    want = np.array([np.bitwise_xor.reduce(m[b * w:(b + 1) * w]) if b * w < m.size else 0 for b in range(grid)],
                    np.uint32)
    assert np.array_equal(got, want)
