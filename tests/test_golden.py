"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py):
the oracle must reproduce them exactly (CPU) and the GPU must match them (gpu)."""
from pathlib import Path

import numpy as np
import pytest

from tests._oracle import max_abs, rel_l2

GOLD = Path(__file__).resolve().parent / "golden"
GEMV = sorted(GOLD.glob("gemv_*.npz"))
FFN = GOLD / "ffn_q4_0_256x512_m4.npz"


def load(p):
    return dict(np.load(p, allow_pickle=False))


@pytest.mark.parametrize("path", GEMV, ids=lambda p: p.stem)
def test_oracle_reproduces_gemv_fixture(orc, path):
    f = load(path)
    t, n, k = int(f["type"]), int(f["n"]), int(f["k"])
    st, deq = orc.dequantize(t, f["w"], n * k)
    assert st == 0 and np.array_equal(deq.view(np.uint32), f["dequant"].view(np.uint32))
    assert np.array_equal(orc.matvec_f64(t, f["w"], f["x"], n, k)[1], f["y_f64"])
    y32 = orc.matvec_f32(t, f["w"], f["x"], n, k)[1]
    assert np.array_equal(y32.view(np.uint32), f["y_f32_scalar_order"].view(np.uint32))


def test_oracle_reproduces_ffn_fixture(orc):
    f = load(FFN)
    out = orc.ffn_rows_f64(int(f["type"]), f["gate"], f["up"], f["down"], int(f["hidden"]),
                           int(f["n_ff"]), f["gamma"], float(f["eps"]), f["x"], np.arange(int(f["m"])))
    assert np.array_equal(out, f["out_f64"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", GEMV, ids=lambda p: p.stem)
def test_gpu_matches_gemv_fixture(gpu, path):
    from tests._gpu import down, gemv, up
    from woolly_amd import ops
    from woolly_amd.device import DeviceBuffer

    f = load(path)
    t, n, k = int(f["type"]), int(f["n"]), int(f["k"])
    wb, wp = up(f["w"])
    db = DeviceBuffer(4 * n * k)
    ops.dequantize(t, wp, f["w"].nbytes, n * k, db.ptr)
    assert np.array_equal(down(db, np.float32, n * k).view(np.uint32), f["dequant"].view(np.uint32))
    y = gemv(t, f["w"], f["x"], n, k)
    assert rel_l2(y, f["y_f64"]) <= 1e-4 and max_abs(y, f["y_f64"]) <= 1e-3


@pytest.mark.gpu
def test_gpu_matches_ffn_fixture(gpu):
    from tests.test_gpu_ffn import run_ffn

    f = load(FFN)
    L = {kk: f[kk] for kk in ("gate", "up", "down", "gamma", "x")}
    got = run_ffn(int(f["type"]), L, int(f["hidden"]), int(f["n_ff"]), int(f["m"]))
    assert rel_l2(got, f["out_f64"]) <= 1e-4 and max_abs(got, f["out_f64"]) <= 1e-3
