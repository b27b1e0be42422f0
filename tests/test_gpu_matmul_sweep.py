"""wh_quantized_matmul and wh_ffn_swiglu over seeded random shapes against the
f64 oracle.

The call dispatches on the token count and the shape: one token streams the
weights once (matrix-core GEMV), 2..16 tokens the several-token GEMV, more
the tiled MFMA GEMM with 16-, 32-, 64- or 128-token tiles (split-K where the
tiles are few, stream-K where they would leave CUs idle), a K that is not a
multiple of 64 the fallback GEMM, and the K-quant formats a conversion to
32-element blocks first.  The fixed cases of the other tests sit on chosen
shapes; these draw n, k and the token count at random (a fixed seed, so the
list is the same on every run) around each of those thresholds, rows that
are not a multiple of 16 or 256 included, and check sampled tokens
(Gemm::compute on the dequantized weights, ops/matmul.rs:83-259).  The FFN
cases compose those paths with the RMSNorm and SwiGLU packings
(lazy_transformer.rs:1073-1123)."""
import numpy as np
import pytest

from tests._gpu import down, report, up
from tests._oracle import max_abs, rel_l2
from woolly_amd import ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14
REL_L2 = 1e-4
TOKENS = [1, 2, 3, 5, 8, 13, 16, 17, 24, 31, 32, 33, 48, 63, 64, 65, 96, 127, 128, 129, 200, 257, 300]


def max_abs_bar(ref) -> float:
    """max-abs <= 1e-3 against the f64 reference, relative to the output RMS
    above an RMS of 300."""
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    return 1e-3 * max(1.0, rms / 300.0)


def cases(count: int = 100, seed: int = 20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        t = [Q4_0, Q4_1, Q8_0, Q4_K, Q6_K][i % 5]
        m = int(TOKENS[rng.integers(len(TOKENS))])
        if t in (Q4_K, Q6_K):
            k = 256 * int(rng.integers(1, 17))            # 256 .. 4096
        else:
            k = 32 * int(rng.integers(1, 129))            # 32 .. 4096, odd block counts included
        n = int(rng.integers(1, 2049))
        out.append((t, n, k, m))
    return out


@pytest.mark.parametrize("t,n,k,m", cases())
def test_matmul_random_shape(gpu, orc, t, n, k, m):
    print(f"[case] matmul sweep type={t} m={m} n={n} k={k}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n * 7 + k + t)
    x = synth.activations(m * k, seed=m * 3 + k).reshape(m, k)
    wb, wp = up(w)
    xb, xp = up(x)
    yb = DeviceBuffer(4 * m * n)
    wsz = ops.matmul_workspace_bytes(t, n, k, m)
    ws = DeviceBuffer(max(wsz, 1))
    ops.quantized_matmul(t, wp, w.nbytes, n, k, xp, m, yb.ptr, ws, wsz)
    got = down(yb, np.float32, m * n).reshape(m, n)
    rows = np.array(sorted({0, m // 2, m - 1}), dtype=np.int64)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, rows)
    g = got[rows]
    r, a = rel_l2(g, ref), max_abs(g, ref)
    report(f"matmul sweep t={t} m={m} n={n} k={k}", r, a, ref)
    assert np.all(np.isfinite(got))
    assert r <= REL_L2 and a <= max_abs_bar(ref)


def ffn_cases(count: int = 25, seed: int = 20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        t = [Q4_0, Q4_1, Q8_0, Q4_K, Q6_K][i % 5]
        m = int(TOKENS[rng.integers(len(TOKENS))])
        unit = 256 if t in (Q4_K, Q6_K) else 32
        hidden = unit * int(rng.integers(1, 4096 // unit + 1))
        n_ff = unit * int(rng.integers(1, 6144 // unit + 1))
        out.append((t, hidden, n_ff, m))
    return out


@pytest.mark.parametrize("t,hidden,n_ff,m", ffn_cases())
def test_ffn_random_shape(gpu, orc, t, hidden, n_ff, m):
    print(f"[case] ffn sweep type={t} hidden={hidden} n_ff={n_ff} m={m}", flush=True)
    L = synth.ffn_layer(t, hidden, n_ff, m, seed=hidden + n_ff + m + t)
    bufs = {key: up(v) for key, v in L.items()}
    ob = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m, t)
    ws = DeviceBuffer(max(wsz, 1))
    ops.ffn_swiglu(t, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], m, ob.ptr, ws.ptr, wsz)
    got = down(ob, np.float32, m * hidden).reshape(m, hidden)
    rows = sorted({0, m // 2, m - 1})
    ref = orc.ffn_rows_f64(t, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5, L["x"], rows)
    g = got[rows]
    r, a = rel_l2(g, ref), max_abs(g, ref)
    report(f"ffn sweep t={t} m={m} hidden={hidden} n_ff={n_ff}", r, a, ref)
    assert np.all(np.isfinite(got))
    assert r <= REL_L2 and a <= max_abs_bar(ref)
