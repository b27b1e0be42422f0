"""Several-token (2..16) matrix-core GEMV: wh_quantized_matmul and
wh_ffn_swiglu with a few tokens stream the weights once for all of them
(gemv_mt_kernel, Q4_0, Q4_1, Q8_0, Q4_K and Q6_K), against the f64 oracle on
the same seeded inputs.

The reference runs these token counts through its naive GEMM on dequantized
weights (crates/woolly-tensor/src/ops/matmul.rs:113-115, 608-646) and the FFN
of compute_simd_swiglu_ffn (crates/woolly-core/src/model/lazy_transformer.rs:1073-1123).
Token counts that are not a multiple of four leave empty rows in the last
group of four; K = 4096 and K = 14336 cover one and four K-segments (Q8_0 at
K = 4096: two), so both the in-register and the several-segment A operands
run (Q6_K's 210-byte blocks at K = 14336: segments that start inside a
16-byte piece); counts beyond a shape's limit take the tiled GEMM and are
checked the same way.  The FFN-layer gate/up shape 14336 x 4096 is checked at
full size for the formats added after Q4_0 and Q8_0.  Non-finite activations in some tokens propagate as in the
reference and leave the other tokens exact."""
import numpy as np
import pytest

from tests._gpu import down, report, up
from tests._oracle import max_abs, rel_l2
from woolly_amd import ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14
TYPES = [Q4_0, Q4_1, Q8_0, Q4_K, Q6_K]
REL_L2 = 1e-4


def max_abs_bar(ref) -> float:
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    return 1e-3 * max(1.0, rms / 300.0)


def matmul(t, w, n, k, x, m):
    wb, wp = up(w)
    xb, xp = up(x)
    yb = DeviceBuffer(4 * m * n)
    wsz = ops.matmul_workspace_bytes(t, n, k, m)
    ws = DeviceBuffer(max(wsz, 1))
    ops.quantized_matmul(t, wp, w.nbytes, n, k, xp, m, yb.ptr, ws, wsz)
    return down(yb, np.float32, m * n).reshape(m, n)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,k", [(300, 4096), (200, 14336)])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 7, 8, 9, 12, 13, 16])
def test_mt_matmul_parity(gpu, orc, t, n, k, m):
    print(f"[case] mt matmul type={t} m={m} n={n} k={k}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n + k + t)
    x = synth.activations(m * k, seed=100 + m).reshape(m, k)
    got = matmul(t, w, n, k, x, m)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"mt matmul t={t} m={m} n={n} k={k}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)


@pytest.mark.parametrize("t", TYPES)
def test_mt_matmul_nonfinite_tokens(gpu, orc, t):
    """inf / NaN in tokens 1, 4 and 5: those rows are non-finite exactly where
    the f64 reference is (same signs of inf); tokens 0, 2 and 3 stay within the
    bars, unaffected by their neighbours in the same group of four."""
    m, n, k = 6, 256, 4096
    w = synth.quantized_weight(t, n, k, seed=7)
    x = synth.activations(m * k, seed=8).reshape(m, k)
    x[1, 100] = np.inf
    x[4, 3000] = np.nan
    x[5, 5] = -np.inf
    x[5, 2000] = np.inf
    got = matmul(t, w, n, k, x, m)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    for tok in (1, 4, 5):
        assert np.array_equal(np.isnan(got[tok]), np.isnan(ref[tok])), tok
        assert np.array_equal(np.isposinf(got[tok]), np.isposinf(ref[tok])), tok
        assert np.array_equal(np.isneginf(got[tok]), np.isneginf(ref[tok])), tok
        fin = np.isfinite(ref[tok])
        if fin.any():
            assert max_abs(got[tok][fin], ref[tok][fin]) <= max_abs_bar(ref[tok][fin])
    ok = [0, 2, 3]
    r, a = rel_l2(got[ok], ref[ok]), max_abs(got[ok], ref[ok])
    report(f"mt matmul nonfinite t={t}", r, a, ref[ok])
    assert r <= REL_L2 and a <= max_abs_bar(ref[ok])


@pytest.mark.parametrize("t", [Q4_K, Q4_1, Q6_K])
@pytest.mark.parametrize("m", [2, 8, 16])
def test_mt_matmul_full_size(gpu, orc, t, m):
    """The FFN gate/up shape (N = 14336, K = 4096) at full size, every output row."""
    n, k = 14336, 4096
    print(f"[case] mt matmul full size type={t} m={m}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=200 + t)
    x = synth.activations(m * k, seed=300 + m).reshape(m, k)
    got = matmul(t, w, n, k, x, m)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"mt matmul full t={t} m={m} {n}x{k}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("hidden,n_ff", [(4096, 1024), (1024, 2048)])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8, 16])
def test_mt_ffn_parity(gpu, orc, t, hidden, n_ff, m):
    print(f"[case] mt ffn type={t} hidden={hidden} n_ff={n_ff} m={m}", flush=True)
    L = synth.ffn_layer(t, hidden, n_ff, m, seed=hidden + n_ff + m)
    bufs = {key: up(v) for key, v in L.items()}
    ob = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m, ggml_type=t)
    ws = DeviceBuffer(wsz)
    ops.ffn_swiglu(t, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], m, ob.ptr, ws.ptr, wsz)
    got = down(ob, np.float32, m * hidden).reshape(m, hidden)
    ref = orc.ffn_rows_f64(t, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5,
                           L["x"], np.arange(m))
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"mt ffn t={t} {hidden}/{n_ff} m={m}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)


@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_mt_ffn_nonfinite_token(gpu, orc, bad):
    """One token's x holds an inf or a NaN: its RMSNorm scale is inf / NaN, so
    the reference's x_hat is NaN there and every output of that token is NaN;
    the fused kernels divide each token's rows by its own rms at the finish, so
    the other tokens of the same group stay within the bars."""
    t, hidden, n_ff, m = Q4_0, 4096, 1024, 4
    print(f"[case] mt ffn nonfinite {bad}", flush=True)
    L = synth.ffn_layer(t, hidden, n_ff, m, seed=77)
    L["x"] = L["x"].copy()
    L["x"].reshape(m, hidden)[1, 1234] = bad
    bufs = {key: up(v) for key, v in L.items()}
    ob = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m)
    ws = DeviceBuffer(wsz)
    ops.ffn_swiglu(t, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], m, ob.ptr, ws.ptr, wsz)
    got = down(ob, np.float32, m * hidden).reshape(m, hidden)
    ref = orc.ffn_rows_f64(t, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5,
                           L["x"], np.arange(m))
    assert np.all(np.isnan(ref[1])) and np.all(np.isnan(got[1]))
    ok = [0, 2, 3]
    r, a = rel_l2(got[ok], ref[ok]), max_abs(got[ok], ref[ok])
    report(f"mt ffn nonfinite {bad}", r, a, ref[ok])
    assert r <= REL_L2 and a <= max_abs_bar(ref[ok])
