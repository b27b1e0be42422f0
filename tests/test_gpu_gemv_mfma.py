"""GPU matrix-core GEMV (int8 MFMA on exact limbs of the activations) against
the f64 oracle, at the north-star bar (rel-L2 <= 1e-4, max-abs <= 1e-3), for
the shapes the kernel takes: every segment count (K = 1536 .. 14336), ragged
row counts, the three block formats, the fused variants (RMSNorm + stacked
Q/K/V, residual add, gate/up with SwiGLU), activations over 60 decades, zero
and non-finite chunks, and agreement with the streaming kernels
(quantized_matvec, quantization.rs:869-909, 1100-1163)."""
import numpy as np
import pytest

from tests._gpu import down, gemv, up
from tests._oracle import max_abs, rel_l2
from woolly_amd import ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0 = 2, 3, 8
REL_L2, MAX_ABS = 1e-4, 1e-3


def check(got, ref, tag, abs_bar=MAX_ABS):
    r, a = rel_l2(got, ref), max_abs(got, ref)
    print(f"[result] {tag} rel_l2={r:.3e} max_abs={a:.3e}", flush=True)
    assert r <= REL_L2 and a <= abs_bar, (tag, r, a)


# (m, k): K = 1536 .. 14336 covers 1 (1536, 2048, 3072, 4096), 2 (6144, 8192),
# 3 (12288) and 4 (14336) K-segments; m is ragged against the 16-row steps
SHAPES = [(64, 1536), (100, 2048), (96, 3072), (1000, 4096), (4100, 4096), (200, 6144), (333, 8192),
          (80, 12288), (64, 14336), (257, 14336)]


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("m,k", SHAPES)
def test_mfma_gemv_parity(gpu, orc, t, m, k):
    print(f"[case] mfma gemv type={t} m={m} k={k}", flush=True)
    w = synth.quantized_weight(t, m, k, seed=m * 3 + k)
    x = synth.activations(k, seed=m + 2 * k)
    got = gemv(t, w, x, m, k)
    check(got, orc.matvec_f64(t, w, x, m, k)[1], f"mfma t={t} {m}x{k}")


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
def test_mfma_matches_streaming_kernels(gpu, orc, t):
    m, k = 777, 4096
    w = synth.quantized_weight(t, m, k, seed=9)
    x = synth.activations(k, seed=10)
    got = gemv(t, w, x, m, k)
    prev = ops.gemv_select(ops.GEMV_STREAM)
    try:
        ref_stream = gemv(t, w, x, m, k)
    finally:
        ops.gemv_select(prev)
    ref = orc.matvec_f64(t, w, x, m, k)[1]
    check(got, ref, f"mfma t={t}")
    check(ref_stream, ref, f"stream t={t}")
    # two f32 computations of the same sum in different orders
    assert rel_l2(got, ref_stream) <= 1e-5


@pytest.mark.parametrize("scale", [1e-30, 1e-12, 1e-3, 1e3, 1e12, 1e30])
def test_mfma_activation_scales(gpu, orc, scale):
    """The per-chunk exponent keeps 22 bits of every chunk's largest element at
    any scale: rel-L2 stays at f32 level over 60 decades."""
    m, k = 300, 4096
    w = synth.quantized_weight(Q4_0, m, k, seed=13)
    x = (synth.activations(k, seed=14) * np.float32(scale)).astype(np.float32)
    got = gemv(Q4_0, w, x, m, k)
    ref = orc.matvec_f64(Q4_0, w, x, m, k)[1]
    r = rel_l2(got, ref)
    print(f"[result] scale={scale:g} rel_l2={r:.3e}", flush=True)
    assert r <= REL_L2
    assert max_abs(got, ref) <= MAX_ABS * max(1.0, float(np.sqrt(np.mean(ref ** 2))) / 300.0)


def test_mfma_wide_dynamic_range_within_chunk(gpu, orc):
    """Elements 2^-20 of their chunk's largest lose precision on the limb grid
    (absolute 2^-23 of the chunk maximum); the product stays within the bar."""
    m, k = 256, 4096
    w = synth.quantized_weight(Q8_0, m, k, seed=15)
    x = synth.activations(k, seed=16)
    x[::256] *= 1e6  # one huge element per 256-element chunk
    got = gemv(Q8_0, w, x, m, k)
    ref = orc.matvec_f64(Q8_0, w, x, m, k)[1]
    r = rel_l2(got, ref)
    print(f"[result] wide range rel_l2={r:.3e}", flush=True)
    assert r <= REL_L2


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
def test_mfma_zero_chunks(gpu, orc, t):
    m, k = 128, 8192
    w = synth.quantized_weight(t, m, k, seed=17)
    x = synth.activations(k, seed=18)
    x[:1024] = 0.0          # whole chunks of zeros
    x[3000:3003] = 0.0
    got = gemv(t, w, x, m, k)
    check(got, orc.matvec_f64(t, w, x, m, k)[1], f"zero chunks t={t}")
    zero = gemv(t, w, np.zeros(k, np.float32), m, k)
    assert np.all(zero == 0.0)


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
def test_mfma_nonfinite_chunks(gpu, orc, t):
    """inf / NaN in some chunks: those chunks are summed per element like the
    reference, the others on the matrix cores; the outputs carry +-inf or NaN
    exactly where the order-exact scalar path does."""
    m, k = 100, 4096
    w = synth.quantized_weight(t, m, k, seed=19)
    x = synth.activations(k, seed=20)
    x[300] = np.inf
    got = gemv(t, w, x, m, k)
    ref = orc.matvec_f32(t, w, x, m, k)[1]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(np.isinf(got[fin]), np.isinf(ref[fin]))
    assert np.array_equal(np.sign(got[fin]), np.sign(ref[fin]))
    x[4000] = np.nan
    assert np.all(np.isnan(gemv(t, w, x, m, k)))


def test_mfma_in_graph_and_deterministic(gpu, orc):
    from woolly_amd.device import Graph, Stream

    m, k = 14336, 4096
    w = synth.quantized_weight(Q4_0, m, k, seed=3)
    wb, wp = up(w)
    xb = DeviceBuffer(4 * k)
    yb = DeviceBuffer(4 * m)
    s = Stream()
    with Graph.capture(s) as g:
        ops.quantized_matvec(Q4_0, wp, w.nbytes, xb.ptr, yb.ptr, m, k, s)
    first = None
    for rep in range(3):
        x = synth.activations(k, seed=200 + (rep % 2))
        xb.upload(x)
        g.launch(s)
        s.synchronize()
        got = down(yb, np.float32, m)
        check(got, orc.matvec_f64(Q4_0, w, x, m, k)[1], f"graph {rep}")
        if rep == 0:
            first = got.copy()
        if rep == 2:  # same input as replay 0: bit-identical
            assert np.array_equal(first.view(np.uint32), got.view(np.uint32))
    g.destroy()
    s.destroy()


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("hidden,q_rows,kv_rows", [(2048, 2048, 256), (4096, 4096, 1024), (3072, 3072, 1024)])
def test_mfma_fused_norm_stacked_qkv(gpu, orc, t, hidden, q_rows, kv_rows):
    """RMSNorm prologue + three row-stacked matrices in one launch (the decode
    step's Q/K/V projection), rows of one step straddling the matrices."""
    wq = synth.quantized_weight(t, q_rows, hidden, seed=21)
    wk = synth.quantized_weight(t, kv_rows, hidden, seed=22)
    wv = synth.quantized_weight(t, kv_rows, hidden, seed=23)
    x = synth.activations(hidden, seed=24) * 3
    g = (1 + 0.1 * np.random.default_rng(25).standard_normal(hidden)).astype(np.float32)
    bufs = [up(a)[0] for a in (wq, wk, wv, x, g)]
    out = DeviceBuffer(4 * (q_rows + 2 * kv_rows))
    wsz = ops.attention_qkv_workspace_bytes(hidden)
    ws = DeviceBuffer(wsz)
    ops.attention_qkv(t, *bufs[:3], q_rows, kv_rows, hidden, bufs[4], 1e-5, bufs[3], out, ws, wsz)
    got = down(out, np.float32, q_rows + 2 * kv_rows)
    xn = np.zeros((1, hidden))
    orc.lib.orc_rms_norm_f64(x.ctypes.data, g.ctypes.data, 1e-5, 1, hidden, xn.ctypes.data)
    xn32 = xn.astype(np.float32).ravel()
    ref = np.concatenate([orc.matvec_f64(t, w, xn32, n, hidden)[1]
                          for w, n in ((wq, q_rows), (wk, kv_rows), (wv, kv_rows))])
    check(got, ref, f"qkv t={t} {hidden}")


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_1])
@pytest.mark.parametrize("m,k", [(1000, 2048), (4096, 14336), (130, 4096)])
def test_mfma_residual_in_place(gpu, orc, t, m, k):
    w = synth.quantized_weight(t, m, k, seed=m + k + 1)
    x = synth.activations(k, seed=27)
    r = synth.activations(m, seed=28) * 10
    wb, xb, rb = up(w)[0], up(x)[0], up(r)[0]
    ops.quantized_matvec_residual(t, wb, w.nbytes, xb, rb, rb, m, k)   # y aliases the residual
    got = down(rb, np.float32, m)
    check(got, r.astype(np.float64) + orc.matvec_f64(t, w, x, m, k)[1], f"residual t={t} {m}x{k}")


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("hidden,n_ff", [(1024, 2816), (2048, 5632)])
def test_mfma_ffn_gate_up_m1(gpu, orc, t, hidden, n_ff):
    """The M = 1 FFN: RMSNorm + gate and up rows streamed side by side on the
    matrix cores with the SwiGLU epilogue, then the down projection."""
    L = synth.ffn_layer(t, hidden, n_ff, 1, seed=hidden + t)
    b = {kk: up(v)[0] for kk, v in L.items()}
    out = DeviceBuffer(4 * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, 1)
    ws = DeviceBuffer(wsz)
    ops.ffn_swiglu(t, b["gate"], b["up"], b["down"], hidden, n_ff, b["gamma"], 1e-5, b["x"], 1, out, ws, wsz)
    got = down(out, np.float32, hidden)
    ref = orc.ffn_rows_f64(t, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5, L["x"], [0])[0]
    rms = float(np.sqrt(np.mean(ref ** 2)))
    check(got, ref, f"ffn m=1 t={t} {hidden}/{n_ff}", abs_bar=MAX_ABS * max(1.0, rms / 300.0))


def test_gemv_select_rejects_unknown_mode(gpu):
    from woolly_amd import WoollyHipError
    with pytest.raises(WoollyHipError):
        ops.gemv_select(7)
    assert ops.gemv_select(ops.GEMV_AUTO) == ops.GEMV_AUTO
