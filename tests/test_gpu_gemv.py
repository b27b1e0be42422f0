"""GPU quantized GEMV against the f64 oracle (rel-L2 <= 1e-4 and
max-abs <= 1e-3), at the reference's shapes, the benchmark shapes and the edge
cases of quantized_matvec (quantization.rs:869-909, 1100-1163)."""
import numpy as np
import pytest

from tests._gpu import down, gemv, up
from tests._oracle import max_abs, rel_l2
from tests.test_oracle import block_q4_0
from woolly_amd import ops, quantization, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0 = 2, 3, 8
REL_L2, MAX_ABS = 1e-4, 1e-3  # BASELINE.json north_star tolerance vs the f64 reference


def check(got, ref, tag):
    r, a = rel_l2(got, ref), max_abs(got, ref)
    print(f"[result] {tag} rel_l2={r:.3e} max_abs={a:.3e}", flush=True)
    assert r <= REL_L2 and a <= MAX_ABS, (tag, r, a)


SHAPES = [(1, 32), (3, 64), (64, 256), (17, 4096), (4096, 4096), (130, 14336), (33, 8192),
          (5, 96), (9, 1056), (7, 20480), (1000, 2048)]


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("m,k", SHAPES)
def test_gemv_parity(gpu, orc, t, m, k):
    print(f"[case] gemv type={t} m={m} k={k}", flush=True)
    w = synth.quantized_weight(t, m, k, seed=m * 7 + k)
    x = synth.activations(k, seed=m + k)
    got = gemv(t, w, x, m, k)
    st, ref = orc.matvec_f64(t, w, x, m, k)
    assert st == 0
    check(got, ref, f"t={t} {m}x{k}")
    st, ref32 = orc.matvec_f32(t, w, x, m, k)
    print(f"[info] vs order-exact f32 scalar: max_abs={max_abs(got, ref32):.3e}", flush=True)


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("w_off", [1, 2])
def test_gemv_unaligned_weights(gpu, orc, t, w_off):
    m, k = 37, 4096
    w = synth.quantized_weight(t, m, k, seed=11)
    x = synth.activations(k, seed=12)
    got = gemv(t, w, x, m, k, w_offset=w_off)
    check(got, orc.matvec_f64(t, w, x, m, k)[1], f"unaligned+{w_off}")


@pytest.mark.parametrize("t,m,k", [(Q4_0, 14336, 4096), (Q4_0, 4096, 4096), (Q8_0, 14336, 4096),
                                   (Q4_1, 14336, 4096), (Q4_0, 4096, 14336),
                                   (Q4_0, 1024, 4096),      # k/v projections (8 KV heads x 128)
                                   (Q8_0, 128256, 4096)])   # Q8_0 output head (vocab 128256)
def test_gemv_benchmark_shapes(gpu, orc, t, m, k):
    print(f"[case] gemv full type={t} {m}x{k}", flush=True)
    w = synth.quantized_weight(t, m, k, seed=3)
    x = synth.activations(k, seed=3)
    got = gemv(t, w, x, m, k)
    check(got, orc.matvec_f64(t, w, x, m, k)[1], f"full t={t} {m}x{k}")


def test_gemv_closed_form(gpu):
    # constant nibbles c per block and x = 1: y[r] = sum_b d_b (c_b - 8) * 32
    rng = np.random.default_rng(5)
    m, nb = 9, 64
    c = rng.integers(0, 16, (m, nb))
    d = np.float16(np.abs(rng.standard_normal((m, nb))) * 0.05)
    w = np.concatenate([block_q4_0(float(d[r, b]), [int(c[r, b]) * 17] * 16)
                        for r in range(m) for b in range(nb)])
    got = gemv(Q4_0, w, np.ones(nb * 32, np.float32), m, nb * 32)
    ref = (d.astype(np.float64) * (c - 8) * 32).sum(axis=1)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-5)


def test_gemv_through_reference_api(gpu, orc):
    # simd::quantized_matvec(&QuantizedStorage, input, output, m, k)
    m, k = 48, 512
    for t, make in ((Q4_0, quantization.QuantizedStorage.Q4_0),
                    (Q8_0, quantization.QuantizedStorage.Q8_0),
                    (Q4_1, quantization.QuantizedStorage.Q4_1)):
        w = synth.quantized_weight(t, m, k, seed=t)
        x = synth.activations(k, seed=t)
        out = np.zeros(m, np.float32)
        quantization.simd.quantized_matvec(make(w), x, out, m, k)
        check(out, orc.matvec_f64(t, w, x, m, k)[1], f"ref-api t={t}")


def test_gemv_edge_cases(gpu):
    w = synth.quantized_weight(Q4_0, 4, 64, seed=1)
    # k == 0: every row is an empty sum
    yb = DeviceBuffer(16)
    yb.upload(np.full(4, 7.0, np.float32))
    ops.quantized_matvec(Q4_0, 0, 0, 0, yb.ptr, 4, 0)
    assert np.all(down(yb, np.float32, 4) == 0.0)
    # m == 0: no-op
    ops.quantized_matvec(Q4_0, 0, 0, 0, 0, 0, 64)
    # k % 32 != 0 and unknown type raise like the reference
    from woolly_amd import WoollyHipError
    with pytest.raises(WoollyHipError):
        gemv(Q4_0, w, np.zeros(64, np.float32), 4, 48)
    with pytest.raises(WoollyHipError):
        gemv(12, w, np.zeros(64, np.float32), 4, 64)


def test_gemv_deterministic(gpu):
    m, k = 4096, 14336
    w = synth.quantized_weight(Q4_0, m, k, seed=21)
    x = synth.activations(k, seed=21)
    wb, wp = up(w)
    xb, xp = up(x)
    outs = []
    for _ in range(3):
        yb = DeviceBuffer(4 * m)
        ops.quantized_matvec(Q4_0, wp, w.nbytes, xp, yb.ptr, m, k)
        outs.append(down(yb, np.float32, m))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("k", [256, 14336])
def test_gemv_nonfinite_propagates(gpu, orc, t, k):
    # inf / NaN activations propagate like the reference's per-element
    # (w * d) * x sum: +-inf, or NaN where a weight is exactly zero.
    m = 64
    w = synth.quantized_weight(t, m, k, seed=2)
    x = synth.activations(k, seed=2)
    x[5] = np.inf
    x[k - 3] = -np.inf if k > 256 else x[k - 3]
    got = gemv(t, w, x, m, k)
    ref = orc.matvec_f32(t, w, x, m, k)[1]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin], ref[fin])  # +-inf with matching signs
    x[7] = np.nan
    got = gemv(t, w, x, m, k)
    assert np.all(np.isnan(got))


def test_gemv_graph_replay(gpu, orc):
    """A captured GEMV replays correctly several times, with eager work between."""
    from woolly_amd.device import Graph, Stream

    m, k = 4096, 4096
    w = synth.quantized_weight(Q4_0, m, k, seed=31)
    wb, wp = up(w)
    xb = DeviceBuffer(4 * k)
    yb = DeviceBuffer(4 * m)
    s = Stream()
    with Graph.capture(s) as g:
        ops.quantized_matvec(Q4_0, wp, w.nbytes, xb.ptr, yb.ptr, m, k, s)
    for rep in range(3):
        x = synth.activations(k, seed=100 + rep)
        xb.upload(x)
        g.launch(s)
        s.synchronize()
        got = down(yb, np.float32, m)
        eager = gemv(Q4_0, w, x, m, k)
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))
        check(got, orc.matvec_f64(Q4_0, w, x, m, k)[1], f"graph replay {rep}")
    g.destroy()
    s.destroy()
