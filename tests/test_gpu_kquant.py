"""Q4_K / Q6_K on the GPU (woolly_gguf::dequantize, dequantize.rs:380-536):
dequantization bit for bit against the oracle and the closed forms the oracle
is pinned on, ragged element counts, unaligned outputs, every byte random (f16
fields included), the short-data error; the GEMV (dequantize-then-dot, no
reference kernel) against the f64 oracle at the north-star bar."""
import numpy as np
import pytest

from tests._gpu import down, gemv, up
from tests._oracle import max_abs, rel_l2
from tests.test_oracle_kquant import np_q4_k, np_q6_k, q4k_block, q6k_block
from woolly_amd import gguf, ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
TS = {Q4_K: 144, Q6_K: 210}


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same(a, b):
    with np.errstate(invalid="ignore"):
        return np.all((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b)))


def gpu_dequant(t, data, n, out_offset=0):
    db, dp = up(data)
    ob = DeviceBuffer(4 * n + out_offset + 16)
    ops.dequantize(t, dp, data.nbytes, n, ob.ptr + out_offset)
    return down(ob, np.float32, n, out_offset)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("n", [1, 255, 256, 257, 4096 + 100, 1 << 20])
def test_kquant_dequant_bit_exact(gpu, orc, t, n):
    print(f"[case] kquant dequant type={t} n={n}", flush=True)
    nb = (n + 255) // 256
    data = synth.quantized_weight(t, nb, 256, seed=n + 7 * t)
    got = gpu_dequant(t, data, n)
    st, ref = orc.dequantize(t, data, n)
    assert st == 0 and same(got, ref)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_dequant_random_bytes_unaligned_out(gpu, orc, t):
    """Every byte random (d / dmin may be NaN, inf or subnormal); output at a
    4-byte (not 16-byte) aligned address."""
    rng = np.random.default_rng(11 + t)
    n = 300 * 256 - 5
    data = rng.integers(0, 256, 300 * TS[t], dtype=np.uint8)
    got = gpu_dequant(t, data, n, out_offset=4)
    st, ref = orc.dequantize(t, data, n)
    assert st == 0 and same(got, ref)
    assert same(got, (np_q4_k if t == Q4_K else np_q6_k)(data)[:n])


def test_kquant_closed_forms_on_gpu(gpu):
    # Q4_K 6-bit scale packing: scales 5, 14, 10, 23, 17, 61, 63, 50 per 32 elements
    sb = np.array([0x05, 0x87, 0x03, 0x0A, 0xC0, 0x05, 0x11, 0x40, 0x0F, 0x3F, 0x80, 0x0C], np.uint8)
    v = gpu_dequant(Q4_K, q4k_block(sb, 1.0, 0.0, np.full(128, 0x11, np.uint8)), 256)
    assert v.reshape(8, 32)[:, 0].tolist() == [5.0, 14.0, 10.0, 23.0, 17.0, 61.0, 63.0, 50.0]
    # even elements take the low nibble, dmin added last
    v = gpu_dequant(Q4_K, q4k_block(np.full(12, 0xFF, np.uint8), 0.5, 0.25, np.full(128, 0x21, np.uint8)), 256)
    assert np.all(v[0::2] == np.float32(31.75)) and np.all(v[1::2] == np.float32(63.25))
    # Q6_K: qh = 0xFF gives q = 48 everywhere except the last element (q = 0)
    v = gpu_dequant(Q6_K, q6k_block(np.zeros(128, np.uint8), np.full(64, 0xFF, np.uint8),
                                    np.ones(16, np.uint8), 0.5), 256)
    assert np.all(v[:255] == np.float32(0.125)) and v[255] == np.float32(-0.25)
    # unsigned scales
    v = gpu_dequant(Q6_K, q6k_block(np.zeros(128, np.uint8), np.zeros(64, np.uint8),
                                    np.full(16, 0xC8, np.uint8), 0.5), 256)
    assert np.all(v == np.float32(-50.0))


def test_kquant_short_data_is_invalid_tensor_info(gpu):
    with pytest.raises(gguf.InvalidTensorInfo):
        gguf.dequantize(np.zeros(2 * 144 - 1, np.uint8), gguf.GGMLType.Q4_K, 257)
    v = gguf.dequantize(synth.quantized_weight(Q6_K, 2, 256, seed=5), gguf.GGMLType.Q6_K, 300)
    assert v.shape == (300,)


# (m, k): ragged row counts, one to 56 blocks per row
GEMV_SHAPES = [(1, 256), (63, 512), (300, 4096), (1024, 4096), (97, 14336)]


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("m,k", GEMV_SHAPES)
def test_kquant_gemv_parity(gpu, orc, t, m, k):
    print(f"[case] kquant gemv type={t} m={m} k={k}", flush=True)
    w = synth.quantized_weight(t, m, k, seed=m + k + t)
    x = synth.activations(k, seed=m * 5 + k)
    got = gemv(t, w, x, m, k)
    ref = orc.matvec_f64(t, w, x, m, k)[1]
    r, a = rel_l2(got, ref), max_abs(got, ref)
    print(f"[result] kquant t={t} {m}x{k} rel_l2={r:.3e} max_abs={a:.3e}", flush=True)
    assert r <= 1e-4 and a <= 1e-3


def test_kquant_gemv_matches_dequantized_dot(gpu):
    """The GEMV is the dequantization followed by the dot product: the same
    numbers as the GPU's own dequantized matrix times x, within f32 summation."""
    m, k = 200, 2048
    w = synth.quantized_weight(Q6_K, m, k, seed=4)
    x = synth.activations(k, seed=5)
    deq = gpu_dequant(Q6_K, w, m * k).reshape(m, k).astype(np.float64)
    got = gemv(Q6_K, w, x, m, k)
    assert rel_l2(got, deq @ x.astype(np.float64)) <= 1e-6


# K = 2048 .. 16384: 1 .. 4 K-segments of the matrix-core kernel (Q6_K at
# K = 14336: four segments of 14 blocks that start 4, 8, 12 bytes past a
# 16-byte boundary); K = 2560 and 5120 (Q6_K rows not a multiple of 16 bytes)
# run on the simple kernel
MFMA_K = [2048, 2560, 4096, 5120, 8192, 12288, 14336, 16384]


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("k", MFMA_K)
def test_kquant_mfma_matches_simple_kernel(gpu, orc, t, k):
    print(f"[case] kquant mfma type={t} k={k}", flush=True)
    m = 200
    w = synth.quantized_weight(t, m, k, seed=k + t)
    x = synth.activations(k, seed=k + 1)
    got = gemv(t, w, x, m, k)
    prev = ops.gemv_select(ops.GEMV_STREAM)
    try:
        simple = gemv(t, w, x, m, k)
    finally:
        ops.gemv_select(prev)
    ref = orc.matvec_f64(t, w, x, m, k)[1]
    for name, y in (("auto", got), ("simple", simple)):
        r, a = rel_l2(y, ref), max_abs(y, ref)
        print(f"[result] kquant {name} t={t} k={k} rel_l2={r:.3e} max_abs={a:.3e}", flush=True)
        assert r <= 1e-4 and a <= 1e-3
    assert rel_l2(got, simple) <= 1e-5


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("scale", [1e-30, 1e30])
def test_kquant_mfma_activation_scales(gpu, orc, t, scale):
    m, k = 256, 4096
    w = synth.quantized_weight(t, m, k, seed=31)
    x = (synth.activations(k, seed=32) * np.float32(scale)).astype(np.float32)
    got = gemv(t, w, x, m, k)
    ref = orc.matvec_f64(t, w, x, m, k)[1]
    assert rel_l2(got, ref) <= 1e-4


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_mfma_nonfinite_and_zero_chunks(gpu, orc, t):
    m, k = 128, 4096
    w = synth.quantized_weight(t, m, k, seed=33)
    x = synth.activations(k, seed=34)
    x[:512] = 0.0
    got = gemv(t, w, x, m, k)
    assert rel_l2(got, orc.matvec_f64(t, w, x, m, k)[1]) <= 1e-4
    x[700] = np.inf
    got = gemv(t, w, x, m, k)
    ref = orc.matvec_f32(t, w, x, m, k)[1]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(np.isinf(got[fin]), np.isinf(ref[fin]))
    assert np.array_equal(np.sign(got[fin]), np.sign(ref[fin]))


# ---------------------------------------------------------------- prefill
# More than two tokens: the matrix is repacked into 32-element blocks with f32
# scales (Q4_K: (d * scale) q + dmin; Q6_K: 16-element halves, (d * scale / 64)
# (q - 32), padded to 32 with zeros) and multiplied on the tiled MFMA kernel.
# (m, n, k): one to 56 super-blocks per row, ragged token and row counts,
# token tiles of 16 .. 128, split-K
KQ_MATMUL = [(3, 300, 4096), (8, 1024, 2048), (17, 768, 256), (64, 129, 4096), (130, 200, 512),
             (257, 384, 1024), (512, 256, 14336)]


def kq_matmul(t, w, x, m, n, k, w_offset=0):
    wb, wp = up(w, offset=w_offset)
    xb, xp = up(x)
    yb = DeviceBuffer(4 * m * n)
    wsz = ops.matmul_workspace_bytes(t, n, k, m)
    ws = DeviceBuffer(max(wsz, 1))
    ops.quantized_matmul(t, wp, w.nbytes, n, k, xp, m, yb.ptr, ws, wsz)
    return down(yb, np.float32, m * n).reshape(m, n)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("m,n,k", KQ_MATMUL)
def test_kquant_matmul_parity(gpu, orc, t, m, n, k):
    print(f"[case] kquant matmul type={t} m={m} n={n} k={k}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n + k + t)
    x = synth.activations(m * k, seed=m + t).reshape(m, k)
    got = kq_matmul(t, w, x, m, n, k)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    r, a = rel_l2(got, ref), max_abs(got, ref)
    print(f"[result] kquant matmul t={t} rel_l2={r:.3e} max_abs={a:.3e}", flush=True)
    assert r <= 1e-4 and a <= 1e-3


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_matmul_matches_gemv(gpu, t):
    """The tiled path (5 tokens) and the per-token GEMV agree on every token."""
    m, n, k = 5, 520, 4096
    w = synth.quantized_weight(t, n, k, seed=77 + t)
    x = synth.activations(m * k, seed=78).reshape(m, k)
    got = kq_matmul(t, w, x, m, n, k)
    for i in range(m):
        assert rel_l2(got[i], gemv(t, w, x[i], n, k)) <= 1e-5


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("hidden,n_ff,m", [(256, 512, 1), (512, 1024, 4), (4096, 1024, 64), (256, 20480, 5)])
def test_kquant_ffn_parity(gpu, orc, t, hidden, n_ff, m):
    """The SwiGLU FFN layer on K-quant weights: decode (fused gate/up GEMV) and
    prefill (RMSNorm and SwiGLU packed into the tiled GEMM's activations, each
    matrix repacked in turn into one workspace region)."""
    print(f"[case] kquant ffn t={t} hidden={hidden} n_ff={n_ff} m={m}", flush=True)
    L = synth.ffn_layer(t, hidden, n_ff, m, seed=hidden + n_ff + t)
    bufs = {name: up(v) for name, v in L.items()}
    ob = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m, ggml_type=t)
    ws = DeviceBuffer(wsz)
    ops.ffn_swiglu(t, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], m, ob.ptr, ws.ptr, wsz)
    got = down(ob, np.float32, m * hidden).reshape(m, hidden)
    rows = sorted({0, m // 2, m - 1})
    ref = orc.ffn_rows_f64(t, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5, L["x"], rows)
    r, a = rel_l2(got[rows], ref), max_abs(got[rows], ref)
    rms = float(np.sqrt(np.mean(ref ** 2)))
    print(f"[result] kquant ffn rel_l2={r:.3e} max_abs={a:.3e} rms={rms:.3e}", flush=True)
    assert r <= 1e-4 and a <= 1e-3 * max(1.0, rms / 300.0)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_matmul_unaligned_weights(gpu, orc, t):
    """Weights 4 bytes past a 16-byte boundary cannot be repacked with 16-byte
    loads: the call takes one GEMV per token instead, same results."""
    m, n, k = 6, 256, 2048
    w = synth.quantized_weight(t, n, k, seed=91 + t)
    x = synth.activations(m * k, seed=92).reshape(m, k)
    got = kq_matmul(t, w, x, m, n, k, w_offset=4)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    assert rel_l2(got, ref) <= 1e-4 and max_abs(got, ref) <= 1e-3
    assert rel_l2(got, kq_matmul(t, w, x, m, n, k)) <= 1e-5


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_prepared_prefill(gpu, orc, t):
    """wh_weight_prepare_prefill converts a handle's blocks once (the reference's
    convert-once cache, dequantization_cache.rs:121-165); matmul and FFN calls
    on the handle's data then skip the per-call conversion and give the same
    bits as the converting call, at the north-star bar against the f64 oracle.
    Preparing again is a no-op; a Q4_0 handle needs no copy."""
    m, n, k = 64, 512, 4096
    w = synth.quantized_weight(t, n, k, seed=500 + t)
    x = synth.activations(m * k, seed=501).reshape(m, k)
    plain = kq_matmul(t, w, x, m, n, k)
    wh = ops.Weight(t, n, k, w)
    size = wh.prepare_prefill()
    # Q4_K: 20-byte blocks, then the fp16 dmin table with rows of k / 256 rounded up to 8
    assert size == (n * (k // 32 * 20 + (k // 256 + 7) // 8 * 8 * 2) if t == Q4_K else n * k // 16 * 20)
    assert wh.prepare_prefill() == size
    xb, xp = up(x)
    yb = DeviceBuffer(4 * m * n)
    wsz = ops.matmul_workspace_bytes(t, n, k, m)
    ws = DeviceBuffer(wsz)
    ops.quantized_matmul(t, wh.ptr, wh.nbytes, n, k, xp, m, yb.ptr, ws, wsz)
    got = down(yb, np.float32, m * n).reshape(m, n)
    assert same(got, plain)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, np.arange(m))
    assert rel_l2(got, ref) <= 1e-4 and max_abs(got, ref) <= 1e-3
    # the FFN layer with prepared gate / up / down handles against the converting call
    hidden, n_ff, mf = 4096, 1024, 64
    L = synth.ffn_layer(t, hidden, n_ff, mf, seed=510 + t)
    bufs = {name: up(v) for name, v in L.items()}
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, mf, ggml_type=t)
    ws = DeviceBuffer(wsz)
    ob = DeviceBuffer(4 * mf * hidden)
    ops.ffn_swiglu(t, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], mf, ob.ptr, ws.ptr, wsz)
    base = down(ob, np.float32, mf * hidden)
    hw = {name: ops.Weight(t, *((n_ff, hidden) if name != "down" else (hidden, n_ff)), L[name])
          for name in ("gate", "up", "down")}
    for h in hw.values():
        assert h.prepare_prefill() > 0
    ob2 = DeviceBuffer(4 * mf * hidden)
    ops.ffn_swiglu(t, hw["gate"].ptr, hw["up"].ptr, hw["down"].ptr, hidden, n_ff,
                   bufs["gamma"][1], 1e-5, bufs["x"][1], mf, ob2.ptr, ws.ptr, wsz)
    assert same(down(ob2, np.float32, mf * hidden), base)
    for h in hw.values():
        h.free()
    wh.free()
    q = ops.Weight(2, 64, 256, synth.quantized_weight(2, 64, 256, seed=1))
    assert q.prepare_prefill() == 0
    q.free()
