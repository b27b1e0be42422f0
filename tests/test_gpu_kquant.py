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
