"""Bit-exact GPU dequantization against the oracle and the reference's KATs."""
import numpy as np
import pytest

from tests._gpu import down, up
from tests.test_oracle import block_q4_0, block_q4_1, block_q5_0, block_q5_1, block_q8_0
from woolly_amd import gguf, ops, quantization, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0 = 2, 3, 8
Q5_0, Q5_1 = 6, 7


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(b)
    return (a.shape == b.shape and np.array_equal(np.isnan(a), nan)
            and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


# --- the reference's own unit tests (quantization.rs:1294-1409), run on the GPU
def test_q4_0_dequantization(gpu):
    blocks = np.frombuffer(block_q4_0(2.0, [0] * 16).tobytes(), quantization.BlockQ4_0)
    result = quantization.dequantize_q4_0(blocks)
    assert len(result) == 32 and np.all(np.abs(result - (-16.0)) < 1e-6)


def test_q4_1_dequantization(gpu):
    blocks = np.frombuffer(block_q4_1(1.0, 5.0, [0x01] * 16).tobytes(), quantization.BlockQ4_1)
    result = quantization.dequantize_q4_1(blocks)
    assert len(result) == 32
    for i in range(16):
        assert abs(result[i] - 6.0) < 1e-6 and abs(result[i + 16] - 5.0) < 1e-6


def test_q8_0_dequantization(gpu):
    qs = np.zeros(32, np.int8)
    qs[0], qs[1] = 10, -5
    blocks = np.frombuffer(block_q8_0(0.5, qs).tobytes(), quantization.BlockQ8_0)
    result = quantization.dequantize_q8_0(blocks)
    assert len(result) == 32 and abs(result[0] - 5.0) < 1e-6 and abs(result[1] + 2.5) < 1e-6


def test_q5_0_dequantization(gpu):
    # quantization.rs:1410-1427
    blocks = np.frombuffer(block_q5_0(0.5, [0xFF] * 4, [0xFF] * 16).tobytes(), quantization.BlockQ5_0)
    result = quantization.dequantize_q5_0(blocks)
    assert len(result) == 32 and np.all(np.abs(result - 7.5) < 1e-6)


def test_q5_1_dequantization(gpu):
    # quantization.rs:1429-1446
    blocks = np.frombuffer(block_q5_1(1.0, 10.0, [0] * 4, [0x11] * 16).tobytes(), quantization.BlockQ5_1)
    result = quantization.dequantize_q5_1(blocks)
    assert len(result) == 32 and np.all(np.abs(result - 11.0) < 1e-6)


def test_q5_storage_dispatch(gpu, orc):
    # optimized::dequantize_blocks takes Q5 storage (quantization.rs:1187-1200);
    # simd::quantized_matvec does not (UnsupportedScheme, :905-907)
    for t, make in ((Q5_0, quantization.QuantizedStorage.Q5_0), (Q5_1, quantization.QuantizedStorage.Q5_1)):
        data = synth.quantized_weight(t, 1, 8 * 32, seed=t)
        got = quantization.optimized.dequantize_blocks(make(data))
        st, ref = orc.dequantize(t, data, 8 * 32)
        assert st == 0 and same_bits(got, ref)
        with pytest.raises(quantization.QuantizationError.UnsupportedScheme):
            quantization.simd.quantized_matvec(make(data), np.zeros(256, np.float32), np.zeros(1, np.float32),
                                               1, 256)


def test_optimized_dispatcher(gpu):
    data = np.concatenate([block_q4_0(1.0, [0x11] * 16), block_q4_0(2.0, [0x22] * 16)])
    storage = quantization.QuantizedStorage.Q4_0(data)
    result = quantization.optimized.dequantize_blocks(storage)
    assert len(result) == 64
    assert np.all(np.abs(result[:32] + 7.0) < 1e-6) and np.all(np.abs(result[32:] + 12.0) < 1e-6)


def test_simd_batch_processing(gpu):
    data = np.concatenate([block_q4_0(i + 1.0, [0] * 16) for i in range(8)])
    blocks = np.frombuffer(data.tobytes(), quantization.BlockQ4_0)
    simd_r = quantization.simd.dequantize_q4_0_batch(blocks)
    assert np.array_equal(simd_r, np.repeat(-8.0 * (np.arange(8) + 1), 32).astype(np.float32))


def test_parallel_quantization_correctness(gpu, orc):
    # woolly-core/tests/parallel_inference_integration.rs:159-210
    q4 = np.concatenate([block_q4_0(0.1 + i * 0.001, [i % 16] * 16) for i in range(64)])
    q8 = np.concatenate([block_q8_0(0.1 + i * 0.001, [i % 127] * 32) for i in range(64)])
    for t, data in ((Q4_0, q4), (Q8_0, q8)):
        got = gguf.dequantize(data, gguf.GGMLType(t), 64 * 32)
        st, ref = orc.dequantize(t, data, 64 * 32)
        assert st == 0 and same_bits(got, ref)


# --- bit-exact parity with the oracle
@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0, Q5_0, Q5_1])
@pytest.mark.parametrize("n", [1, 4, 31, 32, 33, 100, 4096, 100003])
@pytest.mark.parametrize("in_off,out_off", [(0, 0), (2, 4), (1, 8)])
def test_dequant_bit_exact(gpu, orc, t, n, in_off, out_off):
    print(f"[case] dequant type={t} n={n} in_off={in_off} out_off={out_off}", flush=True)
    data = synth.quantized_weight(t, 1, (n + 31) // 32 * 32, seed=n + t)
    db, dp = up(data, offset=in_off)
    ob = DeviceBuffer(4 * n + out_off)
    ops.dequantize(t, dp, data.nbytes, n, ob.ptr + out_off)
    got = down(ob, np.float32, n, out_off)
    st, ref = orc.dequantize(t, data, n)
    assert st == 0 and same_bits(got, ref)


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0, Q5_0, Q5_1])
def test_dequant_every_f16_scale(gpu, orc, t):
    nb = 65536
    ts = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q5_0: 22, Q5_1: 24}[t]
    rng = np.random.default_rng(t)
    data = rng.integers(0, 256, (nb, ts), dtype=np.uint8)
    data[:, 0:2] = np.arange(nb, dtype=np.uint16).view(np.uint8).reshape(nb, 2)
    if t in (Q4_1, Q5_1):  # every pattern as the min too
        data[:, 2:4] = np.arange(nb, dtype=np.uint16)[::-1].copy().view(np.uint8).reshape(nb, 2)
    data = data.reshape(-1)
    got = gguf.dequantize(data, gguf.GGMLType(t), nb * 32)
    st, ref = orc.dequantize(t, data, nb * 32)
    assert st == 0 and same_bits(got, ref)


def test_dequant_f16_f32(gpu):
    vals = np.arange(65536, dtype=np.uint16)
    got = gguf.dequantize(vals.view(np.uint8), gguf.GGMLType.F16, 65536)
    ref = vals.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    f = np.random.default_rng(0).standard_normal(1001).astype(np.float32)
    assert np.array_equal(gguf.dequantize(f.view(np.uint8), gguf.GGMLType.F32, 1001), f)


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_1])
def test_dequant_full_size(gpu, orc, t):
    n_rows, k = 14336, 4096
    print(f"[case] dequant full type={t} {n_rows}x{k}", flush=True)
    w = synth.quantized_weight(t, n_rows, k, seed=3)
    wb, wp = up(w)
    ob = DeviceBuffer(4 * n_rows * k)
    ops.dequantize(t, wp, w.nbytes, n_rows * k, ob.ptr)
    got = down(ob, np.float32, n_rows * k)
    st, ref = orc.dequantize(t, w, n_rows * k)
    assert st == 0 and same_bits(got, ref)
