"""The device copies behind the synchronous host-memory entry points
(wh_host_cache_*): the device-side counterpart of the reference's per-tensor
DequantizationCache::get_or_dequantize
(crates/woolly-core/src/model/dequantization_cache.rs:121-165).

CPU tests cover the bookkeeping that needs no device (budget, stats, evicting
and clearing an empty cache); the GPU tests cover a miss then a hit, results
identical to an uncached call and to the oracle, eviction by host range,
least-recently-used eviction beyond the budget, and an input larger than the
budget that is never cached."""
import numpy as np
import pytest

from tests._oracle import max_abs, rel_l2
from woolly_amd import synth
from woolly_amd.quantization import QuantizationScheme, QuantizedStorage, device_cache, dequantize_q4_0, simd

Q4_0 = 2


@pytest.fixture
def cache_off():
    device_cache.configure(0)
    yield
    device_cache.configure(0)


def _delta(before, after):
    return {k: after[k] - before[k] for k in ("hits", "misses", "evictions")}


def test_cache_bookkeeping_without_gpu(cache_off):
    assert device_cache.stats()["max_bytes"] == 0
    device_cache.configure(1 << 20)
    st = device_cache.stats()
    assert st["max_bytes"] == 1 << 20 and st["entries"] == 0 and st["bytes"] == 0
    assert device_cache.evict(np.zeros(16, np.float32)) == 0
    device_cache.clear()
    assert device_cache.stats()["max_bytes"] == 1 << 20  # clear keeps the budget
    device_cache.configure(0)
    assert device_cache.stats()["max_bytes"] == 0


def _matvec(w, x, m, k):
    y = np.zeros(m, np.float32)
    simd.quantized_matvec(QuantizedStorage(QuantizationScheme.Q4_0, w), x, y, m, k)
    return y


@pytest.mark.gpu
def test_cached_matvec_hit_miss_evict(gpu, orc, cache_off):
    m, k = 512, 4096
    w = synth.quantized_weight(Q4_0, m, k, seed=21)
    x = synth.activations(k, seed=22)
    x2 = synth.activations(k, seed=23)
    uncached = _matvec(w, x, m, k)
    device_cache.configure(64 << 20)
    s0 = device_cache.stats()
    first = _matvec(w, x, m, k)            # miss: uploads and keeps the copy
    s1 = device_cache.stats()
    assert _delta(s0, s1) == {"hits": 0, "misses": 1, "evictions": 0}
    assert s1["entries"] == 1 and s1["bytes"] == w.nbytes
    second = _matvec(w, x2, m, k)          # hit: new activations, same weights
    s2 = device_cache.stats()
    assert _delta(s1, s2) == {"hits": 1, "misses": 0, "evictions": 0}
    assert np.array_equal(first, uncached)
    ref2 = orc.matvec_f64(Q4_0, w, x2, m, k)[1]
    assert rel_l2(second, ref2) <= 1e-4 and max_abs(second, ref2) <= 1e-3
    # evicting a range inside the array drops its entry; the next call misses
    assert device_cache.evict(w[10:20]) == 1
    assert device_cache.stats()["entries"] == 0
    s3 = device_cache.stats()
    third = _matvec(w, x2, m, k)
    assert _delta(s3, device_cache.stats())["misses"] == 1
    assert np.array_equal(third, second)


@pytest.mark.gpu
def test_cache_lru_and_oversized(gpu, orc, cache_off):
    m, k = 256, 4096
    ws = [synth.quantized_weight(Q4_0, m, k, seed=30 + i) for i in range(3)]
    x = synth.activations(k, seed=33)
    nb = ws[0].nbytes
    device_cache.configure(2 * nb)         # room for two matrices
    for w in ws[:2]:
        _matvec(w, x, m, k)
    _matvec(ws[0], x, m, k)                # ws[0] is now the most recent
    s0 = device_cache.stats()
    _matvec(ws[2], x, m, k)                # evicts ws[1], the least recently used
    s1 = device_cache.stats()
    assert _delta(s0, s1) == {"hits": 0, "misses": 1, "evictions": 1}
    assert s1["entries"] == 2 and s1["bytes"] == 2 * nb
    _matvec(ws[0], x, m, k)
    assert _delta(s1, device_cache.stats())["hits"] == 1
    s2 = device_cache.stats()
    y1 = _matvec(ws[1], x, m, k)
    assert _delta(s2, device_cache.stats())["misses"] == 1
    ref = orc.matvec_f64(Q4_0, ws[1], x, m, k)[1]
    assert rel_l2(y1, ref) <= 1e-4 and max_abs(y1, ref) <= 1e-3
    # an input larger than the budget is uploaded per call and never cached
    device_cache.clear()
    device_cache.configure(nb // 2)
    s3 = device_cache.stats()
    for _ in range(2):
        _matvec(ws[0], x, m, k)
    st = device_cache.stats()
    assert st["entries"] == 0 and _delta(s3, st) == {"hits": 0, "misses": 2, "evictions": 0}


@pytest.mark.gpu
def test_cached_dequantize_bit_exact(gpu, orc, cache_off):
    w = synth.quantized_weight(Q4_0, 64, 4096, seed=40)
    blocks = w.view(np.uint8).view(np.dtype([("d", "<u2"), ("qs", "u1", (16,))]))
    plain = dequantize_q4_0(blocks)
    device_cache.configure(16 << 20)
    a = dequantize_q4_0(blocks)
    b = dequantize_q4_0(blocks)
    st = device_cache.stats()
    assert st["hits"] >= 1 and st["entries"] == 1
    exp = orc.dequantize(Q4_0, w, 64 * 4096)[1]
    for got in (plain, a, b):
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
