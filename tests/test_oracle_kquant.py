"""The oracle's Q4_K / Q6_K restatement (woolly_gguf::dequantize,
crates/woolly-gguf/src/dequantize.rs:380-536), pinned without the reference's
own vectors (it has none for these formats):

* block and type sizes: dequantize.rs:630-631 (256 elements) and
  tensor_info.rs:136,163,165 (144 and 210 bytes);
* closed forms hand-derived from dequantize.rs for byte patterns that isolate
  one rule each (where d, dmin and the scales sit in the block, which nibble an
  even element takes, the 6-bit scale packing, Q6_K's unsigned scales, its
  (q - 32) / 64 and the qh wrap-around at the block's last element);
* an independent vectorised numpy decoder (whole-array index arithmetic instead
  of the C loop) on random blocks, bit for bit, and the f64 GEMV on top of it;
* planted mistakes each fail one of the closed forms.

woolly decodes both formats its own way: its Q4_K reads 8 scales from bytes
0..11 and d, dmin at 12..15 and adds dmin, and its Q6_K reads the scales as
unsigned bytes; neither is ggml's layout.  The oracle follows woolly."""
import numpy as np
import pytest

from woolly_amd import synth

Q4_K, Q6_K = 12, 14
INVALID_TENSOR_INFO = 11


def f16b(v) -> np.ndarray:
    return np.array([v], np.float32).astype(np.float16).view(np.uint8)


def q4k_block(scales12, d, dmin, qs128) -> np.ndarray:
    b = np.zeros(144, np.uint8)
    b[0:12] = scales12
    b[12:14] = f16b(d)
    b[14:16] = f16b(dmin)
    b[16:144] = qs128
    return b


def q6k_block(ql128, qh64, scales16, d) -> np.ndarray:
    b = np.zeros(210, np.uint8)
    b[0:128] = ql128
    b[128:192] = qh64
    b[192:208] = scales16
    b[208:210] = f16b(d)
    return b


def np_q4_k(blocks: np.ndarray) -> np.ndarray:
    """Whole-array restatement of dequantize_q4_k_scalar (dequantize.rs:404-458)."""
    b = blocks.reshape(-1, 144).astype(np.int64)
    i = np.arange(8)
    src = (3 * i) // 2
    lo6 = b[:, src] & 63
    hi6 = ((b[:, src] >> 6) | ((b[:, np.minimum(src + 1, 11)] & 15) << 2)) & 63
    scales = np.where(i % 2 == 0, lo6, hi6).astype(np.float32)            # (nb, 8)
    d = blocks.reshape(-1, 144)[:, 12:14].copy().view(np.float16).astype(np.float32)  # (nb, 1)
    dmin = blocks.reshape(-1, 144)[:, 14:16].copy().view(np.float16).astype(np.float32)
    qs = b[:, 16:144]
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 256).astype(np.float32)  # even: low nibble
    scale = np.repeat(scales, 32, axis=1)
    return ((d * scale) * q + dmin).astype(np.float32).reshape(-1)


def np_q6_k(blocks: np.ndarray) -> np.ndarray:
    """Whole-array restatement of dequantize_q6_k (dequantize.rs:460-536)."""
    b = blocks.reshape(-1, 210)
    ql, qh, sc = b[:, :128].astype(np.int64), b[:, 128:192].astype(np.int64), b[:, 192:208].astype(np.float32)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)
    i = np.arange(256)
    ql_idx = 64 * (i // 128) + 32 * ((i % 128) // 64) + 16 * ((i % 64) // 32) + i % 16
    qh_idx = 32 * (i // 128) + 16 * ((i % 128) // 64) + 8 * ((i % 64) // 32) + (i % 32) // 4
    shift = 2 * ((i % 32) % 4)
    qhv = qh[:, qh_idx]
    e1 = (qhv >> shift) & 3
    nxt = np.where(qh_idx + 1 < 64, qh[:, np.minimum(qh_idx + 1, 63)] & 3, 0)
    e2 = np.where(shift < 6, (qhv >> np.minimum(shift + 2, 7)) & 3, nxt)
    qlv = ql[:, ql_idx]
    q = np.where(i < 128, (qlv & 15) | (e1 << 4), (qlv >> 4) | (e2 << 4))
    s = sc[:, i // 16]
    return (((d * s) * (q - 32).astype(np.float32)) / np.float32(64.0)).astype(np.float32).reshape(-1)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_kquant_sizes(orc):
    assert (orc.block_size(Q4_K), orc.type_size(Q4_K)) == (256, 144)
    assert (orc.block_size(Q6_K), orc.type_size(Q6_K)) == (256, 210)


def test_q4_k_closed_forms(orc):
    # all scales 0: every element is d * 0 * q + dmin = dmin (d at 12..13, dmin at 14..15)
    blk = q4k_block(np.zeros(12, np.uint8), 3.0, -0.75, np.full(128, 0xAB, np.uint8))
    st, v = orc.dequantize(Q4_K, blk, 256)
    assert st == 0 and np.all(v == np.float32(-0.75))
    # scale bytes 0xFF: even scales b & 63 = 63, odd ((0xFF >> 6) | (0x0F << 2)) & 63 = 63;
    # qs = 0x21: even elements take the low nibble 1, odd the high nibble 2
    blk = q4k_block(np.full(12, 0xFF, np.uint8), 0.5, 0.25, np.full(128, 0x21, np.uint8))
    st, v = orc.dequantize(Q4_K, blk, 256)
    assert np.all(v[0::2] == np.float32(0.5 * 63 * 1 + 0.25))
    assert np.all(v[1::2] == np.float32(0.5 * 63 * 2 + 0.25))
    # 6-bit packing, scale i from byte src = 3i/2: even i -> b[src] & 63, odd i ->
    # (b[src] >> 6) | ((b[src+1] & 15) << 2); with the bytes below the eight scales are
    # 5, (0x87>>6)|(3<<2) = 14, 10, (0xC0>>6)|(5<<2) = 23, 17, (0x40>>6)|(15<<2) = 61,
    # 63, (0x80>>6)|(12<<2) = 50; groups of 32 elements, q = 1 everywhere, d = 1, dmin = 0
    sb = np.array([0x05, 0x87, 0x03, 0x0A, 0xC0, 0x05, 0x11, 0x40, 0x0F, 0x3F, 0x80, 0x0C], np.uint8)
    blk = q4k_block(sb, 1.0, 0.0, np.full(128, 0x11, np.uint8))
    st, v = orc.dequantize(Q4_K, blk, 256)
    assert v.reshape(8, 32)[:, 0].tolist() == [5.0, 14.0, 10.0, 23.0, 17.0, 61.0, 63.0, 50.0]
    assert np.all(v.reshape(8, 32) == v.reshape(8, 32)[:, :1])


def test_q6_k_closed_forms(orc):
    d = 0.5
    scales = np.arange(1, 17, dtype=np.uint8)
    # ql = qh = 0: q = 0 everywhere, value = d * s * (-32) / 64 = -d * s / 2, s = scales[i / 16]
    st, v = orc.dequantize(Q6_K, q6k_block(np.zeros(128, np.uint8), np.zeros(64, np.uint8), scales, d), 256)
    assert st == 0 and np.array_equal(v, np.float32(-d / 2) * np.repeat(scales, 16).astype(np.float32))
    # scales are unsigned: 0xC8 = 200, not -56
    st, v = orc.dequantize(Q6_K, q6k_block(np.zeros(128, np.uint8), np.zeros(64, np.uint8),
                                           np.full(16, 0xC8, np.uint8), d), 256)
    assert np.all(v == np.float32(-d * 200 / 2))
    # ql = 0xF0: elements below 128 take the low nibble (q = 0), the rest the high one (q = 15)
    st, v = orc.dequantize(Q6_K, q6k_block(np.full(128, 0xF0, np.uint8), np.zeros(64, np.uint8),
                                           np.ones(16, np.uint8), d), 256)
    assert np.all(v[:128] == np.float32(d * -32 / 64)) and np.all(v[128:] == np.float32(d * -17 / 64))
    # qh = 0xFF: every 2-bit extension is 3 (q = 48) except element 255, whose
    # extension would come from a 65th qh byte and is 0 there (q = 0)
    st, v = orc.dequantize(Q6_K, q6k_block(np.zeros(128, np.uint8), np.full(64, 0xFF, np.uint8),
                                           np.ones(16, np.uint8), d), 256)
    assert np.all(v[:255] == np.float32(d * 16 / 64)) and v[255] == np.float32(d * -32 / 64)


@pytest.mark.parametrize("t,n", [(Q4_K, 256), (Q4_K, 4096 + 100), (Q6_K, 256), (Q6_K, 8 * 256 - 3)])
def test_kquant_matches_numpy(orc, t, n):
    nb = (n + 255) // 256
    data = synth.quantized_weight(t, nb, 256, seed=n + t)
    st, v = orc.dequantize(t, data, n)
    ref = (np_q4_k if t == Q4_K else np_q6_k)(data)[:n]
    assert st == 0 and np.array_equal(bits(v), bits(ref))


def test_kquant_random_bytes_and_scales(orc):
    """Every byte of the blocks random (f16 fields included, NaN/inf/subnormal
    patterns among them): bit-exact, NaN compared as NaN."""
    rng = np.random.default_rng(3)
    for t, ts, fn in ((Q4_K, 144, np_q4_k), (Q6_K, 210, np_q6_k)):
        data = rng.integers(0, 256, 64 * ts, dtype=np.uint8)
        st, v = orc.dequantize(t, data, 64 * 256)
        ref = fn(data)
        with np.errstate(invalid="ignore"):
            same = (bits(v) == bits(ref)) | (np.isnan(v) & np.isnan(ref))
        assert st == 0 and np.all(same)


def test_kquant_errors(orc):
    st, _ = orc.dequantize(Q4_K, np.zeros(143, np.uint8), 256)
    assert st == INVALID_TENSOR_INFO
    st, _ = orc.dequantize(Q6_K, np.zeros(210, np.uint8), 257)  # two blocks needed
    assert st == INVALID_TENSOR_INFO
    w = synth.quantized_weight(Q4_K, 2, 256, seed=1)
    st, _ = orc.matvec_f64(Q4_K, w, np.zeros(128, np.float32), 2, 128)
    assert st != 0


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_kquant_matvec_f64(orc, t):
    m, k = 7, 1024
    w = synth.quantized_weight(t, m, k, seed=9)
    x = synth.activations(k, seed=9)
    st, y = orc.matvec_f64(t, w, x, m, k)
    deq = (np_q4_k if t == Q4_K else np_q6_k)(w).reshape(m, k).astype(np.float64)
    assert st == 0 and np.allclose(y, deq @ x.astype(np.float64), rtol=1e-12, atol=1e-12)
    st32, y32 = orc.matvec_f32(t, w, x, m, k)
    assert st32 == 0 and np.allclose(y32, y, rtol=1e-5, atol=1e-5)


def np_q4_k_bug(blocks, bug):
    b = blocks.reshape(-1, 144)
    if bug == "ggml_layout":  # d, dmin first, then the scales
        b = np.concatenate([b[:, 4:16], b[:, 0:4], b[:, 16:]], axis=1)
    v = np_q4_k(b)
    if bug == "nibble_parity":
        v = v.reshape(-1, 2)[:, ::-1].reshape(-1)
    return v


def np_q6_k_bug(blocks, bug):
    b = blocks.reshape(-1, 210).copy()
    if bug == "signed_scales":
        d = b[:, 208:210].copy().view(np.float16).astype(np.float32)
        s = b[:, 192:208].view(np.int8).astype(np.float32)
        base = np_q6_k(b).reshape(-1, 256) / np.repeat(b[:, 192:208].astype(np.float32), 16, axis=1)
        return (base * np.repeat(s, 16, axis=1)).reshape(-1)
    if bug == "no_wrap":  # e2 of shift 6 taken from the same byte (always 0)
        v = np_q6_k(b).reshape(-1, 256)
        i = np.arange(256)
        hit = (i >= 128) & ((i % 32) % 4 == 3)
        d = b[:, 208:210].copy().view(np.float16).astype(np.float32)
        q = (b[:, :128].astype(np.int64)[:, (64 * (i // 128) + 32 * ((i % 128) // 64) + 16 * ((i % 64) // 32) + i % 16)] >> 4)
        s = b[:, 192:208].astype(np.float32)[:, i // 16]
        alt = (((d * s) * (q - 32).astype(np.float32)) / np.float32(64.0)).astype(np.float32)
        return np.where(hit, alt, v).reshape(-1)
    return np_q6_k(b)


def test_kquant_planted_bugs_fail():
    """ggml's Q4_K field order, swapped nibble parity, signed Q6_K scales and a
    Q6_K decoder without the cross-byte extension each fail a closed form."""
    zero_scales = q4k_block(np.zeros(12, np.uint8), 3.0, -0.75, np.full(128, 0xAB, np.uint8))
    assert not np.all(np_q4_k_bug(zero_scales, "ggml_layout") == np.float32(-0.75))
    parity = q4k_block(np.full(12, 0xFF, np.uint8), 0.5, 0.25, np.full(128, 0x21, np.uint8))
    v = np_q4_k_bug(parity, "nibble_parity")
    assert not (np.all(v[0::2] == np.float32(0.5 * 63 + 0.25)) and np.all(v[1::2] == np.float32(0.5 * 126 + 0.25)))
    unsigned = q6k_block(np.zeros(128, np.uint8), np.zeros(64, np.uint8), np.full(16, 0xC8, np.uint8), 0.5)
    assert not np.all(np_q6_k_bug(unsigned, "signed_scales") == np.float32(-0.5 * 200 / 2))
    wrap = q6k_block(np.zeros(128, np.uint8), np.full(64, 0xFF, np.uint8), np.ones(16, np.uint8), 0.5)
    v = np_q6_k_bug(wrap, "no_wrap")
    assert not np.all(v[:255] == np.float32(0.5 * 16 / 64))
    # the correct decoders pass the same checks
    assert np.all(np_q4_k(zero_scales) == np.float32(-0.75))
    assert np.all(np_q6_k(wrap)[:255] == np.float32(0.5 * 16 / 64))
