"""Pins the decode-step part of the CPU oracle (RoPE frequencies, single-token
GQA attention over an f16 KV cache, one transformer layer, the output head)
against closed forms and an independent numpy float64 implementation written
here from the reference's formulas:
  RoPE::apply_f32            crates/woolly-tensor/src/ops/mod.rs:472-530
  compute_optimized_gqa_attention  crates/woolly-core/src/model/lazy_transformer.rs:261-456
  process_layer / forward    lazy_transformer.rs:98-258, 1155-1335
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.test_oracle import np_dequant
from tests.test_oracle_kquant import np_q4_k, np_q6_k
from woolly_amd import synth

Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14


def np_rope(x: np.ndarray, pos: int, inv_freq: np.ndarray) -> np.ndarray:
    """numpy restatement: pairs (i, i + d/2), angle = f32(pos * inv_freq[i])."""
    d = x.size
    h = d // 2
    ang = (np.float32(pos) * inv_freq.astype(np.float32)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[:h].astype(np.float64), x[h:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c])


def f16(v) -> np.ndarray:
    return np.asarray(v, np.float64).astype(np.float32).astype(np.float16)


def np_attention(qkv, kc, vc, pos, n_heads, n_kv, d, inv_freq):
    """Independent numpy float64 attention; kc / vc float16 [ctx][n_kv][d],
    returns (out, new k row, new v row)."""
    G = n_heads // n_kv
    q = qkv[: n_heads * d].reshape(n_heads, d)
    k = qkv[n_heads * d: n_heads * d + n_kv * d].reshape(n_kv, d)
    v = qkv[n_heads * d + n_kv * d:].reshape(n_kv, d)
    kc, vc = kc.copy(), vc.copy()
    kc[pos] = f16(np.stack([np_rope(k[j], pos, inv_freq) for j in range(n_kv)]))
    vc[pos] = f16(v)
    K = kc[: pos + 1].astype(np.float64)
    V = vc[: pos + 1].astype(np.float64)
    out = np.zeros((n_heads, d))
    for h in range(n_heads):
        qr = np_rope(q[h], pos, inv_freq)
        s = K[:, h // G, :] @ qr / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[:, h // G, :]
    return out.ravel(), kc[pos], vc[pos]


def rand_cache(rng, ctx, n_kv, d):
    return (rng.standard_normal((ctx, n_kv, d)).astype(np.float16),
            rng.standard_normal((ctx, n_kv, d)).astype(np.float16))


def test_rope_inv_freq(orc):
    for base, d in ((10000.0, 128), (500000.0, 128), (10000.0, 64)):
        f = orc.rope_inv_freq(base, d)
        ref = 1.0 / np.power(base, 2.0 * np.arange(d // 2) / d)
        assert f[0] == 1.0
        assert np.max(np.abs(f / ref - 1)) < 2e-6


def test_attention_pos0_is_v(orc):
    # one position: softmax weight 1, out = the (f16) new v of the head's group
    n_heads, n_kv, d = 8, 2, 64
    rng = np.random.default_rng(1)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * d)
    kc, vc = np.zeros((4, n_kv, d), np.uint16), np.zeros((4, n_kv, d), np.uint16)
    out = orc.attention_decode_f64(qkv, kc, vc, 0, n_heads, n_kv, d, orc.rope_inv_freq(1e4, d))
    v = qkv[(n_heads + n_kv) * d:].reshape(n_kv, d)
    for h in range(n_heads):
        assert np.array_equal(out[h * d:(h + 1) * d], f16(v[h // 4]).astype(np.float64))
    assert np.array_equal(vc[0].view(np.float16), f16(v))


def test_attention_zero_query_averages_v_and_groups(orc):
    # q = 0: equal scores, out = mean of V over positions 0..pos of the head's
    # KV group; KV head of query head h is h // (n_heads / n_kv)
    n_heads, n_kv, d, pos = 4, 2, 64, 9
    qkv = np.zeros((n_heads + 2 * n_kv) * d)
    qkv[(n_heads + n_kv) * d:] = np.repeat([1.0, 2.0], d)      # new v: group 0 -> 1, group 1 -> 2
    kc = np.zeros((16, n_kv, d), np.float16)
    vc = np.zeros((16, n_kv, d), np.float16)
    vc[:pos, 0, :] = 1.0
    vc[:pos, 1, :] = 2.0
    kc, vc = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    out = orc.attention_decode_f64(qkv, kc, vc, pos, n_heads, n_kv, d, orc.rope_inv_freq(1e4, d))
    assert np.all(out[: 2 * d] == 1.0) and np.all(out[2 * d:] == 2.0)


def test_attention_rope_pairing_closed_form(orc):
    # pos 1, cached key k_0 = e_{d/2}, new key 0, v_0 = 1, v_1 = 0, q = a e_0:
    # rotated q = a (cos 1 e_0 + sin 1 e_{d/2}) (pairs (i, i + d/2), inv_freq[0] = 1),
    # so s_0 = a sin(1) / sqrt(d), s_1 = 0 and out = e^{s_0} / (e^{s_0} + 1).
    d, a = 64, 3.0
    qkv = np.zeros(3 * d)
    qkv[0] = a
    kc = np.zeros((2, 1, d), np.float16)
    vc = np.zeros((2, 1, d), np.float16)
    kc[0, 0, d // 2] = 1.0
    vc[0, 0, :] = 1.0
    kc, vc = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    out = orc.attention_decode_f64(qkv, kc, vc, 1, 1, 1, d, orc.rope_inv_freq(1e4, d))
    s0 = a * np.sin(np.float64(np.float32(1.0))) / np.sqrt(d)
    assert np.allclose(out, np.exp(s0) / (np.exp(s0) + 1.0), rtol=1e-14)


@pytest.mark.parametrize("n_heads,n_kv,d,pos", [(4, 4, 64, 5), (8, 2, 64, 37), (32, 8, 128, 130)])
def test_attention_matches_numpy(orc, n_heads, n_kv, d, pos):
    rng = np.random.default_rng(pos)
    inv = orc.rope_inv_freq(500000.0, d)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * d)
    kc, vc = rand_cache(rng, pos + 3, n_kv, d)
    ref, krow, vrow = np_attention(qkv, kc, vc, pos, n_heads, n_kv, d, inv)
    kb, vb = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    out = orc.attention_decode_f64(qkv, kb, vb, pos, n_heads, n_kv, d, inv)
    assert np.max(np.abs(out - ref)) < 1e-12
    assert np.array_equal(kb[pos], krow.view(np.uint16)) and np.array_equal(vb[pos], vrow.view(np.uint16))
    assert np.array_equal(kb[:pos], kc[:pos].view(np.uint16))   # rows before pos untouched


def np_rms(x, g, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * g.astype(np.float64)


def small_layer(t, hidden, n_heads, n_kv, d, n_ff, seed):
    w = lambda n, k, s: synth.quantized_weight(t, n, k, seed=seed * 10 + s)
    rng = np.random.default_rng(seed)
    return {
        "wq": w(n_heads * d, hidden, 1), "wk": w(n_kv * d, hidden, 2), "wv": w(n_kv * d, hidden, 3),
        "wo": w(hidden, n_heads * d, 4), "w_gate": w(n_ff, hidden, 5), "w_up": w(n_ff, hidden, 6),
        "w_down": w(hidden, n_ff, 7),
        "attn_norm": (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
        "ffn_norm": (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
    }


PROJ = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def np_dequant_any(t, blocks, n):
    if t == Q4_K:
        return np_q4_k(blocks)[:n]
    if t == Q6_K:
        return np_q6_k(blocks)[:n]
    return np_dequant(t, blocks, n)


def np_layer(t, L, dims, inv, kc, vc, pos, x):
    """t: one block type, or a dict of types per projection."""
    hidden, n_heads, n_kv, d, n_ff, eps = dims
    ty = t if isinstance(t, dict) else {name: t for name in PROJ}
    dq = lambda name, n, k: np_dequant_any(ty[name], L[name], n * k).astype(np.float64).reshape(n, k)
    xn = np_rms(x, L["attn_norm"], eps)
    qkv = np.concatenate([dq("wq", n_heads * d, hidden) @ xn, dq("wk", n_kv * d, hidden) @ xn,
                          dq("wv", n_kv * d, hidden) @ xn])
    att, krow, vrow = np_attention(qkv, kc, vc, pos, n_heads, n_kv, d, inv)
    x = x + dq("wo", hidden, n_heads * d) @ att
    xn = np_rms(x, L["ffn_norm"], eps)
    g = dq("w_gate", n_ff, hidden) @ xn
    u = dq("w_up", n_ff, hidden) @ xn
    h = g * (1.0 / (1.0 + np.exp(-g))) * u
    return x + dq("w_down", hidden, n_ff) @ h, krow, vrow


@pytest.mark.parametrize("t", [Q4_0, Q8_0])
def test_layer_matches_numpy(orc, t):
    hidden, n_heads, n_kv, d, n_ff, pos = 256, 4, 2, 64, 512, 6
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    L = small_layer(t, hidden, n_heads, n_kv, d, n_ff, seed=3)
    inv = orc.rope_inv_freq(10000.0, d)
    rng = np.random.default_rng(4)
    kc, vc = rand_cache(rng, 8, n_kv, d)
    x = rng.standard_normal(hidden)
    ref, krow, vrow = np_layer(t, L, dims, inv, kc, vc, pos, x)
    kb, vb = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    got = orc.llama_layer_decode_f64(t, L, dims, inv, kb, vb, pos, x)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-12
    assert np.array_equal(kb[pos], krow.view(np.uint16))


# the tensor types of a Q4_K_M file: attn_v and ffn_down in Q6_K, the rest Q4_K
MIXED = {"wq": Q4_K, "wk": Q4_K, "wv": Q6_K, "wo": Q4_K, "w_gate": Q4_K, "w_up": Q4_K, "w_down": Q6_K}


def mixed_layer(types, hidden, n_heads, n_kv, d, n_ff, seed):
    shapes = {"wq": (n_heads * d, hidden), "wk": (n_kv * d, hidden), "wv": (n_kv * d, hidden),
              "wo": (hidden, n_heads * d), "w_gate": (n_ff, hidden), "w_up": (n_ff, hidden),
              "w_down": (hidden, n_ff)}
    rng = np.random.default_rng(seed)
    L = {name: synth.quantized_weight(types[name], *shapes[name], seed=seed * 10 + i)
         for i, name in enumerate(PROJ)}
    L["attn_norm"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    L["ffn_norm"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    return L


def test_layer_mixed_types_matches_numpy(orc):
    """A block type per projection (orc_llama_layer_decode_types_f64) against
    the numpy layer over each tensor's own dequantization."""
    hidden, n_heads, n_kv, d, n_ff, pos = 512, 4, 2, 128, 768, 5
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    L = mixed_layer(MIXED, hidden, n_heads, n_kv, d, n_ff, seed=9)
    inv = orc.rope_inv_freq(500000.0, d)
    rng = np.random.default_rng(10)
    kc, vc = rand_cache(rng, 8, n_kv, d)
    x = rng.standard_normal(hidden)
    ref, krow, vrow = np_layer(MIXED, L, dims, inv, kc, vc, pos, x)
    kb, vb = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    got = orc.llama_layer_decode_f64([MIXED[n] for n in PROJ], L, dims, inv, kb, vb, pos, x)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-12
    assert np.array_equal(vb[pos], vrow.view(np.uint16))
    # each projection is read with its own type: v's Q6_K bytes read as Q4_K differ
    wrong = dict(MIXED, wv=Q4_K)
    bad = orc.llama_layer_decode_f64([wrong[n] for n in PROJ], L, dims, inv, kc.view(np.uint16).copy(),
                                     vc.view(np.uint16).copy(), pos, x)
    assert not np.allclose(bad, ref, rtol=1e-3, atol=1e-3)


def test_output_head_matches_numpy(orc):
    hidden, vocab = 256, 300
    w = synth.quantized_weight(Q8_0, vocab, hidden, seed=8)
    g = np.linspace(0.5, 1.5, hidden).astype(np.float32)
    x = np.random.default_rng(9).standard_normal(hidden)
    ref = np_dequant(Q8_0, w, vocab * hidden).astype(np.float64).reshape(vocab, hidden) @ np_rms(x, g, 1e-5)
    got = orc.output_head_f64(Q8_0, w, g, 1e-5, x, hidden, vocab)
    assert np.max(np.abs(got - ref)) < 1e-9


def test_attention_store_new_false_uses_given_row(orc):
    # store_new = False: row pos already in the caches is attended to as is
    n_heads, n_kv, d, pos = 4, 2, 64, 5
    rng = np.random.default_rng(12)
    inv = orc.rope_inv_freq(1e4, d)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * d)
    kc, vc = rand_cache(rng, 8, n_kv, d)
    kb, vb = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    out = orc.attention_decode_f64(qkv, kb, vb, pos, n_heads, n_kv, d, inv, store_new=False)
    assert np.array_equal(kb, kc.view(np.uint16)) and np.array_equal(vb, vc.view(np.uint16))
    G = n_heads // n_kv
    q = qkv[: n_heads * d].reshape(n_heads, d)
    K, V = kc[: pos + 1].astype(np.float64), vc[: pos + 1].astype(np.float64)
    ref = []
    for h in range(n_heads):
        s_ = K[:, h // G] @ np_rope(q[h], pos, inv) / np.sqrt(d)
        w = np.exp(s_ - s_.max())
        ref.append((w / w.sum()) @ V[:, h // G])
    assert np.max(np.abs(out - np.concatenate(ref))) < 1e-12


@pytest.mark.parametrize("t", [Q4_0, Q8_0])
def test_layer_f32_order_close_to_f64(orc, t):
    # the reference-order f32 layer: same computation, f32 rounding only
    hidden, n_heads, n_kv, d, n_ff, pos = 256, 4, 2, 64, 512, 6
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    L = small_layer(t, hidden, n_heads, n_kv, d, n_ff, seed=5)
    inv = orc.rope_inv_freq(10000.0, d)
    rng = np.random.default_rng(6)
    kc, vc = rand_cache(rng, 8, n_kv, d)
    x = rng.standard_normal(hidden).astype(np.float32)
    k64, v64 = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    k32, v32 = kc.view(np.uint16).copy(), vc.view(np.uint16).copy()
    ref = orc.llama_layer_decode_f64(t, L, dims, inv, k64, v64, pos, x.astype(np.float64))
    got = orc.llama_layer_decode_f32(t, L, dims, inv, k32, v32, pos, x)
    assert np.sqrt(np.sum((got - ref) ** 2) / np.sum(ref ** 2)) < 1e-5
    # the stored rows agree to one f16 rounding step
    a, b = k32[pos].view(np.float16).astype(np.float64), k64[pos].view(np.float16).astype(np.float64)
    assert np.all(np.abs(a - b) <= np.spacing(np.abs(b).astype(np.float16)).astype(np.float64))
