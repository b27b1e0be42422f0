"""GPU decode step (config 4 pieces) against the f64 oracle: fused RMSNorm +
Q/K/V projection, single-token GQA attention over an f16 KV cache with RoPE,
residual projections, one layer, several steps and the whole step with the
output head.  Bars: rel-L2 <= 1e-4 and max-abs <= 1e-3 of the f64 oracle
(north_star) for projections, attention and logits; hidden states (residual
sums, RMS up to ~2e4 here, where one f32 ulp of the largest elements exceeds
1e-3) to max-abs <= 1e-3 per 300 of their RMS; cache rows written by the step
within one f16 ulp of the oracle's."""
import numpy as np
import pytest

from tests._gpu import down, report, up
from tests._oracle import max_abs, rel_l2
from tests.test_oracle_decode import MIXED, PROJ, mixed_layer, small_layer
from woolly_amd import ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14
REL_L2 = 1e-4


def hidden_bar(ref) -> float:
    """max-abs bar of a hidden state (a residual sum): 1e-3 per 300 of its RMS,
    the rule the FFN tests apply to outputs larger than config 3's (RMS ~ 300);
    1e-3 for anything smaller.  Logits and projections use 1e-3 itself."""
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    return 1e-3 * max(1.0, rms / 300.0)


def check(got, ref, tag, abs_bar=1e-3):
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(tag, r, a, ref, abs_bar=float(abs_bar))
    assert r <= REL_L2 and a <= abs_bar, (tag, r, a)


def f16_ulp_close(got_bits, ref_bits, slack=0.0):
    """Cache rows: within one f16 ulp, plus `slack` x the row's largest
    magnitude for rows computed from activations that already differ
    upstream (a later layer)."""
    g = got_bits.view(np.float16).astype(np.float64)
    r = ref_bits.view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float64)
    return np.all(np.abs(g - r) <= ulp + slack * np.max(np.abs(r)))


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_1])
@pytest.mark.parametrize("hidden,q_rows,kv_rows", [(4096, 4096, 1024), (256, 256, 128), (512, 384, 64)])
def test_attention_qkv_fused(gpu, orc, t, hidden, q_rows, kv_rows):
    print(f"[case] qkv t={t} hidden={hidden} q={q_rows} kv={kv_rows}", flush=True)
    wq = synth.quantized_weight(t, q_rows, hidden, seed=1)
    wk = synth.quantized_weight(t, kv_rows, hidden, seed=2)
    wv = synth.quantized_weight(t, kv_rows, hidden, seed=3)
    x = synth.activations(hidden, seed=4)
    g = (1 + 0.1 * np.random.default_rng(5).standard_normal(hidden)).astype(np.float32)
    bufs = [up(a)[0] for a in (wq, wk, wv, x, g)]
    out = DeviceBuffer(4 * (q_rows + 2 * kv_rows))
    ws = DeviceBuffer(ops.attention_qkv_workspace_bytes(hidden))
    ops.attention_qkv(t, *bufs[:3], q_rows, kv_rows, hidden, bufs[4], 1e-5, bufs[3], out, ws,
                      ops.attention_qkv_workspace_bytes(hidden))
    got = down(out, np.float32, q_rows + 2 * kv_rows)
    xn = np.zeros((1, hidden))
    orc.lib.orc_rms_norm_f64(x.ctypes.data, g.ctypes.data, 1e-5, 1, hidden, xn.ctypes.data)
    xn32 = xn.astype(np.float32).ravel()
    ref = np.concatenate([orc.matvec_f64(t, w, xn32, n, hidden)[1]
                          for w, n in ((wq, q_rows), (wk, kv_rows), (wv, kv_rows))])
    # the oracle's f64 x_hat rounded to f32 for its input: a 2^-24 relative
    # perturbation, far inside the bar
    check(got, ref, f"qkv t={t} {hidden}")


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_attention_qkv_nonfinite(gpu, orc, bad):
    """One inf or NaN in x: rms_norm's rms is then inf or NaN, x_hat is NaN at
    that element (inf / inf, NaN) and 0 or NaN elsewhere, so every projection
    is NaN in the reference (tensor_utils.rs:446-480 followed by the matvec);
    the fused kernel (W (x * gamma)) / rms gives NaN everywhere as well.  A
    finite x whose squares overflow (rms = inf) gives x_hat = 0 and zeros."""
    hidden, q_rows, kv_rows = 4096, 4096, 1024
    print(f"[case] qkv nonfinite {bad}", flush=True)
    ws = [synth.quantized_weight(Q4_0, n, hidden, seed=30 + i) for i, n in enumerate((q_rows, kv_rows, kv_rows))]
    g = (1 + 0.1 * np.random.default_rng(5).standard_normal(hidden)).astype(np.float32)
    wb = [up(w)[0] for w in ws]
    gb = up(g)[0]
    out = DeviceBuffer(4 * (q_rows + 2 * kv_rows))
    wsb = DeviceBuffer(ops.attention_qkv_workspace_bytes(hidden))
    x = synth.activations(hidden, seed=6)
    x[1234] = bad
    ops.attention_qkv(Q4_0, *wb, q_rows, kv_rows, hidden, gb, 1e-5, up(x)[0], out, wsb,
                      ops.attention_qkv_workspace_bytes(hidden))
    got = down(out, np.float32, q_rows + 2 * kv_rows)
    xn = np.zeros((1, hidden))
    orc.lib.orc_rms_norm_f64(x.ctypes.data, g.ctypes.data, 1e-5, 1, hidden, xn.ctypes.data)
    ref = np.concatenate([orc.matvec_f64(Q4_0, w, xn.astype(np.float32).ravel(), n, hidden)[1]
                          for w, n in zip(ws, (q_rows, kv_rows, kv_rows))])
    assert np.all(np.isnan(ref)) and np.all(np.isnan(got))
    # squares that overflow f32 (|x| ~ 1e30): rms = inf in f32, x_hat = 0
    big = (synth.activations(hidden, seed=7) * np.float32(1e30)).astype(np.float32)
    ops.attention_qkv(Q4_0, *wb, q_rows, kv_rows, hidden, gb, 1e-5, up(big)[0], out, wsb,
                      ops.attention_qkv_workspace_bytes(hidden))
    got = down(out, np.float32, q_rows + 2 * kv_rows)
    assert np.all(got == 0.0)


@pytest.mark.parametrize("t", [Q4_0, Q8_0])
@pytest.mark.parametrize("m,k", [(4096, 4096), (4096, 14336), (300, 96)])
def test_matvec_residual_in_place(gpu, orc, t, m, k):
    w = synth.quantized_weight(t, m, k, seed=m + k)
    x = synth.activations(k, seed=7)
    r = synth.activations(m, seed=8) * 10
    wb, xb, rb = up(w)[0], up(x)[0], up(r)[0]
    ops.quantized_matvec_residual(t, wb, w.nbytes, xb, rb, rb, m, k)   # in place
    got = down(rb, np.float32, m)
    ref = r.astype(np.float64) + orc.matvec_f64(t, w, x, m, k)[1]
    check(got, ref, f"residual t={t} {m}x{k}")


# (8, 1, 128) at 8191: 128 chunks per head, so each combine lane merges two load batches
@pytest.mark.parametrize("n_heads,n_kv,d,pos", [(n, k, d, p) for (n, k, d) in
                                                ((32, 8, 128), (8, 2, 64), (4, 4, 64), (16, 2, 128), (8, 1, 128))
                                                for p in (0, 1, 63, 64, 200, 1000, 4095, 8191)] +
                         # long contexts with 8 KV heads: 192- and 256-position chunks
                         [(32, 8, 128, 12000), (32, 8, 128, 40000), (32, 8, 128, 64319), (16, 8, 64, 20000)])
def test_attention_decode(gpu, orc, n_heads, n_kv, d, pos):
    print(f"[case] attention heads={n_heads}/{n_kv} d={d} pos={pos}", flush=True)
    rng = np.random.default_rng(pos + d)
    ctx = max(4096, pos + 1)
    inv = orc.rope_inv_freq(500000.0, d)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * d).astype(np.float32)
    kc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
    kcb, vcb = up(kc)[0], up(vc)[0]
    qb, fb = up(qkv)[0], up(inv)[0]
    out = DeviceBuffer(4 * n_heads * d)
    wsz = ops.attention_workspace_bytes(n_heads, n_kv, d, ctx)
    ws = DeviceBuffer(wsz)
    ops.attention_decode(qb, kcb, vcb, pos, n_heads, n_kv, d, fb, out, ws, wsz)
    got = down(out, np.float32, n_heads * d)
    kg = down(kcb, np.uint16, kc.size).reshape(kc.shape)
    vg = down(vcb, np.uint16, vc.size).reshape(vc.shape)
    # the stored row: within one f16 ulp of the oracle's own rounding (v exact)
    kr, vr = kc.copy(), vc.copy()
    orc.attention_decode_f64(qkv.astype(np.float64), kr, vr, pos, n_heads, n_kv, d, inv)
    assert f16_ulp_close(kg[pos], kr[pos]) and np.array_equal(vg[pos], vr[pos])
    # the output, attending to the stored row (an f16 rounding flip of the new
    # k is not an arithmetic difference)
    ref = orc.attention_decode_f64(qkv.astype(np.float64), kg.copy(), vg.copy(), pos, n_heads, n_kv, d, inv,
                                   store_new=False)
    check(got, ref, f"attn {n_heads}/{n_kv} d={d} pos={pos}")
    # every other cache row untouched
    assert np.array_equal(np.delete(kg, pos, 0), np.delete(kc, pos, 0))
    assert np.array_equal(np.delete(vg, pos, 0), np.delete(vc, pos, 0))


def upload_layer(t, L, ctx, n_kv, d, rng):
    dev = {k: up(v)[0] for k, v in L.items()}
    kc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
    dev["k_cache"], dev["v_cache"] = up(kc)[0], up(vc)[0]
    return dev, kc, vc


@pytest.mark.parametrize("t", [Q4_0, Q8_0])
def test_layers_and_steps_small_model(gpu, orc, t):
    """Two layers and a Q8_0 head, six consecutive steps (positions 0..5) on
    empty caches, against the f64 oracle stepping the same model."""
    hidden, n_heads, n_kv, d, n_ff, vocab, ctx = 256, 4, 2, 64, 512, 300, 16
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    rng = np.random.default_rng(0)
    Ls = [small_layer(t, hidden, n_heads, n_kv, d, n_ff, seed=20 + i) for i in range(2)]
    devs, caches = [], []
    for L in Ls:
        dev, kc, vc = upload_layer(t, L, ctx, n_kv, d, rng)
        kc[:] = 0
        vc[:] = 0
        dev["k_cache"].upload(kc)
        dev["v_cache"].upload(vc)
        devs.append(dev)
        caches.append((kc, vc))
    inv = orc.rope_inv_freq(10000.0, d)
    head = synth.quantized_weight(Q8_0, vocab, hidden, seed=30)
    onorm = np.linspace(0.8, 1.2, hidden).astype(np.float32)
    model = ops.LlamaModel(t, dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff,
                                   max_ctx=ctx, vocab=vocab, eps=1e-5),
                           devs, up(inv)[0], up(onorm)[0], up(head)[0], Q8_0)
    ws = DeviceBuffer(model.workspace_bytes())
    xb, lb = DeviceBuffer(4 * hidden), DeviceBuffer(4 * vocab)
    for pos in range(6):
        x0 = synth.activations(hidden, seed=100 + pos)
        xb.upload(x0)
        model.decode_step(pos, xb, lb, ws, model.workspace_bytes())
        got_x = down(xb, np.float32, hidden)
        got_l = down(lb, np.float32, vocab)
        gcache = [(down(dv["k_cache"], np.uint16, kc.size).reshape(kc.shape),
                   down(dv["v_cache"], np.uint16, vc.size).reshape(vc.shape)) for dv, (kc, vc) in zip(devs, caches)]
        # rows stored at pos: within one f16 ulp of the oracle's own (its
        # caches hold the GPU's earlier rows, carried over below)
        x = x0.astype(np.float64)
        for li, (L, (kc, vc), (kg, vg)) in enumerate(zip(Ls, caches, gcache)):
            x = orc.llama_layer_decode_f64(t, L, dims, inv, kc, vc, pos, x)
            slack = 0.0 if li == 0 else 1e-4   # later layers: inputs differ by earlier rows' rounding
            assert f16_ulp_close(kg[pos], kc[pos], slack) and f16_ulp_close(vg[pos], vc[pos], slack), (pos, li)
        # the comparison run attends to the GPU's stored rows
        x = x0.astype(np.float64)
        for L, (kg, vg) in zip(Ls, gcache):
            x = orc.llama_layer_decode_f64(t, L, dims, inv, kg.copy(), vg.copy(), pos, x, store_new=False)
        logits = orc.output_head_f64(Q8_0, head, onorm, 1e-5, x, hidden, vocab)
        print(f"[info] step pos={pos} max|x|={np.max(np.abs(x)):.3e} max|logits|={np.max(np.abs(logits)):.3e}",
              flush=True)
        check(got_x, x, f"step t={t} pos={pos} hidden", abs_bar=hidden_bar(x))
        check(got_l, logits, f"step t={t} pos={pos} logits", abs_bar=1e-3)
        for (kc, vc), (kg, vg) in zip(caches, gcache):
            kc[:] = kg
            vc[:] = vg


def test_layer_llama3_8b_shape_ctx4096(gpu, orc):
    """Config 4 at one layer: Llama-3-8B shapes (4096 hidden, 32/8 heads of 128,
    n_ff 14336, Q4_0), position 4095 over a cache filled ~N(0,1)."""
    hidden, n_heads, n_kv, d, n_ff, ctx, pos = 4096, 32, 8, 128, 14336, 4096, 4095
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    rng = np.random.default_rng(6)
    L = small_layer(Q4_0, hidden, n_heads, n_kv, d, n_ff, seed=6)
    dev, kc, vc = upload_layer(Q4_0, L, ctx, n_kv, d, rng)
    inv = orc.rope_inv_freq(500000.0, d)
    model = ops.LlamaModel(Q4_0, dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d,
                                      n_ff=n_ff, max_ctx=ctx, vocab=0, eps=1e-5),
                           [dev], up(inv)[0])
    ws = DeviceBuffer(model.workspace_bytes())
    x0 = synth.activations(hidden, seed=7)
    xb = up(x0)[0]
    model.layer_decode(0, pos, xb, ws, model.workspace_bytes())
    got = down(xb, np.float32, hidden)
    kg = down(dev["k_cache"], np.uint16, kc.size).reshape(kc.shape)
    vg = down(dev["v_cache"], np.uint16, vc.size).reshape(vc.shape)
    kr, vr = kc.copy(), vc.copy()
    orc.llama_layer_decode_f64(Q4_0, L, dims, inv, kr, vr, pos, x0.astype(np.float64))
    assert f16_ulp_close(kg[pos], kr[pos]) and f16_ulp_close(vg[pos], vr[pos])
    assert np.array_equal(kg[:pos], kc[:pos]) and np.array_equal(vg[:pos], vc[:pos])
    ref = orc.llama_layer_decode_f64(Q4_0, L, dims, inv, kg.copy(), vg.copy(), pos, x0.astype(np.float64),
                                     store_new=False)
    err = np.abs(got - ref)
    i = int(np.argmax(err))
    print(f"[info] layer 8B: rms(ref)={np.sqrt(np.mean(ref ** 2)):.3e} max|ref|={np.max(np.abs(ref)):.3e} "
          f"worst element {i}: ref={ref[i]:.6e} got={got[i]:.6e} err={err[i]:.3e} "
          f"(f32 ulp there {np.spacing(np.float32(abs(ref[i]))):.3e}); "
          f"99.9th pct err={np.percentile(err, 99.9):.3e}", flush=True)
    # the reference's own f32 evaluation order on the same input (same stored rows)
    ref32 = orc.llama_layer_decode_f32(Q4_0, L, dims, inv, kg.copy(), vg.copy(), pos, x0, store_new=False)
    ref32_err = max_abs(ref32, ref)
    print(f"[info] layer 8B: reference-order f32 vs f64 max_abs={ref32_err:.3e} rel_l2={rel_l2(ref32, ref):.3e}; "
          f"GPU vs reference-order f32 max_abs={max_abs(got, ref32):.3e}", flush=True)
    # bar: rel-L2 1e-4 and the hidden-state max-abs rule (the reference's own
    # f32 order is several times further from f64 on this input: ref32_err)
    check(got, ref, "layer 8B ctx4096", abs_bar=hidden_bar(ref))


# K-quant models: every matrix Q4_K, every matrix Q6_K, or the per-tensor mix of
# a Q4_K_M file (attn_v and ffn_down Q6_K); the model's type is Q4_K and the
# layers name their own types where they differ
KQ_MODELS = {"q4_k": {n: Q4_K for n in PROJ}, "q6_k": {n: Q6_K for n in PROJ}, "q4_k_m": MIXED}


def kq_model(types, dims, ctx, vocab, inv, n_layers, head, onorm, rng, seed):
    hidden, n_heads, n_kv, d, n_ff, _ = dims
    Ls, devs, caches = [], [], []
    for i in range(n_layers):
        L = mixed_layer(types, hidden, n_heads, n_kv, d, n_ff, seed=seed + i)
        dev, kc, vc = upload_layer(None, L, ctx, n_kv, d, rng)
        for name in PROJ:
            dev[name + "_type"] = types[name] if types[name] != Q4_K else 0   # 0: the model's type
        Ls.append(L)
        devs.append(dev)
        caches.append((kc, vc))
    model = ops.LlamaModel(Q4_K, dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff,
                                      max_ctx=ctx, vocab=vocab, eps=1e-5),
                           devs, up(inv)[0], up(onorm)[0] if onorm is not None else None,
                           up(head)[0] if head is not None else None, Q6_K)
    return model, Ls, devs, caches


@pytest.mark.parametrize("kind", list(KQ_MODELS))
def test_kquant_model_steps(gpu, orc, kind):
    """Two K-quant layers and a Q6_K head, three steps on ~N(0,1) caches,
    against the f64 oracle with each tensor's own type."""
    types = KQ_MODELS[kind]
    tl = [types[n] for n in PROJ]
    hidden, n_heads, n_kv, d, n_ff, vocab, ctx = 512, 4, 2, 128, 768, 300, 8
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    rng = np.random.default_rng(1)
    inv = orc.rope_inv_freq(500000.0, d)
    head = synth.quantized_weight(Q6_K, vocab, hidden, seed=40)
    onorm = np.linspace(0.8, 1.2, hidden).astype(np.float32)
    model, Ls, devs, caches = kq_model(types, dims, ctx, vocab, inv, 2, head, onorm, rng, seed=50)
    ws = DeviceBuffer(model.workspace_bytes())
    xb, lb = DeviceBuffer(4 * hidden), DeviceBuffer(4 * vocab)
    for pos in range(3):
        print(f"[case] kquant model {kind} pos={pos}", flush=True)
        x0 = synth.activations(hidden, seed=200 + pos)
        xb.upload(x0)
        model.decode_step(pos, xb, lb, ws, model.workspace_bytes())
        got_x = down(xb, np.float32, hidden)
        got_l = down(lb, np.float32, vocab)
        gcache = [(down(dv["k_cache"], np.uint16, kc.size).reshape(kc.shape),
                   down(dv["v_cache"], np.uint16, vc.size).reshape(vc.shape)) for dv, (kc, vc) in zip(devs, caches)]
        x = x0.astype(np.float64)
        for li, (L, (kc, vc), (kg, vg)) in enumerate(zip(Ls, caches, gcache)):
            x = orc.llama_layer_decode_f64(tl, L, dims, inv, kc, vc, pos, x)
            slack = 0.0 if li == 0 else 1e-4
            assert f16_ulp_close(kg[pos], kc[pos], slack) and f16_ulp_close(vg[pos], vc[pos], slack), (pos, li)
        x = x0.astype(np.float64)
        for L, (kg, vg) in zip(Ls, gcache):
            x = orc.llama_layer_decode_f64(tl, L, dims, inv, kg.copy(), vg.copy(), pos, x, store_new=False)
        logits = orc.output_head_f64(Q6_K, head, onorm, 1e-5, x, hidden, vocab)
        check(got_x, x, f"kquant {kind} pos={pos} hidden", abs_bar=hidden_bar(x))
        check(got_l, logits, f"kquant {kind} pos={pos} logits", abs_bar=1e-3)
        for (kc, vc), (kg, vg) in zip(caches, gcache):
            kc[:] = kg
            vc[:] = vg


def test_kquant_m_layer_llama3_8b_shape(gpu, orc):
    """One Llama-3-8B-shaped layer with Q4_K_M's per-tensor types at position
    1000: the matrix-core GEMVs on K-quants with RMSNorm, residual and the
    fused gate/up + SwiGLU, q / k / v as separate GEMVs (v is Q6_K)."""
    hidden, n_heads, n_kv, d, n_ff, ctx, pos = 4096, 32, 8, 128, 14336, 1024, 1000
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    rng = np.random.default_rng(8)
    inv = orc.rope_inv_freq(500000.0, d)
    model, Ls, devs, caches = kq_model(MIXED, dims, ctx, 0, inv, 1, None, None, rng, seed=60)
    ws = DeviceBuffer(model.workspace_bytes())
    x0 = synth.activations(hidden, seed=9)
    xb = up(x0)[0]
    model.layer_decode(0, pos, xb, ws, model.workspace_bytes())
    got = down(xb, np.float32, hidden)
    kc, vc = caches[0]
    kg = down(devs[0]["k_cache"], np.uint16, kc.size).reshape(kc.shape)
    vg = down(devs[0]["v_cache"], np.uint16, vc.size).reshape(vc.shape)
    tl = [MIXED[n] for n in PROJ]
    kr, vr = kc.copy(), vc.copy()
    orc.llama_layer_decode_f64(tl, Ls[0], dims, inv, kr, vr, pos, x0.astype(np.float64))
    assert f16_ulp_close(kg[pos], kr[pos]) and f16_ulp_close(vg[pos], vr[pos])
    ref = orc.llama_layer_decode_f64(tl, Ls[0], dims, inv, kg.copy(), vg.copy(), pos, x0.astype(np.float64),
                                     store_new=False)
    check(got, ref, "kquant q4_k_m layer 8B", abs_bar=hidden_bar(ref))


def test_llama_model_from_gguf_q4_k_m(gpu, orc, tmp_path):
    """A two-layer Q4_K_M-typed model written as a GGUF file (llama.* metadata,
    blk.N.* tensors, Q6_K output head), loaded with LlamaModel.from_gguf and
    stepped three times from empty caches, against the f64 oracle."""
    from tests.test_gguf import MockGGUFBuilder, load
    from woolly_amd.gguf import GGMLType, MetadataValueType as VT

    hidden, n_heads, n_kv, d, n_ff, vocab, ctx = 512, 4, 2, 128, 768, 300, 8
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    Ls = [mixed_layer(MIXED, hidden, n_heads, n_kv, d, n_ff, seed=70 + i) for i in range(2)]
    head = synth.quantized_weight(Q6_K, vocab, hidden, seed=72)
    onorm = np.linspace(0.9, 1.1, hidden).astype(np.float32)
    b = MockGGUFBuilder().add_metadata("general.architecture", VT.String, "llama")
    for key, vt, v in (("embedding_length", VT.UInt32, hidden), ("block_count", VT.UInt32, 2),
                       ("attention.head_count", VT.UInt32, n_heads), ("attention.head_count_kv", VT.UInt32, n_kv),
                       ("feed_forward_length", VT.UInt32, n_ff), ("context_length", VT.UInt32, ctx),
                       ("rope.freq_base", VT.Float32, 500000.0), ("attention.layer_norm_epsilon", VT.Float32, 1e-5)):
        b.add_metadata("llama." + key, vt, v)
    gnames = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "w_gate": "ffn_gate",
              "w_up": "ffn_up", "w_down": "ffn_down"}
    shapes = {"wq": (n_heads * d, hidden), "wk": (n_kv * d, hidden), "wv": (n_kv * d, hidden),
              "wo": (hidden, n_heads * d), "w_gate": (n_ff, hidden), "w_up": (n_ff, hidden), "w_down": (hidden, n_ff)}
    for i, L in enumerate(Ls):
        b.add_tensor(f"blk.{i}.attn_norm.weight", [hidden], GGMLType.F32, L["attn_norm"].tobytes())
        b.add_tensor(f"blk.{i}.ffn_norm.weight", [hidden], GGMLType.F32, L["ffn_norm"].tobytes())
        for key, nm in gnames.items():
            n, k = shapes[key]
            b.add_tensor(f"blk.{i}.{nm}.weight", [k, n], GGMLType(MIXED[key]), L[key].tobytes())
    b.add_tensor("output_norm.weight", [hidden], GGMLType.F32, onorm.tobytes())
    b.add_tensor("output.weight", [hidden, vocab], GGMLType.Q6_K, head.tobytes())
    ld = load(b.build(), tmp_path)
    model = ops.LlamaModel.from_gguf(ld)
    assert model.dims == dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff, max_ctx=ctx,
                              vocab=vocab, eps=float(np.float32(1e-5)))
    ws = DeviceBuffer(model.workspace_bytes())
    xb, lb = DeviceBuffer(4 * hidden), DeviceBuffer(4 * vocab)
    tl = [MIXED[n] for n in PROJ]
    inv = orc.rope_inv_freq(500000.0, d)
    caches = [(np.zeros((ctx, n_kv, d), np.uint16), np.zeros((ctx, n_kv, d), np.uint16)) for _ in Ls]
    for pos in range(3):
        print(f"[case] gguf q4_k_m model pos={pos}", flush=True)
        x0 = synth.activations(hidden, seed=300 + pos)
        xb.upload(x0)
        model.decode_step(pos, xb, lb, ws, model.workspace_bytes())
        got_x, got_l = down(xb, np.float32, hidden), down(lb, np.float32, vocab)
        x = x0.astype(np.float64)
        for L, (kc, vc) in zip(Ls, caches):
            x = orc.llama_layer_decode_f64(tl, L, dims, inv, kc, vc, pos, x)
        logits = orc.output_head_f64(Q6_K, head, onorm, 1e-5, x, hidden, vocab)
        check(got_x, x, f"gguf q4_k_m pos={pos} hidden", abs_bar=hidden_bar(x))
        check(got_l, logits, f"gguf q4_k_m pos={pos} logits", abs_bar=1e-3)


EMB_TYPES = [0, 1, Q4_0, Q4_1, 6, 7, Q8_0, Q4_K, Q6_K]  # F32, F16, the 32- and 256-element blocks


def emb_table(t, vocab, hidden, seed):
    if t == 0:
        return synth.activations(vocab * hidden, seed=seed).view(np.uint8)
    if t == 1:
        return synth.activations(vocab * hidden, seed=seed).astype(np.float16).view(np.uint8)
    return synth.quantized_weight(t, vocab, hidden, seed=seed)


@pytest.mark.parametrize("t", EMB_TYPES)
def test_embedding_lookup_bit_exact(gpu, orc, t):
    """embedding_lookup (tensor_utils.rs:548-590) on the device: every requested
    row equals the oracle's dequantization of the table, bit for bit; an id past
    the vocabulary gives a NaN row from the C ABI and ValueError from the host
    mirror, as the reference's TENSOR_EMBEDDING_TOKEN_OUT_OF_RANGE."""
    from woolly_amd import _lib

    vocab, hidden = 300, 512
    tab = emb_table(t, vocab, hidden, seed=40 + t)
    st, full = orc.dequantize(t, tab, vocab * hidden)
    assert st == 0
    full = full.reshape(vocab, hidden)
    ids = [0, 1, 299, 150, 7, 7]
    tb = up(tab)[0]
    out = DeviceBuffer(4 * len(ids) * hidden)
    keep = ops.embedding_lookup(t, tb, vocab, hidden, ids, out)
    got = down(out, np.float32, len(ids) * hidden).reshape(len(ids), hidden)
    assert np.array_equal(got.view(np.uint32), full[ids].view(np.uint32)), t
    del keep
    with pytest.raises(ValueError):
        ops.embedding_lookup(t, tb, vocab, hidden, [3, vocab], out)
    idb = up(np.array([2, vocab, 5], np.uint32))[0]
    _lib.check(_lib.load().wh_embedding_lookup(t, tb.ptr, vocab, hidden, idb.ptr, 3, out.ptr, None))
    got = down(out, np.float32, 3 * hidden).reshape(3, hidden)
    assert np.array_equal(got[0].view(np.uint32), full[2].view(np.uint32))
    assert np.all(np.isnan(got[1]))
    assert np.array_equal(got[2].view(np.uint32), full[5].view(np.uint32))


def test_forward_token_tied_head_gguf(gpu, orc, tmp_path):
    """A GGUF file without output.weight (the head tied to token_embd.weight,
    lazy_transformer.rs:1301-1316), loaded with LlamaModel.from_gguf and run
    from token ids held on the device (forward for one token, :1155-1230):
    three steps against the f64 oracle starting from the dequantized embedding
    rows, and each step equal bit for bit to decode_step on the uploaded row."""
    from tests.test_gguf import _llama_gguf, load

    hidden, n_heads, n_kv, d, n_ff, vocab = 256, 4, 2, 64, 512, 64
    ld = load(_llama_gguf(hidden, n_heads, n_kv, n_ff, vocab, output=False).build(), tmp_path)
    model = ops.LlamaModel.from_gguf(ld, max_ctx=8)
    assert model.tied_head and model.dims["vocab"] == vocab
    L = {k: np.array(ld.tensor_data(f"blk.0.{nm}.weight")) for k, nm in
         {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "w_gate": "ffn_gate",
          "w_up": "ffn_up", "w_down": "ffn_down"}.items()}
    L["attn_norm"] = L["ffn_norm"] = np.ones(hidden, np.float32)
    embd = np.array(ld.tensor_data("token_embd.weight"))
    onorm = np.ones(hidden, np.float32)
    st, rows = orc.dequantize(Q8_0, embd, vocab * hidden)
    rows = rows.reshape(vocab, hidden)
    inv = orc.rope_inv_freq(10000.0, d)
    dims = (hidden, n_heads, n_kv, d, n_ff, 1e-5)
    ws = DeviceBuffer(model.workspace_bytes())
    xb, lb, x2, l2 = DeviceBuffer(4 * hidden), DeviceBuffer(4 * vocab), DeviceBuffer(4 * hidden), DeviceBuffer(4 * vocab)
    tok = DeviceBuffer(4)
    cache_dev = model._keep[0][0]
    for pos, token in enumerate([5, 17, 63]):
        print(f"[case] forward_token tied pos={pos} token={token}", flush=True)
        tok.upload(np.array([token], np.uint32))
        # decode_step on the uploaded row first (it writes the same cache row)
        x2.upload(rows[token])
        model.decode_step(pos, x2, l2, ws, model.workspace_bytes())
        model.forward_token(tok, pos, xb, lb, ws, model.workspace_bytes())
        got_x, got_l = down(xb, np.float32, hidden), down(lb, np.float32, vocab)
        assert np.array_equal(got_x.view(np.uint32), down(x2, np.float32, hidden).view(np.uint32))
        assert np.array_equal(got_l.view(np.uint32), down(l2, np.float32, vocab).view(np.uint32))
        # the oracle attends to the rows the GPU stored (an f16 rounding flip of
        # a new k or v is not an arithmetic difference)
        kc = down(cache_dev["k_cache"], np.uint16, 8 * n_kv * d).reshape(8, n_kv, d)
        vc = down(cache_dev["v_cache"], np.uint16, 8 * n_kv * d).reshape(8, n_kv, d)
        x = orc.llama_layer_decode_f64(Q8_0, L, dims, inv, kc, vc, pos, rows[token].astype(np.float64),
                                       store_new=False)
        logits = orc.output_head_f64(Q8_0, embd, onorm, 1e-5, x, hidden, vocab)
        check(got_l, logits, f"forward_token tied head pos={pos} logits")
