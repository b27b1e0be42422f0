"""wh_llama_decode_step_noalloc (the decode step on the library's static
scratch, for callers that cannot allocate) against wh_llama_decode_step with a
caller workspace, through the C ABI: identical x, logits and stored cache rows,
bit for bit, on two calls in a row (the second on a smaller model at an
earlier position), a HIP-graph capture of it replayed three times, and a
position whose workspace would exceed the scratch rejected before anything is
launched."""
import ctypes as C

import numpy as np
import pytest

from tests._gpu import down, up
from tests.test_oracle_decode import small_layer
from woolly_amd import _lib, ops, synth
from woolly_amd.device import DeviceBuffer, Graph, Stream

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 8


class Model:
    """A random Llama-shaped model with two identical sets of KV caches, one
    per entry point, so both start from the same state."""

    def __init__(self, hidden, n_heads, n_kv, d, n_ff, n_layers, vocab, ctx, seed):
        rng = np.random.default_rng(seed)
        self.dims = dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff, max_ctx=ctx,
                         vocab=vocab, eps=1e-5)
        self.hidden, self.vocab, self.row = hidden, vocab, n_kv * d
        self.keep = []
        layers = [[], []]
        for li in range(n_layers):
            L = small_layer(Q4_0, hidden, n_heads, n_kv, d, n_ff, seed=seed + li)
            dev = {k: up(v)[0] for k, v in L.items()}
            self.keep.append(dev)
            kc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
            vc = rng.standard_normal((ctx, n_kv, d)).astype(np.float16).view(np.uint16)
            for copy in layers:
                c = dict(dev)
                c["k_cache"], c["v_cache"] = up(kc)[0], up(vc)[0]
                copy.append(c)
        inv = up(ops.rope_inv_freq(500000.0, d))[0]
        head = up(synth.quantized_weight(Q8_0, vocab, hidden, seed=seed + 99))[0]
        onorm = up((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))[0]
        self.keep += [inv, head, onorm]
        self.ref = ops.LlamaModel(Q4_0, self.dims, layers[0], inv, onorm, head, Q8_0)
        self.noalloc = ops.LlamaModel(Q4_0, self.dims, layers[1], inv, onorm, head, Q8_0)
        self.layers = layers

    def cache_rows(self, copy, pos):
        return [down(L[k], np.uint16, self.row, offset=pos * self.row * 2)
                for L in self.layers[copy] for k in ("k_cache", "v_cache")]


def run_noalloc(model, pos, xb, lb, stream=None):
    return _lib.load().wh_llama_decode_step_noalloc(C.byref(model.model), pos, xb.ptr, lb.ptr,
                                                    stream.handle if stream else None)


def compare(m, pos, seed):
    x0 = synth.activations(m.hidden, seed=seed)
    xr, lr = up(x0)[0], DeviceBuffer(4 * m.vocab)
    xn, ln = up(x0)[0], DeviceBuffer(4 * m.vocab)
    wsz = m.ref.workspace_bytes()
    ws = DeviceBuffer(wsz)
    m.ref.decode_step(pos, xr, lr, ws, wsz)
    _lib.check(run_noalloc(m.noalloc, pos, xn, ln))
    for a, b in ((xr, xn), (lr, ln)):
        n = a.nbytes // 4
        assert np.array_equal(down(a, np.uint32, n), down(b, np.uint32, n))
    for ra, rb in zip(m.cache_rows(0, pos), m.cache_rows(1, pos)):
        assert np.array_equal(ra, rb)
    return x0, down(ln, np.float32, m.vocab)


def test_noalloc_step_matches_workspace_step(gpu):
    print("[case] noalloc: 3-layer model hidden 512 at pos 40, then 2-layer hidden 256 at pos 5", flush=True)
    big = Model(512, 8, 2, 64, 1024, 3, 500, 64, seed=10)
    compare(big, 40, seed=1)
    small = Model(256, 4, 2, 64, 512, 2, 300, 16, seed=20)
    compare(small, 5, seed=2)
    # the first model again, at a later position: the scratch keeps no state
    compare(big, 41, seed=3)


def test_noalloc_step_graph_replays(gpu):
    """Captured into a HIP graph (the caller it is for) and replayed three
    times, with eager work in between: each replay equals the eager step."""
    print("[case] noalloc: graph capture and replays", flush=True)
    m = Model(256, 4, 2, 64, 512, 2, 300, 16, seed=30)
    other = Model(512, 8, 2, 64, 1024, 1, 200, 16, seed=31)
    x0, eager = compare(m, 7, seed=4)
    stream = Stream()
    xb, lb = up(x0)[0], DeviceBuffer(4 * m.vocab)
    with Graph.capture(stream) as g:
        _lib.check(run_noalloc(m.noalloc, 7, xb, lb, stream))
    for rep in range(3):
        xb.upload(x0)
        g.launch(stream)
        stream.synchronize()
        assert np.array_equal(down(lb, np.float32, m.vocab).view(np.uint32), eager.view(np.uint32)), rep
        # eager work between replays: another model's step on the same scratch
        # (the replay must not depend on what an earlier call left there)
        _lib.check(run_noalloc(other.noalloc, 3 + rep, up(synth.activations(512, seed=rep))[0],
                               DeviceBuffer(4 * other.vocab)))
    g.destroy()
    stream.destroy()


def test_noalloc_step_scratch_limit(gpu):
    """32 query heads of 128 at a position whose attention partials exceed the
    scratch: WH_ERR_BUFFER_TOO_SMALL and x untouched; the largest position that
    fits runs and matches the workspace step."""
    hidden, n_heads, n_kv, d, n_ff = 256, 32, 8, 128, 256
    limit = _lib.LLAMA_DECODE_NOALLOC_MAX_BYTES
    per_chunk = n_heads * (d + 2) * 4           # attention partials of 64 positions
    fixed = sum((4 * n + 255) // 256 * 256 for n in (n_heads * d + 2 * n_kv * d, n_heads * d, n_ff, n_ff,
                                                     max(hidden, n_ff)))
    chunks_ok = (limit - fixed) // per_chunk
    pos_ok = 64 * chunks_ok - 1
    pos_bad = pos_ok + 1
    ctx = pos_bad + 1
    print(f"[case] noalloc limit: ctx {ctx}, pos_ok {pos_ok}, pos_bad {pos_bad}", flush=True)
    m = Model(hidden, n_heads, n_kv, d, n_ff, 1, 64, ctx, seed=40)
    x0 = synth.activations(hidden, seed=5)
    xb, lb = up(x0)[0], DeviceBuffer(4 * 64)
    st = run_noalloc(m.noalloc, pos_bad, xb, lb)
    assert st == _lib.WH_ERR_BUFFER_TOO_SMALL, st
    assert b"static scratch" in _lib.load().wh_last_error()
    assert np.array_equal(down(xb, np.float32, hidden), x0)
    compare(m, pos_ok, seed=6)
