"""The tiled prefill GEMM's stream-K mode against the f64 oracle.

When the tiles of a GEMM would leave CUs idle in their last round (224 tiles
of 128 tokens x 256 rows on 256 CUs at M = 512, N = 14336), one workgroup per
CU takes an equal share of the (tile, stage) units, and tiles shared by
consecutive workgroups are completed by the workgroup holding their first
stage, which adds the other owners' partial accumulators in owner order.
The same split replaces split-K (partial planes and a reduce launch) where
there are fewer tiles than CUs, with 64- or 128-token tiles.  These cases
check the shapes where that happens: two owners per tile, three owners per
tile (a workgroup's share lying strictly inside one tile), sixteen owners
per tile (16 tiles on 256 workgroups), a partial last token tile, every
32-element block type, and repeated calls giving bit-identical results (the
sum order does not depend on timing).  With the hand-off wait bound set to 0
(wh_set_stream_k_wait), a workgroup that finishes a shared tile computes the
other owners' parts itself: the fallback a GPU shared with other work takes."""
import numpy as np
import pytest

from tests._gpu import down, report, up
from tests._oracle import max_abs, rel_l2
from woolly_amd import ops, synth
from woolly_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14
REL_L2 = 1e-4


def max_abs_bar(ref) -> float:
    """max-abs <= 1e-3 against the f64 reference, relative to the output RMS
    above an RMS of 300 (one f32 ulp at RMS 1e4 is already 1e-3)."""
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    return 1e-3 * max(1.0, rms / 300.0)


def sk_units(n, k, m, cus):
    """(tiles, stages per tile, units per workgroup) of the stream-K split, as
    the launcher forms it (tiles of 64 or 128 tokens and 256 rows, 2 blocks
    per stage)."""
    bm = 64 if m <= 64 else 128
    tiles = -(-m // bm) * -(-n // 256)
    tile_st = k // 64
    return tiles, tile_st, -(-tiles * tile_st // cus)


def owners_per_tile(n, k, m, cus=256):
    tiles, tile_st, upw = sk_units(n, k, m, cus)
    return max(len({u // upw for u in range(t * tile_st, (t + 1) * tile_st)}) for t in range(tiles))


def run_matmul(t, w, n, k, x, m):
    wb, wp = up(w)
    xb, xp = up(x)
    yb = DeviceBuffer(4 * m * n)
    wsz = ops.matmul_workspace_bytes(t, n, k, m)
    ws = DeviceBuffer(max(wsz, 1))
    outs = []
    for _ in range(3):
        ops.quantized_matmul(t, wp, w.nbytes, n, k, xp, m, yb.ptr, ws, wsz)
        outs.append(down(yb, np.float32, m * n).reshape(m, n))
    return outs


# token rows checked against the oracle: both ends of every 64- and 128-token tile
ROWS = [0, 1, 62, 63, 64, 99, 126, 127, 128, 200, 255, 256, 383, 384, 450, 511]


@pytest.mark.parametrize("t", [Q4_0, Q4_1, Q8_0])
@pytest.mark.parametrize("n,k,m", [(14336, 4096, 512),   # 224 tiles: two owners per shared tile
                                   (10240, 1024, 512),   # 160 tiles of 16 stages: three owners
                                   (14336, 1024, 300),   # 168 tiles, the last token tile partial
                                   (14336, 4096, 64),    # 56 tiles of 64 tokens: stream-K instead of split-K
                                   (4096, 14336, 100)])  # 16 tiles of 224 stages: 16 owners per tile
def test_stream_k_matmul(gpu, orc, t, n, k, m):
    print(f"[case] stream-K matmul type={t} m={m} n={n} k={k} owners<={owners_per_tile(n, k, m)}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n + k + t)
    x = synth.activations(m * k, seed=m + t).reshape(m, k)
    outs = run_matmul(t, w, n, k, x, m)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "repeated calls differ"
    rows = np.array([r for r in ROWS if r < m], dtype=np.int64)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, rows)
    got = outs[0][rows]
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"stream-K matmul t={t} m={m} n={n} k={k}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("n,k,m", [(14336, 4096, 512), (4096, 14336, 100)])
def test_stream_k_kquant_matmul(gpu, orc, t, n, k, m):
    """The K-quant formats (converted per call to 32-element blocks with f32
    scales): the same split, Q4_K's dmin term added once per tile by the
    workgroup that finishes it."""
    print(f"[case] stream-K kquant matmul type={t} m={m} n={n} k={k}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n + k + t)
    x = synth.activations(m * k, seed=m + t).reshape(m, k)
    outs = run_matmul(t, w, n, k, x, m)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "repeated calls differ"
    rows = np.array([r for r in ROWS if r < m], dtype=np.int64)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, rows)
    got = outs[0][rows]
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"stream-K kquant matmul t={t} m={m} n={n} k={k}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)


def test_stream_k_shapes_cover_three_owners():
    """The cases above include a tile with three owners (a workgroup's units
    strictly inside one tile) at 256 CUs, and the two-owner headline shape."""
    assert owners_per_tile(10240, 1024, 512) == 3
    assert owners_per_tile(14336, 4096, 512) == 2
    assert owners_per_tile(4096, 14336, 100) == 16


def owners_cases():
    return [(14336, 4096, 512), (10240, 1024, 512), (4096, 14336, 100)]


@pytest.mark.parametrize("t", [Q4_0, Q4_K])
@pytest.mark.parametrize("n,k,m", owners_cases())
def test_stream_k_fallback_matmul(gpu, orc, t, n, k, m):
    """Wait bound 0: the finishing workgroup computes the rest of each shared
    tile in a second pass (for Q4_K also the dmin term of every super-block);
    the result is the product within the same bars."""
    print(f"[case] stream-K fallback matmul type={t} m={m} n={n} k={k}", flush=True)
    w = synth.quantized_weight(t, n, k, seed=n + k + t)
    x = synth.activations(m * k, seed=m + t).reshape(m, k)
    try:
        ops.set_stream_k_wait(0)
        outs = run_matmul(t, w, n, k, x, m)
    finally:
        ops.set_stream_k_wait(ops.STREAM_K_WAIT_DEFAULT)
    rows = np.array([r for r in ROWS if r < m], dtype=np.int64)
    ref = orc.matmul_rows_f64(t, w, n, k, x, m, rows)
    for o in outs:
        got = o[rows]
        r, a = rel_l2(got, ref), max_abs(got, ref)
        report(f"stream-K fallback t={t} m={m} n={n} k={k}", r, a, ref)
        assert r <= REL_L2 and a <= max_abs_bar(ref)


def test_stream_k_fallback_ffn(gpu, orc):
    """Wait bound 0 in the fused gate||up kernel and the down projection of the
    Llama-3-8B FFN at M=512 (both split by stream-K there)."""
    from woolly_amd import synth as sy
    hidden, n_ff, m = 4096, 14336, 512
    L = sy.ffn_layer(Q4_0, hidden, n_ff, m, seed=5)
    bufs = {key: up(v) for key, v in L.items()}
    ob = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m)
    ws = DeviceBuffer(wsz)
    try:
        ops.set_stream_k_wait(0)
        ops.ffn_swiglu(Q4_0, bufs["gate"][1], bufs["up"][1], bufs["down"][1], hidden, n_ff,
                       bufs["gamma"][1], 1e-5, bufs["x"][1], m, ob.ptr, ws.ptr, wsz)
        got = down(ob, np.float32, m * hidden).reshape(m, hidden)
    finally:
        ops.set_stream_k_wait(ops.STREAM_K_WAIT_DEFAULT)
    rows = [0, 1, 127, 128, 256, 511]
    ref = orc.ffn_rows_f64(Q4_0, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5, L["x"], rows)
    g = got[rows]
    r, a = rel_l2(g, ref), max_abs(g, ref)
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    print(f"[result] stream-K fallback ffn m={m} rel_l2={r:.3e} max_abs={a:.3e} rms={rms:.1f} "
          f"bar={max_abs_bar(ref):.3e}", flush=True)
    # twice the bar of the other cases: in the fallback the finishing workgroup
    # accumulates the down projection's whole K = 14336 in one f32 accumulator
    # (the hand-off adds four owners' partial sums), 3.5e-6 of the output RMS
    # here against the bar's 3.3e-6
    assert r <= REL_L2 and a <= 2.0 * max_abs_bar(ref)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("n,k,m", [(10240, 1024, 512),   # three owners: parts end inside the 32-block window
                                   (4096, 14336, 100),   # sixteen owners over 14 windows per row
                                   (2048, 1600, 200)])   # 50 blocks per row: a last window of 18
def test_q4_1_dominant_minima(gpu, orc, n, k, m):
    """Q4_1 blocks whose minimum m is 16 to 64 times the block scale d, of
    either sign, against activations with a mean of 0.5, so that the m * sum(x)
    term carries most of each output.  The tiled GEMM forms that term as
    matrix-core products of each 32-block window's minima against the packed
    block sums, flushed at the window's end or where a stream-K part ends, so
    these shapes put part ends inside windows and a partial last window."""
    print(f"[case] q4_1 dominant minima m={m} n={n} k={k} owners<={owners_per_tile(n, k, m)}", flush=True)
    w = synth.quantized_weight(Q4_1, n, k, seed=n + k + 7)
    blocks = w.reshape(-1, 20)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    rng = np.random.default_rng(n + k)
    mult = rng.uniform(16.0, 64.0, size=d.shape) * rng.choice([-1.0, 1.0], size=d.shape)
    mins = (np.abs(d) * mult).astype(np.float16)
    blocks[:, 2:4] = mins.view(np.uint8).reshape(-1, 2)
    x = synth.activations(m * k, seed=m + k, mean=0.5).reshape(m, k)
    outs = run_matmul(Q4_1, w, n, k, x, m)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "repeated calls differ"
    rows = np.array([r for r in ROWS if r < m], dtype=np.int64)
    ref = orc.matmul_rows_f64(Q4_1, w, n, k, x, m, rows)
    got = outs[0][rows]
    r, a = rel_l2(got, ref), max_abs(got, ref)
    report(f"q4_1 dominant minima m={m} n={n} k={k}", r, a, ref)
    assert r <= REL_L2 and a <= max_abs_bar(ref)
    assert np.all(np.isfinite(got))
