"""Decode attention over seeded random head layouts and positions against the
f64 oracle (compute_optimized_gqa_attention, lazy_transformer.rs:261-456).

The fixed cases of test_gpu_decode.py use five head layouts; these draw the
query heads per KV head (1..8: the 4- and 8-head query tiles, rows past the
group masked), KV head counts that are and are not multiples of 8 (the
combine's XCD-affine and plain workgroup maps), both head sizes and random
positions (chunk boundaries and partial last chunks), with the same checks:
the stored k / v row, the untouched cache rows and the output."""
import numpy as np
import pytest

from tests.test_gpu_decode import test_attention_decode as _attention_case

pytestmark = pytest.mark.gpu


def cases(count: int = 30, seed: int = 20261204):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        g = int(rng.integers(1, 9))
        n_kv = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
        d = int(rng.choice([64, 128]))
        pos = int(rng.integers(0, 10000))
        out.append((g * n_kv, n_kv, d, pos))
    return out


@pytest.mark.parametrize("n_heads,n_kv,d,pos", cases())
def test_attention_random_layout(gpu, orc, n_heads, n_kv, d, pos):
    _attention_case(gpu, orc, n_heads, n_kv, d, pos)
