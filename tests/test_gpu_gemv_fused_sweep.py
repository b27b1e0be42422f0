"""The single-token GEMV's fused modes over seeded random shapes against the
f64 oracle: RMSNorm + stacked q / k / v (the attention projections of
process_layer, lazy_transformer.rs:98-258, with rms_norm tensor_utils.rs:446-480)
and y = residual + W x in place (the residual adds of the same function).
The fixed cases of test_gpu_decode.py use three and two shapes; these draw
the hidden size and the row counts at random (a fixed seed), row counts that
are not a multiple of 16 and hidden sizes with odd block counts included, so
the matrix-core kernel's partial row groups, its several-segment rows and the
streaming fallbacks all run."""
import numpy as np
import pytest

from tests.test_gpu_decode import test_attention_qkv_fused as _qkv_case
from tests.test_gpu_decode import test_matvec_residual_in_place as _residual_case

pytestmark = pytest.mark.gpu
Q4_0, Q4_1, Q8_0 = 2, 3, 8


def qkv_cases(count: int = 24, seed: int = 20261205):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        t = [Q4_0, Q8_0, Q4_1][i % 3]
        hidden = 32 * int(rng.integers(1, 257))           # 32 .. 8192
        q_rows = int(rng.integers(1, 4097))
        kv_rows = int(rng.integers(1, 1025))
        out.append((t, hidden, q_rows, kv_rows))
    return out


def residual_cases(count: int = 16, seed: int = 20261206):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        t = [Q4_0, Q8_0][i % 2]
        m = int(rng.integers(1, 8193))
        k = 32 * int(rng.integers(1, 513))                # 32 .. 16384
        out.append((t, m, k))
    return out


@pytest.mark.parametrize("t,hidden,q_rows,kv_rows", qkv_cases())
def test_attention_qkv_random_shape(gpu, orc, t, hidden, q_rows, kv_rows):
    _qkv_case(gpu, orc, t, hidden, q_rows, kv_rows)


@pytest.mark.parametrize("t,m,k", residual_cases())
def test_matvec_residual_random_shape(gpu, orc, t, m, k):
    print(f"[case] residual t={t} {m}x{k}", flush=True)
    _residual_case(gpu, orc, t, m, k)
