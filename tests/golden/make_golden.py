"""Writes the committed golden fixtures in tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Inputs come from woolly_amd.synth (seeded); outputs from oracle/ (built on demand).
The fixtures pin the oracle against regressions and give the GPU tests vectors that do
not need the oracle at run time.  Nothing from /root/reference is imported or run.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from tests._oracle import Oracle  # noqa: E402
from woolly_amd import synth  # noqa: E402

Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 2, 3, 8, 12, 14
NAMES = {Q4_0: "q4_0", Q4_1: "q4_1", Q8_0: "q8_0"}
# 256-element K-quant blocks: two blocks per row
K_NAMES = {Q4_K: "q4_k", Q6_K: "q6_k"}


def main() -> None:
    orc = Oracle()
    for t, name in {**NAMES, **K_NAMES}.items():
        n, k = (64, 256) if t in NAMES else (16, 512)
        w = synth.quantized_weight(t, n, k, seed=1000 + t)
        x = synth.activations(k, seed=2000 + t)
        st, deq = orc.dequantize(t, w, n * k)
        assert st == 0
        _, y64 = orc.matvec_f64(t, w, x, n, k)
        _, y32 = orc.matvec_f32(t, w, x, n, k)
        np.savez_compressed(HERE / f"gemv_{name}_{n}x{k}.npz", type=t, n=n, k=k, w=w, x=x,
                            dequant=deq, y_f64=y64, y_f32_scalar_order=y32)
    hidden, n_ff, m = 256, 512, 4
    L = synth.ffn_layer(Q4_0, hidden, n_ff, m, seed=3000)
    out = orc.ffn_rows_f64(Q4_0, L["gate"], L["up"], L["down"], hidden, n_ff, L["gamma"], 1e-5,
                           L["x"], np.arange(m))
    np.savez_compressed(HERE / "ffn_q4_0_256x512_m4.npz", type=Q4_0, hidden=hidden, n_ff=n_ff,
                        m=m, eps=1e-5, out_f64=out, **L)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
