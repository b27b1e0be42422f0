"""Seeded synthetic inputs for the benchmark configurations.

Counter-based SplitMix64 (output i of a stream is mix(seed_state + (i+1) *
0x9E3779B97F4A7C15)) so that any slice of any array can be regenerated
independently; Box-Muller turns uniforms into normals.  Scales are rounded to
f16 with numpy's round-to-nearest-even.  The same generator feeds the GPU
runs, the CPU oracle and the golden fixtures, so all of them see identical
bytes for a given (config, seed).

Block layouts (crates/woolly-tensor/src/quantization.rs:98-151):
  Q4_0  {u16 d; u8 qs[16]}            18 B
  Q4_1  {u16 d; u16 m; u8 qs[16]}     20 B
  Q8_0  {u16 d; i8 qs[32]}            34 B
and the 256-element K-quant blocks as woolly-gguf reads them
(crates/woolly-gguf/src/dequantize.rs:404-536):
  Q4_K  {u8 scales[12]; u16 d; u16 dmin; u8 qs[128]}              144 B
  Q6_K  {u8 ql[128]; u8 qh[64]; u8 scales[16]; u16 d}              210 B
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

GGML_Q4_0, GGML_Q4_1, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 2, 3, 8, 12, 14
GGML_Q5_0, GGML_Q5_1 = 6, 7
TYPE_SIZE = {GGML_Q4_0: 18, GGML_Q4_1: 20, GGML_Q5_0: 22, GGML_Q5_1: 24, GGML_Q8_0: 34, GGML_Q4_K: 144,
             GGML_Q6_K: 210}
BLOCK_ELEMS = {GGML_Q4_0: 32, GGML_Q4_1: 32, GGML_Q5_0: 32, GGML_Q5_1: 32, GGML_Q8_0: 32, GGML_Q4_K: 256,
               GGML_Q6_K: 256}
TYPE_NAME = {GGML_Q4_0: "Q4_0", GGML_Q4_1: "Q4_1", GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K"}


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def stream_seed(seed: int, stream: int) -> np.uint64:
    """Independent sub-stream of `seed` (one per generated array)."""
    with np.errstate(over="ignore"):
        s = (np.array([seed], dtype=np.uint64) * np.uint64(0x2545F4914F6CDD1D)
             + np.array([stream], dtype=np.uint64) * GOLDEN)
        return _mix(s)[0]


def u64(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start + n - 1 of the stream, in cache-sized chunks with
    in-place operations (the same values as _mix(base + idx * GOLDEN))."""
    base = stream_seed(seed, stream)
    out = np.empty(n, np.uint64)
    chunk = 1 << 16
    tmp = np.empty(min(n, chunk), np.uint64)
    with np.errstate(over="ignore"):
        for c0 in range(0, n, chunk):
            c1 = min(n, c0 + chunk)
            z, t = out[c0:c1], tmp[: c1 - c0]
            z[:] = np.arange(start + c0 + 1, start + c1 + 1, dtype=np.uint64)
            np.multiply(z, GOLDEN, out=z)
            np.add(z, base, out=z)
            for sh, mul in ((30, M1), (27, M2), (31, None)):
                np.right_shift(z, np.uint64(sh), out=t)
                np.bitwise_xor(z, t, out=z)
                if mul is not None:
                    np.multiply(z, mul, out=z)
    return out


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    """Uniform float64 in [0, 1)."""
    return (u64(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Normal float64 via Box-Muller on two uniforms per output."""
    m = (n + 1) // 2
    u = uniform(seed, stream, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return mean + std * z[:n]


def f16_bits(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def quantized_weight(ggml_type: int, n_rows: int, k: int, seed: int, stream: int = 0,
                     d_std: float | None = None) -> np.ndarray:
    """N x K weight in the GGUF block layout, as a flat uint8 array.

    Q4_0: d = f16(|N(0, 0.02)|), qs bytes uniform 0..255 (two uniform nibbles).
    Q8_0: d = f16(|N(0, 0.02)|), qs int8 uniform in [-127, 127].
    Q4_1: d, m = f16(N(0, 0.01)), qs bytes uniform 0..255.
    Q5_0: d = f16(|N(0, 0.02)|), qh and qs bytes uniform 0..255 (dequantization only).
    Q5_1: d, m = f16(N(0, 0.01)), qh and qs bytes uniform 0..255 (dequantization only).
    Q4_K: scale bytes uniform, d = f16(|N(0, 0.0005)|), dmin = f16(N(0, 0.01)), quant bytes uniform.
    Q6_K: ql, qh, scale bytes uniform, d = f16(|N(0, 0.0001)|).
    """
    be = BLOCK_ELEMS.get(ggml_type, 0)
    if be == 0:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    if k % be:
        raise ValueError(f"k must be a multiple of {be}")
    nb = n_rows * (k // be)
    ts = TYPE_SIZE[ggml_type]
    out = np.empty((nb, ts), dtype=np.uint8)
    s0 = 16 * stream
    if ggml_type == GGML_Q4_K:
        out[:, :] = (u64(seed, s0 + 2, nb * ts) & np.uint64(0xFF)).astype(np.uint8).reshape(nb, ts)
        d = np.abs(normal(seed, s0 + 1, nb, 0.0, 0.0005 if d_std is None else d_std))
        out[:, 12:14] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        out[:, 14:16] = f16_bits(normal(seed, s0 + 3, nb, 0.0, 0.01)).view(np.uint8).reshape(nb, 2)
        return out.reshape(-1)
    if ggml_type == GGML_Q6_K:
        out[:, :] = (u64(seed, s0 + 2, nb * ts) & np.uint64(0xFF)).astype(np.uint8).reshape(nb, ts)
        d = np.abs(normal(seed, s0 + 1, nb, 0.0, 0.0001 if d_std is None else d_std))
        out[:, 208:210] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        return out.reshape(-1)
    if ggml_type == GGML_Q4_0:
        d = np.abs(normal(seed, s0 + 1, nb, 0.0, 0.02 if d_std is None else d_std))
        out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        out[:, 2:18] = u64(seed, s0 + 2, nb * 2).view(np.uint8).reshape(nb, 16)
    elif ggml_type == GGML_Q4_1:
        d = normal(seed, s0 + 1, nb, 0.0, 0.01 if d_std is None else d_std)
        m = normal(seed, s0 + 3, nb, 0.0, 0.01)
        out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        out[:, 2:4] = f16_bits(m).view(np.uint8).reshape(nb, 2)
        out[:, 4:20] = u64(seed, s0 + 2, nb * 2).view(np.uint8).reshape(nb, 16)
    elif ggml_type in (GGML_Q5_0, GGML_Q5_1):
        # d (and m), then 20 random bytes: qh[4], qs[16]
        h = 2 if ggml_type == GGML_Q5_0 else 4
        if ggml_type == GGML_Q5_0:
            d = np.abs(normal(seed, s0 + 1, nb, 0.0, 0.02 if d_std is None else d_std))
        else:
            d = normal(seed, s0 + 1, nb, 0.0, 0.01 if d_std is None else d_std)
            out[:, 2:4] = f16_bits(normal(seed, s0 + 3, nb, 0.0, 0.01)).view(np.uint8).reshape(nb, 2)
        out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        out[:, h:h + 20] = u64(seed, s0 + 2, nb * 3).view(np.uint8).reshape(nb, 24)[:, :20]
    elif ggml_type == GGML_Q8_0:
        d = np.abs(normal(seed, s0 + 1, nb, 0.0, 0.02 if d_std is None else d_std))
        out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
        # u % 255 of each 64-bit draw, from the sum of its 8 bytes (2^8 = 1 mod 255)
        u = u64(seed, s0 + 2, nb * 32)
        q = (u.view(np.uint8).reshape(-1, 8).sum(axis=1, dtype=np.uint32) % np.uint32(255)).astype(np.int16) - 127
        out[:, 2:34] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    else:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    return out.reshape(-1)


def activations(n: int, seed: int, stream: int = 100, mean: float = 0.0,
                std: float = 1.0) -> np.ndarray:
    return normal(seed, stream, n, mean, std).astype(np.float32)


def ffn_layer(ggml_type: int, hidden: int, n_ff: int, m: int, seed: int) -> dict:
    """Config 3: RMSNorm gamma ~ N(1, 0.1), gate/up [n_ff, hidden], down [hidden, n_ff]."""
    return {
        "gate": quantized_weight(ggml_type, n_ff, hidden, seed, stream=1),
        "up": quantized_weight(ggml_type, n_ff, hidden, seed, stream=2),
        "down": quantized_weight(ggml_type, hidden, n_ff, seed, stream=3),
        "gamma": activations(hidden, seed, stream=200, mean=1.0, std=0.1),
        "x": activations(m * hidden, seed, stream=201).reshape(m, hidden),
    }
