"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module, and only as the checker.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "_build" / "liboracle.so"

_p = C.c_void_p
_sz = C.c_size_t


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self, lib_path: Path | None = None):
        """The oracle library (oracle/_build/liboracle.so, built on demand), or
        another build of the same sources at lib_path (the mutation tests load
        copies with a planted mistake)."""
        if lib_path is None:
            if not ORACLE_LIB.exists():
                subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
            lib_path = ORACLE_LIB
        lib = C.CDLL(str(lib_path))
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32_array": (None, [_p, _sz, _p]),
            "orc_f32_to_f16_array": (None, [_p, _sz, _p]),
            "orc_block_size": (_sz, [C.c_int]),
            "orc_type_size": (_sz, [C.c_int]),
            "orc_dequantize": (C.c_int, [C.c_int, _p, _sz, _sz, _p]),
            "orc_matvec_f32": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz]),
            "orc_matvec_f64": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz]),
            "orc_matmul_f64": (C.c_int, [C.c_int, _p, _sz, _sz, _p, _sz, _p]),
            "orc_matmul_rows_f64": (C.c_int, [C.c_int, _p, _sz, _sz, _p, _sz, _p, _sz, _p]),
            "orc_gemm_f32": (None, [_p, _p, _p, _sz, _sz, _sz, C.c_float, C.c_float]),
            "orc_rms_norm_f32": (None, [_p, _p, C.c_float, _sz, _sz, _p]),
            "orc_rms_norm_f64": (None, [_p, _p, C.c_double, _sz, _sz, _p]),
            "orc_swiglu_f32": (None, [_p, _p, _sz, _p]),
            "orc_swiglu_f64": (None, [_p, _p, _sz, _p]),
            "orc_ffn_f64": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz, _p, C.c_double, _p, _sz, _p]),
            "orc_ffn_rows_f64": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz, _p, C.c_double, _p, _p,
                                           _sz, _p]),
            "orc_ffn_f32": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz, _p, C.c_float, _p, _sz, _p]),
            "orc_rope_inv_freq": (C.c_int, [C.c_float, _sz, _p]),
            "orc_attention_decode_f64": (C.c_int, [_p, _p, _p, _sz, _sz, _sz, _sz, _p, C.c_int, _p]),
            "orc_llama_layer_decode_f64": (C.c_int, [C.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz,
                                                     _sz, _sz, _sz, _sz, C.c_double, _p, _p, _p, _sz,
                                                     C.c_int, _p]),
            "orc_llama_layer_decode_types_f64": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz,
                                                           _sz, _sz, _sz, _sz, C.c_double, _p, _p, _p, _sz,
                                                           C.c_int, _p]),
            "orc_output_head_f64": (C.c_int, [C.c_int, _p, _p, C.c_double, _p, _sz, _sz, _p]),
            "orc_llama_layer_decode_f32": (C.c_int, [C.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz,
                                                     _sz, _sz, _sz, _sz, C.c_float, _p, _p, _p, _sz,
                                                     C.c_int, _p]),
            "orc_simd_available": (C.c_int, []),
            "orc_matvec_simd_mt": (C.c_int, [C.c_int, _p, _p, _p, _sz, _sz, C.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib

    # --- scalar helpers
    def f16_to_f32(self, bits: np.ndarray) -> np.ndarray:
        b = np.ascontiguousarray(bits, dtype=np.uint16)
        out = np.empty(b.size, dtype=np.float32)
        self.lib.orc_f16_to_f32_array(_ptr(b), b.size, _ptr(out))
        return out

    def f32_to_f16(self, vals: np.ndarray) -> np.ndarray:
        v = np.ascontiguousarray(vals, dtype=np.float32)
        out = np.empty(v.size, dtype=np.uint16)
        self.lib.orc_f32_to_f16_array(_ptr(v), v.size, _ptr(out))
        return out

    def type_size(self, t: int) -> int:
        return int(self.lib.orc_type_size(t))

    def block_size(self, t: int) -> int:
        return int(self.lib.orc_block_size(t))

    # --- kernels
    def dequantize(self, t: int, data: np.ndarray, n: int) -> tuple[int, np.ndarray]:
        d = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.zeros(n, dtype=np.float32)
        st = self.lib.orc_dequantize(t, _ptr(d), d.nbytes, n, _ptr(out))
        return st, out

    def matvec_f32(self, t, w, x, m, k):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(m, dtype=np.float32)
        st = self.lib.orc_matvec_f32(t, _ptr(w), _ptr(x), _ptr(y), m, k)
        return st, y

    # --- decode step
    def rope_inv_freq(self, base: float, head_dim: int) -> np.ndarray:
        out = np.zeros(head_dim // 2, np.float32)
        assert self.lib.orc_rope_inv_freq(base, head_dim, _ptr(out)) == 0
        return out

    def attention_decode_f64(self, qkv, k_cache, v_cache, pos, n_heads, n_kv, d, inv_freq, store_new=True):
        """Returns out (f64 [n_heads*d]); k_cache / v_cache (uint16 f16 bits,
        [ctx][n_kv][d], C-contiguous) are updated at row pos in place, or with
        store_new=False the row already there is attended to."""
        q = np.ascontiguousarray(qkv, dtype=np.float64)
        f = np.ascontiguousarray(inv_freq, dtype=np.float32)
        assert k_cache.dtype == np.uint16 and k_cache.flags.c_contiguous
        assert v_cache.dtype == np.uint16 and v_cache.flags.c_contiguous
        out = np.zeros(n_heads * d, np.float64)
        st = self.lib.orc_attention_decode_f64(_ptr(q), _ptr(k_cache), _ptr(v_cache), pos, n_heads, n_kv,
                                               d, _ptr(f), int(store_new), _ptr(out))
        assert st == 0, st
        return out

    def llama_layer_decode_f64(self, t, L, dims, inv_freq, k_cache, v_cache, pos, x, store_new=True):
        """One layer on x (f64, updated copy returned); L: dict of the layer's
        weights (uint8 blocks) and norms (f32); dims: hidden, n_heads, n_kv, d,
        n_ff, eps; t: one block type, or seven (q, k, v, o, gate, up, down)."""
        hidden, n_heads, n_kv, d, n_ff, eps = dims
        xx = np.array(x, dtype=np.float64, copy=True)
        a = {k: np.ascontiguousarray(v) for k, v in L.items()}
        f = np.ascontiguousarray(inv_freq, dtype=np.float32)
        types = np.ascontiguousarray(np.broadcast_to(np.asarray(t, dtype=np.int32), (7,)))
        st = self.lib.orc_llama_layer_decode_types_f64(
            _ptr(types), _ptr(a["wq"]), _ptr(a["wk"]), _ptr(a["wv"]), _ptr(a["wo"]), _ptr(a["attn_norm"]),
            _ptr(a["w_gate"]), _ptr(a["w_up"]), _ptr(a["w_down"]), _ptr(a["ffn_norm"]), hidden, n_heads,
            n_kv, d, n_ff, eps, _ptr(f), _ptr(k_cache), _ptr(v_cache), pos, int(store_new), _ptr(xx))
        assert st == 0, st
        return xx

    def llama_layer_decode_f32(self, t, L, dims, inv_freq, k_cache, v_cache, pos, x, store_new=True):
        """The reference's own f32 evaluation order of the same layer."""
        hidden, n_heads, n_kv, d, n_ff, eps = dims
        xx = np.array(x, dtype=np.float32, copy=True)
        a = {k: np.ascontiguousarray(v) for k, v in L.items()}
        f = np.ascontiguousarray(inv_freq, dtype=np.float32)
        st = self.lib.orc_llama_layer_decode_f32(
            t, _ptr(a["wq"]), _ptr(a["wk"]), _ptr(a["wv"]), _ptr(a["wo"]), _ptr(a["attn_norm"]),
            _ptr(a["w_gate"]), _ptr(a["w_up"]), _ptr(a["w_down"]), _ptr(a["ffn_norm"]), hidden, n_heads,
            n_kv, d, n_ff, eps, _ptr(f), _ptr(k_cache), _ptr(v_cache), pos, int(store_new), _ptr(xx))
        assert st == 0, st
        return xx

    def output_head_f64(self, t, w, norm, eps, x, hidden, vocab):
        ww = np.ascontiguousarray(w)
        nn = np.ascontiguousarray(norm, dtype=np.float32)
        xx = np.ascontiguousarray(x, dtype=np.float64)
        out = np.zeros(vocab, np.float64)
        st = self.lib.orc_output_head_f64(t, _ptr(ww), _ptr(nn), eps, _ptr(xx), hidden, vocab, _ptr(out))
        assert st == 0, st
        return out

    def simd_available(self) -> bool:
        return bool(self.lib.orc_simd_available())

    def matvec_simd_mt(self, t, w, x, m, k, threads):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(m, dtype=np.float32)
        st = self.lib.orc_matvec_simd_mt(t, _ptr(w), _ptr(x), _ptr(y), m, k, threads)
        return st, y

    def matvec_f64(self, t, w, x, m, k):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(m, dtype=np.float64)
        st = self.lib.orc_matvec_f64(t, _ptr(w), _ptr(x), _ptr(y), m, k)
        return st, y

    def matmul_rows_f64(self, t, w, n, k, x, m, rows):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        r = np.ascontiguousarray(rows, dtype=np.int64)
        y = np.zeros((r.size, n), dtype=np.float64)
        st = self.lib.orc_matmul_rows_f64(t, _ptr(w), n, k, _ptr(x), m, _ptr(r), r.size, _ptr(y))
        assert st == 0
        return y

    def gemm_f32(self, a, b, c, m, n, k, alpha=1.0, beta=0.0):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        c = np.array(c, dtype=np.float32, copy=True)
        self.lib.orc_gemm_f32(_ptr(a), _ptr(b), _ptr(c), m, n, k, alpha, beta)
        return c

    def rms_norm_f32(self, x, w, eps, tokens, hidden):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.zeros(tokens * hidden, dtype=np.float32)
        self.lib.orc_rms_norm_f32(_ptr(x), _ptr(w), eps, tokens, hidden, _ptr(out))
        return out

    def rms_norm_f64(self, x, w, eps, tokens, hidden):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.zeros(tokens * hidden, dtype=np.float64)
        self.lib.orc_rms_norm_f64(_ptr(x), _ptr(w), eps, tokens, hidden, _ptr(out))
        return out

    def swiglu_f32(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        out = np.zeros(g.size, dtype=np.float32)
        self.lib.orc_swiglu_f32(_ptr(g), _ptr(u), g.size, _ptr(out))
        return out

    def swiglu_f64(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float64)
        u = np.ascontiguousarray(u, dtype=np.float64)
        out = np.zeros(g.size, dtype=np.float64)
        self.lib.orc_swiglu_f64(_ptr(g), _ptr(u), g.size, _ptr(out))
        return out

    def ffn_rows_f64(self, t, gate, up, down, hidden, n_ff, gamma, eps, x, tokens):
        tok = np.ascontiguousarray(tokens, dtype=np.int64)
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((tok.size, hidden), dtype=np.float64)
        st = self.lib.orc_ffn_rows_f64(t, _ptr(gate), _ptr(up), _ptr(down), hidden, n_ff,
                                       _ptr(np.ascontiguousarray(gamma, dtype=np.float32)), eps,
                                       _ptr(x), _ptr(tok), tok.size, _ptr(out))
        assert st == 0
        return out

    def ffn_f32(self, t, gate, up, down, hidden, n_ff, gamma, eps, x, m):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((m, hidden), dtype=np.float32)
        st = self.lib.orc_ffn_f32(t, _ptr(gate), _ptr(up), _ptr(down), hidden, n_ff,
                                  _ptr(np.ascontiguousarray(gamma, dtype=np.float32)), eps,
                                  _ptr(x), m, _ptr(out))
        assert st == 0
        return out


def rel_l2(a, ref) -> float:
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(a - ref) / den) if den > 0 else float(np.linalg.norm(a - ref))


def max_abs(a, ref) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(ref, np.float64)))) if np.size(a) else 0.0
