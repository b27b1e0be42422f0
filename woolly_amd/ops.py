"""Device-level entry points (DeviceBuffer in, DeviceBuffer out, stream-ordered).

Thin wrappers over the C ABI: each call validates nothing itself; the library
returns the reference's error semantics (see include/woolly_hip.h), raised here
as WoollyHipError.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .device import DeviceBuffer, Stream

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0 = 0, 1, 2, 3, 8
GGML_Q4_K, GGML_Q6_K = 12, 14


def _s(stream: Stream | None):
    return stream.handle if stream else None


def _p(buf) -> int:
    """Device address of a DeviceBuffer, a Weight handle or a plain integer."""
    if buf is None:
        return 0
    ptr = getattr(buf, "ptr", None)
    return int(ptr) if ptr is not None else int(buf)


def type_size(ggml_type: int) -> int:
    return int(_lib.load().wh_type_size(ggml_type))


def block_size(ggml_type: int) -> int:
    return int(_lib.load().wh_block_size(ggml_type))


def tensor_nbytes(ggml_type: int, nelements: int) -> int:
    out = C.c_uint64()
    _lib.check(_lib.load().wh_tensor_nbytes(ggml_type, nelements, C.byref(out)))
    return int(out.value)


def dequantize(ggml_type: int, data, nbytes: int, nelements: int, out,
               stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_dequantize(ggml_type, _p(data), nbytes, nelements, _p(out),
                                         _s(stream)))


def quantized_matvec(ggml_type: int, weights, weight_nbytes: int, x, y, m: int, k: int,
                     stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_quantized_matvec(ggml_type, _p(weights), weight_nbytes, _p(x),
                                               _p(y), m, k, _s(stream)))


GEMV_AUTO, GEMV_STREAM = 0, 1


def gemv_select(mode: int) -> int:
    """Chooses the single-token GEMV kernels (GEMV_AUTO: the int8 matrix-core
    kernel where the shape fits, GEMV_STREAM: the streaming kernels only);
    returns the previous mode."""
    prev = C.c_int(0)
    _lib.check(_lib.load().wh_gemv_select(int(mode), C.byref(prev)))
    return int(prev.value)


def matmul_workspace_bytes(ggml_type: int, n_rows: int, k: int, n_tokens: int) -> int:
    return int(_lib.load().wh_quantized_matmul_workspace_bytes(ggml_type, n_rows, k, n_tokens))


def quantized_matmul(ggml_type: int, weights, weight_nbytes: int, n_rows: int, k: int, x,
                     n_tokens: int, y, workspace=None, workspace_bytes: int = 0,
                     stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_quantized_matmul(ggml_type, _p(weights), weight_nbytes, n_rows, k,
                                               _p(x), n_tokens, _p(y), _p(workspace) or None,
                                               workspace_bytes, _s(stream)))


def rms_norm(x, weight, eps: float, tokens: int, hidden: int, out,
             stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_rms_norm(_p(x), _p(weight), eps, tokens, hidden, _p(out),
                                       _s(stream)))


def swiglu(gate, up, n: int, out, stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_swiglu(_p(gate), _p(up), n, _p(out), _s(stream)))


def ffn_workspace_bytes(hidden: int, n_ff: int, m: int, ggml_type: int | None = None) -> int:
    """Workspace of ffn_swiglu; without a type, enough for Q4_0, Q4_1 and Q8_0."""
    if ggml_type is None:
        return int(_lib.load().wh_ffn_workspace_bytes(hidden, n_ff, m))
    return int(_lib.load().wh_ffn_workspace_bytes_for_type(ggml_type, hidden, n_ff, m))


def ffn_swiglu(ggml_type: int, gate, up, down, hidden: int, n_ff: int, gamma, eps: float, x,
               m: int, out, workspace, workspace_bytes: int,
               stream: Stream | None = None) -> None:
    w = _lib.wh_ffn_weights(ggml_type, _p(gate), _p(up), _p(down), hidden, n_ff)
    _lib.check(_lib.load().wh_ffn_swiglu(C.byref(w), _p(gamma), eps, _p(x), m, _p(out),
                                         _p(workspace), workspace_bytes, _s(stream)))


class Weight:
    """A device-resident quantized tensor (wh_weight_upload / wh_weight_free)."""

    def __init__(self, ggml_type: int, n_rows: int, k: int, host_bytes) -> None:
        import numpy as np

        arr = np.ascontiguousarray(np.frombuffer(host_bytes, dtype=np.uint8)
                                   if not isinstance(host_bytes, np.ndarray) else host_bytes)
        h = C.c_void_p()
        _lib.check(_lib.load().wh_weight_upload(ggml_type, n_rows, k, arr.ctypes.data, arr.nbytes,
                                                C.byref(h)))
        self.handle = h.value
        self.ggml_type, self.n_rows, self.k = ggml_type, n_rows, k

    @classmethod
    def from_handle(cls, handle: int) -> "Weight":
        """Wraps a wh_weight* made by another entry point (wh_gguf_upload)."""
        w = cls.__new__(cls)
        w.handle = handle
        t, n, k = C.c_int(), C.c_size_t(), C.c_size_t()
        _lib.check(_lib.load().wh_weight_info(handle, C.byref(t), C.byref(n), C.byref(k), None))
        w.ggml_type, w.n_rows, w.k = t.value, n.value, k.value
        return w

    @property
    def ptr(self) -> int:
        return int(_lib.load().wh_weight_data(self.handle) or 0)

    @property
    def nbytes(self) -> int:
        nb = C.c_size_t()
        _lib.check(_lib.load().wh_weight_info(self.handle, None, None, None, C.byref(nb)))
        return int(nb.value)

    def free(self) -> None:
        if self.handle:
            _lib.check(_lib.load().wh_weight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                _lib.load().wh_weight_free(self.handle)
                self.handle = None
        except Exception:
            pass


# ------------------------------------------------------------ decode step
def rope_inv_freq(base: float, head_dim: int):
    """RoPE inverse frequencies 1 / base^(2i/d) in f32 (host array)."""
    import numpy as np

    out = np.zeros(head_dim // 2, np.float32)
    _lib.check(_lib.load().wh_rope_inv_freq(base, head_dim, out.ctypes.data))
    return out


def attention_qkv_workspace_bytes(hidden: int) -> int:
    return int(_lib.load().wh_attention_qkv_workspace_bytes(hidden))


def attention_qkv(ggml_type: int, wq, wk, wv, q_rows: int, kv_rows: int, hidden: int, gamma,
                  eps: float, x, qkv, workspace=None, workspace_bytes: int = 0,
                  stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_attention_qkv(ggml_type, _p(wq), _p(wk), _p(wv), q_rows, kv_rows, hidden,
                                            _p(gamma), eps, _p(x), _p(qkv), _p(workspace) or None,
                                            workspace_bytes, _s(stream)))


def attention_workspace_bytes(n_heads: int, n_kv_heads: int, head_dim: int, max_ctx: int) -> int:
    return int(_lib.load().wh_attention_workspace_bytes(n_heads, n_kv_heads, head_dim, max_ctx))


def attention_decode(qkv, k_cache, v_cache, pos: int, n_heads: int, n_kv_heads: int, head_dim: int,
                     inv_freq, out, workspace, workspace_bytes: int,
                     stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_attention_decode(_p(qkv), _p(k_cache), _p(v_cache), pos, n_heads,
                                               n_kv_heads, head_dim, _p(inv_freq), _p(out),
                                               _p(workspace), workspace_bytes, _s(stream)))


def quantized_matvec_residual(ggml_type: int, weights, weight_nbytes: int, x, residual, y, m: int,
                              k: int, stream: Stream | None = None) -> None:
    _lib.check(_lib.load().wh_quantized_matvec_residual(ggml_type, _p(weights), weight_nbytes, _p(x),
                                                        _p(residual), _p(y), m, k, _s(stream)))


class LlamaModel:
    """A Llama-shaped model on the device for the decode step: `layers` is a
    list of dicts of device buffers (attn_norm, wq, wk, wv, wo, ffn_norm,
    w_gate, w_up, w_down, k_cache, v_cache) and optionally a block type per
    matrix (wq_type .. w_down_type; absent or 0: ggml_type); wraps wh_llama_model."""

    def __init__(self, ggml_type: int, dims: dict, layers: list, inv_freq_dev, output_norm=None,
                 output=None, output_type: int = GGML_Q8_0) -> None:
        self._keep = (layers, inv_freq_dev, output_norm, output)
        arr = (_lib.wh_llama_layer * len(layers))()
        for i, L in enumerate(layers):
            for name, _ in _lib.wh_llama_layer._fields_:
                if name.endswith("_type"):
                    setattr(arr[i], name, int(L.get(name, 0)))
                else:
                    setattr(arr[i], name, _p(L[name]) or None)
        self._layers = arr
        m = _lib.wh_llama_model()
        m.type = ggml_type
        for key in ("hidden", "n_heads", "n_kv_heads", "head_dim", "n_ff", "max_ctx", "vocab"):
            setattr(m, key, dims[key])
        m.n_layers = len(layers)
        m.eps = dims.get("eps", 1e-5)
        m.rope_inv_freq = _p(inv_freq_dev)
        m.layers = C.cast(arr, C.POINTER(_lib.wh_llama_layer))
        m.output_norm = _p(output_norm) or None
        m.output_type = output_type
        m.output = _p(output) or None
        self.model = m

    @staticmethod
    def config_from_gguf(ld, max_ctx: int | None = None) -> dict:
        """The model config of a GGUF file (gguf.GGUFLoader) from the
        `{arch}.*` metadata keys GGUFModelLoader reads (model/loader.rs:110-150):
        embedding_length, block_count, attention.head_count[_kv] (default: the
        head count), feed_forward_length (default 4 x hidden), context_length
        (default 2048; max_ctx overrides it), rope.freq_base (default 10000),
        attention.layer_norm_epsilon or layer_norm_epsilon (default 1e-5)."""
        md = ld.metadata()
        arch = md.get_string("general.architecture") or "llama"

        def u32(key, default=None):
            v = md.get_u32(f"{arch}.{key}")
            if v is None and default is None:
                raise ValueError(f"GGUF metadata {arch}.{key} missing")
            return int(v if v is not None else default)

        def f32(keys, default):
            for key in keys:
                v = md.get_f32(f"{arch}.{key}")
                if v is not None:
                    return float(v)
            return default

        hidden, n_layers, n_heads = u32("embedding_length"), u32("block_count"), u32("attention.head_count")
        return dict(hidden=hidden, n_layers=n_layers, n_heads=n_heads,
                    n_kv_heads=u32("attention.head_count_kv", n_heads), head_dim=hidden // n_heads,
                    n_ff=u32("feed_forward_length", 4 * hidden),
                    max_ctx=int(max_ctx) if max_ctx else u32("context_length", 2048),
                    rope_base=f32(["rope.freq_base"], 10000.0),
                    eps=f32(["attention.layer_norm_epsilon", "layer_norm_epsilon"], 1e-5))

    @classmethod
    def from_gguf(cls, ld, max_ctx: int | None = None) -> "LlamaModel":
        """The decode model of a GGUF file (gguf.GGUFLoader): the config of
        config_from_gguf and the tensors load_layer_weights / load_model_weights
        name (model/loader.rs:370-520: blk.N.{attn_norm, attn_q, attn_k, attn_v,
        attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down}.weight,
        output_norm.weight, output.weight).  Every matrix is uploaded from the
        mapping with its own block type (Q4_K_M files mix Q4_K and Q6_K); the
        f16 KV caches (max_ctx rows) start zeroed."""
        from .device import DeviceBuffer

        cfg = cls.config_from_gguf(ld, max_ctx)
        hidden, n_layers, n_heads, n_kv = cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"]
        n_ff, ctx, base, eps = cfg["n_ff"], cfg["max_ctx"], cfg["rope_base"], cfg["eps"]
        d = hidden // n_heads
        names = {"attn_norm": "attn_norm", "wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
                 "ffn_norm": "ffn_norm", "w_gate": "ffn_gate", "w_up": "ffn_up", "w_down": "ffn_down"}
        layers = []
        for i in range(n_layers):
            L = {}
            for key, nm in names.items():
                name = f"blk.{i}.{nm}.weight"
                L[key] = ld.upload(name)
                if key.startswith("w"):
                    L[key + "_type"] = int(ld.tensor_info(name).ggml_type)
            for key in ("k_cache", "v_cache"):
                L[key] = DeviceBuffer(ctx * n_kv * d * 2)
                L[key].fill(0)
            layers.append(L)
        inv = DeviceBuffer.from_array(rope_inv_freq(base, d))
        out_norm = ld.upload("output_norm.weight")
        head = ld.upload("output.weight")
        head_info = ld.tensor_info("output.weight")
        dims = dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff, max_ctx=ctx,
                    vocab=int(head_info.shape()[1]), eps=eps)
        m = cls(layers[0]["wq_type"] if layers else GGML_Q4_0, dims, layers, inv, out_norm, head,
                int(head_info.ggml_type))
        m.dims = dims
        return m

    def workspace_bytes(self) -> int:
        return int(_lib.load().wh_llama_decode_workspace_bytes(C.byref(self.model)))

    def layer_decode(self, layer: int, pos: int, x, workspace, workspace_bytes: int,
                     stream: Stream | None = None) -> None:
        _lib.check(_lib.load().wh_llama_layer_decode(C.byref(self.model), layer, pos, _p(x),
                                                     _p(workspace), workspace_bytes, _s(stream)))

    def decode_step(self, pos: int, x, logits, workspace, workspace_bytes: int,
                    stream: Stream | None = None) -> None:
        _lib.check(_lib.load().wh_llama_decode_step(C.byref(self.model), pos, _p(x),
                                                    _p(logits) or None, _p(workspace), workspace_bytes,
                                                    _s(stream)))
