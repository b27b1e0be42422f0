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


TYPE_BF16 = 30  # activation type of quantized_matmul_x (GGMLType::BF16)


def matmul_x_workspace_bytes(ggml_type: int, n_rows: int, k: int, n_tokens: int, x_dtype: int) -> int:
    return int(_lib.load().wh_quantized_matmul_x_workspace_bytes(ggml_type, n_rows, k, n_tokens, x_dtype))


def quantized_matmul_x(ggml_type: int, weights, weight_nbytes: int, n_rows: int, k: int, x, x_dtype: int,
                       n_tokens: int, y, workspace=None, workspace_bytes: int = 0,
                       stream: Stream | None = None) -> None:
    """Y = X W^T with X of x_dtype (0: f32, TYPE_BF16: bfloat16 [n_tokens][k])."""
    _lib.check(_lib.load().wh_quantized_matmul_x(ggml_type, _p(weights), weight_nbytes, n_rows, k, _p(x),
                                                 x_dtype, n_tokens, _p(y), _p(workspace) or None,
                                                 workspace_bytes, _s(stream)))


def set_stream_k_wait(ticks: int) -> None:
    """Bound of the prefill GEMM's stream-K hand-off wait, in ticks of the GPU's
    100 MHz clock (default 100000 = 1 ms); 0 makes a workgroup that finishes a
    shared tile compute the other owners' parts itself (wh_set_stream_k_wait)."""
    _lib.check(_lib.load().wh_set_stream_k_wait(int(ticks)))


STREAM_K_WAIT_DEFAULT = 100000


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

    def prepare_prefill(self, stream: Stream | None = None) -> int:
        """wh_weight_prepare_prefill: Q4_K / Q6_K blocks converted once into the
        tiled GEMM's layout and kept with the handle; returns the copy's bytes."""
        nb = C.c_size_t()
        _lib.check(_lib.load().wh_weight_prepare_prefill(self.handle, _s(stream), C.byref(nb)))
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


def embedding_lookup(ggml_type: int, table, vocab: int, hidden: int, input_ids, out,
                     stream: Stream | None = None):
    """embedding_lookup (crates/woolly-core/src/tensor_utils.rs:548-590) with the
    table on the device: out (device, [len(input_ids)][hidden] f32) receives the
    dequantized rows.  Token ids are checked on the host first and an id >=
    vocab raises ValueError with the reference's message
    (TENSOR_EMBEDDING_TOKEN_OUT_OF_RANGE); returns the device buffer of ids."""
    import numpy as np

    from .device import DeviceBuffer

    ids = np.ascontiguousarray(np.asarray(input_ids, dtype=np.int64))
    for t in ids.tolist():
        if t < 0 or t >= vocab:
            raise ValueError(f"Token ID {t} exceeds vocabulary size {vocab}")
    idb = DeviceBuffer.from_array(ids.astype(np.uint32), stream)
    _lib.check(_lib.load().wh_embedding_lookup(ggml_type, _p(table), vocab, hidden, idb.ptr, ids.size, _p(out),
                                               _s(stream)))
    return idb


class LlamaModel:
    """A Llama-shaped model on the device for the decode step: `layers` is a
    list of dicts of device buffers (attn_norm, wq, wk, wv, wo, ffn_norm,
    w_gate, w_up, w_down, k_cache, v_cache) and optionally a block type per
    matrix (wq_type .. w_down_type; absent or 0: ggml_type); wraps wh_llama_model."""

    def __init__(self, ggml_type: int, dims: dict, layers: list, inv_freq_dev, output_norm=None,
                 output=None, output_type: int = GGML_Q8_0, token_embd=None, token_embd_type: int = 0) -> None:
        self._keep = (layers, inv_freq_dev, output_norm, output, token_embd)
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
        m.token_embd_type = token_embd_type
        m.token_embd = _p(token_embd) or None
        self.model = m

    @staticmethod
    def config_from_gguf(ld, max_ctx: int | None = None) -> dict:
        """The model config of a GGUF file (gguf.GGUFLoader), read as
        GGUFModelLoader::extract_config does (model/loader.rs:104-150): the
        architecture from general.architecture (ValueError when absent, like
        the reference's "No architecture specified in GGUF"), then, each with
        its fallback key and default:
          hidden    {arch}.embedding_length, {arch}.embed_dim            4096
          n_layers  {arch}.block_count, {arch}.layer_count               32
          n_heads   {arch}.attention.head_count                          32
          n_kv      {arch}.attention.head_count_kv                       n_heads
          n_ff      {arch}.feed_forward_length                           4 x hidden
          max_ctx   {arch}.context_length, tokenizer.ggml.context_length 2048 (max_ctx overrides)
          vocab     {arch}.vocab_size, tokenizer.ggml.tokens.len         32000
          rope_base {arch}.rope.freq_base, {arch}.attention.rope_theta   10000
          eps       {arch}.attention.layer_norm_epsilon, {arch}.layer_norm_epsilon  1e-5"""
        md = ld.metadata()
        arch = md.get_string("general.architecture")
        if not arch:
            raise ValueError("No architecture specified in GGUF")

        def first(get, keys, default):
            for key in keys:
                v = get(key)
                if v is not None:
                    return v
            return default

        u32 = lambda keys, default: int(first(md.get_u32, keys, default))
        f32 = lambda keys, default: float(first(md.get_f32, keys, default))
        hidden = u32([f"{arch}.embedding_length", f"{arch}.embed_dim"], 4096)
        n_heads = u32([f"{arch}.attention.head_count"], 32)
        return dict(hidden=hidden, n_layers=u32([f"{arch}.block_count", f"{arch}.layer_count"], 32),
                    n_heads=n_heads, n_kv_heads=u32([f"{arch}.attention.head_count_kv"], n_heads),
                    head_dim=hidden // n_heads, n_ff=u32([f"{arch}.feed_forward_length"], 4 * hidden),
                    max_ctx=int(max_ctx) if max_ctx else u32([f"{arch}.context_length",
                                                              "tokenizer.ggml.context_length"], 2048),
                    vocab=u32([f"{arch}.vocab_size", "tokenizer.ggml.tokens.len"], 32000),
                    rope_base=f32([f"{arch}.rope.freq_base", f"{arch}.attention.rope_theta"], 10000.0),
                    eps=f32([f"{arch}.attention.layer_norm_epsilon", f"{arch}.layer_norm_epsilon"], 1e-5))

    @classmethod
    def from_gguf(cls, ld, max_ctx: int | None = None) -> "LlamaModel":
        """The decode model of a GGUF file (gguf.GGUFLoader): the config of
        config_from_gguf and the tensors load_layer_weights / load_model_weights
        name (model/loader.rs:370-520: token_embd.weight, blk.N.{attn_norm,
        attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up,
        ffn_down}.weight, output_norm.weight, output.weight).  Every matrix is
        uploaded from the mapping with its own block type (Q4_K_M files mix Q4_K
        and Q6_K) after its dims are checked against the config (ValueError on a
        mismatch, before anything reads past a tensor); without output.weight
        the head is token_embd.weight, tied as in lazy_transformer.rs:1301-1316.
        The f16 KV caches (max_ctx rows) start zeroed."""
        from .device import DeviceBuffer

        cfg = cls.config_from_gguf(ld, max_ctx)
        hidden, n_layers, n_heads, n_kv = cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"]
        n_ff, ctx, base, eps = cfg["n_ff"], cfg["max_ctx"], cfg["rope_base"], cfg["eps"]
        if n_heads == 0 or hidden % n_heads:
            raise ValueError(f"hidden size {hidden} is not a multiple of {n_heads} heads")
        d = hidden // n_heads
        # GGUF dims: [ne0 = K (fastest), ne1 = rows]
        shapes = {"attn_norm": [hidden], "wq": [hidden, n_heads * d], "wk": [hidden, n_kv * d],
                  "wv": [hidden, n_kv * d], "wo": [n_heads * d, hidden], "ffn_norm": [hidden],
                  "w_gate": [hidden, n_ff], "w_up": [hidden, n_ff], "w_down": [n_ff, hidden]}
        names = {"attn_norm": "attn_norm", "wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
                 "ffn_norm": "ffn_norm", "w_gate": "ffn_gate", "w_up": "ffn_up", "w_down": "ffn_down"}

        def info(name, want=None):
            ti = ld.tensor_info(name)
            if ti is None:
                from .gguf import TensorNotFound
                raise TensorNotFound(name)
            got = [int(v) for v in ti.shape()]
            if want is not None and got != want:
                raise ValueError(f"tensor {name} has dims {got}, the config needs {want}")
            return ti

        for i in range(n_layers):
            for key, nm in names.items():
                info(f"blk.{i}.{nm}.weight", shapes[key])
        embd = info("token_embd.weight") if ld.has_tensor("token_embd.weight") else None
        if embd is not None and (len(embd.shape()) != 2 or int(embd.shape()[0]) != hidden):
            raise ValueError(f"token_embd.weight has dims {list(embd.shape())}, the config needs [{hidden}, vocab]")
        tied = not ld.has_tensor("output.weight")
        if tied and embd is None:
            raise ValueError("GGUF file has neither output.weight nor token_embd.weight")
        head_info = embd if tied else info("output.weight")
        # the head is a quantized GEMV of one of these block types (a tied
        # F32 / F16 / Q5 embedding table would fail at the first logits step)
        head_types = (GGML_Q4_0, GGML_Q4_1, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K)
        if int(head_info.ggml_type) not in head_types:
            raise ValueError(f"output head {'token_embd.weight (tied)' if tied else 'output.weight'} has ggml type "
                             f"{int(head_info.ggml_type)}; the head GEMV takes Q4_0, Q4_1, Q8_0, Q4_K or Q6_K")
        if len(head_info.shape()) != 2 or int(head_info.shape()[0]) != hidden:
            raise ValueError(f"output head has dims {list(head_info.shape())}, the config needs [{hidden}, vocab]")
        vocab = int(head_info.shape()[1])
        if embd is not None and int(embd.shape()[1]) != vocab:
            raise ValueError(f"token_embd.weight has {int(embd.shape()[1])} rows, the head {vocab}")
        info("output_norm.weight", [hidden])

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
        embd_dev = ld.upload("token_embd.weight") if embd is not None else None
        head = embd_dev if tied else ld.upload("output.weight")
        dims = dict(hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=d, n_ff=n_ff, max_ctx=ctx,
                    vocab=vocab, eps=eps)
        m = cls(layers[0]["wq_type"] if layers else GGML_Q4_0, dims, layers, inv, out_norm, head,
                int(head_info.ggml_type), embd_dev, int(embd.ggml_type) if embd is not None else 0)
        m.dims = dims
        m.tied_head = tied
        return m

    def workspace_bytes(self) -> int:
        return int(_lib.load().wh_llama_decode_workspace_bytes(C.byref(self.model)))

    def layer_decode(self, layer: int, pos: int, x, workspace, workspace_bytes: int,
                     stream: Stream | None = None) -> None:
        _lib.check(_lib.load().wh_llama_layer_decode(C.byref(self.model), layer, pos, _p(x),
                                                     _p(workspace), workspace_bytes, _s(stream)))

    def forward_token(self, token_dev, pos: int, x, logits, workspace, workspace_bytes: int,
                      stream: Stream | None = None) -> None:
        """The step from a token id held in device memory (uint32 at token_dev):
        x = its embedding row, then decode_step (LazyTransformer::forward for
        one token, lazy_transformer.rs:1155-1336)."""
        _lib.check(_lib.load().wh_llama_forward_token(C.byref(self.model), _p(token_dev), pos, _p(x),
                                                      _p(logits) or None, _p(workspace), workspace_bytes,
                                                      _s(stream)))

    def decode_step(self, pos: int, x, logits, workspace, workspace_bytes: int,
                    stream: Stream | None = None) -> None:
        _lib.check(_lib.load().wh_llama_decode_step(C.byref(self.model), pos, _p(x),
                                                    _p(logits) or None, _p(workspace), workspace_bytes,
                                                    _s(stream)))
