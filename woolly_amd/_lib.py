"""ctypes binding of libwoolly_hip.so (the C ABI in include/woolly_hip.h).

The shared library is built in-tree by woolly_amd.build.  Loading it does not
touch the GPU; every entry point that needs one fails with WH_ERR_NO_DEVICE
(or a HIP error) when none is present.  There is no CPU fallback: if the
library is missing, load() raises.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwoolly_hip.so"

WH_OK = 0
WH_ERR_UNSUPPORTED_TYPE = 1
WH_ERR_INVALID_SHAPE = 2
WH_ERR_BUFFER_TOO_SMALL = 3
WH_ERR_INVALID_ARGUMENT = 4
WH_ERR_HIP = 5
WH_ERR_OOM = 6
WH_ERR_NO_DEVICE = 7
WH_ERR_IO = 8
WH_ERR_INVALID_MAGIC = 9
WH_ERR_UNSUPPORTED_VERSION = 10
WH_ERR_INVALID_METADATA = 11
WH_ERR_NOT_FOUND = 12
WH_ERR_TYPE_MISMATCH = 13

# WH_LLAMA_DECODE_NOALLOC_MAX_BYTES: the static scratch of wh_llama_decode_step_noalloc
LLAMA_DECODE_NOALLOC_MAX_BYTES = 16 << 20

STATUS_NAMES = {
    0: "WH_OK",
    1: "WH_ERR_UNSUPPORTED_TYPE",
    2: "WH_ERR_INVALID_SHAPE",
    3: "WH_ERR_BUFFER_TOO_SMALL",
    4: "WH_ERR_INVALID_ARGUMENT",
    5: "WH_ERR_HIP",
    6: "WH_ERR_OOM",
    7: "WH_ERR_NO_DEVICE",
    8: "WH_ERR_IO",
    9: "WH_ERR_INVALID_MAGIC",
    10: "WH_ERR_UNSUPPORTED_VERSION",
    11: "WH_ERR_INVALID_METADATA",
    12: "WH_ERR_NOT_FOUND",
    13: "WH_ERR_TYPE_MISMATCH",
}


class WoollyHipError(RuntimeError):
    """A non-zero wh_status returned by the C ABI."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.message = message
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class wh_ffn_weights(C.Structure):
    _fields_ = [
        ("type", C.c_int),
        ("gate", C.c_void_p),
        ("up", C.c_void_p),
        ("down", C.c_void_p),
        ("hidden", C.c_size_t),
        ("n_ff", C.c_size_t),
    ]


GGUF_MAX_DIMS = 8


class wh_gguf_header(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("tensor_count", C.c_uint64),
        ("metadata_kv_count", C.c_uint64),
        ("alignment", C.c_uint32),
        ("data_offset", C.c_uint64),
        ("file_size", C.c_uint64),
        ("total_tensor_size", C.c_uint64),
    ]


class wh_gguf_tensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("n_dims", C.c_uint32),
        ("dims", C.c_uint64 * GGUF_MAX_DIMS),
        ("ggml_type", C.c_int),
        ("offset", C.c_uint64),
        ("n_elements", C.c_uint64),
        ("data_size", C.c_uint64),
    ]


class wh_host_cache_stats(C.Structure):
    _fields_ = [
        ("hits", C.c_uint64),
        ("misses", C.c_uint64),
        ("evictions", C.c_uint64),
        ("entries", C.c_size_t),
        ("bytes", C.c_size_t),
        ("max_bytes", C.c_size_t),
    ]


class wh_llama_layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate",
                                          "w_up", "w_down", "k_cache", "v_cache")] + \
               [(n, C.c_int) for n in ("wq_type", "wk_type", "wv_type", "wo_type", "w_gate_type",
                                       "w_up_type", "w_down_type")]


class wh_llama_model(C.Structure):
    _fields_ = [
        ("type", C.c_int),
        ("n_layers", C.c_size_t), ("hidden", C.c_size_t), ("n_heads", C.c_size_t),
        ("n_kv_heads", C.c_size_t), ("head_dim", C.c_size_t), ("n_ff", C.c_size_t),
        ("max_ctx", C.c_size_t), ("vocab", C.c_size_t),
        ("eps", C.c_float),
        ("rope_inv_freq", C.c_void_p),
        ("layers", C.POINTER(wh_llama_layer)),
        ("output_norm", C.c_void_p),
        ("output_type", C.c_int),
        ("output", C.c_void_p),
        ("token_embd_type", C.c_int),
        ("token_embd", C.c_void_p),
    ]


_sz = C.c_size_t
_vp = C.c_void_p
_int = C.c_int
_f32p = C.c_void_p  # float* passed as raw addresses

# name -> (restype, argtypes).  This table is the list of exported symbols;
# tests check that it matches the declarations in include/woolly_hip.h.
SIGNATURES = {
    "wh_status_string": (C.c_char_p, [_int]),
    "wh_last_error": (C.c_char_p, []),
    "wh_version": (_int, []),
    "wh_gemv_select": (_int, [_int, C.POINTER(_int)]),
    "wh_init": (_int, [_int]),
    "wh_device_count": (_int, [C.POINTER(_int)]),
    "wh_device_name": (_int, [C.c_char_p, _sz]),
    "wh_malloc": (_int, [C.POINTER(_vp), _sz]),
    "wh_free": (_int, [_vp]),
    "wh_memcpy_h2d": (_int, [_vp, _vp, _sz, _vp]),
    "wh_memcpy_d2h": (_int, [_vp, _vp, _sz, _vp]),
    "wh_memcpy_d2d": (_int, [_vp, _vp, _sz, _vp]),
    "wh_fill_bytes": (_int, [_vp, _int, _sz, _vp]),
    "wh_read_probe": (_int, [_vp, _sz, _sz, _int, _vp, _vp]),
    "wh_stream_create": (_int, [C.POINTER(_vp)]),
    "wh_stream_destroy": (_int, [_vp]),
    "wh_stream_synchronize": (_int, [_vp]),
    "wh_device_synchronize": (_int, []),
    "wh_event_create": (_int, [C.POINTER(_vp)]),
    "wh_event_destroy": (_int, [_vp]),
    "wh_event_record": (_int, [_vp, _vp]),
    "wh_event_synchronize": (_int, [_vp]),
    "wh_event_elapsed_ms": (_int, [C.POINTER(C.c_float), _vp, _vp]),
    "wh_graph_begin_capture": (_int, [_vp]),
    "wh_graph_end_capture": (_int, [_vp, C.POINTER(_vp)]),
    "wh_graph_launch": (_int, [_vp, _vp]),
    "wh_graph_destroy": (_int, [_vp]),
    "wh_block_size": (_sz, [_int]),
    "wh_type_size": (_sz, [_int]),
    "wh_tensor_nbytes": (_int, [_int, C.c_uint64, C.POINTER(C.c_uint64)]),
    "wh_dequantize": (_int, [_int, _vp, _sz, _sz, _f32p, _vp]),
    "wh_quantized_matvec": (_int, [_int, _vp, _sz, _f32p, _f32p, _sz, _sz, _vp]),
    "wh_quantized_matmul_workspace_bytes": (_sz, [_int, _sz, _sz, _sz]),
    "wh_quantized_matmul": (_int, [_int, _vp, _sz, _sz, _sz, _f32p, _sz, _f32p, _vp, _sz, _vp]),
    "wh_quantized_matmul_x_workspace_bytes": (_sz, [_int, _sz, _sz, _sz, _int]),
    "wh_quantized_matmul_x": (_int, [_int, _vp, _sz, _sz, _sz, _vp, _int, _sz, _f32p, _vp, _sz, _vp]),
    "wh_set_stream_k_wait": (_int, [C.c_uint32]),
    "wh_rms_norm": (_int, [_f32p, _f32p, C.c_float, _sz, _sz, _f32p, _vp]),
    "wh_swiglu": (_int, [_f32p, _f32p, _sz, _f32p, _vp]),
    "wh_ffn_workspace_bytes": (_sz, [_sz, _sz, _sz]),
    "wh_ffn_workspace_bytes_for_type": (_sz, [_int, _sz, _sz, _sz]),
    "wh_ffn_swiglu": (_int, [C.POINTER(wh_ffn_weights), _f32p, C.c_float, _f32p, _sz, _f32p,
                             _vp, _sz, _vp]),
    "wh_weight_upload": (_int, [_int, _sz, _sz, _vp, _sz, C.POINTER(_vp)]),
    "wh_weight_free": (_int, [_vp]),
    "wh_weight_data": (_vp, [_vp]),
    "wh_weight_info": (_int, [_vp, C.POINTER(_int), C.POINTER(_sz), C.POINTER(_sz),
                              C.POINTER(_sz)]),
    "wh_weight_prepare_prefill": (_int, [_vp, _vp, C.POINTER(_sz)]),
    "wh_dequantize_host": (_int, [_int, _vp, _sz, _sz, _f32p]),
    "wh_quantized_matvec_host": (_int, [_int, _vp, _sz, _f32p, _f32p, _sz, _sz]),
    "wh_host_cache_configure": (_int, [_sz]),
    "wh_host_cache_evict": (_int, [_vp, _sz, C.POINTER(_sz)]),
    "wh_host_cache_clear": (_int, []),
    "wh_host_cache_get_stats": (_int, [C.POINTER(wh_host_cache_stats)]),
    "wh_rope_inv_freq": (_int, [C.c_float, _sz, _vp]),
    "wh_attention_qkv_workspace_bytes": (_sz, [_sz]),
    "wh_attention_qkv": (_int, [_int, _vp, _vp, _vp, _sz, _sz, _sz, _f32p, C.c_float, _f32p, _f32p,
                                _vp, _sz, _vp]),
    "wh_attention_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
    "wh_attention_decode": (_int, [_f32p, _vp, _vp, _sz, _sz, _sz, _sz, _f32p, _f32p, _vp, _sz, _vp]),
    "wh_quantized_matvec_residual": (_int, [_int, _vp, _sz, _f32p, _f32p, _f32p, _sz, _sz, _vp]),
    "wh_llama_decode_workspace_bytes": (_sz, [C.POINTER(wh_llama_model)]),
    "wh_llama_layer_decode": (_int, [C.POINTER(wh_llama_model), _sz, _sz, _f32p, _vp, _sz, _vp]),
    "wh_llama_decode_step": (_int, [C.POINTER(wh_llama_model), _sz, _f32p, _f32p, _vp, _sz, _vp]),
    "wh_llama_forward_token": (_int, [C.POINTER(wh_llama_model), _vp, _sz, _f32p, _f32p, _vp, _sz, _vp]),
    "wh_embedding_lookup": (_int, [_int, _vp, _sz, _sz, _vp, _sz, _f32p, _vp]),
    "wh_llama_decode_step_noalloc": (_int, [C.POINTER(wh_llama_model), _sz, _f32p, _f32p, _vp]),
    "wh_gguf_open": (_int, [C.c_char_p, C.POINTER(_vp)]),
    "wh_gguf_open_buffer": (_int, [_vp, _sz, C.POINTER(_vp)]),
    "wh_gguf_close": (_int, [_vp]),
    "wh_gguf_get_header": (_int, [_vp, C.POINTER(wh_gguf_header)]),
    "wh_gguf_tensor_at": (_int, [_vp, C.c_uint64, C.POINTER(wh_gguf_tensor)]),
    "wh_gguf_find_tensor": (_int, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "wh_gguf_tensor_data": (_int, [_vp, C.c_uint64, C.POINTER(_vp), C.POINTER(_sz)]),
    "wh_gguf_upload": (_int, [_vp, C.c_uint64, C.POINTER(_vp)]),
    "wh_gguf_kv_at": (_int, [_vp, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(_int)]),
    "wh_gguf_find_kv": (_int, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "wh_gguf_get_u32": (_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "wh_gguf_get_u64": (_int, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "wh_gguf_get_i32": (_int, [_vp, C.c_char_p, C.POINTER(C.c_int32)]),
    "wh_gguf_get_f32": (_int, [_vp, C.c_char_p, C.POINTER(C.c_float)]),
    "wh_gguf_get_bool": (_int, [_vp, C.c_char_p, C.POINTER(_int)]),
    "wh_gguf_get_string": (_int, [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(_sz)]),
    "wh_gguf_kv_scalar": (_int, [_vp, C.c_uint64, C.POINTER(_int), _vp]),
    "wh_gguf_kv_array": (_int, [_vp, C.c_uint64, C.POINTER(_int), C.POINTER(C.c_uint64),
                                C.POINTER(_vp)]),
    "wh_gguf_kv_array_string": (_int, [_vp, C.c_uint64, C.c_uint64, C.POINTER(_vp),
                                       C.POINTER(_sz)]),
    "wh_gguf_kv_string": (_int, [_vp, C.c_uint64, C.POINTER(_vp), C.POINTER(_sz)]),
    "wh_ggml_type_traits": (_int, [_int, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_int)]),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Loads libwoolly_hip.so (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m woolly_amd.build` "
                "(there is no CPU fallback for the HIP path)")
        lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    return load().wh_last_error().decode(errors="replace")


def check(status: int) -> None:
    """Raises WoollyHipError for a non-zero status."""
    if status != WH_OK:
        raise WoollyHipError(status, last_error())
