"""The C ABI library loads, exports every declared symbol, and reports the
reference's error semantics for bad arguments without touching a GPU."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from woolly_amd import _lib, gguf, quantization

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "woolly_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"WH_API\s+[\w\s\*]+?\b(wh_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), f"{n} declared in woolly_hip.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_library_is_gfx950_only():
    data = (ROOT / "woolly_amd" / "libwoolly_hip.so").read_bytes()
    assert b"gfx950" in data


def test_format_queries():
    lib = _lib.load()
    assert lib.wh_type_size(2) == 18 and lib.wh_type_size(3) == 20 and lib.wh_type_size(8) == 34
    assert lib.wh_block_size(2) == 32 and lib.wh_block_size(0) == 1 and lib.wh_block_size(10) == 0
    # dequantize.rs:213, 230-231: Q5_0 / Q5_1 are 32-element blocks of 22 / 24 bytes
    assert lib.wh_block_size(6) == 32 and lib.wh_type_size(6) == 22
    assert lib.wh_block_size(7) == 32 and lib.wh_type_size(7) == 24
    # dequantize.rs:208-242: Q4_K / Q6_K are 256-element blocks of 144 / 210 bytes
    assert lib.wh_block_size(12) == 256 and lib.wh_type_size(12) == 144
    assert lib.wh_block_size(14) == 256 and lib.wh_type_size(14) == 210
    assert gguf.data_size(gguf.GGMLType.Q6_K, 4096 + 1) == 17 * 210
    # tensor_info.rs:292-305: 64x64 Q4_0 -> 2304 bytes; 4x8 F32 -> 128 bytes
    assert gguf.data_size(gguf.GGMLType.Q4_0, 4096) == 2304
    assert gguf.data_size(gguf.GGMLType.F32, 32) == 128
    assert gguf.get_type_size(gguf.GGMLType.Q8_0) == 34
    assert lib.wh_status_string(2) == b"WH_ERR_INVALID_SHAPE"


def test_matvec_argument_errors_need_no_gpu():
    lib = _lib.load()
    w = np.zeros(2 * 18 * 2, np.uint8)
    x = np.zeros(64, np.float32)
    y = np.zeros(2, np.float32)
    # k % 32 != 0 -> the reference's assert_eq! panic becomes WH_ERR_INVALID_SHAPE
    assert lib.wh_quantized_matvec(2, w.ctypes.data, w.nbytes, x.ctypes.data, y.ctypes.data,
                                   2, 48, None) == _lib.WH_ERR_INVALID_SHAPE
    assert b"multiple of the block size" in lib.wh_last_error()
    # unsupported scheme (Q5_0, id 6) -> UnsupportedScheme
    assert lib.wh_quantized_matvec(6, w.ctypes.data, w.nbytes, x.ctypes.data, y.ctypes.data,
                                   2, 64, None) == _lib.WH_ERR_UNSUPPORTED_TYPE
    # Q4_K rows are whole 256-element blocks
    assert lib.wh_quantized_matvec(12, w.ctypes.data, w.nbytes, x.ctypes.data, y.ctypes.data,
                                   2, 64, None) == _lib.WH_ERR_INVALID_SHAPE
    assert b"block size 256" in lib.wh_last_error()
    assert lib.wh_quantized_matvec(14, w.ctypes.data, 2 * 210 - 1, x.ctypes.data, y.ctypes.data,
                                   2, 256, None) == _lib.WH_ERR_BUFFER_TOO_SMALL
    # too few weight bytes -> BufferTooSmall{needed, available}
    assert lib.wh_quantized_matvec(2, w.ctypes.data, 71, x.ctypes.data, y.ctypes.data,
                                   2, 64, None) == _lib.WH_ERR_BUFFER_TOO_SMALL
    assert b"needed 72 bytes, available 71" in lib.wh_last_error()
    # m == 0 is a no-op
    assert lib.wh_quantized_matvec(2, None, 0, None, None, 0, 64, None) == _lib.WH_OK
    # null output with work to do
    assert lib.wh_quantized_matvec(2, w.ctypes.data, w.nbytes, x.ctypes.data, None,
                                   2, 64, None) == _lib.WH_ERR_INVALID_ARGUMENT


def test_dequant_argument_errors_need_no_gpu():
    with pytest.raises(gguf.BufferTooSmall) as e:
        gguf.dequantize(bytes(35), gguf.GGMLType.Q4_0, 64)
    assert e.value.needed == 36 and e.value.available == 35
    with pytest.raises(gguf.InvalidTensorType):
        gguf.dequantize(bytes(84), gguf.GGMLType.Q2_K, 256)
    # Q5_0 / Q5_1 blocks are 22 / 24 bytes (quantization.rs:1353-1354)
    with pytest.raises(gguf.BufferTooSmall) as e:
        gguf.dequantize(bytes(43), gguf.GGMLType.Q5_0, 64)
    assert e.value.needed == 44 and e.value.available == 43
    with pytest.raises(gguf.BufferTooSmall) as e:
        gguf.dequantize(bytes(23), gguf.GGMLType.Q5_1, 32)
    assert e.value.needed == 24
    # a short K-quant block is InvalidTensorInfo (dequantize.rs:416-418, 472-474)
    with pytest.raises(gguf.InvalidTensorInfo):
        gguf.dequantize(bytes(143), gguf.GGMLType.Q4_K, 256)
    with pytest.raises(gguf.InvalidTensorInfo):
        gguf.dequantize(bytes(210), gguf.GGMLType.Q6_K, 257)
    with pytest.raises(gguf.BufferTooSmall):
        gguf.dequantize(bytes(10), gguf.GGMLType.F32, 4)   # F32 needs exactly 16 bytes
    assert gguf.dequantize(b"", gguf.GGMLType.Q4_0, 0).size == 0


def test_python_mirror_errors_need_no_gpu():
    st = quantization.QuantizedStorage(quantization.QuantizationScheme.Q5_0, np.zeros(22, np.uint8))
    with pytest.raises(quantization.QuantizationError.UnsupportedScheme):
        quantization.simd.quantized_matvec(st, np.zeros(32, np.float32), np.zeros(1, np.float32),
                                           1, 32)
    st = quantization.QuantizedStorage.Q4_0(np.zeros(18, np.uint8))
    with pytest.raises(quantization.QuantizationError.InvalidParameters):
        quantization.simd.quantized_matvec(st, np.zeros(48, np.float32), np.zeros(1, np.float32),
                                           1, 48)


def test_ffn_and_weight_argument_errors_need_no_gpu():
    lib = _lib.load()
    w = _lib.wh_ffn_weights(2, 1, 1, 1, 4096, 14336)
    assert lib.wh_ffn_swiglu(C.byref(w), 1, 1e-5, 1, 1, 1, 1, 0, None) == _lib.WH_ERR_BUFFER_TOO_SMALL
    w = _lib.wh_ffn_weights(2, 1, 1, 1, 4010, 14336)
    assert lib.wh_ffn_swiglu(C.byref(w), 1, 1e-5, 1, 1, 1, 1, 1 << 40, None) == _lib.WH_ERR_INVALID_SHAPE
    assert lib.wh_ffn_workspace_bytes(4096, 14336, 1) >= 4 * (4096 + 3 * 14336)
    # K-quant FFN and GEMM: whole 256-element blocks; no GEMM workspace for 1-2 tokens
    w = _lib.wh_ffn_weights(14, 1, 1, 1, 4096 + 32, 14336)
    assert lib.wh_ffn_swiglu(C.byref(w), 1, 1e-5, 1, 1, 1, 1, 1 << 40, None) == _lib.WH_ERR_INVALID_SHAPE
    assert b"block size 256" in lib.wh_last_error()
    assert lib.wh_ffn_workspace_bytes_for_type(12, 4096, 14336, 1) == lib.wh_ffn_workspace_bytes(4096, 14336, 1)
    assert lib.wh_quantized_matmul_workspace_bytes(12, 4096, 4096, 2) == 0
    assert lib.wh_quantized_matmul(12, 1, 1 << 40, 8, 64, 1, 4, 1, None, 0, None) == _lib.WH_ERR_INVALID_SHAPE
    h = C.c_void_p()
    assert lib.wh_weight_upload(2, 4, 48, None, 0, C.byref(h)) == _lib.WH_ERR_INVALID_SHAPE
    assert lib.wh_weight_upload(2, 4, 64, None, 10, C.byref(h)) == _lib.WH_ERR_BUFFER_TOO_SMALL
    # K-quants: 256-element blocks, 144 / 210 bytes each
    assert lib.wh_weight_upload(12, 4, 64, None, 0, C.byref(h)) == _lib.WH_ERR_INVALID_SHAPE
    assert lib.wh_weight_upload(14, 4, 256, None, 4 * 210 - 1, C.byref(h)) == _lib.WH_ERR_BUFFER_TOO_SMALL
    assert h.value is None


def test_cpp_mirror_header_compiles_and_links():
    """include/woolly_hip.hpp compiles stand-alone (C++17, -Werror) and the
    mirror's test program links against the library (no GPU needed to build)."""
    import subprocess

    root = Path(__file__).resolve().parent.parent
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-x",
                    "c++", "-I", str(root / "include"), "-"],
                   input=b'#include "woolly_hip.hpp"\n', check=True)
    subprocess.run(["make", "-s", "-C", str(root / "tests" / "cpp")], check=True)
    assert (root / "tests" / "cpp" / "_build" / "test_mirror").exists()


def _fake_model(n_layers=2, null_field=None, output_type=8, logits_head=True):
    """A wh_llama_model whose device pointers are fake non-null addresses: the
    step's checks must reject it before any launch."""
    layers = (_lib.wh_llama_layer * n_layers)()
    for L in layers:
        for name, _ in _lib.wh_llama_layer._fields_:
            if not name.endswith("_type"):
                setattr(L, name, 0x10000)
    if null_field is not None:
        setattr(layers[n_layers - 1], null_field, None)
    m = _lib.wh_llama_model()
    m.type = 2
    m.n_layers, m.hidden, m.n_heads, m.n_kv_heads, m.head_dim = n_layers, 256, 4, 2, 64
    m.n_ff, m.max_ctx, m.vocab, m.eps = 512, 16, 300, 1e-5
    m.rope_inv_freq = 0x10000
    m.layers = C.cast(layers, C.POINTER(_lib.wh_llama_layer))
    m.output_norm = 0x10000 if logits_head else None
    m.output_type = output_type
    m.output = 0x10000
    return m, layers


@pytest.mark.parametrize("field", ["attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down"])
def test_decode_step_rejects_null_layer_pointers(field):
    """Every matrix and norm of every layer must be non-null: a null pointer is
    WH_ERR_INVALID_ARGUMENT naming it, reported before anything is launched."""
    lib = _lib.load()
    m, keep = _fake_model(null_field=field)
    st = lib.wh_llama_decode_step(C.byref(m), 0, 0x10000, 0x10000, 0x10000, 1 << 30, None)
    assert st == _lib.WH_ERR_INVALID_ARGUMENT
    assert f"layer 1 {field} is a null pointer".encode() in lib.wh_last_error()


def test_decode_step_checks_the_head_before_any_layer():
    """A bad output head (unsupported type, null output_norm) fails before the
    first layer is launched, so x and the caches are left as they were: with
    fake device pointers a launch would report a HIP error instead."""
    lib = _lib.load()
    m, keep = _fake_model(output_type=6)
    assert lib.wh_llama_decode_step(C.byref(m), 0, 0x10000, 0x10000, 0x10000, 1 << 30, None) == \
        _lib.WH_ERR_UNSUPPORTED_TYPE
    assert b"output head" in lib.wh_last_error()
    m, keep = _fake_model(logits_head=False)
    assert lib.wh_llama_decode_step(C.byref(m), 0, 0x10000, 0x10000, 0x10000, 1 << 30, None) == \
        _lib.WH_ERR_INVALID_ARGUMENT
    assert b"output_norm" in lib.wh_last_error()
    # forward_token without a token_embd table
    m, keep = _fake_model()
    assert lib.wh_llama_forward_token(C.byref(m), 0x10000, 0, 0x10000, 0x10000, 0x10000, 1 << 30, None) == \
        _lib.WH_ERR_INVALID_ARGUMENT
    assert b"token_embd" in lib.wh_last_error()


def test_embedding_lookup_argument_errors_need_no_gpu():
    lib = _lib.load()
    # Q2_K (10) has no embedding decoder; Q5_0 (6) has one, so its shape is checked next
    assert lib.wh_embedding_lookup(10, 0x10000, 10, 256, 0x10000, 1, 0x10000, None) == _lib.WH_ERR_UNSUPPORTED_TYPE
    assert lib.wh_embedding_lookup(6, 0x10000, 10, 48, 0x10000, 1, 0x10000, None) == _lib.WH_ERR_INVALID_SHAPE
    assert lib.wh_embedding_lookup(12, 0x10000, 10, 128, 0x10000, 1, 0x10000, None) == _lib.WH_ERR_INVALID_SHAPE
    assert lib.wh_embedding_lookup(2, None, 10, 256, 0x10000, 1, 0x10000, None) == _lib.WH_ERR_INVALID_ARGUMENT
    assert lib.wh_embedding_lookup(2, 0x10000, 10, 256, 0x10000, 0, 0x10000, None) == _lib.WH_OK
    from woolly_amd import ops
    with pytest.raises(ValueError, match="Token ID 10 exceeds vocabulary size 10"):
        ops.embedding_lookup(2, 0x10000, 10, 256, [3, 10], 0x10000)
