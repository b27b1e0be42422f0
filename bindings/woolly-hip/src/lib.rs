//! `woolly-hip`: Rust bindings of libwoolly_hip.so, the MI355X (gfx950)
//! backend of woolly's quantized matmul hot path.
//!
//! The raw declarations at the crate root are one-to-one with
//! `include/woolly_hip.h` (every `WH_API` entry point, every `#[repr(C)]`
//! struct with its fields in header order, and the status / type constants).
//! The `safe` module wraps the entry points woolly's call sites need in
//! woolly's own shapes: `Result` instead of status codes, slices instead of
//! pointer/length pairs, and RAII handles for device memory, streams and
//! uploaded weights.
//!
//! Call sites this crate serves (reference files):
//! * `simd::quantized_matvec` (crates/woolly-tensor/src/quantization.rs:869-909)
//!   and `dequantize_q4_0/_q4_1/_q8_0` (quantization.rs:466-590):
//!   [`wh_quantized_matvec`], [`wh_quantized_matvec_host`], [`wh_dequantize`],
//!   [`wh_dequantize_host`];
//! * `woolly_gguf::dequantize` (crates/woolly-gguf/src/dequantize.rs:189-205) and the
//!   GGUF loader (crates/woolly-gguf/src/loader.rs:111-295): [`wh_dequantize`],
//!   the `wh_gguf_*` functions, [`wh_gguf_upload`];
//! * `compute_simd_swiglu_ffn` / `process_layer` / `forward`
//!   (crates/woolly-core/src/model/lazy_transformer.rs:98-258, 1073-1123, 1155-1335):
//!   [`wh_ffn_swiglu`], [`wh_quantized_matmul`], [`wh_attention_qkv`],
//!   [`wh_attention_decode`], [`wh_llama_decode_step`], [`wh_llama_forward_token`].
//!
//! All device pointers are addresses from [`wh_malloc`] (or any HIP device
//! allocation); kernel entry points are asynchronous on the given stream.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_float, c_int, c_void};

// ------------------------------------------------------------------ status codes
pub const WH_OK: c_int = 0;
pub const WH_ERR_UNSUPPORTED_TYPE: c_int = 1;
pub const WH_ERR_INVALID_SHAPE: c_int = 2;
pub const WH_ERR_BUFFER_TOO_SMALL: c_int = 3;
pub const WH_ERR_INVALID_ARGUMENT: c_int = 4;
pub const WH_ERR_HIP: c_int = 5;
pub const WH_ERR_OOM: c_int = 6;
pub const WH_ERR_NO_DEVICE: c_int = 7;
pub const WH_ERR_IO: c_int = 8;
pub const WH_ERR_INVALID_MAGIC: c_int = 9;
pub const WH_ERR_UNSUPPORTED_VERSION: c_int = 10;
pub const WH_ERR_INVALID_METADATA: c_int = 11;
pub const WH_ERR_NOT_FOUND: c_int = 12;
pub const WH_ERR_TYPE_MISMATCH: c_int = 13;

// ------------------------------------------------- GGMLType ids (tensor_info.rs:15-30)
pub const WH_TYPE_F32: c_int = 0;
pub const WH_TYPE_F16: c_int = 1;
pub const WH_TYPE_Q4_0: c_int = 2;
pub const WH_TYPE_Q4_1: c_int = 3;
pub const WH_TYPE_Q5_0: c_int = 6;
pub const WH_TYPE_Q5_1: c_int = 7;
pub const WH_TYPE_Q8_0: c_int = 8;
pub const WH_TYPE_Q4_K: c_int = 12;
pub const WH_TYPE_Q6_K: c_int = 14;
pub const WH_TYPE_BF16: c_int = 30;

// ------------------------------------------------------- single-token GEMV kernels
pub const WH_GEMV_AUTO: c_int = 0;
pub const WH_GEMV_STREAM: c_int = 1;

// --------------------------------------------------------------------- limits
pub const WH_LLAMA_DECODE_NOALLOC_MAX_BYTES: usize = 16 << 20;
pub const WH_GGUF_MAX_DIMS: usize = 8;

// ------------------------------------------ GGUF metadata value types (metadata.rs:13-42)
pub const WH_GGUF_U8: c_int = 0;
pub const WH_GGUF_I8: c_int = 1;
pub const WH_GGUF_U16: c_int = 2;
pub const WH_GGUF_I16: c_int = 3;
pub const WH_GGUF_U32: c_int = 4;
pub const WH_GGUF_I32: c_int = 5;
pub const WH_GGUF_F32: c_int = 6;
pub const WH_GGUF_BOOL: c_int = 7;
pub const WH_GGUF_STRING: c_int = 8;
pub const WH_GGUF_ARRAY: c_int = 9;
pub const WH_GGUF_U64: c_int = 10;
pub const WH_GGUF_I64: c_int = 11;
pub const WH_GGUF_F64: c_int = 12;

// ---------------------------------------------------------------- opaque handles
#[repr(C)]
pub struct wh_stream_opaque {
    _private: [u8; 0],
}
#[repr(C)]
pub struct wh_event_opaque {
    _private: [u8; 0],
}
#[repr(C)]
pub struct wh_graph_opaque {
    _private: [u8; 0],
}
/// A device-resident quantized tensor (`wh_weight_upload`).
#[repr(C)]
pub struct wh_weight {
    _private: [u8; 0],
}
/// A parsed, memory-mapped GGUF file (`wh_gguf_open`).
#[repr(C)]
pub struct wh_gguf {
    _private: [u8; 0],
}
/// A hipStream_t; null is the device's null stream.
pub type wh_stream_t = *mut wh_stream_opaque;
/// A hipEvent_t.
pub type wh_event_t = *mut wh_event_opaque;
/// An instantiated hipGraphExec_t.
pub type wh_graph_t = *mut wh_graph_opaque;

// ------------------------------------------------------------------------ structs
/// The weights of one SwiGLU feed-forward layer (`wh_ffn_swiglu`).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct wh_ffn_weights {
    pub r#type: c_int,
    pub gate: *const c_void,
    pub up: *const c_void,
    pub down: *const c_void,
    pub hidden: usize,
    pub n_ff: usize,
}

/// Counters of the device copies kept behind the `*_host` variants.
#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct wh_host_cache_stats {
    pub hits: u64,
    pub misses: u64,
    pub evictions: u64,
    pub entries: usize,
    pub bytes: usize,
    pub max_bytes: usize,
}

/// One decoder layer (device pointers); a `*_type` of 0 means the model's type.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct wh_llama_layer {
    pub attn_norm: *const c_float,
    pub wq: *const c_void,
    pub wk: *const c_void,
    pub wv: *const c_void,
    pub wo: *const c_void,
    pub ffn_norm: *const c_float,
    pub w_gate: *const c_void,
    pub w_up: *const c_void,
    pub w_down: *const c_void,
    pub k_cache: *mut c_void,
    pub v_cache: *mut c_void,
    pub wq_type: c_int,
    pub wk_type: c_int,
    pub wv_type: c_int,
    pub wo_type: c_int,
    pub w_gate_type: c_int,
    pub w_up_type: c_int,
    pub w_down_type: c_int,
}

/// A Llama-shaped model for the decode step; `layers` is a host array.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct wh_llama_model {
    pub r#type: c_int,
    pub n_layers: usize,
    pub hidden: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub head_dim: usize,
    pub n_ff: usize,
    pub max_ctx: usize,
    pub vocab: usize,
    pub eps: c_float,
    pub rope_inv_freq: *const c_float,
    pub layers: *const wh_llama_layer,
    pub output_norm: *const c_float,
    pub output_type: c_int,
    pub output: *const c_void,
    pub token_embd_type: c_int,
    pub token_embd: *const c_void,
}

/// GGUF header and layout figures (`wh_gguf_get_header`).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct wh_gguf_header {
    pub version: u32,
    pub tensor_count: u64,
    pub metadata_kv_count: u64,
    pub alignment: u32,
    pub data_offset: u64,
    pub file_size: u64,
    pub total_tensor_size: u64,
}

/// One tensor of a GGUF file (`wh_gguf_tensor_at`); `name` lives with the handle.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct wh_gguf_tensor {
    pub name: *const c_char,
    pub n_dims: u32,
    pub dims: [u64; WH_GGUF_MAX_DIMS],
    pub ggml_type: c_int,
    pub offset: u64,
    pub n_elements: u64,
    pub data_size: u64,
}

// -------------------------------------------------------------------- entry points
extern "C" {
    // errors and version
    pub fn wh_status_string(status: c_int) -> *const c_char;
    pub fn wh_last_error() -> *const c_char;
    pub fn wh_version() -> c_int;

    // device, memory, streams, events
    pub fn wh_init(device: c_int) -> c_int;
    pub fn wh_device_count(count: *mut c_int) -> c_int;
    pub fn wh_device_name(buf: *mut c_char, len: usize) -> c_int;
    pub fn wh_malloc(dptr: *mut *mut c_void, nbytes: usize) -> c_int;
    pub fn wh_free(dptr: *mut c_void) -> c_int;
    pub fn wh_memcpy_h2d(dst: *mut c_void, src: *const c_void, nbytes: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_memcpy_d2h(dst: *mut c_void, src: *const c_void, nbytes: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_memcpy_d2d(dst: *mut c_void, src: *const c_void, nbytes: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_fill_bytes(dst: *mut c_void, value: c_int, nbytes: usize, stream: wh_stream_t) -> c_int;
    // measurement aid (no counterpart in the reference)
    pub fn wh_read_probe(src: *const c_void, row_bytes: usize, n_rows: usize, mode: c_int, out: *mut u32,
                         stream: wh_stream_t) -> c_int;
    pub fn wh_stream_create(out: *mut wh_stream_t) -> c_int;
    pub fn wh_stream_destroy(stream: wh_stream_t) -> c_int;
    pub fn wh_stream_synchronize(stream: wh_stream_t) -> c_int;
    pub fn wh_device_synchronize() -> c_int;
    pub fn wh_event_create(out: *mut wh_event_t) -> c_int;
    pub fn wh_event_destroy(event: wh_event_t) -> c_int;
    pub fn wh_event_record(event: wh_event_t, stream: wh_stream_t) -> c_int;
    pub fn wh_event_synchronize(event: wh_event_t) -> c_int;
    pub fn wh_event_elapsed_ms(ms: *mut c_float, start: wh_event_t, end: wh_event_t) -> c_int;

    // HIP graphs of the launch-only entry points
    pub fn wh_graph_begin_capture(stream: wh_stream_t) -> c_int;
    pub fn wh_graph_end_capture(stream: wh_stream_t, out: *mut wh_graph_t) -> c_int;
    pub fn wh_graph_launch(graph: wh_graph_t, stream: wh_stream_t) -> c_int;
    pub fn wh_graph_destroy(graph: wh_graph_t) -> c_int;

    // formats (dequantize.rs:208-242, tensor_info.rs:244-255)
    pub fn wh_block_size(r#type: c_int) -> usize;
    pub fn wh_type_size(r#type: c_int) -> usize;
    pub fn wh_tensor_nbytes(r#type: c_int, nelements: u64, nbytes: *mut u64) -> c_int;

    // dequantization (dequantize.rs:189-205, quantization.rs:466-590)
    pub fn wh_dequantize(r#type: c_int, data: *const c_void, nbytes: usize, nelements: usize, out: *mut c_float,
                         stream: wh_stream_t) -> c_int;

    // quantized GEMV (quantization.rs:869-909)
    pub fn wh_quantized_matvec(r#type: c_int, weights: *const c_void, weight_nbytes: usize, input: *const c_float,
                               output: *mut c_float, m: usize, k: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_gemv_select(mode: c_int, previous: *mut c_int) -> c_int;

    // quantized GEMM (ops/matmul.rs:83-259 on dequantized weights)
    pub fn wh_quantized_matmul_workspace_bytes(r#type: c_int, n_rows: usize, k: usize, n_tokens: usize) -> usize;
    pub fn wh_quantized_matmul(r#type: c_int, weights: *const c_void, weight_nbytes: usize, n_rows: usize, k: usize,
                               x: *const c_float, n_tokens: usize, y: *mut c_float, workspace: *mut c_void,
                               workspace_bytes: usize, stream: wh_stream_t) -> c_int;

    pub fn wh_quantized_matmul_x_workspace_bytes(r#type: c_int, n_rows: usize, k: usize, n_tokens: usize,
                                                 x_dtype: c_int) -> usize;
    pub fn wh_quantized_matmul_x(r#type: c_int, weights: *const c_void, weight_nbytes: usize, n_rows: usize, k: usize,
                                 x: *const c_void, x_dtype: c_int, n_tokens: usize, y: *mut c_float,
                                 workspace: *mut c_void, workspace_bytes: usize, stream: wh_stream_t) -> c_int;
    // tuning knob (no counterpart in the reference)
    pub fn wh_set_stream_k_wait(ticks: u32) -> c_int;

    // elementwise (tensor_utils.rs:446-480, 512-532)
    pub fn wh_rms_norm(x: *const c_float, weight: *const c_float, eps: c_float, tokens: usize, hidden: usize,
                       out: *mut c_float, stream: wh_stream_t) -> c_int;
    pub fn wh_swiglu(gate: *const c_float, up: *const c_float, n: usize, out: *mut c_float,
                     stream: wh_stream_t) -> c_int;

    // SwiGLU FFN layer (lazy_transformer.rs:1073-1123)
    pub fn wh_ffn_workspace_bytes(hidden: usize, n_ff: usize, m: usize) -> usize;
    pub fn wh_ffn_workspace_bytes_for_type(r#type: c_int, hidden: usize, n_ff: usize, m: usize) -> usize;
    pub fn wh_ffn_swiglu(weights: *const wh_ffn_weights, gamma: *const c_float, eps: c_float, x: *const c_float,
                         m: usize, out: *mut c_float, workspace: *mut c_void, workspace_bytes: usize,
                         stream: wh_stream_t) -> c_int;

    // device-resident weights (loader.rs:274-291)
    pub fn wh_weight_upload(r#type: c_int, n_rows: usize, k: usize, host_bytes: *const c_void, nbytes: usize,
                            out: *mut *mut wh_weight) -> c_int;
    pub fn wh_weight_free(weight: *mut wh_weight) -> c_int;
    pub fn wh_weight_data(weight: *const wh_weight) -> *const c_void;
    pub fn wh_weight_info(weight: *const wh_weight, r#type: *mut c_int, n_rows: *mut usize, k: *mut usize,
                          nbytes: *mut usize) -> c_int;
    // convert-once copy for prefill (dequantization_cache.rs:121-165)
    pub fn wh_weight_prepare_prefill(weight: *mut wh_weight, stream: wh_stream_t, prepared_bytes: *mut usize)
                                     -> c_int;

    // synchronous host-memory variants
    pub fn wh_dequantize_host(r#type: c_int, data: *const c_void, nbytes: usize, nelements: usize,
                              out: *mut c_float) -> c_int;
    pub fn wh_quantized_matvec_host(r#type: c_int, weights: *const c_void, weight_nbytes: usize,
                                    input: *const c_float, output: *mut c_float, m: usize, k: usize) -> c_int;
    // device copies of host weights behind the host variants (dequantization_cache.rs:121-165)
    pub fn wh_host_cache_configure(max_bytes: usize) -> c_int;
    pub fn wh_host_cache_evict(host_ptr: *const c_void, nbytes: usize, evicted: *mut usize) -> c_int;
    pub fn wh_host_cache_clear() -> c_int;
    pub fn wh_host_cache_get_stats(out: *mut wh_host_cache_stats) -> c_int;

    // decode step (lazy_transformer.rs:98-456, 1155-1335)
    pub fn wh_rope_inv_freq(base: c_float, head_dim: usize, out_host: *mut c_float) -> c_int;
    pub fn wh_attention_qkv_workspace_bytes(hidden: usize) -> usize;
    pub fn wh_attention_qkv(r#type: c_int, wq: *const c_void, wk: *const c_void, wv: *const c_void, q_rows: usize,
                            kv_rows: usize, hidden: usize, gamma: *const c_float, eps: c_float, x: *const c_float,
                            qkv: *mut c_float, workspace: *mut c_void, workspace_bytes: usize,
                            stream: wh_stream_t) -> c_int;
    pub fn wh_attention_workspace_bytes(n_heads: usize, n_kv_heads: usize, head_dim: usize, max_ctx: usize) -> usize;
    pub fn wh_attention_decode(qkv: *const c_float, k_cache: *mut c_void, v_cache: *mut c_void, pos: usize,
                               n_heads: usize, n_kv_heads: usize, head_dim: usize, inv_freq: *const c_float,
                               out: *mut c_float, workspace: *mut c_void, workspace_bytes: usize,
                               stream: wh_stream_t) -> c_int;
    pub fn wh_quantized_matvec_residual(r#type: c_int, weights: *const c_void, weight_nbytes: usize,
                                        input: *const c_float, residual: *const c_float, output: *mut c_float,
                                        m: usize, k: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_llama_decode_workspace_bytes(model: *const wh_llama_model) -> usize;
    pub fn wh_llama_layer_decode(model: *const wh_llama_model, layer: usize, pos: usize, x: *mut c_float,
                                 workspace: *mut c_void, workspace_bytes: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_llama_decode_step(model: *const wh_llama_model, pos: usize, x: *mut c_float, logits: *mut c_float,
                                workspace: *mut c_void, workspace_bytes: usize, stream: wh_stream_t) -> c_int;
    pub fn wh_llama_forward_token(model: *const wh_llama_model, token: *const u32, pos: usize, x: *mut c_float,
                                  logits: *mut c_float, workspace: *mut c_void, workspace_bytes: usize,
                                  stream: wh_stream_t) -> c_int;
    /// No counterpart in woolly: the step for callers that cannot allocate
    /// (graph capture, allocation-free serving loops); workspace in a static
    /// device array of `WH_LLAMA_DECODE_NOALLOC_MAX_BYTES` per device.
    pub fn wh_llama_decode_step_noalloc(model: *const wh_llama_model, pos: usize, x: *mut c_float,
                                        logits: *mut c_float, stream: wh_stream_t) -> c_int;
    pub fn wh_embedding_lookup(r#type: c_int, table: *const c_void, vocab: usize, hidden: usize, ids: *const u32,
                               n_tokens: usize, out: *mut c_float, stream: wh_stream_t) -> c_int;

    // GGUF files (loader.rs:111-295, format.rs, metadata.rs, tensor_info.rs)
    pub fn wh_gguf_open(path: *const c_char, out: *mut *mut wh_gguf) -> c_int;
    pub fn wh_gguf_open_buffer(data: *const c_void, nbytes: usize, out: *mut *mut wh_gguf) -> c_int;
    pub fn wh_gguf_close(g: *mut wh_gguf) -> c_int;
    pub fn wh_gguf_get_header(g: *const wh_gguf, out: *mut wh_gguf_header) -> c_int;
    pub fn wh_gguf_tensor_at(g: *const wh_gguf, i: u64, out: *mut wh_gguf_tensor) -> c_int;
    pub fn wh_gguf_find_tensor(g: *const wh_gguf, name: *const c_char, index: *mut u64) -> c_int;
    pub fn wh_gguf_tensor_data(g: *const wh_gguf, i: u64, data: *mut *const c_void, nbytes: *mut usize) -> c_int;
    pub fn wh_gguf_upload(g: *const wh_gguf, i: u64, out: *mut *mut wh_weight) -> c_int;
    pub fn wh_gguf_kv_at(g: *const wh_gguf, i: u64, key: *mut *const c_char, value_type: *mut c_int) -> c_int;
    pub fn wh_gguf_find_kv(g: *const wh_gguf, key: *const c_char, index: *mut u64) -> c_int;
    pub fn wh_gguf_get_u32(g: *const wh_gguf, key: *const c_char, out: *mut u32) -> c_int;
    pub fn wh_gguf_get_u64(g: *const wh_gguf, key: *const c_char, out: *mut u64) -> c_int;
    pub fn wh_gguf_get_i32(g: *const wh_gguf, key: *const c_char, out: *mut i32) -> c_int;
    pub fn wh_gguf_get_f32(g: *const wh_gguf, key: *const c_char, out: *mut c_float) -> c_int;
    pub fn wh_gguf_get_bool(g: *const wh_gguf, key: *const c_char, out: *mut c_int) -> c_int;
    pub fn wh_gguf_get_string(g: *const wh_gguf, key: *const c_char, data: *mut *const c_char,
                              len: *mut usize) -> c_int;
    pub fn wh_gguf_kv_scalar(g: *const wh_gguf, i: u64, value_type: *mut c_int, out8: *mut c_void) -> c_int;
    pub fn wh_gguf_kv_array(g: *const wh_gguf, i: u64, elem_type: *mut c_int, count: *mut u64,
                            data: *mut *const c_void) -> c_int;
    pub fn wh_gguf_kv_array_string(g: *const wh_gguf, i: u64, j: u64, data: *mut *const c_char,
                                   len: *mut usize) -> c_int;
    pub fn wh_gguf_kv_string(g: *const wh_gguf, i: u64, data: *mut *const c_char, len: *mut usize) -> c_int;
    pub fn wh_ggml_type_traits(ggml_type: c_int, block_size: *mut usize, type_size: *mut usize,
                               is_quantized: *mut c_int) -> c_int;
}

/// Safe wrappers in woolly's shapes.
pub mod safe {
    use super::*;
    use std::ffi::CStr;
    use std::fmt;
    use std::ptr;

    /// A failed call: the status code and the library's message for it.
    #[derive(Clone, Debug, PartialEq, Eq)]
    pub struct Error {
        pub status: c_int,
        pub message: String,
    }

    impl fmt::Display for Error {
        fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
            write!(f, "woolly-hip status {}: {}", self.status, self.message)
        }
    }

    impl std::error::Error for Error {}

    /// The message of the last failure on this thread.
    pub fn last_error() -> String {
        // wh_last_error returns a thread-local NUL-terminated string (never null)
        unsafe { CStr::from_ptr(wh_last_error()).to_string_lossy().into_owned() }
    }

    /// Maps a status code to `Ok` or an `Error` carrying the last message.
    pub fn check(status: c_int) -> Result<(), Error> {
        if status == WH_OK {
            Ok(())
        } else {
            Err(Error { status, message: last_error() })
        }
    }

    /// Selects and initialises a device (0 for the first gfx950 GPU).
    pub fn init(device: i32) -> Result<(), Error> {
        check(unsafe { wh_init(device) })
    }

    /// `y = W x` on host slices (`simd::quantized_matvec`,
    /// quantization.rs:869-909): `weights` holds `m` rows of `k` elements in
    /// the GGUF block layout of `ggml_type`.
    pub fn quantized_matvec_host(ggml_type: i32, weights: &[u8], input: &[f32], output: &mut [f32], m: usize,
                                 k: usize) -> Result<(), Error> {
        if input.len() < k || output.len() < m {
            return Err(Error {
                status: WH_ERR_INVALID_ARGUMENT,
                message: format!("input holds {} of {} elements, output {} of {}", input.len(), k, output.len(), m),
            });
        }
        check(unsafe {
            wh_quantized_matvec_host(ggml_type, weights.as_ptr() as *const c_void, weights.len(), input.as_ptr(),
                                     output.as_mut_ptr(), m, k)
        })
    }

    /// `dequantize(data, ggml_type, nelements)` (dequantize.rs:189-205) on
    /// host memory: bit-exact with the reference.
    pub fn dequantize_host(ggml_type: i32, data: &[u8], nelements: usize) -> Result<Vec<f32>, Error> {
        let mut out = vec![0f32; nelements];
        check(unsafe {
            wh_dequantize_host(ggml_type, data.as_ptr() as *const c_void, data.len(), nelements, out.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// Device memory owned until drop.
    pub struct DeviceBuffer {
        ptr: *mut c_void,
        len: usize,
    }

    impl DeviceBuffer {
        pub fn new(len: usize) -> Result<Self, Error> {
            let mut ptr = ptr::null_mut();
            check(unsafe { wh_malloc(&mut ptr, len) })?;
            Ok(DeviceBuffer { ptr, len })
        }
        pub fn from_slice<T: Copy>(data: &[T], stream: &Stream) -> Result<Self, Error> {
            let bytes = std::mem::size_of_val(data);
            let buf = Self::new(bytes)?;
            check(unsafe { wh_memcpy_h2d(buf.ptr, data.as_ptr() as *const c_void, bytes, stream.raw()) })?;
            Ok(buf)
        }
        pub fn copy_to<T: Copy>(&self, out: &mut [T], stream: &Stream) -> Result<(), Error> {
            let bytes = std::mem::size_of_val(out).min(self.len);
            check(unsafe { wh_memcpy_d2h(out.as_mut_ptr() as *mut c_void, self.ptr, bytes, stream.raw()) })?;
            stream.synchronize()
        }
        pub fn as_ptr(&self) -> *const c_void {
            self.ptr
        }
        pub fn as_mut_ptr(&mut self) -> *mut c_void {
            self.ptr
        }
        pub fn len(&self) -> usize {
            self.len
        }
        pub fn is_empty(&self) -> bool {
            self.len == 0
        }
    }

    impl Drop for DeviceBuffer {
        fn drop(&mut self) {
            unsafe {
                wh_free(self.ptr);
            }
        }
    }

    /// A HIP stream owned until drop.
    pub struct Stream(wh_stream_t);

    impl Stream {
        pub fn new() -> Result<Self, Error> {
            let mut s = ptr::null_mut();
            check(unsafe { wh_stream_create(&mut s) })?;
            Ok(Stream(s))
        }
        pub fn raw(&self) -> wh_stream_t {
            self.0
        }
        pub fn synchronize(&self) -> Result<(), Error> {
            check(unsafe { wh_stream_synchronize(self.0) })
        }
    }

    impl Drop for Stream {
        fn drop(&mut self) {
            unsafe {
                wh_stream_destroy(self.0);
            }
        }
    }

    /// A quantized tensor uploaded to the device (`wh_weight_upload`),
    /// replacing the to_vec copy and f32 cache of the loader (loader.rs:274-291).
    pub struct Weight(*mut wh_weight);

    impl Weight {
        pub fn upload(ggml_type: i32, n_rows: usize, k: usize, host_bytes: &[u8]) -> Result<Self, Error> {
            let mut w = ptr::null_mut();
            check(unsafe {
                wh_weight_upload(ggml_type, n_rows, k, host_bytes.as_ptr() as *const c_void, host_bytes.len(), &mut w)
            })?;
            Ok(Weight(w))
        }
        pub fn data(&self) -> *const c_void {
            unsafe { wh_weight_data(self.0) }
        }
        /// (type, n_rows, k, nbytes)
        pub fn info(&self) -> Result<(i32, usize, usize, usize), Error> {
            let (mut t, mut n, mut k, mut nb) = (0, 0, 0, 0);
            check(unsafe { wh_weight_info(self.0, &mut t, &mut n, &mut k, &mut nb) })?;
            Ok((t, n, k, nb))
        }
        /// `output = W input` on the device (asynchronous on `stream`).
        pub fn matvec(&self, input: &DeviceBuffer, output: &mut DeviceBuffer, stream: &Stream) -> Result<(), Error> {
            let (t, n, k, nb) = self.info()?;
            if input.len() < 4 * k || output.len() < 4 * n {
                return Err(Error { status: WH_ERR_BUFFER_TOO_SMALL, message: "matvec buffers too small".into() });
            }
            check(unsafe {
                wh_quantized_matvec(t, self.data(), nb, input.as_ptr() as *const f32, output.as_mut_ptr() as *mut f32,
                                    n, k, stream.raw())
            })
        }
    }

    impl Drop for Weight {
        fn drop(&mut self) {
            unsafe {
                wh_weight_free(self.0);
            }
        }
    }
}
