/*
 * woolly_hip.h -- C ABI of the MI355X (gfx950) backend for woolly's quantized
 * matmul hot path: GGUF Q4_0 / Q4_1 / Q8_0 dequantization, quantized GEMV and
 * GEMM, RMSNorm, SwiGLU, and the fused SwiGLU feed-forward layer.
 *
 * Conventions
 *  - Every entry point returns an int status (wh_status).  Nothing panics,
 *    aborts or throws across the ABI; the reference's panics (assert_eq! on
 *    k % 32, quantization.rs:1107) become WH_ERR_INVALID_SHAPE.  The message of
 *    the last failure on the calling thread is available from wh_last_error().
 *  - Plain pointers and sizes only.  Device pointers are addresses returned by
 *    wh_malloc (or any HIP device allocation); "host" variants take host memory.
 *  - Kernel entry points are asynchronous and ordered on the given stream
 *    (NULL = the device's null stream).  The *_host variants are synchronous.
 *  - Weight matrices use ggml's convention: N rows of K elements, each row K/32
 *    consecutive blocks (quantization.rs:730-737; GGUF ne0 = K is fastest), in
 *    the on-disk block format (BlockQ4_0 18 B, BlockQ4_1 20 B, BlockQ8_0 34 B,
 *    quantization.rs:98-151).  Output buffers are always caller-allocated.
 *  - Calls are thread-safe; the library keeps no hidden global streams.
 */
#ifndef WOOLLY_HIP_H
#define WOOLLY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WH_API __attribute__((visibility("default")))

/* Status codes.  Mirrors QuantizationError (quantization.rs:8-26),
 * woolly_gguf::Error (crates/woolly-gguf/src/error.rs:11-64) and the panics of
 * the scalar kernels. */
typedef enum wh_status {
  WH_OK = 0,
  WH_ERR_UNSUPPORTED_TYPE = 1,  /* UnsupportedScheme / Error::InvalidTensorType */
  WH_ERR_INVALID_SHAPE = 2,     /* k % 32 != 0 (assert_eq! at quantization.rs:729,1107) */
  WH_ERR_BUFFER_TOO_SMALL = 3,  /* Error::BufferTooSmall{needed, available} */
  WH_ERR_INVALID_ARGUMENT = 4,  /* QuantizationError::InvalidParameters, null/misaligned */
  WH_ERR_HIP = 5,               /* a HIP runtime call failed */
  WH_ERR_OOM = 6,               /* device allocation failed */
  WH_ERR_NO_DEVICE = 7,         /* no usable gfx950 device */
  WH_ERR_IO = 8,                /* Error::Io (open/map failure, unexpected end of file) */
  WH_ERR_INVALID_MAGIC = 9,     /* Error::InvalidMagic */
  WH_ERR_UNSUPPORTED_VERSION = 10, /* Error::UnsupportedVersion */
  WH_ERR_INVALID_METADATA = 11, /* Error::InvalidMetadata / InvalidString / InvalidTensorInfo */
  WH_ERR_NOT_FOUND = 12,        /* Error::TensorNotFound, or a metadata key that is absent */
  WH_ERR_TYPE_MISMATCH = 13     /* metadata value of another type (the reference's get_* -> None) */
} wh_status;

/* GGMLType ids (crates/woolly-gguf/src/tensor_info.rs:15-30). */
typedef enum wh_type {
  WH_TYPE_F32 = 0,
  WH_TYPE_F16 = 1,
  WH_TYPE_Q4_0 = 2,
  WH_TYPE_Q4_1 = 3,
  /* BlockQ5_0 {f16 d; u8 qh[4]; u8 qs[16]} (22 B) and BlockQ5_1 {f16 d; f16 m;
   * u8 qh[4]; u8 qs[16]} (24 B), quantization.rs:117-140: dequantization only
   * (dequantize_q5_0 / _q5_1, quantization.rs:515-575) */
  WH_TYPE_Q5_0 = 6,
  WH_TYPE_Q5_1 = 7,
  WH_TYPE_Q8_0 = 8,
  /* 256-element K-quant blocks in woolly-gguf's layout (dequantize.rs:404-536,
   * which differs from ggml's): dequantization, GEMV, GEMM, the FFN layer and
   * the decode step (rows a multiple of 256 elements). */
  WH_TYPE_Q4_K = 12,
  WH_TYPE_Q6_K = 14,
  /* bfloat16 (GGMLType::BF16, tensor_info.rs:72-73): activations of
   * wh_quantized_matmul_x only */
  WH_TYPE_BF16 = 30
} wh_type;

typedef struct wh_stream_opaque* wh_stream_t; /* a hipStream_t */
typedef struct wh_event_opaque* wh_event_t;   /* a hipEvent_t */
typedef struct wh_weight wh_weight;           /* device-resident quantized tensor */
typedef struct wh_graph_opaque* wh_graph_t;   /* an instantiated hipGraphExec_t */

/* ------------------------------------------------------------------ errors */
WH_API const char* wh_status_string(int status);
WH_API const char* wh_last_error(void);
WH_API int wh_version(void);

/* ------------------------------------------------- device, memory, streams */
/* Selects the device for the calling thread and checks that it is gfx950. */
WH_API int wh_init(int device);
WH_API int wh_device_count(int* count);
WH_API int wh_device_name(char* buf, size_t len);
WH_API int wh_malloc(void** dptr, size_t nbytes);
WH_API int wh_free(void* dptr);
WH_API int wh_memcpy_h2d(void* dst, const void* src, size_t nbytes, wh_stream_t stream);
WH_API int wh_memcpy_d2h(void* dst, const void* src, size_t nbytes, wh_stream_t stream);
WH_API int wh_memcpy_d2d(void* dst, const void* src, size_t nbytes, wh_stream_t stream);
/* Fills nbytes with the byte value using a kernel (safe under graph capture). */
WH_API int wh_fill_bytes(void* dst, int value, size_t nbytes, wh_stream_t stream);
WH_API int wh_stream_create(wh_stream_t* out);
WH_API int wh_stream_destroy(wh_stream_t stream);
WH_API int wh_stream_synchronize(wh_stream_t stream);
WH_API int wh_device_synchronize(void);
WH_API int wh_event_create(wh_event_t* out);
WH_API int wh_event_destroy(wh_event_t event);
WH_API int wh_event_record(wh_event_t event, wh_stream_t stream);
WH_API int wh_event_synchronize(wh_event_t event);
WH_API int wh_event_elapsed_ms(float* ms, wh_event_t start, wh_event_t end);

/* HIP graphs: capture a sequence of stream-ordered calls once, replay it with
 * one launch (e.g. a decode step's projections).  Capture needs a non-null
 * stream; the entry points above record only kernel launches (no memset
 * nodes), so every replay recomputes from the buffers' current contents. */
WH_API int wh_graph_begin_capture(wh_stream_t stream);
WH_API int wh_graph_end_capture(wh_stream_t stream, wh_graph_t* out);
WH_API int wh_graph_launch(wh_graph_t graph, wh_stream_t stream);
WH_API int wh_graph_destroy(wh_graph_t graph);

/* Measurement aid, no counterpart in the reference (for benchmarks of the
 * GEMV): reads an n_rows x row_bytes device matrix (row_bytes <= 4096) in the
 * geometry of the single-token matrix-core GEMV (workgroups of 16 waves, one
 * row per wave per step, 16-byte loads) without storing or computing
 * anything but a checksum per workgroup: out is a device array of at least
 * ceil(n_rows / 16) dwords.  mode 0: one step in flight per wave, as the
 * GEMV; mode 1: up to four; mode 2: the matrix read as one flat byte range,
 * one contiguous piece per workgroup (one workgroup per CU, more for
 * matrices past 64 MiB), every load of a lane in flight at once. */
WH_API int wh_read_probe(const void* src, size_t row_bytes, size_t n_rows, int mode, uint32_t* out,
                         wh_stream_t stream);

/* ------------------------------------------------------------------ format */
/* get_block_size / get_type_size, crates/woolly-gguf/src/dequantize.rs:208-242.
 * Return 0 for types this backend does not handle. */
WH_API size_t wh_block_size(int type);
WH_API size_t wh_type_size(int type);
/* TensorInfo::data_size, crates/woolly-gguf/src/tensor_info.rs:244-255. */
WH_API int wh_tensor_nbytes(int type, uint64_t nelements, uint64_t* nbytes);

/* ------------------------------------------------------- dequantization */
/* woolly_gguf::dequantize(data, ggml_type, nelements)
 *   (crates/woolly-gguf/src/dequantize.rs:189-205), and through it
 *   dequantize_q4_0 / dequantize_q4_1 / dequantize_q8_0
 *   (crates/woolly-tensor/src/quantization.rs:466, 490, 576) and
 *   optimized::dequantize_blocks (quantization.rs:1171).
 * Writes exactly nelements f32 values; bit-exact with the reference.
 * F32 and F16 are accepted as in the reference.  WH_ERR_BUFFER_TOO_SMALL when
 * nbytes < ceil(nelements/32) * type_size.
 * Q4_K and Q6_K (dequantize_q4_k_scalar / dequantize_q6_k, dequantize.rs:404-536)
 * decode 256-element blocks; a buffer shorter than ceil(nelements/256) *
 * type_size is Error::InvalidTensorInfo there, WH_ERR_INVALID_METADATA here.
 * Q5_0 and Q5_1 decode as dequantize_q5_0 / dequantize_q5_1
 * (quantization.rs:515-575); woolly_gguf's own Q5 functions (dequantize.rs:538-550)
 * are stubs that return zeros, which this entry point does not reproduce. */
WH_API int wh_dequantize(int type, const void* data, size_t nbytes, size_t nelements,
                         float* out, wh_stream_t stream);

/* ------------------------------------------------------ quantized GEMV */
/* simd::quantized_matvec(weights, input, output, m, k)
 *   (crates/woolly-tensor/src/quantization.rs:869-909):
 *   output[r] = sum_k W[r, k] * input[k] for r < m.
 * Covers Q4_0 and Q8_0 like the reference, and Q4_1, Q4_K and Q6_K, which the
 * reference rejects with UnsupportedScheme (quantization.rs:905-907); those
 * are defined as the reference's dequantization followed by the f32 dot.
 * k must be a multiple of the block size (32, or 256 for Q4_K / Q6_K) and
 * weight_nbytes >= m * (k/block size) * type_size. */
WH_API int wh_quantized_matvec(int type, const void* weights, size_t weight_nbytes,
                               const float* input, float* output, size_t m, size_t k,
                               wh_stream_t stream);

/* Which single-token GEMV kernels the library launches (no counterpart in the
 * reference: a switch for comparing the two implementations on one device).
 * WH_GEMV_AUTO (default): the matrix-core kernel (int8 MFMA on exact limbs of
 * the activations) for the shapes it takes, the streaming VALU kernels
 * otherwise; WH_GEMV_STREAM: streaming kernels only.  Applies to
 * wh_quantized_matvec, the fused decode GEMVs and the M <= 2 FFN gate/up.
 * The setting belongs to the calling thread (other threads keep theirs); the
 * previous setting is stored in *previous when it is not NULL.
 * WH_ERR_INVALID_ARGUMENT for an unknown mode (nothing changes). */
enum { WH_GEMV_AUTO = 0, WH_GEMV_STREAM = 1 };
WH_API int wh_gemv_select(int mode, int* previous);

/* ------------------------------------------------------ quantized GEMM */
/* Y[t, r] = sum_k X[t, k] * W[r, k] for t < n_tokens, r < n_rows.
 * Replaces the projections woolly runs on fully dequantized f32 weights:
 *   simd_matmul_optimized -> Gemm::compute (tensor_utils_simd.rs:855-914,
 *   ops/matmul.rs:83-259) called from simd_ffn_forward
 *   (tensor_utils_simd.rs:605-754) and compute_simd_swiglu_ffn
 *   (model/lazy_transformer.rs:1073-1123), with ggml's [N][K] weight layout
 *   instead of the [K][N] reshape at lazy_transformer.rs:1091-1101.
 * X is row-major [n_tokens][k] f32, Y is row-major [n_tokens][n_rows] f32.
 * Types: Q4_0, Q4_1, Q8_0 (k % 32 == 0) and Q4_K, Q6_K (k % 256 == 0; with
 * more than 2 tokens the matrix is first rewritten into the workspace as
 * 32-element blocks with f32 scales, the values unchanged).
 * The MFMA path (more than 2 tokens) needs a device workspace of
 * wh_quantized_matmul_workspace_bytes(type, n_rows, k, n_tokens) bytes (256-byte
 * aligned); the call itself never allocates.  WH_ERR_BUFFER_TOO_SMALL if it
 * is missing or short.  Where the output tiles would leave CUs idle in their
 * last round (e.g. 14336 rows at 512 tokens), the size includes one f32 tile
 * of 128 tokens x 256 rows per CU and a flag per CU (32 MiB + 1 KiB at 256
 * CUs) for the stream-K split; calls that overlap on one workspace race. */
WH_API size_t wh_quantized_matmul_workspace_bytes(int type, size_t n_rows, size_t k,
                                                  size_t n_tokens);
WH_API int wh_quantized_matmul(int type, const void* weights, size_t weight_nbytes,
                               size_t n_rows, size_t k, const float* x, size_t n_tokens,
                               float* y, void* workspace, size_t workspace_bytes,
                               wh_stream_t stream);

/* The same product with the activations given as x_dtype: WH_TYPE_F32 (as
 * wh_quantized_matmul) or WH_TYPE_BF16 (X row-major [n_tokens][k] bfloat16,
 * 8-byte aligned), the activation types of the prefill benchmark configuration
 * ("f32/bf16", a wh_qgemm(.., X, x_dtype, ..) signature).  bf16 values are
 * widened exactly to f32, so the result equals wh_quantized_matmul on the
 * widened X (bit for bit unless a row holds elements below 2^-31 of its
 * largest: for bf16 the tiled kernel issues the hi-limb products only, and
 * such elements' lo products, each below 2^-39 of the row's largest term,
 * are left out).  The workspace (wh_quantized_matmul_x_workspace_bytes) is needed
 * for bf16 at any token count; WH_ERR_UNSUPPORTED_TYPE for another x_dtype. */
WH_API size_t wh_quantized_matmul_x_workspace_bytes(int type, size_t n_rows, size_t k, size_t n_tokens,
                                                    int x_dtype);
WH_API int wh_quantized_matmul_x(int type, const void* weights, size_t weight_nbytes, size_t n_rows, size_t k,
                                 const void* x, int x_dtype, size_t n_tokens, float* y, void* workspace,
                                 size_t workspace_bytes, wh_stream_t stream);

/* Tuning knob, no counterpart in the reference: the bound of the stream-K
 * hand-off wait of wh_quantized_matmul(_x) and wh_ffn_swiglu, in ticks of
 * the GPU's 100 MHz real-time clock (default 100000 = 1 ms; read at every
 * launch and captured into a graph with it).  A workgroup that finishes a
 * shared output tile waits that long for the other workgroups' parts of the
 * tile (they run at the same time on a GPU the call has to itself), then
 * computes the rest of the tile itself; a GPU shared with other work may
 * want a shorter bound.  0 makes every such workgroup compute the rest
 * without waiting (the results differ from the default's in rounding only).
 * Process-wide; always WH_OK. */
WH_API int wh_set_stream_k_wait(uint32_t ticks);

/* --------------------------------------------------- elementwise / norms */
/* rms_norm (crates/woolly-core/src/tensor_utils.rs:446-480):
 *   out[t, i] = (x[t, i] / sqrt(sum_i x[t, i]^2 / hidden + eps)) * weight[i] */
WH_API int wh_rms_norm(const float* x, const float* weight, float eps, size_t tokens,
                       size_t hidden, float* out, wh_stream_t stream);
/* swiglu (crates/woolly-core/src/tensor_utils.rs:512-532):
 *   out[i] = gate[i] * (1 / (1 + exp(-gate[i]))) * up[i] */
WH_API int wh_swiglu(const float* gate, const float* up, size_t n, float* out,
                     wh_stream_t stream);

/* ------------------------------------------------------ SwiGLU FFN layer */
/* One feed-forward layer with its RMSNorm prologue:
 *   xh = rms_norm(x, gamma, eps); out = W_down (silu(W_gate xh) * (W_up xh))
 * The call site it replaces is compute_simd_swiglu_ffn
 *   (model/lazy_transformer.rs:1073-1123) with the preceding rms_norm of
 *   process_layer (lazy_transformer.rs:98-258); FeedForward::forward
 *   (model/feedforward.rs:93-127) and fused_rmsnorm_ffn
 *   (model/fused_kernels.rs:403-455) compute the same layer.
 * gate and up are [n_ff][hidden], down is [hidden][n_ff], all of `type`
 * (Q4_0, Q4_1, Q8_0, or Q4_K / Q6_K with hidden and n_ff multiples of 256).
 * The workspace must hold wh_ffn_workspace_bytes_for_type(type, hidden, n_ff, m)
 * bytes of device memory (no allocation happens inside the call);
 * wh_ffn_workspace_bytes(hidden, n_ff, m) is enough for Q4_0, Q4_1 and Q8_0. */
typedef struct wh_ffn_weights {
  int type;
  const void* gate;
  const void* up;
  const void* down;
  size_t hidden;
  size_t n_ff;
} wh_ffn_weights;

WH_API size_t wh_ffn_workspace_bytes(size_t hidden, size_t n_ff, size_t m);
WH_API size_t wh_ffn_workspace_bytes_for_type(int type, size_t hidden, size_t n_ff, size_t m);
WH_API int wh_ffn_swiglu(const wh_ffn_weights* weights, const float* gamma, float eps,
                         const float* x, size_t m, float* out, void* workspace,
                         size_t workspace_bytes, wh_stream_t stream);

/* ------------------------------------------------------- weight handles */
/* Uploads one quantized tensor straight from host bytes (e.g. the GGUF mmap
 * slice at data_start_offset + tensor.offset, crates/woolly-gguf/src/loader.rs:274),
 * replacing GGUFLoader::tensor_data's to_vec copy (loader.rs:291) and the f32
 * dequantization cache (model/lazy_loader.rs:599-659).  The handle owns its
 * device memory until wh_weight_free; the host bytes are only read during the
 * call.  The device layout is the GGUF block layout, so the handle's data can
 * be passed to every kernel entry point above.  F32 and F16 tensors (norm
 * weights, embeddings) are accepted as n_rows x k plain elements. */
WH_API int wh_weight_upload(int type, size_t n_rows, size_t k, const void* host_bytes,
                            size_t nbytes, wh_weight** out);
WH_API int wh_weight_free(wh_weight* weight);
WH_API const void* wh_weight_data(const wh_weight* weight);
WH_API int wh_weight_info(const wh_weight* weight, int* type, size_t* n_rows, size_t* k,
                          size_t* nbytes);
/* Converts a Q4_K / Q6_K handle's blocks once, on the stream, into the block
 * layout of the tiled prefill GEMM (the same values: 32-element blocks with
 * f32 scales d * s_j, Q6_K's 16-element halves padded) and keeps that copy
 * with the handle until wh_weight_free; calls of wh_quantized_matmul and
 * wh_ffn_swiglu with more than two tokens whose weight pointer is the
 * handle's data (wh_weight_data) then skip the per-call conversion.  This is
 * the device-side counterpart of the reference's convert-once cache
 * (DequantizationCache::get_or_dequantize,
 * crates/woolly-core/src/model/dequantization_cache.rs:121-165,
 * LazyModelWeights::get_tensor_cached, model/lazy_loader.rs:599-659).  The
 * copy takes 648 bytes per 1024 elements for Q4_K at rows of a multiple of
 * 2048 elements (576 in the file; each row's dmin table is padded to 8
 * super-blocks) and 1280 for Q6_K (840) of device memory.  A no-op for the other block types, whose blocks the
 * GEMM reads directly.  Idempotent; *prepared_bytes (may be null) receives
 * the copy's size. */
WH_API int wh_weight_prepare_prefill(wh_weight* weight, wh_stream_t stream, size_t* prepared_bytes);

/* ------------------------------------- synchronous host-pointer variants */
/* Same semantics as the device entry points, on host memory, blocking.  They
 * mirror the reference's slice-in / Vec-out signatures
 * (dequantize_q4_0(&[BlockQ4_0]) -> Vec<f32>, quantized_matvec(&storage,
 * &[f32], &mut [f32], m, k)). */
WH_API int wh_dequantize_host(int type, const void* data, size_t nbytes, size_t nelements,
                              float* out);
WH_API int wh_quantized_matvec_host(int type, const void* weights, size_t weight_nbytes,
                                    const float* input, float* output, size_t m, size_t k);

/* Device copies of host weights behind the two host variants above.  Off by
 * default: every call then uploads its whole block input (a 33 MB matrix
 * crosses PCIe for an 8 us GEMV).  With a budget above 0, a call's block input
 * is uploaded once per (device, host address, byte count) and later calls with
 * the same key reuse the device copy, so a call moves only its activations and
 * outputs; its small device buffers come from a pool, so a cached call
 * allocates nothing.  This is the device-side counterpart of the reference's
 * per-tensor cache (DequantizationCache::get_or_dequantize,
 * crates/woolly-core/src/model/dequantization_cache.rs:121-165) and assumes, as
 * that cache does, that cached bytes do not change (GGUF mmap slices): a caller
 * that rewrites host memory evicts its range first.  Least recently used
 * entries are dropped beyond the budget; an input larger than the budget is
 * not cached.  Thread-safe: an entry dropped while another call uses it is
 * freed when that call returns.  Device-resident handles (wh_weight_upload)
 * remain the fast path: no PCIe copy and no host synchronisation per call. */
typedef struct wh_host_cache_stats {
  uint64_t hits;      /* calls that found their block input on the device */
  uint64_t misses;    /* calls that uploaded it (cached or not) */
  uint64_t evictions; /* entries dropped by the budget, evict or clear */
  size_t entries;     /* entries held */
  size_t bytes;       /* device bytes held by the entries */
  size_t max_bytes;   /* the budget (0: off) */
} wh_host_cache_stats;
/* Sets the budget; 0 turns the cache off and frees every entry and pooled buffer. */
WH_API int wh_host_cache_configure(size_t max_bytes);
/* Drops every entry whose host range overlaps [host_ptr, host_ptr + nbytes)
 * (nbytes 0: the entries that start at host_ptr), on every device. */
WH_API int wh_host_cache_evict(const void* host_ptr, size_t nbytes, size_t* evicted);
/* Drops every entry and frees the pooled buffers (the budget is kept). */
WH_API int wh_host_cache_clear(void);
WH_API int wh_host_cache_get_stats(wh_host_cache_stats* out);

/* ---------------------------------------------------- decode step (M = 1) */
/* The pieces of one transformer layer for a single new token
 * (LazyTransformer::process_layer, crates/woolly-core/src/model/lazy_transformer.rs:98-258)
 * and the whole step (LazyTransformer::forward, :1155-1335).  All pointers are
 * device memory; calls are asynchronous on the stream. */

/* RoPE inverse frequencies, inv_freq[i] = 1 / base^(2i / head_dim) for
 * i < head_dim / 2, evaluated in f32 exactly as RoPE::apply_f32 does
 * (crates/woolly-tensor/src/ops/mod.rs:490-494).  Host output. */
WH_API int wh_rope_inv_freq(float base, size_t head_dim, float* out_host);

/* Fused RMSNorm + Q/K/V projection of one token (the rms_norm of process_layer,
 * :130-134, then simd_attention_projections, tensor_utils_simd.rs:455-602):
 * qkv = [Wq; Wk; Wv] * rms_norm(x, gamma, eps), laid out q (q_rows) | k | v
 * (kv_rows each), all three matrices of one block type with K = hidden
 * (Q4_0, Q4_1, Q8_0, or Q4_K / Q6_K with hidden a multiple of 256).
 * The workspace (wh_attention_qkv_workspace_bytes) is only used by shapes the
 * fused kernel does not take. */
WH_API size_t wh_attention_qkv_workspace_bytes(size_t hidden);
WH_API int wh_attention_qkv(int type, const void* wq, const void* wk, const void* wv, size_t q_rows,
                            size_t kv_rows, size_t hidden, const float* gamma, float eps,
                            const float* x, float* qkv, void* workspace, size_t workspace_bytes,
                            wh_stream_t stream);

/* Grouped-query attention of one new token at position pos over an f16 KV
 * cache (compute_optimized_gqa_attention, lazy_transformer.rs:261-456, with the
 * RoPE of ops/mod.rs:472-530 applied to q and k): reads qkv (the layout of
 * wh_attention_qkv), rotates q and k by pos, stores k and v (rounded to f16)
 * at cache row pos, and writes out[n_heads * head_dim] = softmax(q k^T / sqrt(d)) v
 * over cache rows 0..pos.  Caches are [max_ctx][n_kv_heads][head_dim] f16.
 * head_dim 64 or 128, n_heads a multiple of n_kv_heads with at most 8 query
 * heads per KV head.  Workspace: wh_attention_workspace_bytes(.., max_ctx). */
WH_API size_t wh_attention_workspace_bytes(size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                           size_t max_ctx);
WH_API int wh_attention_decode(const float* qkv, void* k_cache, void* v_cache, size_t pos,
                               size_t n_heads, size_t n_kv_heads, size_t head_dim,
                               const float* inv_freq, float* out, void* workspace,
                               size_t workspace_bytes, wh_stream_t stream);

/* y = residual + W x for one token (the attention output projection and the
 * FFN down projection with process_layer's residual adds, :186-188, 245-247).
 * y may be the residual buffer itself.  Types as wh_quantized_matvec. */
WH_API int wh_quantized_matvec_residual(int type, const void* weights, size_t weight_nbytes,
                                        const float* input, const float* residual, float* output,
                                        size_t m, size_t k, wh_stream_t stream);

/* A Llama-shaped model for the decode step. */
typedef struct wh_llama_layer {
  const float* attn_norm;  /* f32 [hidden] */
  const void* wq;          /* [n_heads * head_dim][hidden] */
  const void* wk;          /* [n_kv_heads * head_dim][hidden] */
  const void* wv;          /* [n_kv_heads * head_dim][hidden] */
  const void* wo;          /* [hidden][n_heads * head_dim] */
  const float* ffn_norm;   /* f32 [hidden] */
  const void* w_gate;      /* [n_ff][hidden] */
  const void* w_up;        /* [n_ff][hidden] */
  const void* w_down;      /* [hidden][n_ff] */
  void* k_cache;           /* f16 [max_ctx][n_kv_heads][head_dim] */
  void* v_cache;           /* f16 [max_ctx][n_kv_heads][head_dim] */
  /* Block type of each matrix; 0 (zero-initialised) = the model's type.  GGUF
   * files such as Q4_K_M mix types per tensor (attn_v and ffn_down in Q6_K,
   * the rest in Q4_K).  K-quant matrices need their K a multiple of 256. */
  int wq_type, wk_type, wv_type, wo_type, w_gate_type, w_up_type, w_down_type;
} wh_llama_layer;

typedef struct wh_llama_model {
  int type;                    /* block type of the layer matrices (see wh_llama_layer) */
  size_t n_layers, hidden, n_heads, n_kv_heads, head_dim, n_ff, max_ctx, vocab;
  float eps;                   /* RMSNorm epsilon (model/mod.rs:193: 1e-5) */
  const float* rope_inv_freq;  /* device [head_dim / 2], see wh_rope_inv_freq */
  const wh_llama_layer* layers;/* host array of n_layers */
  const float* output_norm;    /* f32 [hidden] */
  int output_type;             /* block type of the output head */
  const void* output;          /* [vocab][hidden] */
  /* Token embeddings (token_embd.weight, [vocab][hidden] of token_embd_type:
   * F32, F16 or a block type) for wh_llama_forward_token; may be NULL for the
   * entry points that take an embedded x.  A GGUF file without output.weight
   * ties the head to this table (lazy_transformer.rs:1301-1316): output =
   * token_embd and output_type = token_embd_type. */
  int token_embd_type;
  const void* token_embd;
} wh_llama_model;

WH_API size_t wh_llama_decode_workspace_bytes(const wh_llama_model* model);
/* One layer for one token at position pos: x (device [hidden]) is updated in
 * place (process_layer, :98-258). */
WH_API int wh_llama_layer_decode(const wh_llama_model* model, size_t layer, size_t pos, float* x,
                                 void* workspace, size_t workspace_bytes, wh_stream_t stream);
/* The whole step (forward, :1155-1335, for one token): every layer on x (in:
 * the token's embedding, out: the last hidden state), then
 * logits = output * rms_norm(x, output_norm) when logits is not NULL.  Launches
 * only (no allocation, no synchronisation): the step can be captured into a
 * HIP graph with wh_graph_begin_capture. */
WH_API int wh_llama_decode_step(const wh_llama_model* model, size_t pos, float* x, float* logits,
                                void* workspace, size_t workspace_bytes, wh_stream_t stream);
/* The step from a token id (forward, :1155-1230, for one token): x = the
 * dequantized row *token of model->token_embd, then wh_llama_decode_step.
 * `token` is device memory (a uint32 the caller or a sampler on the device
 * writes before each step), so a captured step reads the current token at
 * every replay.  An id >= vocab, which the reference rejects with
 * TENSOR_EMBEDDING_TOKEN_OUT_OF_RANGE, makes x and the logits NaN. */
WH_API int wh_llama_forward_token(const wh_llama_model* model, const uint32_t* token, size_t pos, float* x,
                                  float* logits, void* workspace, size_t workspace_bytes,
                                  wh_stream_t stream);

/* wh_llama_decode_step without a workspace argument and without any
 * allocation (no counterpart in the reference: for callers that cannot
 * allocate, such as code under HIP graph capture or a serving loop that
 * forbids hipMalloc).  The step's workspace lives in a static device array of
 * WH_LLAMA_DECODE_NOALLOC_MAX_BYTES bytes, one per device, held until the
 * process ends; wh_init looks up its address.  A step whose
 * workspace at this position exceeds it (about 64K positions for 32 heads of
 * 128) fails with WH_ERR_BUFFER_TOO_SMALL before anything is launched.  All
 * calls on one device share that array: calls that overlap on one device
 * (concurrent streams or threads) race.  Results are identical to
 * wh_llama_decode_step's. */
#define WH_LLAMA_DECODE_NOALLOC_MAX_BYTES ((size_t)16 << 20)
WH_API int wh_llama_decode_step_noalloc(const wh_llama_model* model, size_t pos, float* x, float* logits,
                                        wh_stream_t stream);

/* embedding_lookup (crates/woolly-core/src/tensor_utils.rs:548-590) on the
 * device: out[t, :] = the dequantized row ids[t] of table ([vocab][hidden] of
 * `type`, e.g. token_embd.weight), bit-identical to wh_dequantize of that row,
 * for t < n_tokens (at most 65535).  ids (uint32) and out are device memory,
 * out 16-byte aligned, hidden a multiple of 4 and of the block size.  Rows of
 * ids >= vocab are written as NaN (the reference returns
 * TENSOR_EMBEDDING_TOKEN_OUT_OF_RANGE; the host mirrors check ids first). */
WH_API int wh_embedding_lookup(int type, const void* table, size_t vocab, size_t hidden, const uint32_t* ids,
                               size_t n_tokens, float* out, wh_stream_t stream);

/* --------------------------------------------------------------- GGUF files */
/* A parsed GGUF file: header, metadata key/values and the tensor table of
 * woolly-gguf's GGUFLoader (crates/woolly-gguf/src/loader.rs:111-200), over a
 * read-only memory map.  Parsing follows GGUFHeader::read_from (format.rs:74-103),
 * GGUFMetadata::read_from (metadata.rs:153-178), MetadataValue::read_from
 * (metadata.rs:86-124) and TensorInfo::read_from (tensor_info.rs:203-238); the
 * data section starts at the header's end rounded up to general.alignment
 * (a u32, default 32; loader.rs:148-164, 662-667).  Every read is bounds-checked:
 * a truncated file fails with WH_ERR_IO ("unexpected end of file"), as the
 * reference's Cursor reads do.  Strings must be valid UTF-8 (InvalidString).
 * Keys and tensor names that occur twice resolve to the last occurrence (the
 * reference inserts into a HashMap); the *_at calls enumerate in file order.
 * A handle is immutable after open and may be shared between threads. */
typedef struct wh_gguf wh_gguf;
#define WH_GGUF_MAX_DIMS 8

/* GGUFLoader::from_path (loader.rs:112-133): opens and maps `path`. */
WH_API int wh_gguf_open(const char* path, wh_gguf** out);
/* GGUFLoader::from_mmap (loader.rs:136-200) over caller memory; the bytes are
 * borrowed and must outlive the handle. */
WH_API int wh_gguf_open_buffer(const void* data, size_t nbytes, wh_gguf** out);
WH_API int wh_gguf_close(wh_gguf* g);

typedef struct wh_gguf_header {
  uint32_t version;             /* 1..3 (GGUFVersion::is_supported, format.rs:54-56) */
  uint64_t tensor_count;        /* as stored in the header */
  uint64_t metadata_kv_count;   /* as stored in the header */
  uint32_t alignment;           /* loader.alignment() */
  uint64_t data_offset;         /* absolute offset of the data section */
  uint64_t file_size;           /* loader.file_size() */
  uint64_t total_tensor_size;   /* loader.total_tensor_size(), distinct names */
} wh_gguf_header;
WH_API int wh_gguf_get_header(const wh_gguf* g, wh_gguf_header* out);

/* TensorInfo (tensor_info.rs:187-255). name is NUL-terminated and lives as
 * long as the handle; dims[n_dims..] are 0. */
typedef struct wh_gguf_tensor {
  const char* name;
  uint32_t n_dims;
  uint64_t dims[WH_GGUF_MAX_DIMS];
  int ggml_type;
  uint64_t offset;      /* relative to the data section */
  uint64_t n_elements;  /* TensorInfo::n_elements */
  uint64_t data_size;   /* TensorInfo::data_size */
} wh_gguf_tensor;
/* i-th tensor in file order (i < number of tensors). */
WH_API int wh_gguf_tensor_at(const wh_gguf* g, uint64_t i, wh_gguf_tensor* out);
/* loader.tensor_info(name): index of the tensor; WH_ERR_NOT_FOUND if absent. */
WH_API int wh_gguf_find_tensor(const wh_gguf* g, const char* name, uint64_t* index);
/* loader.tensor_data(name) (loader.rs:230-295) without the copy: a pointer into
 * the mapping and its size; WH_ERR_BUFFER_TOO_SMALL{needed, available} when the
 * tensor runs past the end of the file (loader.rs:276-282). */
WH_API int wh_gguf_tensor_data(const wh_gguf* g, uint64_t i, const void** data, size_t* nbytes);
/* Uploads tensor i to a device weight handle straight from the mapping
 * (wh_weight_upload with K = dims[0], rows = dims[1] * dims[2] * ...):
 * replaces load_tensor_data_direct's to_vec (loader.rs:291) and the f32
 * dequantization cache.  Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, F32 and F16 tensors
 * (the types wh_weight_upload takes). */
WH_API int wh_gguf_upload(const wh_gguf* g, uint64_t i, wh_weight** out);

/* Metadata value types (metadata.rs:13-42). */
typedef enum wh_gguf_value_type {
  WH_GGUF_U8 = 0, WH_GGUF_I8 = 1, WH_GGUF_U16 = 2, WH_GGUF_I16 = 3,
  WH_GGUF_U32 = 4, WH_GGUF_I32 = 5, WH_GGUF_F32 = 6, WH_GGUF_BOOL = 7,
  WH_GGUF_STRING = 8, WH_GGUF_ARRAY = 9, WH_GGUF_U64 = 10, WH_GGUF_I64 = 11,
  WH_GGUF_F64 = 12
} wh_gguf_value_type;
/* i-th key/value in file order: key (NUL-terminated, lives with the handle)
 * and value type. */
WH_API int wh_gguf_kv_at(const wh_gguf* g, uint64_t i, const char** key, int* value_type);
WH_API int wh_gguf_find_kv(const wh_gguf* g, const char* key, uint64_t* index);
/* Typed getters (GGUFMetadata::get_u32 / get_u64 / get_i32 / get_f32 /
 * get_bool / get_string, metadata.rs:186-233): WH_ERR_NOT_FOUND for an absent
 * key, WH_ERR_TYPE_MISMATCH for a value of another type. */
WH_API int wh_gguf_get_u32(const wh_gguf* g, const char* key, uint32_t* out);
WH_API int wh_gguf_get_u64(const wh_gguf* g, const char* key, uint64_t* out);
WH_API int wh_gguf_get_i32(const wh_gguf* g, const char* key, int32_t* out);
WH_API int wh_gguf_get_f32(const wh_gguf* g, const char* key, float* out);
WH_API int wh_gguf_get_bool(const wh_gguf* g, const char* key, int* out);
/* String value: pointer into the mapping (not NUL-terminated) and length. */
WH_API int wh_gguf_get_string(const wh_gguf* g, const char* key, const char** data, size_t* len);
/* Any scalar value (types 0-7, 10-12) of key/value i, as its little-endian
 * bytes in out[0 .. size) (bool: one byte 0/1). */
WH_API int wh_gguf_kv_scalar(const wh_gguf* g, uint64_t i, int* value_type, void* out8);
/* Array value of key/value i: element type and count; for fixed-size element
 * types `data` points at the packed little-endian elements in the mapping
 * (unaligned), for strings and nested arrays it is NULL. */
WH_API int wh_gguf_kv_array(const wh_gguf* g, uint64_t i, int* elem_type, uint64_t* count,
                            const void** data);
/* j-th element of a string array (pointer into the mapping, length). */
WH_API int wh_gguf_kv_array_string(const wh_gguf* g, uint64_t i, uint64_t j, const char** data,
                                   size_t* len);
/* String value of key/value i. */
WH_API int wh_gguf_kv_string(const wh_gguf* g, uint64_t i, const char** data, size_t* len);

/* GGMLType traits for every id the reference knows (tensor_info.rs:75-183):
 * block size, bytes per block (per element for plain types), quantized or not.
 * WH_ERR_UNSUPPORTED_TYPE (Error::InvalidTensorType) for other ids. */
WH_API int wh_ggml_type_traits(int ggml_type, size_t* block_size, size_t* type_size,
                               int* is_quantized);

#ifdef __cplusplus
}
#endif
#endif /* WOOLLY_HIP_H */
