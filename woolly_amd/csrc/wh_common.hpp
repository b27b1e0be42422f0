// wh_common.hpp -- shared host/device helpers of libwoolly_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

#include "../../include/woolly_hip.h"

namespace wh {

// ---------------------------------------------------------------- host side
// Records the message of the last failure on this thread and returns status.
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a failed HIP call to WH_ERR_HIP / WH_ERR_OOM with its message.
int hip_error(hipError_t err, const char* what);

#define WH_HIP_TRY(expr)                                    \
  do {                                                      \
    hipError_t _e = (expr);                                 \
    if (_e != hipSuccess) return ::wh::hip_error(_e, #expr); \
  } while (0)

// Checks the launch that was just issued on this thread.
#define WH_LAUNCH_CHECK(name)                                 \
  do {                                                        \
    hipError_t _e = hipGetLastError();                        \
    if (_e != hipSuccess) return ::wh::hip_error(_e, name);   \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline size_t type_size(int type) {
  switch (type) {
    case WH_TYPE_F32: return 4;
    case WH_TYPE_F16: return 2;
    case WH_TYPE_Q4_0: return 18;
    case WH_TYPE_Q4_1: return 20;
    case WH_TYPE_Q5_0: return 22;
    case WH_TYPE_Q5_1: return 24;
    case WH_TYPE_Q8_0: return 34;
    case WH_TYPE_Q4_K: return 144;
    case WH_TYPE_Q6_K: return 210;
    default: return 0;
  }
}
// Elements per block (1 for the plain types, 0 for unknown ids).
inline size_t block_elems(int type) {
  switch (type) {
    case WH_TYPE_F32:
    case WH_TYPE_F16: return 1;
    case WH_TYPE_Q4_0:
    case WH_TYPE_Q4_1:
    case WH_TYPE_Q5_0:
    case WH_TYPE_Q5_1:
    case WH_TYPE_Q8_0: return 32;
    case WH_TYPE_Q4_K:
    case WH_TYPE_Q6_K: return 256;
    default: return 0;
  }
}
// The 32-element block formats every kernel of the library takes.
inline bool is_block_type(int type) {
  return type == WH_TYPE_Q4_0 || type == WH_TYPE_Q4_1 || type == WH_TYPE_Q8_0;
}
// The 256-element K-quant formats.
inline bool is_kquant(int type) { return type == WH_TYPE_Q4_K || type == WH_TYPE_Q6_K; }

// Block formats of the tiled prefill GEMM that K-quant matrices are repacked
// into (internal ids, never seen at the C ABI):
//   kGemmQ4F {f32 d; u8 qs[16]}: 32 elements d * q, Q4_0 nibble order, followed
//            by the super-blocks' dmin as fp16 [n_rows][q4f_dmin_stride(k)]
//            (zeros past k / 256; the GEMM's epilogue adds dmin * sum(x) per
//            super-block, as matrix-core products over 32 super-blocks)
//   kGemmQ8H {f32 d; i8 q[16]}: 16 elements d * q, which the GEMM reads as a
//            32-element block whose upper half is zero (activations packed to match)
constexpr int kGemmQ4F = 256, kGemmQ8H = 257;
inline int kquant_gemm_type(int type) { return type == WH_TYPE_Q4_K ? kGemmQ4F : kGemmQ8H; }
// The GEMM's reduction length for a K-quant row of k elements.
inline size_t kquant_gemm_k(int type, size_t k) { return type == WH_TYPE_Q4_K ? k : 2 * k; }
// Super-blocks per row of kGemmQ4F's dmin table: k / 256 rounded up to 8
// (16-byte rows).
inline size_t q4f_dmin_stride(size_t k) { return (k / 256 + 7) / 8 * 8; }
inline size_t kquant_repacked_bytes(int type, size_t n_rows, size_t k) {
  return n_rows * (type == WH_TYPE_Q4_K ? k / 32 * 20 + q4f_dmin_stride(k) * 2 : k / 16 * 20);
}
// Rewrites a Q4_K / Q6_K matrix (n_rows x k, 16-byte aligned) into the format above (kquant.hip).
int launch_repack_kquant(int type, const void* w, size_t n_rows, size_t k, void* out, hipStream_t stream);
// The copy of a K-quant matrix in the format above that wh_weight_prepare_prefill
// made for the handle whose data is w (with this type and shape), or null.
const void* prepared_kquant(const void* w, int type, size_t n_rows, size_t k);

// Number of compute units of the current device (cached per device, no lock).
int cu_count();
// Looks up the current device's copy of the no-allocation decode step's
// static scratch (decode.hip); called by wh_init.
int init_step_scratch();
// Largest LDS allocation one workgroup may use on the current device (cached
// per device, no lock).
size_t max_lds_per_block();

// Devices the per-device caches of the library track.
constexpr int kMaxDevices = 64;
// The dynamic LDS limit set so far for one kernel, per device.
struct LdsLimit {
  std::atomic<int> set[kMaxDevices];
};
// Raises fn's dynamic LDS limit on the current device to at least `bytes`.
// hipFuncSetAttribute is called only when a launch needs more than the limit
// already set on this device (it costs microseconds of host time, which every
// eager launch would otherwise pay).  Concurrent first calls may both set it.
int ensure_dynamic_lds(LdsLimit& lim, const void* fn, size_t bytes);
// The same with the kernel's own record, a static of the enclosing launcher
// (one per template instantiation, so one per kernel).  The kernel comes last
// so that template arguments with commas need no parentheses.
#define WH_ENSURE_LDS(bytes, ...)                                                                          \
  do {                                                                                                     \
    static ::wh::LdsLimit _wh_lim;                                                                         \
    const int _wh_st = ::wh::ensure_dynamic_lds(_wh_lim, reinterpret_cast<const void*>(__VA_ARGS__), (bytes)); \
    if (_wh_st != 0) return _wh_st;                                                                        \
  } while (0)

// Launchers implemented in the .hip translation units.  Arguments have been
// validated by the C ABI layer; these only choose kernels and launch them.
int launch_dequantize(int type, const void* data, size_t nelements, float* out,
                      hipStream_t stream);
// Q4_K / Q6_K (kquant.hip): bit-exact dequantization and dequantize-then-dot GEMV
// (y = residual + W x when residual is not null; y may be the residual).
int launch_dequantize_kquant(int type, const void* data, size_t nelements, float* out, hipStream_t stream);
int launch_gemv_kquant(int type, const void* w, const float* x, float* y, size_t n_rows, size_t k,
                       hipStream_t stream, const float* residual = nullptr);
int launch_fill_bytes(void* dst, int value, size_t nbytes, hipStream_t stream);
int launch_gemv(int type, const void* w, const float* x, float* y, size_t n_rows,
                size_t k, hipStream_t stream);
// FFN gate/up for one token with RMSNorm and SwiGLU fused into the streaming
// GEMV; WH_ERR_INVALID_SHAPE (nothing launched) when its layout does not fit.
int launch_ffn_gate_up(int type, const void* gate, const void* up, const float* x,
                       const float* gamma, float eps, float* h, size_t n_ff, size_t hidden,
                       hipStream_t stream);
// Single-token GEMV over up to three row-stacked matrices with the same K,
// optional RMSNorm prologue (gamma != null) and residual add (residual !=
// null); WH_ERR_INVALID_SHAPE (nothing launched) when its layout does not fit.
int launch_gemv_fused(int type, const void* const* mats, const size_t* rows, int n_mats, const float* x,
                      const float* gamma, float eps, const float* residual, float* y, size_t k,
                      hipStream_t stream);
// Single-token GEMV on the int8 matrix cores (gemv_mfma.hip): whether the shape
// fits, and the launch (WH_ERR_INVALID_SHAPE without launching otherwise).
// mats / rows: up to three row-stacked matrices with the same K; ffn: mats =
// {gate, up}, y = silu(gate x_hat) * (up x_hat) over n_out rows.
bool gemv_mfma_ok(int type, size_t n_out, size_t k);
int launch_gemv_mfma(int type, const void* const* mats, const size_t* rows, int n_mats, bool ffn, const float* x,
                     const float* gamma, float eps, const float* residual, float* y, size_t n_out, size_t k,
                     hipStream_t stream);
// Two groups of row-stacked matrices of different types over one x with the
// RMSNorm prologue, in one launch (group a -> y_a, group b -> y_b); taken for
// Q4_K + Q6_K with one-segment rows, WH_ERR_INVALID_SHAPE (nothing launched)
// otherwise.
int launch_gemv_mfma2(int type_a, const void* const* mats_a, const size_t* rows_a, int n_a, int type_b,
                      const void* const* mats_b, const size_t* rows_b, int n_b, const float* x, const float* gamma,
                      float eps, float* y_a, float* y_b, size_t k, hipStream_t stream);
// 2..16 tokens on the matrix cores (gemv_mfma.hip, Q4_0 and Q8_0): plain
// Y[t] = W X[t] (mats = {W}) or, with ffn, H[t] = silu(gate x_hat[t]) *
// (up x_hat[t]) with each token's RMSNorm (mats = {gate, up}); x is [m][k], row
// t of y starts at y + t * ldy.  WH_ERR_INVALID_SHAPE (nothing launched) when
// the shape does not fit.
int launch_gemv_mt(int type, const void* const* mats, bool ffn, const float* x, size_t m, const float* gamma,
                   float eps, float* y, size_t ldy, size_t n_out, size_t k, hipStream_t stream);
// Whether several-token products may take launch_gemv_mt: the calling
// thread's wh_gemv_select mode and the sizes the single-token matrix-core
// kernel needs (gemv.hip).
bool mt_allowed(size_t n_rows, size_t k);
// WH_GEMV_AUTO / WH_GEMV_STREAM (wh_gemv_select); returns the previous mode.
int gemv_mode_exchange(int mode);
// Token counts up to this use one streaming GEMV per token instead of MFMA.
constexpr size_t kGemvTokenLimit = 2;
size_t gemm_workspace_bytes(int type, size_t n_tokens, size_t k);
size_t gemm_workspace_bytes_for(int type, size_t n_rows, size_t n_tokens, size_t k);
int launch_gemm(int type, const void* w, size_t n_rows, size_t k, const float* x,
                size_t n_tokens, float* y, void* workspace, size_t workspace_bytes,
                hipStream_t stream);
// Tiled 16x16x32 MFMA kernel (gemm_tiled.hip): eligibility, workspace, launch.
bool gemm_tiled_ok(int type, const void* w, const float* x, size_t n_rows, size_t k, size_t n_tokens);
size_t gemm_tiled_workspace_bytes(int type, size_t n_rows, size_t n_tokens, size_t k);
int launch_gemm_tiled(int type, const void* w, size_t n_rows, size_t k, const float* x,
                      size_t n_tokens, float* y, void* workspace, hipStream_t stream);
// The tiled GEMM with bfloat16 activations, read directly by its packing.
int launch_gemm_tiled_bf16(int type, const void* w, size_t n_rows, size_t k, const uint16_t* x, size_t n_tokens,
                           float* y, void* workspace, hipStream_t s);
// bfloat16 -> f32 (exact), n elements.
int launch_bf16_to_f32(const uint16_t* x, size_t n, float* out, hipStream_t s);
// Q4_K / Q6_K on the tiled kernel: the matrix repacked into the front of the
// workspace, then the GEMM.
bool gemm_kquant_ok(int type, const void* w, const float* x, size_t n_rows, size_t k, size_t n_tokens);
size_t gemm_kquant_workspace_bytes(int type, size_t n_rows, size_t n_tokens, size_t k);
int launch_gemm_kquant(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                       float* y, void* workspace, hipStream_t stream);
// Workspace of launch_ffn_tiled beyond its g / u scratch, for a K-quant FFN.
size_t ffn_kquant_workspace_bytes(int type, size_t hidden, size_t n_ff, size_t n_tokens);
// FFN for more than kGemvTokenLimit tokens on the tiled kernel, with the
// RMSNorm and SwiGLU fused into its activation packing (g, u: scratch of
// n_tokens x n_ff); WH_ERR_INVALID_SHAPE (nothing launched) when it does not fit.
int launch_ffn_tiled(int type, const void* gate, const void* up, const void* down, size_t hidden, size_t n_ff,
                     const float* x, const float* gamma, float eps, size_t n_tokens, float* g, float* u, float* out,
                     void* workspace, size_t workspace_bytes, hipStream_t s);
// Decode attention (attention.hip).
size_t attention_workspace_bytes(size_t n_heads, size_t head_dim, size_t max_ctx, size_t n_kv_heads);
bool attention_shape_ok(size_t n_heads, size_t n_kv_heads, size_t head_dim);
int launch_attention_decode(const float* qkv, void* k_cache, void* v_cache, size_t pos, size_t n_heads,
                            size_t n_kv_heads, size_t head_dim, const float* inv_freq, float* out, void* ws,
                            hipStream_t stream);
// Token-embedding rows (embed.hip): out[t] = dequantized row ids[t] of a
// [vocab][hidden] table; NaN rows for ids >= vocab.
int check_embedding_args(const char* fn, int type, const void* table, size_t vocab, size_t hidden,
                         const uint32_t* ids, float* out);
int launch_embedding_lookup(int type, const void* table, size_t vocab, size_t hidden, const uint32_t* ids,
                            size_t n_tokens, float* out, hipStream_t stream);
int launch_rms_norm(const float* x, const float* weight, float eps, size_t tokens,
                    size_t hidden, float* out, hipStream_t stream);
int launch_swiglu(const float* gate, const float* up, size_t n, float* out,
                  hipStream_t stream);

}  // namespace wh

// -------------------------------------------------------------- device side
namespace whd {

// IEEE binary16 -> binary32 (v_cvt_f32_f16; exact, denormals preserved).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// Sum of v over the 64 lanes of the wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace whd
