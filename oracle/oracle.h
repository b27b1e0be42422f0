/*
 * oracle.h -- CPU restatement of woolly's quantized dequantize / GEMV / GEMM /
 * SwiGLU-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (woolly_amd, libwoolly_hip.so)
 * never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the Enreign/woolly repository root).  The f32 "order-exact" functions keep
 * the reference's evaluation order and are compiled with -ffp-contract=off,
 * because Rust never contracts `a*b + c` into a fused multiply-add.  The f64
 * functions accumulate in double and are the precision oracle the GPU results
 * are measured against.
 *
 * Parity pinning (how each function is checked, see tests/test_oracle.py):
 *   orc_f16_to_f32        exhaustive 65,536-pattern comparison with numpy's
 *                         independent IEEE binary16 widening.
 *   orc_f32_to_f16        against numpy float16 rounding (RNE) on random and
 *                         edge values.
 *   orc_dequantize        reference KATs (quantization.rs:1294-1386,
 *                         parallel_inference_integration.rs:159-210) and an
 *                         independent vectorised numpy decoder.  Q4_K /
 *                         Q6_K (the reference holds no vectors for them,
 *                         tests/test_oracle_kquant.py): closed forms that
 *                         isolate each layout rule (field offsets, nibble
 *                         order, 6-bit scale packing, unsigned Q6_K scales,
 *                         (q - 32) / 64, the qh wrap at element 255), a
 *                         whole-array numpy decoder on random bytes, and
 *                         planted mistakes that fail the closed forms.
 *   orc_matvec_f32       closed forms on constant-nibble blocks, brute force
 *                         in f64 on tiny shapes, and a numpy float32
 *                         sequential emulation on tiny shapes (order).
 *   orc_matvec_f64 /
 *   orc_matmul_f64        numpy float64 dequant-then-matmul.
 *   orc_gemm_f32          reference GEMM KATs matmul.rs:934-974,
 *                         tensor_utils.rs:608-620.
 *   orc_rms_norm_*        closed forms (constant rows) and numpy float64.
 *   orc_swiglu_*          special values (g=0, large |g|) and numpy float64.
 *   orc_ffn_*             composition of the above against numpy float64.
 *   orc_rope_inv_freq     numpy float64 1/base^(2i/d) within f32 rounding.
 *   orc_attention_decode_f64  closed forms (pos 0: out = v; equal keys:
 *                         mean of V), RoPE norm preservation, an independent
 *                         numpy float64 implementation on small shapes.
 *   orc_llama_layer_decode_f64, orc_llama_layer_decode_types_f64,
 *   orc_output_head_f64  numpy float64 composition on small shapes (the
 *                         types variant with Q4_K_M's per-tensor Q4_K / Q6_K
 *                         mix, each tensor dequantized with its own type; a
 *                         planted type swap fails).
 */
#ifndef WOOLLY_ORACLE_H
#define WOOLLY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGMLType ids, crates/woolly-gguf/src/tensor_info.rs:15-30 */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };

/* Status codes mirror woolly's errors (quantization.rs:8-26, error.rs:11-64). */
enum {
  ORC_OK = 0,
  ORC_ERR_UNSUPPORTED_TYPE = 1,
  ORC_ERR_INVALID_SHAPE = 2,
  ORC_ERR_BUFFER_TOO_SMALL = 3,
  ORC_ERR_INVALID_TENSOR_INFO = 11, /* Error::InvalidTensorInfo ("Q4_K data too small") */
};

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t* h, size_t n, float* out);
void orc_f32_to_f16_array(const float* f, size_t n, uint16_t* out);

size_t orc_block_size(int type);
size_t orc_type_size(int type);

int orc_dequantize(int type, const uint8_t* data, size_t nbytes, size_t nelements,
                   float* out);

int orc_matvec_f32(int type, const uint8_t* w, const float* x, float* y, size_t m,
                   size_t k);
int orc_matvec_f64(int type, const uint8_t* w, const float* x, double* y, size_t m,
                   size_t k);
int orc_matmul_f64(int type, const uint8_t* w, size_t n, size_t k, const float* x,
                   size_t m, double* y);
int orc_matmul_rows_f64(int type, const uint8_t* w, size_t n, size_t k, const float* x,
                        size_t m, const int64_t* rows, size_t nrows, double* y);

void orc_gemm_f32(const float* a, const float* b, float* c, size_t m, size_t n, size_t k,
                  float alpha, float beta);

void orc_rms_norm_f32(const float* x, const float* w, float eps, size_t tokens,
                      size_t hidden, float* out);
void orc_rms_norm_f64(const float* x, const float* w, double eps, size_t tokens,
                      size_t hidden, double* out);
void orc_swiglu_f32(const float* gate, const float* up, size_t n, float* out);
void orc_swiglu_f64(const double* gate, const double* up, size_t n, double* out);

int orc_ffn_f64(int type, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                size_t hidden, size_t n_ff, const float* gamma, double eps, const float* x,
                size_t m, double* out);
int orc_ffn_rows_f64(int type, const uint8_t* w_gate, const uint8_t* w_up,
                     const uint8_t* w_down, size_t hidden, size_t n_ff, const float* gamma,
                     double eps, const float* x, const int64_t* tokens, size_t ntok,
                     double* out);
int orc_ffn_f32(int type, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                size_t hidden, size_t n_ff, const float* gamma, float eps, const float* x,
                size_t m, float* out);

/* Decode step (oracle.c): RoPE inverse frequencies (ops/mod.rs:490-494, f32),
 * single-token GQA attention over an f16 KV cache with RoPE
 * (lazy_transformer.rs:261-456, ops/mod.rs:472-530), one transformer layer
 * (process_layer, lazy_transformer.rs:98-258) and the output head, in f64. */
int orc_rope_inv_freq(float base, size_t head_dim, float* out);
int orc_attention_decode_f64(const double* qkv, uint16_t* k_cache, uint16_t* v_cache, size_t pos,
                             size_t n_heads, size_t n_kv, size_t d, const float* inv_freq, int store_new,
                             double* out);
int orc_llama_layer_decode_f64(int type, const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const uint8_t* wo, const float* attn_norm, const uint8_t* wg,
                               const uint8_t* wu, const uint8_t* wd, const float* ffn_norm,
                               size_t hidden, size_t n_heads, size_t n_kv, size_t d, size_t n_ff,
                               double eps, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache,
                               size_t pos, int store_new, double* x);
int orc_output_head_f64(int type, const uint8_t* w, const float* norm, double eps, const double* x,
                        size_t hidden, size_t vocab, double* logits);
/* The same layer with a block type per projection, types = {q, k, v, o, gate,
 * up, down} (GGUF files such as Q4_K_M mix Q4_K and Q6_K tensors). */
int orc_llama_layer_decode_types_f64(const int* types, const uint8_t* wq, const uint8_t* wk,
                                     const uint8_t* wv, const uint8_t* wo, const float* attn_norm,
                                     const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                                     const float* ffn_norm, size_t hidden, size_t n_heads, size_t n_kv,
                                     size_t d, size_t n_ff, double eps, const float* inv_freq,
                                     uint16_t* k_cache, uint16_t* v_cache, size_t pos, int store_new,
                                     double* x);
/* The same layer in the reference's own f32 evaluation order (x f32 in place). */
int orc_llama_layer_decode_f32(int type, const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const uint8_t* wo, const float* attn_norm, const uint8_t* wg,
                               const uint8_t* wu, const uint8_t* wd, const float* ffn_norm,
                               size_t hidden, size_t n_heads, size_t n_kv, size_t d, size_t n_ff,
                               float eps, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache,
                               size_t pos, int store_new, float* x);

/* Multi-threaded 8-lane restatement of the reference's intended AVX2 GEMV
 * (qmatvec_q4_0_avx2 / qmatvec_q8_0_avx2, quantization.rs:720-840, nibble
 * order fixed), oracle_simd.c; the benchmark's CPU baseline.  Returns
 * ORC_ERR_UNSUPPORTED_TYPE when the CPU lacks AVX2/FMA. */
int orc_simd_available(void);
int orc_matvec_simd_mt(int type, const uint8_t* w, const float* x, float* y, size_t m, size_t k,
                       int threads);

#ifdef __cplusplus
}
#endif
#endif
