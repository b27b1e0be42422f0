/*
 * oracle.c -- CPU restatement of woolly's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of the
 * product.  Build with -O2 -ffp-contract=off (oracle/Makefile) so that every
 * `a*b + c` stays an unfused multiply then add, as in the Rust reference.
 * See oracle.h for the list of functions and how each one is pinned.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE-754 binary16 -> binary32 widening, written from the bit layout.
 * Restates half::f16::to_f32 as used at quantization.rs:470,495-496,581 and
 * dequantize.rs:306,356-357,572 (half 2.x: exact widening, NaNs are quieted
 * and keep their payload). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      /* subnormal: man * 2^-24; normalise so bit 10 is the implicit one */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while (!(man & 0x400u));
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
    if (man) bits |= 0x00400000u;
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  return bits_f32(bits);
}

/* binary32 -> binary16 with round-to-nearest-even (half::f16::from_f32, used
 * by the reference's KATs and by the synthetic-input generators). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) {
    if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13));
    return (uint16_t)(sign | 0x7C00u);
  }
  int e = (int)exp - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t hm = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

void orc_f16_to_f32_array(const uint16_t* h, size_t n, float* out) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}
void orc_f32_to_f16_array(const float* f, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(f[i]);
}

/* get_block_size / get_type_size, crates/woolly-gguf/src/dequantize.rs:208-242 */
size_t orc_block_size(int type) {
  switch (type) {
    case ORC_F32:
    case ORC_F16:
      return 1;
    case ORC_Q4_0:
    case ORC_Q4_1:
    case ORC_Q5_0:
    case ORC_Q5_1:
    case ORC_Q8_0:
      return 32;
    case ORC_Q4_K:
    case ORC_Q6_K:
      return 256;
    default:
      return 0;
  }
}
size_t orc_type_size(int type) {
  switch (type) {
    case ORC_F32:
      return 4;
    case ORC_F16:
      return 2;
    case ORC_Q4_0:
      return 18;
    case ORC_Q4_1:
      return 20;
    case ORC_Q5_0:
      return 22;
    case ORC_Q5_1:
      return 24;
    case ORC_Q8_0:
      return 34;
    case ORC_Q4_K:
      return 144;
    case ORC_Q6_K:
      return 210;
    default:
      return 0;
  }
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Dequantize one block of 32 elements into out[0..32).
 *   Q4_0: quantization.rs:466-486 / dequantize.rs:286-327:
 *         element j<16 = ((qs[j] & 0xF) - 8) * d, element j+16 = ((qs[j] >> 4) - 8) * d
 *   Q4_1: quantization.rs:490-511 / dequantize.rs:337-378: q * d + m
 *   Q5_0: quantization.rs:515-541 (BlockQ5_0 {d, qh[4], qs[16]}, :117-127):
 *         qh = u32::from_le_bytes(qh); for j < 16:
 *         xh_0 = ((qh >> j) << 4) & 0x10, xh_1 = (qh >> (j + 12)) & 0x10,
 *         element j = ((qs[j] & 0xF) | xh_0) - 16) * d, element j+16 = ((qs[j] >> 4) | xh_1) - 16) * d
 *   Q5_1: quantization.rs:545-573 (BlockQ5_1 {d, m, qh[4], qs[16]}, :129-140):
 *         the same x0 / x1 without the -16, value x * d + m (mul, then add)
 *   Q8_0: quantization.rs:576-590 / dequantize.rs:553-586: (int8)qs[j] * d */
static void dequant_block(int type, const uint8_t* b, float* out) {
  if (type == ORC_Q4_0) {
    float d = orc_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    for (int j = 0; j < 16; j++) {
      int x0 = (int)(qs[j] & 0x0F) - 8;
      int x1 = (int)(qs[j] >> 4) - 8;
      out[j] = (float)x0 * d;
      out[j + 16] = (float)x1 * d;
    }
  } else if (type == ORC_Q4_1) {
    float d = orc_f16_to_f32(rd16(b));
    float m = orc_f16_to_f32(rd16(b + 2));
    const uint8_t* qs = b + 4;
    for (int j = 0; j < 16; j++) {
      float x0 = (float)(qs[j] & 0x0F);
      float x1 = (float)(qs[j] >> 4);
      float p0 = x0 * d;
      float p1 = x1 * d;
      out[j] = p0 + m;
      out[j + 16] = p1 + m;
    }
  } else if (type == ORC_Q5_0 || type == ORC_Q5_1) {
    const int q51 = type == ORC_Q5_1;
    float d = orc_f16_to_f32(rd16(b));
    float m = q51 ? orc_f16_to_f32(rd16(b + 2)) : 0.0f;
    const uint8_t* qhp = b + (q51 ? 4 : 2);
    const uint8_t* qs = qhp + 4;
    uint32_t qh = (uint32_t)qhp[0] | ((uint32_t)qhp[1] << 8) | ((uint32_t)qhp[2] << 16) | ((uint32_t)qhp[3] << 24);
    for (int j = 0; j < 16; j++) {
      uint32_t xh_0 = ((qh >> j) << 4) & 0x10;
      uint32_t xh_1 = (qh >> (j + 12)) & 0x10;
      uint32_t x0 = (uint32_t)(qs[j] & 0x0F) | xh_0;
      uint32_t x1 = (uint32_t)(qs[j] >> 4) | xh_1;
      if (q51) {
        float p0 = (float)x0 * d;
        float p1 = (float)x1 * d;
        out[j] = p0 + m;
        out[j + 16] = p1 + m;
      } else {
        out[j] = (float)((int32_t)x0 - 16) * d;
        out[j + 16] = (float)((int32_t)x1 - 16) * d;
      }
    }
  } else { /* ORC_Q8_0 */
    float d = orc_f16_to_f32(rd16(b));
    const int8_t* qs = (const int8_t*)(b + 2);
    for (int j = 0; j < 32; j++) out[j] = (float)qs[j] * d;
  }
}

/* Q4_K as woolly_gguf decodes it (dequantize_q4_k_scalar, dequantize.rs:404-458;
 * the x86 path: the NEON variant is aarch64-only).  This is woolly's own
 * layout, not ggml's: 12 bytes of packed 6-bit scales first (bytes 0..11),
 * then f16 d (12..13) and f16 dmin (14..15), then 128 bytes of quants.
 * Scales: for i < 8, src = 3i/2; even i: s = b[src] & 63; odd i:
 * s = ((b[src] >> 6) | ((b[src+1] & 15) << 2)) & 63.  Element i (0..255):
 * q = qs[i/2] & 15 for even i, qs[i/2] >> 4 for odd i, value
 * d * scale[i/32] * q + dmin, evaluated left to right in f32. */
static void dequant_q4_k_block(const uint8_t* b, float* out) {
  uint8_t scales[16] = {0};
  for (int i = 0; i < 8; i++) {
    int src = (i * 3) / 2;
    if (i % 2 == 0) scales[i] = (uint8_t)(b[src] & 63);
    else scales[i] = (uint8_t)(((b[src] >> 6) | ((b[src + 1] & 15) << 2)) & 63);
  }
  float d = orc_f16_to_f32(rd16(b + 12));
  float dmin = orc_f16_to_f32(rd16(b + 14));
  const uint8_t* qs = b + 16;
  for (int i = 0; i < 256; i++) {
    int q = (i % 2 == 0) ? (qs[i / 2] & 0x0F) : ((qs[i / 2] >> 4) & 0x0F);
    float scale = (float)scales[i / 32];
    float t = d * scale;
    float u = t * (float)q;
    out[i] = u + dmin;
  }
}

/* Q6_K as woolly_gguf decodes it (dequantize_q6_k, dequantize.rs:460-536):
 * ql = bytes 0..127, qh = 128..191, scales = 192..207 (read as u8), f16 d at
 * 208..209.  Element i: is = i/16,
 *   ql_idx = 64(i/128) + 32((i%128)/64) + 16((i%64)/32) + i%16,
 *   qh_idx = 32(i/128) + 16((i%128)/64) + 8((i%64)/32) + (i%32)/4,
 *   shift = 2((i%32)%4), e1 = (qh[qh_idx] >> shift) & 3,
 *   e2 = shift < 6 ? (qh[qh_idx] >> (shift+2)) & 3 : (qh_idx+1 < 64 ? qh[qh_idx+1] & 3 : 0),
 *   q = i < 128 ? (ql[ql_idx] & 15) | (e1 << 4) : (ql[ql_idx] >> 4) | (e2 << 4),
 * value ((d * scales[is]) * (q - 32)) / 64, left to right in f32. */
static void dequant_q6_k_block(const uint8_t* b, float* out) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const uint8_t* sc = b + 192;
  float d = orc_f16_to_f32(rd16(b + 208));
  for (int i = 0; i < 256; i++) {
    int is = i / 16;
    int ql_idx = 64 * (i / 128) + 32 * ((i % 128) / 64) + 16 * ((i % 64) / 32) + (i % 16);
    int qh_idx = 32 * (i / 128) + 16 * ((i % 128) / 64) + 8 * ((i % 64) / 32) + (i % 32) / 4;
    int shift = 2 * ((i % 32) % 4);
    uint8_t qhv = qh[qh_idx];
    uint8_t e1 = (uint8_t)((qhv >> shift) & 3);
    uint8_t e2;
    if (shift < 6) e2 = (uint8_t)((qhv >> (shift + 2)) & 3);
    else e2 = (uint8_t)(qh_idx + 1 < 64 ? (qh[qh_idx + 1] & 3) : 0);
    uint8_t q1 = (uint8_t)((ql[ql_idx] & 0x0F) | (e1 << 4));
    uint8_t q2 = (uint8_t)((ql[ql_idx] >> 4) | (e2 << 4));
    uint8_t q = i < 128 ? q1 : q2;
    float s = (float)sc[is];
    float t = d * s;
    float u = t * (float)((int)(int8_t)q - 32);
    out[i] = u / 64.0f;
  }
}

static void dequant_any_block(int type, const uint8_t* b, float* out) {
  if (type == ORC_Q4_K) dequant_q4_k_block(b, out);
  else if (type == ORC_Q6_K) dequant_q6_k_block(b, out);
  else dequant_block(type, b, out);
}

/* woolly_gguf::dequantize(data, ggml_type, nelements), dequantize.rs:189-205:
 * nblocks = ceil(n / 32); BufferTooSmall when data is shorter than
 * nblocks * type_size; the output is truncated to n elements. */
int orc_dequantize(int type, const uint8_t* data, size_t nbytes, size_t nelements,
                   float* out) {
  size_t ts = orc_type_size(type);
  if (ts == 0) return ORC_ERR_UNSUPPORTED_TYPE;
  if (type == ORC_F32) {
    if (nbytes != nelements * 4) return ORC_ERR_BUFFER_TOO_SMALL;
    memcpy(out, data, nelements * 4);
    return ORC_OK;
  }
  if (type == ORC_F16) {
    if (nbytes != nelements * 2) return ORC_ERR_BUFFER_TOO_SMALL;
    for (size_t i = 0; i < nelements; i++) out[i] = orc_f16_to_f32(rd16(data + 2 * i));
    return ORC_OK;
  }
  size_t bs = orc_block_size(type);
  size_t nb = (nelements + bs - 1) / bs;
  /* Q4_K / Q6_K report a short buffer as InvalidTensorInfo (dequantize.rs:416-418, 472-474) */
  if (nbytes < nb * ts) return bs == 256 ? ORC_ERR_INVALID_TENSOR_INFO : ORC_ERR_BUFFER_TOO_SMALL;
  float tmp[256];
  for (size_t b = 0; b < nb; b++) {
    dequant_any_block(type, data + b * ts, tmp);
    size_t base = b * bs;
    size_t cnt = nelements - base < bs ? nelements - base : bs;
    memcpy(out + base, tmp, cnt * sizeof(float));
  }
  return ORC_OK;
}

static int check_matvec_args(int type, size_t k) {
  if (type != ORC_Q4_0 && type != ORC_Q4_1 && type != ORC_Q8_0 && type != ORC_Q4_K && type != ORC_Q6_K)
    return ORC_ERR_UNSUPPORTED_TYPE;
  if (k % orc_block_size(type) != 0) return ORC_ERR_INVALID_SHAPE;
  return ORC_OK;
}

/* Order-exact f32 quantized matvec, y[row] = sum_k W[row,k] * x[k].
 *   Q4_0: quantized_matvec_q4_0_scalar, quantization.rs:1100-1132
 *         sum += (x0 * d) * input[off + j]; sum += (x1 * d) * input[off + j + 16]
 *   Q8_0: quantized_matvec_q8_0_scalar, quantization.rs:1135-1163
 *   Q4_1: no reference kernel (quantized_matvec returns UnsupportedScheme at
 *         quantization.rs:905-907); defined as dequantize_q4_1
 *         (quantization.rs:490-511) followed by the f32 dot in the Q4_0 order. */
int orc_matvec_f32(int type, const uint8_t* w, const float* x, float* y, size_t m,
                   size_t k) {
  int st = check_matvec_args(type, k);
  if (st) return st;
  if (type == ORC_Q4_K || type == ORC_Q6_K) {
    /* no reference kernel: dequantize (dequantize.rs:404-536) then the f32 dot
     * in element order */
    size_t nbk = k / 256, tsk = orc_type_size(type);
    float deq[256];
    for (size_t row = 0; row < m; row++) {
      float sum = 0.0f;
      for (size_t b = 0; b < nbk; b++) {
        dequant_any_block(type, w + (row * nbk + b) * tsk, deq);
        for (int j = 0; j < 256; j++) {
          float p = deq[j] * x[b * 256 + j];
          sum = sum + p;
        }
      }
      y[row] = sum;
    }
    return ORC_OK;
  }
  size_t nb = k / 32, ts = orc_type_size(type);
  for (size_t row = 0; row < m; row++) {
    float sum = 0.0f;
    const uint8_t* rp = w + row * nb * ts;
    for (size_t b = 0; b < nb; b++) {
      const uint8_t* blk = rp + b * ts;
      const float* in = x + b * 32;
      if (type == ORC_Q4_0) {
        float d = orc_f16_to_f32(rd16(blk));
        const uint8_t* qs = blk + 2;
        for (int j = 0; j < 16; j++) {
          int x0 = (int)(qs[j] & 0x0F) - 8;
          int x1 = (int)(qs[j] >> 4) - 8;
          float w0 = (float)x0 * d;
          float w1 = (float)x1 * d;
          float p0 = w0 * in[j];
          sum = sum + p0;
          float p1 = w1 * in[j + 16];
          sum = sum + p1;
        }
      } else if (type == ORC_Q8_0) {
        float d = orc_f16_to_f32(rd16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        for (int j = 0; j < 32; j++) {
          float wv = (float)qs[j] * d;
          float p = wv * in[j];
          sum = sum + p;
        }
      } else {
        float deq[32];
        dequant_block(ORC_Q4_1, blk, deq);
        for (int j = 0; j < 16; j++) {
          float p0 = deq[j] * in[j];
          sum = sum + p0;
          float p1 = deq[j + 16] * in[j + 16];
          sum = sum + p1;
        }
      }
    }
    y[row] = sum;
  }
  return ORC_OK;
}

/* Same product accumulated in double: every dequantized weight is an exact
 * f32 value and f32*f32 is exact in f64, so this is the precision oracle. */
int orc_matvec_f64(int type, const uint8_t* w, const float* x, double* y, size_t m,
                   size_t k) {
  int st = check_matvec_args(type, k);
  if (st) return st;
  size_t bs = orc_block_size(type), nb = k / bs, ts = orc_type_size(type);
  float deq[256];
  for (size_t row = 0; row < m; row++) {
    double sum = 0.0;
    const uint8_t* rp = w + row * nb * ts;
    for (size_t b = 0; b < nb; b++) {
      dequant_any_block(type, rp + b * ts, deq);
      const float* in = x + b * bs;
      for (size_t j = 0; j < bs; j++) sum += (double)deq[j] * (double)in[j];
    }
    y[row] = sum;
  }
  return ORC_OK;
}

static void dequant_row(int type, const uint8_t* w, size_t row, size_t k, float* out) {
  size_t bs = orc_block_size(type), nb = k / bs, ts = orc_type_size(type);
  const uint8_t* rp = w + row * nb * ts;
  for (size_t b = 0; b < nb; b++) dequant_any_block(type, rp + b * ts, out + b * bs);
}

/* Y[t, n] = sum_k X[t, k] * W[n, k] in double, for a subset of token rows.
 * This is the quantized replacement of the projections in
 * simd_ffn_forward (tensor_utils_simd.rs:605-754) using ggml's [N][K]
 * weight convention (quantization.rs:730-737). */
int orc_matmul_rows_f64(int type, const uint8_t* w, size_t n, size_t k, const float* x,
                        size_t m, const int64_t* rows, size_t nrows, double* y) {
  int st = check_matvec_args(type, k);
  if (st) return st;
  (void)m;
  float* wrow = (float*)malloc(k * sizeof(float));
  if (!wrow) return ORC_ERR_BUFFER_TOO_SMALL;
  for (size_t j = 0; j < n; j++) {
    dequant_row(type, w, j, k, wrow);
    for (size_t r = 0; r < nrows; r++) {
      const float* xr = x + (size_t)rows[r] * k;
      double s = 0.0;
      for (size_t i = 0; i < k; i++) s += (double)xr[i] * (double)wrow[i];
      y[r * n + j] = s;
    }
  }
  free(wrow);
  return ORC_OK;
}

int orc_matmul_f64(int type, const uint8_t* w, size_t n, size_t k, const float* x,
                   size_t m, double* y) {
  int64_t* rows = (int64_t*)malloc((m ? m : 1) * sizeof(int64_t));
  if (!rows) return ORC_ERR_BUFFER_TOO_SMALL;
  for (size_t i = 0; i < m; i++) rows[i] = (int64_t)i;
  int st = orc_matmul_rows_f64(type, w, n, k, x, m, rows, m, y);
  free(rows);
  return st;
}

/* Gemm::compute_naive, crates/woolly-tensor/src/ops/matmul.rs:608-646
 * (no transposes): c[i*n+j] = alpha * sum_l a[i*k+l]*b[l*n+j] + beta * c[i*n+j]. */
void orc_gemm_f32(const float* a, const float* b, float* c, size_t m, size_t n, size_t k,
                  float alpha, float beta) {
  for (size_t i = 0; i < m; i++) {
    for (size_t j = 0; j < n; j++) {
      float sum = 0.0f;
      for (size_t l = 0; l < k; l++) {
        float p = a[i * k + l] * b[l * n + j];
        sum = sum + p;
      }
      float s1 = alpha * sum;
      float s2 = beta * c[i * n + j];
      c[i * n + j] = s1 + s2;
    }
  }
}

/* rms_norm, crates/woolly-core/src/tensor_utils.rs:446-480:
 *   rms = sqrt(sum(x*x) / hidden + eps);  out = (x / rms) * w  */
void orc_rms_norm_f32(const float* x, const float* w, float eps, size_t tokens,
                      size_t hidden, float* out) {
  for (size_t t = 0; t < tokens; t++) {
    const float* xt = x + t * hidden;
    float ss = 0.0f;
    for (size_t i = 0; i < hidden; i++) {
      float sq = xt[i] * xt[i];
      ss = ss + sq;
    }
    float mean = ss / (float)hidden;
    float rms = sqrtf(mean + eps);
    for (size_t i = 0; i < hidden; i++) {
      float nv = xt[i] / rms;
      out[t * hidden + i] = nv * w[i];
    }
  }
}

void orc_rms_norm_f64(const float* x, const float* w, double eps, size_t tokens,
                      size_t hidden, double* out) {
  for (size_t t = 0; t < tokens; t++) {
    const float* xt = x + t * hidden;
    double ss = 0.0;
    for (size_t i = 0; i < hidden; i++) ss += (double)xt[i] * (double)xt[i];
    double rms = sqrt(ss / (double)hidden + eps);
    for (size_t i = 0; i < hidden; i++) out[t * hidden + i] = ((double)xt[i] / rms) * w[i];
  }
}

/* swiglu, crates/woolly-core/src/tensor_utils.rs:512-532:
 *   silu_gate = g * (1 / (1 + exp(-g)));  out = silu_gate * u
 * (the exact SiLU; not the approximations of simd_matmul.rs:1050-1108). */
void orc_swiglu_f32(const float* gate, const float* up, size_t n, float* out) {
  for (size_t i = 0; i < n; i++) {
    float g = gate[i];
    float e = expf(-g);
    float den = 1.0f + e;
    float sig = 1.0f / den;
    float sg = g * sig;
    out[i] = sg * up[i];
  }
}

void orc_swiglu_f64(const double* gate, const double* up, size_t n, double* out) {
  for (size_t i = 0; i < n; i++) {
    double g = gate[i];
    out[i] = g * (1.0 / (1.0 + exp(-g))) * up[i];
  }
}

/* One SwiGLU FFN layer with its RMSNorm prologue, in double:
 *   xh = rms_norm(x, gamma, eps)                 tensor_utils.rs:446-480
 *   g = W_gate xh, u = W_up xh                   lazy_transformer.rs:1073-1123
 *   h = silu(g) * u                              tensor_utils.rs:512-532
 *   out = W_down h                               feedforward.rs:93-127
 * Weights use ggml's [N][K] convention: gate/up are [n_ff][hidden] and down is
 * [hidden][n_ff]. */
int orc_ffn_rows_f64(int type, const uint8_t* w_gate, const uint8_t* w_up,
                     const uint8_t* w_down, size_t hidden, size_t n_ff, const float* gamma,
                     double eps, const float* x, const int64_t* tokens, size_t ntok,
                     double* out) {
  int st = check_matvec_args(type, hidden);
  if (st) return st;
  st = check_matvec_args(type, n_ff);
  if (st) return st;
  double* xh = (double*)malloc(hidden * sizeof(double));
  double* g = (double*)malloc(n_ff * sizeof(double));
  double* u = (double*)malloc(n_ff * sizeof(double));
  double* h = (double*)malloc(n_ff * sizeof(double));
  float* wrow = (float*)malloc((hidden > n_ff ? hidden : n_ff) * sizeof(float));
  if (!xh || !g || !u || !h || !wrow) {
    free(xh); free(g); free(u); free(h); free(wrow);
    return ORC_ERR_BUFFER_TOO_SMALL;
  }
  for (size_t t = 0; t < ntok; t++) {
    orc_rms_norm_f64(x + (size_t)tokens[t] * hidden, gamma, eps, 1, hidden, xh);
    for (size_t j = 0; j < n_ff; j++) {
      double sg = 0.0, su = 0.0;
      dequant_row(type, w_gate, j, hidden, wrow);
      for (size_t i = 0; i < hidden; i++) sg += (double)wrow[i] * xh[i];
      dequant_row(type, w_up, j, hidden, wrow);
      for (size_t i = 0; i < hidden; i++) su += (double)wrow[i] * xh[i];
      g[j] = sg;
      u[j] = su;
    }
    orc_swiglu_f64(g, u, n_ff, h);
    for (size_t i = 0; i < hidden; i++) {
      double s = 0.0;
      dequant_row(type, w_down, i, n_ff, wrow);
      for (size_t j = 0; j < n_ff; j++) s += (double)wrow[j] * h[j];
      out[t * hidden + i] = s;
    }
  }
  free(xh); free(g); free(u); free(h); free(wrow);
  return ORC_OK;
}

int orc_ffn_f64(int type, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                size_t hidden, size_t n_ff, const float* gamma, double eps, const float* x,
                size_t m, double* out) {
  int64_t* rows = (int64_t*)malloc((m ? m : 1) * sizeof(int64_t));
  if (!rows) return ORC_ERR_BUFFER_TOO_SMALL;
  for (size_t i = 0; i < m; i++) rows[i] = (int64_t)i;
  int st = orc_ffn_rows_f64(type, w_gate, w_up, w_down, hidden, n_ff, gamma, eps, x, rows,
                            m, out);
  free(rows);
  return st;
}

/* The same layer on woolly's CPU f32 path: rms_norm (f32 order), the
 * order-exact scalar quantized matvec for each projection and token, and the
 * exact SwiGLU.  This is the CPU baseline the GPU FFN is timed beside. */
int orc_ffn_f32(int type, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                size_t hidden, size_t n_ff, const float* gamma, float eps, const float* x,
                size_t m, float* out) {
  int st = check_matvec_args(type, hidden);
  if (st) return st;
  st = check_matvec_args(type, n_ff);
  if (st) return st;
  float* xh = (float*)malloc(hidden * sizeof(float));
  float* g = (float*)malloc(n_ff * sizeof(float));
  float* u = (float*)malloc(n_ff * sizeof(float));
  float* h = (float*)malloc(n_ff * sizeof(float));
  if (!xh || !g || !u || !h) {
    free(xh); free(g); free(u); free(h);
    return ORC_ERR_BUFFER_TOO_SMALL;
  }
  for (size_t t = 0; t < m; t++) {
    orc_rms_norm_f32(x + t * hidden, gamma, eps, 1, hidden, xh);
    orc_matvec_f32(type, w_gate, xh, g, n_ff, hidden);
    orc_matvec_f32(type, w_up, xh, u, n_ff, hidden);
    orc_swiglu_f32(g, u, n_ff, h);
    orc_matvec_f32(type, w_down, h, out + t * hidden, hidden, n_ff);
  }
  free(xh); free(g); free(u); free(h);
  return ORC_OK;
}

/* ------------------------------------------------------------ decode step */

/* RoPE inverse frequencies, RoPE::apply_f32 (crates/woolly-tensor/src/ops/mod.rs:490-494):
 * freqs[i] = 1.0 / base.powf(2.0 * i as f32 / head_dim as f32), all in f32. */
int orc_rope_inv_freq(float base, size_t head_dim, float* out) {
  if (head_dim == 0 || head_dim % 2) return ORC_ERR_INVALID_SHAPE;
  for (size_t i = 0; i < head_dim / 2; i++) {
    float e = (2.0f * (float)i) / (float)head_dim;
    out[i] = 1.0f / powf(base, e);
  }
  return ORC_OK;
}

/* Rotation of one head (ops/mod.rs:500-524): pairs (i, i + d/2), angle =
 * pos * freq in f32 (the reference multiplies in f32), sin/cos and the
 * rotation in double. */
static void rope_head_d(const double* in, double* out, size_t d, size_t pos, const float* inv_freq) {
  size_t h = d / 2;
  for (size_t i = 0; i < h; i++) {
    float ang = (float)pos * inv_freq[i];
    double c = cos((double)ang), s = sin((double)ang);
    double x1 = in[i], x2 = in[i + h];
    out[i] = x1 * c - x2 * s;
    out[i + h] = x1 * s + x2 * c;
  }
}

/* Attention of one new token at position pos over an f16 KV cache
 * ([ctx][n_kv][d] half bits), compute_optimized_gqa_attention
 * (crates/woolly-core/src/model/lazy_transformer.rs:261-456) with RoPE on q
 * and k: q head h uses KV head h / (n_heads / n_kv) (:380-388); the new k
 * (rotated) and v are rounded to f16 and stored at row pos (:326-345), then
 * s_p = (q . k_p) / sqrt(d) for p <= pos, softmax with the maximum
 * subtracted (:407-420), out = sum_p w_p v_p (:423-433).  qkv = q | k | v. */
int orc_attention_decode_f64(const double* qkv, uint16_t* k_cache, uint16_t* v_cache, size_t pos,
                             size_t n_heads, size_t n_kv, size_t d, const float* inv_freq, int store_new,
                             double* out) {
  if (n_kv == 0 || n_heads % n_kv || d == 0 || d % 2) return ORC_ERR_INVALID_SHAPE;
  size_t G = n_heads / n_kv, kvd = n_kv * d;
  double* rot = (double*)malloc(d * sizeof(double));
  double* sc = (double*)malloc((pos + 1) * sizeof(double));
  if (!rot || !sc) {
    free(rot);
    free(sc);
    return ORC_ERR_BUFFER_TOO_SMALL;
  }
  for (size_t kh = 0; kh < n_kv && store_new; kh++) {
    rope_head_d(qkv + n_heads * d + kh * d, rot, d, pos, inv_freq);
    for (size_t i = 0; i < d; i++) {
      k_cache[(pos * n_kv + kh) * d + i] = orc_f32_to_f16((float)rot[i]);
      v_cache[(pos * n_kv + kh) * d + i] = orc_f32_to_f16((float)qkv[n_heads * d + kvd + kh * d + i]);
    }
  }
  double scale = 1.0 / sqrt((double)d);
  for (size_t h = 0; h < n_heads; h++) {
    size_t kh = h / G;
    rope_head_d(qkv + h * d, rot, d, pos, inv_freq);
    double mx = -INFINITY;
    for (size_t p = 0; p <= pos; p++) {
      const uint16_t* kr = k_cache + (p * n_kv + kh) * d;
      double s = 0.0;
      for (size_t i = 0; i < d; i++) s += rot[i] * (double)orc_f16_to_f32(kr[i]);
      sc[p] = s * scale;
      if (sc[p] > mx) mx = sc[p];
    }
    double sum = 0.0;
    for (size_t p = 0; p <= pos; p++) {
      sc[p] = exp(sc[p] - mx);
      sum += sc[p];
    }
    for (size_t i = 0; i < d; i++) {
      double a = 0.0;
      for (size_t p = 0; p <= pos; p++) a += sc[p] * (double)orc_f16_to_f32(v_cache[(p * n_kv + kh) * d + i]);
      out[h * d + i] = a / sum;
    }
  }
  free(rot);
  free(sc);
  return ORC_OK;
}

/* y = W x with an f64 input (weights dequantized exactly). */
static int matvec_dd(int type, const uint8_t* w, const double* x, double* y, size_t m, size_t k) {
  float* wrow = (float*)malloc(k * sizeof(float));
  if (!wrow) return ORC_ERR_BUFFER_TOO_SMALL;
  for (size_t r = 0; r < m; r++) {
    dequant_row(type, w, r, k, wrow);
    double s = 0.0;
    for (size_t i = 0; i < k; i++) s += (double)wrow[i] * x[i];
    y[r] = s;
  }
  free(wrow);
  return ORC_OK;
}

static void rms_norm_dd(const double* x, const float* g, double eps, size_t n, double* out) {
  double ss = 0.0;
  for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
  double rms = sqrt(ss / (double)n + eps);
  for (size_t i = 0; i < n; i++) out[i] = (x[i] / rms) * (double)g[i];
}

/* One layer for one token, LazyTransformer::process_layer
 * (lazy_transformer.rs:98-258): x += Wo attn(qkv(rms_norm(x, attn_norm)));
 * x += Wd (silu(Wg x_hat) * (Wu x_hat)), x_hat = rms_norm(x, ffn_norm).  x in
 * f64, updated in place; the caches are updated at row pos. */
int orc_llama_layer_decode_types_f64(const int* types, const uint8_t* wq, const uint8_t* wk,
                                     const uint8_t* wv, const uint8_t* wo, const float* attn_norm,
                                     const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                                     const float* ffn_norm, size_t hidden, size_t n_heads, size_t n_kv,
                                     size_t d, size_t n_ff, double eps, const float* inv_freq,
                                     uint16_t* k_cache, uint16_t* v_cache, size_t pos, int store_new,
                                     double* x) {
  size_t qd = n_heads * d, kvd = n_kv * d;
  /* reduction length of each projection: q, k, v, gate, up read x_hat; o reads
   * the attention output, down the SwiGLU */
  const size_t kdim[7] = {hidden, hidden, hidden, qd, hidden, hidden, n_ff};
  int st = ORC_OK;
  for (int i = 0; i < 7; i++)
    if ((st = check_matvec_args(types[i], kdim[i]))) return st;
  size_t big = hidden > n_ff ? hidden : n_ff;
  double* xn = (double*)malloc(big * sizeof(double));
  double* qkv = (double*)malloc((qd + 2 * kvd) * sizeof(double));
  double* att = (double*)malloc(qd * sizeof(double));
  double* g = (double*)malloc(n_ff * sizeof(double));
  double* u = (double*)malloc(n_ff * sizeof(double));
  double* y = (double*)malloc(hidden * sizeof(double));
  if (!xn || !qkv || !att || !g || !u || !y) {
    st = ORC_ERR_BUFFER_TOO_SMALL;
    goto done;
  }
  rms_norm_dd(x, attn_norm, eps, hidden, xn);
  if ((st = matvec_dd(types[0], wq, xn, qkv, qd, hidden))) goto done;
  if ((st = matvec_dd(types[1], wk, xn, qkv + qd, kvd, hidden))) goto done;
  if ((st = matvec_dd(types[2], wv, xn, qkv + qd + kvd, kvd, hidden))) goto done;
  if ((st = orc_attention_decode_f64(qkv, k_cache, v_cache, pos, n_heads, n_kv, d, inv_freq, store_new, att)))
    goto done;
  if ((st = matvec_dd(types[3], wo, att, y, hidden, qd))) goto done;
  for (size_t i = 0; i < hidden; i++) x[i] += y[i];
  rms_norm_dd(x, ffn_norm, eps, hidden, xn);
  if ((st = matvec_dd(types[4], wg, xn, g, n_ff, hidden))) goto done;
  if ((st = matvec_dd(types[5], wu, xn, u, n_ff, hidden))) goto done;
  orc_swiglu_f64(g, u, n_ff, g);
  if ((st = matvec_dd(types[6], wd, g, y, hidden, n_ff))) goto done;
  for (size_t i = 0; i < hidden; i++) x[i] += y[i];
done:
  free(xn);
  free(qkv);
  free(att);
  free(g);
  free(u);
  free(y);
  return st;
}

int orc_llama_layer_decode_f64(int type, const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const uint8_t* wo, const float* attn_norm, const uint8_t* wg,
                               const uint8_t* wu, const uint8_t* wd, const float* ffn_norm,
                               size_t hidden, size_t n_heads, size_t n_kv, size_t d, size_t n_ff,
                               double eps, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache,
                               size_t pos, int store_new, double* x) {
  const int types[7] = {type, type, type, type, type, type, type};
  return orc_llama_layer_decode_types_f64(types, wq, wk, wv, wo, attn_norm, wg, wu, wd, ffn_norm, hidden,
                                          n_heads, n_kv, d, n_ff, eps, inv_freq, k_cache, v_cache, pos,
                                          store_new, x);
}

/* logits = W rms_norm(x, norm) with f64 x (the end of forward,
 * lazy_transformer.rs:1281-1316). */
int orc_output_head_f64(int type, const uint8_t* w, const float* norm, double eps, const double* x,
                        size_t hidden, size_t vocab, double* logits) {
  int st = check_matvec_args(type, hidden);
  if (st) return st;
  double* xn = (double*)malloc(hidden * sizeof(double));
  if (!xn) return ORC_ERR_BUFFER_TOO_SMALL;
  rms_norm_dd(x, norm, eps, hidden, xn);
  st = matvec_dd(type, w, xn, logits, vocab, hidden);
  free(xn);
  return st;
}

/* Order-exact f32 restatement of the reference's decode layer on an f16 KV
 * cache: rms_norm (tensor_utils.rs:446-480), the scalar quantized matvecs
 * (quantization.rs:1100-1163), RoPE in f32 (ops/mod.rs:506-521: x1*cos - x2*sin,
 * x1*sin + x2*cos, unfused), the attention loops of
 * compute_optimized_gqa_attention (lazy_transformer.rs:380-433: sequential dot,
 * * scale, max, exp(s - max), sequential sum, inv_sum = 1 / sum,
 * out += (e * inv_sum) * v), swiglu (tensor_utils.rs:512-532) and the residual
 * adds of process_layer (:186-188, 245-247).  The checker of how accurate the
 * reference's own f32 path is on the same input; x (f32) is updated in place
 * and the new k / v (f16) are stored at row pos. */
int orc_llama_layer_decode_f32(int type, const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const uint8_t* wo, const float* attn_norm, const uint8_t* wg,
                               const uint8_t* wu, const uint8_t* wd, const float* ffn_norm,
                               size_t hidden, size_t n_heads, size_t n_kv, size_t d, size_t n_ff,
                               float eps, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache,
                               size_t pos, int store_new, float* x) {
  int st = check_matvec_args(type, hidden);
  if (st) return st;
  if ((n_heads * d) % 32 || n_ff % 32 || n_kv == 0 || n_heads % n_kv || d % 2) return ORC_ERR_INVALID_SHAPE;
  size_t qd = n_heads * d, kvd = n_kv * d, G = n_heads / n_kv, h2 = d / 2;
  size_t big = hidden > n_ff ? hidden : n_ff;
  float* xn = (float*)malloc(big * sizeof(float));
  float* qkv = (float*)malloc((qd + 2 * kvd) * sizeof(float));
  float* att = (float*)calloc(qd, sizeof(float));
  float* g = (float*)malloc(n_ff * sizeof(float));
  float* u = (float*)malloc(n_ff * sizeof(float));
  float* y = (float*)malloc(big * sizeof(float));
  float* sc = (float*)malloc((pos + 1) * sizeof(float));
  float* rq = (float*)malloc(d * sizeof(float));
  if (!xn || !qkv || !att || !g || !u || !y || !sc || !rq) {
    st = ORC_ERR_BUFFER_TOO_SMALL;
    goto done;
  }
  orc_rms_norm_f32(x, attn_norm, eps, 1, hidden, xn);
  if ((st = orc_matvec_f32(type, wq, xn, qkv, qd, hidden))) goto done;
  if ((st = orc_matvec_f32(type, wk, xn, qkv + qd, kvd, hidden))) goto done;
  if ((st = orc_matvec_f32(type, wv, xn, qkv + qd + kvd, kvd, hidden))) goto done;
  /* RoPE in f32 */
  for (size_t h = 0; h < n_heads + n_kv; h++) {
    float* v = qkv + h * d;
    for (size_t i = 0; i < h2; i++) {
      float ang = (float)pos * inv_freq[i];
      float c = cosf(ang), s = sinf(ang);
      float x1 = v[i], x2 = v[i + h2];
      float a1 = x1 * c, a2 = x2 * s, b1 = x1 * s, b2 = x2 * c;
      v[i] = a1 - a2;
      v[i + h2] = b1 + b2;
    }
  }
  if (store_new) {
    for (size_t i = 0; i < kvd; i++) {
      k_cache[pos * kvd + i] = orc_f32_to_f16(qkv[qd + i]);
      v_cache[pos * kvd + i] = orc_f32_to_f16(qkv[qd + kvd + i]);
    }
  }
  {
    float scale = 1.0f / sqrtf((float)d);
    for (size_t h = 0; h < n_heads; h++) {
      size_t kh = h / G;
      for (size_t p = 0; p <= pos; p++) {
        float s = 0.0f;
        for (size_t i = 0; i < d; i++) {
          float pr = qkv[h * d + i] * orc_f16_to_f32(k_cache[(p * n_kv + kh) * d + i]);
          s = s + pr;
        }
        sc[p] = s * scale;
      }
      float mx = -INFINITY;
      for (size_t p = 0; p <= pos; p++) mx = sc[p] > mx ? sc[p] : mx;
      float sum = 0.0f;
      for (size_t p = 0; p <= pos; p++) {
        sc[p] = expf(sc[p] - mx);
        sum = sum + sc[p];
      }
      float inv = 1.0f / sum;
      for (size_t p = 0; p <= pos; p++) {
        float w = sc[p] * inv;
        for (size_t i = 0; i < d; i++) {
          float pr = w * orc_f16_to_f32(v_cache[(p * n_kv + kh) * d + i]);
          att[h * d + i] = att[h * d + i] + pr;
        }
      }
    }
  }
  (void)rq;
  if ((st = orc_matvec_f32(type, wo, att, y, hidden, qd))) goto done;
  for (size_t i = 0; i < hidden; i++) x[i] = x[i] + y[i];
  orc_rms_norm_f32(x, ffn_norm, eps, 1, hidden, xn);
  if ((st = orc_matvec_f32(type, wg, xn, g, n_ff, hidden))) goto done;
  if ((st = orc_matvec_f32(type, wu, xn, u, n_ff, hidden))) goto done;
  orc_swiglu_f32(g, u, n_ff, g);
  if ((st = orc_matvec_f32(type, wd, g, y, hidden, n_ff))) goto done;
  for (size_t i = 0; i < hidden; i++) x[i] = x[i] + y[i];
done:
  free(xn);
  free(qkv);
  free(att);
  free(g);
  free(u);
  free(y);
  free(sc);
  free(rq);
  return st;
}
