// wh_blocks.hpp -- GGUF block formats on the device (BlockQ4_0 / BlockQ4_1 /
// BlockQ5_0 / BlockQ5_1 / BlockQ8_0, crates/woolly-tensor/src/quantization.rs:98-151).
#pragma once

#include "wh_common.hpp"

namespace whd {

template <int TYPE>
struct BlockFmt;
template <>
struct BlockFmt<WH_TYPE_Q4_0> {
  static constexpr int BYTES = 18;
};
template <>
struct BlockFmt<WH_TYPE_Q4_1> {
  static constexpr int BYTES = 20;
};
template <>
struct BlockFmt<WH_TYPE_Q5_0> {
  static constexpr int BYTES = 22;
};
template <>
struct BlockFmt<WH_TYPE_Q5_1> {
  static constexpr int BYTES = 24;
};
template <>
struct BlockFmt<WH_TYPE_Q8_0> {
  static constexpr int BYTES = 34;
};

// Decodes one block at any byte alignment into v[0..32) (byte loads; used by
// the generic kernels only).  Same arithmetic as the dequantization kernels.
template <int TYPE>
__device__ __forceinline__ void decode_block_bytes(const uint8_t* b, float v[32]) {
  if constexpr (TYPE == WH_TYPE_Q4_0) {
    const float d = f16_bits_to_f32(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t q = b[2 + j];
      v[j] = static_cast<float>(static_cast<int>(q & 15u) - 8) * d;
      v[j + 16] = static_cast<float>(static_cast<int>(q >> 4) - 8) * d;
    }
  } else if constexpr (TYPE == WH_TYPE_Q4_1) {
    const float d = f16_bits_to_f32(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
    const float m = f16_bits_to_f32(static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8));
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t q = b[4 + j];
      v[j] = __fadd_rn(__fmul_rn(static_cast<float>(q & 15u), d), m);
      v[j + 16] = __fadd_rn(__fmul_rn(static_cast<float>(q >> 4), d), m);
    }
  } else {
    const float d = f16_bits_to_f32(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = static_cast<float>(static_cast<int8_t>(b[2 + j])) * d;
  }
}

// ---- per-quad decoders (4 consecutive elements of a block), bit-exact with
// dequantize_q4_0 / _q4_1 / _q5_0 / _q5_1 / _q8_0 (quantization.rs:466-590) and
// dequantize_q4_k_scalar / dequantize_q6_k (dequantize.rs:404-536).

// Little-endian 16- / 32-bit loads at a pointer with ALIGN-byte alignment.
template <int ALIGN>
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) {
  if constexpr (ALIGN >= 2) {
    return *reinterpret_cast<const uint16_t*>(p);
  } else {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
  }
}

template <int ALIGN>
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) {
  if constexpr (ALIGN >= 4) {
    return *reinterpret_cast<const uint32_t*>(p);
  } else {
    return ld16<ALIGN>(p) | (ld16<ALIGN>(p + 2) << 16);
  }
}

// Decodes quad c (0..7) of block `blk` into v[0..4).
template <int TYPE, int ALIGN>
__device__ __forceinline__ void decode_quad(const uint8_t* blk, int c, float v[4]) {
  if constexpr (TYPE == WH_TYPE_Q4_0) {
    const float d = f16_bits_to_f32(ld16<ALIGN>(blk));
    const uint32_t w = ld32<(ALIGN >= 2 ? 2 : 1)>(blk + 2 + 4 * (c & 3));
    const uint32_t nib = (c >= 4) ? ((w >> 4) & 0x0F0F0F0Fu) : (w & 0x0F0F0F0Fu);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = static_cast<int>((nib >> (8 * i)) & 0xFFu) - 8;
      v[i] = static_cast<float>(q) * d;
    }
  } else if constexpr (TYPE == WH_TYPE_Q4_1) {
    const uint32_t dm = ld32<ALIGN>(blk);
    const float d = f16_bits_to_f32(dm & 0xFFFFu);
    const float m = f16_bits_to_f32(dm >> 16);
    const uint32_t w = ld32<ALIGN>(blk + 4 + 4 * (c & 3));
    const uint32_t nib = (c >= 4) ? ((w >> 4) & 0x0F0F0F0Fu) : (w & 0x0F0F0F0Fu);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float q = static_cast<float>((nib >> (8 * i)) & 0xFFu);
      v[i] = __fadd_rn(__fmul_rn(q, d), m);
    }
  } else if constexpr (TYPE == WH_TYPE_Q5_0 || TYPE == WH_TYPE_Q5_1) {
    // quantization.rs:515-575: element e (< 16: low nibble of qs[e], >= 16: high
    // nibble of qs[e - 16]) takes bit e of the little-endian qh as its 5th bit
    // (((qh >> j) << 4) & 0x10 and (qh >> (j + 12)) & 0x10 are both bit e);
    // Q5_0: (x - 16) * d, Q5_1: x * d + m
    constexpr int QH = TYPE == WH_TYPE_Q5_0 ? 2 : 4;
    const float d = f16_bits_to_f32(ld16<ALIGN>(blk));
    const uint32_t qh = ld32<(ALIGN >= 2 ? 2 : 1)>(blk + QH) >> (4 * c);
    const uint32_t w = ld32<(ALIGN >= 2 ? 2 : 1)>(blk + QH + 4 + 4 * (c & 3));
    const uint32_t nib = (c >= 4) ? ((w >> 4) & 0x0F0F0F0Fu) : (w & 0x0F0F0F0Fu);
    if constexpr (TYPE == WH_TYPE_Q5_0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int q = static_cast<int>(((nib >> (8 * i)) & 0xFFu) | (((qh >> i) & 1u) << 4)) - 16;
        v[i] = static_cast<float>(q) * d;
      }
    } else {
      const float m = f16_bits_to_f32(ld16<ALIGN>(blk + 2));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float q = static_cast<float>(((nib >> (8 * i)) & 0xFFu) | (((qh >> i) & 1u) << 4));
        v[i] = __fadd_rn(__fmul_rn(q, d), m);
      }
    }
  } else {  // Q8_0
    const float d = f16_bits_to_f32(ld16<ALIGN>(blk));
    const uint32_t w = ld32<(ALIGN >= 2 ? 2 : 1)>(blk + 2 + 4 * c);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = static_cast<int>(static_cast<int8_t>((w >> (8 * i)) & 0xFFu));
      v[i] = static_cast<float>(q) * d;
    }
  }
}

// ---- K-quant elements (woolly_gguf's layout)
__device__ __forceinline__ uint32_t b16(const uint8_t* p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

// 6-bit scale j (0..7) of a Q4_K block at b.
__device__ __forceinline__ uint32_t q4k_scale(const uint8_t* b, int j) {
  const int src = (3 * j) >> 1;
  return (j & 1) ? (((b[src] >> 6) | ((b[src + 1] & 15u) << 2)) & 63u) : (b[src] & 63u);
}

// Element i (0..255) of a Q4_K block at b.
__device__ __forceinline__ float q4k_elem(const uint8_t* b, int i, float d, float dmin) {
  const uint32_t s = q4k_scale(b, i >> 5);
  const uint32_t qb = b[16 + (i >> 1)];
  const uint32_t q = (i & 1) ? ((qb >> 4) & 15u) : (qb & 15u);
  return __fadd_rn(__fmul_rn(__fmul_rn(d, static_cast<float>(s)), static_cast<float>(q)), dmin);
}

// The 6-bit quant q (0..63) of element i (0..255) of a Q6_K block at b.
__device__ __forceinline__ uint32_t q6k_quant(const uint8_t* b, int i) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const int ql_idx = 64 * (i >> 7) + 32 * ((i & 127) >> 6) + 16 * ((i & 63) >> 5) + (i & 15);
  const int qh_idx = 32 * (i >> 7) + 16 * ((i & 127) >> 6) + 8 * ((i & 63) >> 5) + ((i & 31) >> 2);
  const int shift = 2 * (i & 3);
  const uint32_t qhv = qh[qh_idx];
  if (i < 128) return (ql[ql_idx] & 15u) | (((qhv >> shift) & 3u) << 4);
  const uint32_t e2 = shift < 6 ? ((qhv >> (shift + 2)) & 3u) : (qh_idx + 1 < 64 ? (qh[qh_idx + 1] & 3u) : 0u);
  return (ql[ql_idx] >> 4) | (e2 << 4);
}

// Element i (0..255) of a Q6_K block at b.
__device__ __forceinline__ float q6k_elem(const uint8_t* b, int i, float d) {
  const uint32_t q = q6k_quant(b, i);
  const float s = static_cast<float>(b[192 + (i >> 4)]);
  return __fmul_rn(__fmul_rn(__fmul_rn(d, s), static_cast<float>(static_cast<int>(q) - 32)), 0.015625f);
}

template <int TYPE>
__device__ __forceinline__ void kq_quad(const uint8_t* b, int c, float v[4]) {
  if constexpr (TYPE == WH_TYPE_Q4_K) {
    const float d = f16_bits_to_f32(b16(b + 12));
    const float dmin = f16_bits_to_f32(b16(b + 14));
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = q4k_elem(b, 4 * c + t, d, dmin);
  } else {
    const float d = f16_bits_to_f32(b16(b + 208));
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = q6k_elem(b, 4 * c + t, d);
  }
}

}  // namespace whd
