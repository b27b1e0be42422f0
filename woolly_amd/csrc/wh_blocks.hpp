// wh_blocks.hpp -- GGUF block formats on the device (BlockQ4_0 / BlockQ4_1 /
// BlockQ8_0, crates/woolly-tensor/src/quantization.rs:98-151).
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

}  // namespace whd
