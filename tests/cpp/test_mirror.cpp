// Unit tests of the C++ mirror (include/woolly_hip.hpp), written after the
// reference's own Rust unit tests so the two read side by side:
//   crates/woolly-tensor/src/quantization.rs:1293-1407
//   crates/woolly-gguf/src/dequantize.rs:613-633
// plus closed-form checks of simd::quantized_matvec and of the error mapping.
// Every computation runs on the GPU through libwoolly_hip.  Exit status 0 iff
// all tests pass; one line per test.
#include <cmath>
#include <cstdio>
#include <functional>
#include <vector>

#include "woolly_hip.hpp"

using namespace woolly;
using namespace woolly::tensor::quantization;

namespace {

int g_failed = 0;

#define EXPECT(cond)                                                          \
  do {                                                                        \
    if (!(cond)) {                                                            \
      std::fprintf(stderr, "  %s:%d: expectation failed: %s\n", __FILE__,     \
                   __LINE__, #cond);                                          \
      throw std::runtime_error("expectation failed");                         \
    }                                                                         \
  } while (0)

void run(const char* name, const std::function<void()>& fn) {
  try {
    fn();
    std::printf("ok   %s\n", name);
  } catch (const std::exception& e) {
    ++g_failed;
    std::printf("FAIL %s: %s\n", name, e.what());
  }
  std::fflush(stdout);
}

BlockQ4_0 q4_0(float d, uint8_t fill) {
  BlockQ4_0 b;
  b.d = f16::from_f32(d);
  std::memset(b.qs, fill, sizeof b.qs);
  return b;
}

}  // namespace

int main() {
  if (wh_init(0) != WH_OK) {
    std::printf("FAIL init: %s\n", wh_last_error());
    return 2;
  }

  run("f16_from_f32_bits", [] {
    EXPECT(f16::from_f32(2.0f).bits == 0x4000);
    EXPECT(f16::from_f32(1.0f).bits == 0x3C00);
    EXPECT(f16::from_f32(5.0f).bits == 0x4500);
    EXPECT(f16::from_f32(0.5f).bits == 0x3800);
    EXPECT(f16::from_f32(-16.0f).bits == 0xCC00);
    EXPECT(f16::from_f32(65520.0f).bits == 0x7C00);     // rounds to +inf
    EXPECT(f16::from_f32(1.0f + 1.0f / 2048).bits == 0x3C00);  // tie to even
    EXPECT(f16::from_f32(5.9604645e-8f).bits == 0x0001);  // smallest subnormal
  });

  // quantization.rs:1293-1307
  run("test_q4_0_dequantization", [] {
    const auto result = dequantize_q4_0({q4_0(2.0f, 0x00)});
    EXPECT(result.size() == 32);
    for (float v : result) EXPECT(std::fabs(v - (-16.0f)) < 1e-6f);
  });

  // quantization.rs:1309-1326
  run("test_q4_1_dequantization", [] {
    BlockQ4_1 b;
    b.d = f16::from_f32(1.0f);
    b.m = f16::from_f32(5.0f);
    std::memset(b.qs, 0x01, sizeof b.qs);
    const auto result = dequantize_q4_1({b});
    EXPECT(result.size() == 32);
    for (int i = 0; i < 16; ++i) {
      EXPECT(std::fabs(result[i] - 6.0f) < 1e-6f);
      EXPECT(std::fabs(result[i + 16] - 5.0f) < 1e-6f);
    }
  });

  // quantization.rs:1328-1344
  run("test_q8_0_dequantization", [] {
    BlockQ8_0 b;
    b.d = f16::from_f32(0.5f);
    std::memset(b.qs, 0, sizeof b.qs);
    b.qs[0] = 10;
    b.qs[1] = -5;
    const auto result = dequantize_q8_0({b});
    EXPECT(result.size() == 32);
    EXPECT(std::fabs(result[0] - 5.0f) < 1e-6f);
    EXPECT(std::fabs(result[1] - (-2.5f)) < 1e-6f);
    for (int i = 2; i < 32; ++i) EXPECT(result[i] == 0.0f);
  });

  // quantization.rs:1346-1356 (the block formats on this path)
  run("test_block_sizes", [] {
    EXPECT(sizeof(BlockQ4_0) == 18);
    EXPECT(sizeof(BlockQ4_1) == 20);
    EXPECT(sizeof(BlockQ8_0) == 34);
  });

  // quantization.rs:1358-1386
  run("test_optimized_dispatcher", [] {
    const auto storage = QuantizedStorage::Q4_0({q4_0(1.0f, 0x11), q4_0(2.0f, 0x22)});
    const auto result = optimized::dequantize_blocks(storage);
    EXPECT(result.size() == 64);
    for (int i = 0; i < 32; ++i) EXPECT(std::fabs(result[i] - (-7.0f)) < 1e-6f);
    for (int i = 32; i < 64; ++i) EXPECT(std::fabs(result[i] - (-12.0f)) < 1e-6f);
  });

  // quantization.rs:1388-1407
  run("test_simd_batch_processing", [] {
    std::vector<BlockQ4_0> blocks;
    for (int i = 0; i < 8; ++i) blocks.push_back(q4_0(float(i) + 1.0f, 0x00));
    const auto result_simd = simd::dequantize_q4_0_batch(blocks);
    const auto result_regular = dequantize_q4_0(blocks);
    EXPECT(result_simd.size() == result_regular.size());
    for (size_t i = 0; i < result_simd.size(); ++i)
      EXPECT(std::fabs(result_simd[i] - result_regular[i]) < 1e-6f);
    for (size_t i = 0; i < result_regular.size(); ++i)
      EXPECT(result_regular[i] == -8.0f * float(i / 32 + 1));
  });

  // Closed form: a Q4_0 row whose nibbles are all q has every weight d*(q-8),
  // so output[r] = d_r * (q_r - 8) * sum(x); with small integer x the sum is exact.
  run("quantized_matvec_closed_form", [] {
    const size_t m = 5, k = 96;
    std::vector<BlockQ4_0> blocks;
    for (size_t r = 0; r < m; ++r)
      for (size_t b = 0; b < k / 32; ++b) blocks.push_back(q4_0(float(r + 1), uint8_t(0x11 * (3 * r + 1))));
    std::vector<float> x(k), y(m, -1.0f);
    float sx = 0;
    for (size_t i = 0; i < k; ++i) sx += (x[i] = float(int(i % 7) - 3));
    simd::quantized_matvec(QuantizedStorage::Q4_0(blocks), x, y, m, k);
    for (size_t r = 0; r < m; ++r) EXPECT(y[r] == float(r + 1) * (float(3 * r + 1) - 8.0f) * sx);
  });

  // Q8_0 and Q4_1 closed forms, and the k % 32 rule (quantization.rs:1107).
  run("quantized_matvec_q8_0_q4_1_and_shape", [] {
    const size_t m = 2, k = 64;
    std::vector<BlockQ8_0> q8(m * k / 32);
    for (size_t b = 0; b < q8.size(); ++b) {
      q8[b].d = f16::from_f32(0.25f);
      for (int j = 0; j < 32; ++j) q8[b].qs[j] = int8_t(j - 16);
    }
    std::vector<BlockQ4_1> q41(m * k / 32);
    for (auto& b : q41) {
      b.d = f16::from_f32(2.0f);
      b.m = f16::from_f32(-1.0f);
      std::memset(b.qs, 0x53, sizeof b.qs);  // low nibble 3, high nibble 5
    }
    std::vector<float> x(k, 1.0f), y(m);
    simd::quantized_matvec(QuantizedStorage::Q8_0(q8), x, y, m, k);
    // per block: 0.25 * sum(j - 16, j < 32) = 0.25 * -16 = -4
    for (size_t r = 0; r < m; ++r) EXPECT(y[r] == -8.0f);
    simd::quantized_matvec(QuantizedStorage::Q4_1(q41), x, y, m, k);
    // per block: 16 * (2*3 - 1) + 16 * (2*5 - 1) = 80 + 144 = 224
    for (size_t r = 0; r < m; ++r) EXPECT(y[r] == 448.0f);
    bool threw = false;
    try {
      std::vector<float> x2(48);
      simd::quantized_matvec(QuantizedStorage::Q8_0(q8), x2, y, 1, 48);
    } catch (const QuantizationError& e) {
      threw = e.kind == QuantizationError::Kind::InvalidParameters;
    }
    EXPECT(threw);
  });

  // dequantize.rs:613-624
  run("test_f32_dequantization", [] {
    const float data[4] = {0.0f, 1.0f, -1.0f, 3.14f};
    std::vector<uint8_t> bytes(sizeof data);
    std::memcpy(bytes.data(), data, sizeof data);
    const auto result = gguf::dequantize(bytes, gguf::GGMLType::F32, 4);
    EXPECT(result.size() == 4);
    EXPECT(result[0] == 0.0f && result[1] == 1.0f && result[2] == -1.0f);
    EXPECT(std::fabs(result[3] - 3.14f) < 0.001f);
  });

  // dequantize.rs:626-632
  run("test_gguf_block_sizes", [] {
    EXPECT(gguf::get_block_size(gguf::GGMLType::F32) == 1);
    EXPECT(gguf::get_block_size(gguf::GGMLType::Q4_0) == 32);
    EXPECT(gguf::get_block_size(gguf::GGMLType::Q4_K) == 256);
    EXPECT(gguf::get_block_size(gguf::GGMLType::Q6_K) == 256);
    EXPECT(gguf::get_type_size(gguf::GGMLType::Q4_0) == 18);
    EXPECT(gguf::get_type_size(gguf::GGMLType::Q8_0) == 34);
  });

  // error.rs:11-64 through dequantize.rs:189-205
  run("gguf_errors", [] {
    std::vector<uint8_t> bytes(18 * 2 - 1);
    bool too_small = false, invalid = false;
    try {
      gguf::dequantize(bytes, gguf::GGMLType::Q4_0, 64);
    } catch (const gguf::BufferTooSmall& e) {
      too_small = e.needed == 36 && e.available == 35;
    }
    try {
      gguf::dequantize(bytes, gguf::GGMLType::Q4_K, 256);
    } catch (const gguf::InvalidTensorType& e) {
      invalid = e.type_id == 12;
    }
    EXPECT(too_small && invalid);
    // A partial trailing block decodes the elements asked for.
    std::vector<uint8_t> one(18, 0x00);
    one[0] = 0x00, one[1] = 0x3C;  // d = 1.0
    const auto r = gguf::dequantize(one, gguf::GGMLType::Q4_0, 20);
    EXPECT(r.size() == 20);
    for (float v : r) EXPECT(v == -8.0f);
  });

  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "PASSED", g_failed);
  return g_failed ? 1 : 0;
}
