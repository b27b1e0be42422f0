// Unit tests of the C++ mirror (include/woolly_hip.hpp), written after the
// reference's own Rust unit tests so the two read side by side:
//   crates/woolly-tensor/src/quantization.rs:1293-1407
//   crates/woolly-gguf/src/dequantize.rs:613-633
//   crates/woolly-gguf/tests/load_model.rs:214-300 (GGUF loader, on a file
//     written here with the same layout as its MockGGUFBuilder)
// plus closed-form checks of simd::quantized_matvec and of the error mapping.
// Every computation runs on the GPU through libwoolly_hip.  Exit status 0 iff
// all tests pass; one line per test.
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
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

// GGUF bytes in the layout of load_model.rs:15-145 (version 3, padding to 32).
struct GgufWriter {
  std::vector<uint8_t> b;
  void u32(uint32_t v) { b.insert(b.end(), reinterpret_cast<uint8_t*>(&v), reinterpret_cast<uint8_t*>(&v) + 4); }
  void u64(uint64_t v) { b.insert(b.end(), reinterpret_cast<uint8_t*>(&v), reinterpret_cast<uint8_t*>(&v) + 8); }
  void str(const std::string& s) {
    u64(s.size());
    b.insert(b.end(), s.begin(), s.end());
  }
};

std::string write_temp(const std::vector<uint8_t>& bytes) {
  char path[] = "/tmp/woolly_mirror_XXXXXX";
  const int fd = mkstemp(path);
  if (fd < 0) throw std::runtime_error("mkstemp failed");
  const ssize_t n = write(fd, bytes.data(), bytes.size());
  close(fd);
  if (n != static_cast<ssize_t>(bytes.size())) throw std::runtime_error("short write");
  return path;
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

  // quantization.rs:1409-1427
  run("test_q5_0_dequantization", [] {
    BlockQ5_0 b;
    b.d = f16::from_f32(0.5f);
    std::memset(b.qh, 0xFF, sizeof b.qh);
    std::memset(b.qs, 0xFF, sizeof b.qs);
    const auto result = dequantize_q5_0({b});
    EXPECT(result.size() == 32);
    for (float v : result) EXPECT(std::fabs(v - 7.5f) < 1e-6f);
  });

  // quantization.rs:1429-1446
  run("test_q5_1_dequantization", [] {
    BlockQ5_1 b;
    b.d = f16::from_f32(1.0f);
    b.m = f16::from_f32(10.0f);
    std::memset(b.qh, 0x00, sizeof b.qh);
    std::memset(b.qs, 0x11, sizeof b.qs);
    const auto result = optimized::dequantize_blocks(QuantizedStorage::Q5_1({b}));
    EXPECT(result.size() == 32);
    for (float v : result) EXPECT(std::fabs(v - 11.0f) < 1e-6f);
  });

  // quantization.rs:1346-1356
  run("test_block_sizes", [] {
    EXPECT(sizeof(BlockQ4_0) == 18);
    EXPECT(sizeof(BlockQ4_1) == 20);
    EXPECT(sizeof(BlockQ5_0) == 22);
    EXPECT(sizeof(BlockQ5_1) == 24);
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
    bool too_small = false, invalid = false, short_k = false;
    try {
      gguf::dequantize(bytes, gguf::GGMLType::Q4_0, 64);
    } catch (const gguf::BufferTooSmall& e) {
      too_small = e.needed == 36 && e.available == 35;
    }
    try {
      gguf::dequantize(bytes, gguf::GGMLType::Q2_K, 256);
    } catch (const gguf::InvalidTensorType& e) {
      invalid = e.type_id == 10;
    }
    try {
      gguf::dequantize(bytes, gguf::GGMLType::Q4_K, 256);  // 35 of 144 bytes
    } catch (const gguf::InvalidTensorInfo&) {
      short_k = true;
    }
    EXPECT(too_small && invalid && short_k);
    // A partial trailing block decodes the elements asked for.
    std::vector<uint8_t> one(18, 0x00);
    one[0] = 0x00, one[1] = 0x3C;  // d = 1.0
    const auto r = gguf::dequantize(one, gguf::GGMLType::Q4_0, 20);
    EXPECT(r.size() == 20);
    for (float v : r) EXPECT(v == -8.0f);
  });

  // load_model.rs:214-300 (tensors, mapped access, quantized tensors) and the
  // upload of a mapped Q4_0 tensor, whose GEMV must equal the host-pointer one.
  run("gguf_loader_tensors_and_upload", [] {
    const int rows = 4, k = 64;
    std::vector<BlockQ4_0> w;
    for (int r = 0; r < rows; r++)
      for (int b = 0; b < k / 32; b++) w.push_back(q4_0(0.25f * (r + 1), static_cast<uint8_t>(0x1F + 16 * b + r)));
    GgufWriter g;
    g.b = {'G', 'G', 'U', 'F'};
    g.u32(3);
    g.u64(2);  // tensors
    g.u64(2);  // metadata
    g.str("general.architecture");
    g.u32(8);
    g.str("llama");
    g.str("llama.block_count");
    g.u32(4);
    g.u32(32);
    g.str("blk.0.ffn_gate.weight");
    g.u32(2);
    g.u64(k);
    g.u64(rows);
    g.u32(2);
    g.u64(0);
    g.str("output_norm.weight");
    g.u32(1);
    g.u64(16);
    g.u32(0);
    g.u64(w.size() * sizeof(BlockQ4_0));
    while (g.b.size() % 32) g.b.push_back(0);
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(w.data());
    g.b.insert(g.b.end(), wb, wb + w.size() * sizeof(BlockQ4_0));
    for (int i = 0; i < 16; i++) {
      const float v = 0.5f * i;
      const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
      g.b.insert(g.b.end(), p, p + 4);
    }
    const std::string path = write_temp(g.b);
    auto ld = gguf::GGUFLoader::from_path(path);
    unlink(path.c_str());
    EXPECT(ld.version() == 3 && ld.tensor_count() == 2 && ld.metadata_kv_count() == 2);
    EXPECT(ld.architecture() == "llama");
    uint32_t nl = 0;
    EXPECT(ld.get_u32("llama.block_count", &nl) && nl == 32);
    uint64_t nl64 = 0;
    EXPECT(!ld.get_u64("llama.block_count", &nl64));  // other type -> none
    gguf::TensorInfo ti;
    EXPECT(ld.tensor_info("blk.0.ffn_gate.weight", &ti));
    EXPECT(ti.shape().size() == 2 && ti.dims[0] == 64 && ti.dims[1] == 4 && ti.ggml_type == 2);
    EXPECT(ti.n_elements == 256 && ti.data_size == 8 * 18);
    EXPECT(!ld.tensor_info("missing", &ti));
    bool not_found = false;
    try {
      ld.tensor_data("missing");
    } catch (const gguf::TensorNotFound&) {
      not_found = true;
    }
    EXPECT(not_found);
    const auto norm = ld.tensor_data("output_norm.weight");
    EXPECT(norm.second == 64);
    float f7;
    std::memcpy(&f7, norm.first + 28, 4);
    EXPECT(f7 == 3.5f);
    EXPECT(ld.total_tensor_size() == 8 * 18 + 64 && ld.file_size() == g.b.size());
    // device upload from the mapping; GEMV vs the host-pointer path
    wh_weight* dw = ld.upload("blk.0.ffn_gate.weight");
    std::vector<float> x(k);
    for (int i = 0; i < k; i++) x[i] = std::sin(0.3f * i);
    float *dx, *dy;
    EXPECT(wh_malloc(reinterpret_cast<void**>(&dx), 4 * k) == WH_OK);
    EXPECT(wh_malloc(reinterpret_cast<void**>(&dy), 4 * rows) == WH_OK);
    EXPECT(wh_memcpy_h2d(dx, x.data(), 4 * k, nullptr) == WH_OK);
    EXPECT(wh_quantized_matvec(2, wh_weight_data(dw), 8 * 18, dx, dy, rows, k, nullptr) == WH_OK);
    std::vector<float> y(rows), yh(rows);
    EXPECT(wh_memcpy_d2h(y.data(), dy, 4 * rows, nullptr) == WH_OK);
    EXPECT(wh_stream_synchronize(nullptr) == WH_OK);
    simd::quantized_matvec(QuantizedStorage::Q4_0(w), x, yh, rows, k);
    for (int r = 0; r < rows; r++) EXPECT(y[r] == yh[r]);
    wh_free(dx);
    wh_free(dy);
    wh_weight_free(dw);
    // load_model.rs:300-330 error cases
    bool io = false, magic = false;
    try {
      gguf::GGUFLoader::from_path("/non/existent/file.gguf");
    } catch (const gguf::Io&) {
      io = true;
    }
    const std::string bad = write_temp(std::vector<uint8_t>{'B', 'A', 'D', '!', 0, 0, 0, 0, 0, 0, 0, 0,
                                                            0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0});
    try {
      gguf::GGUFLoader::from_path(bad);
    } catch (const gguf::InvalidMagic&) {
      magic = true;
    }
    unlink(bad.c_str());
    EXPECT(io && magic);
  });

  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "PASSED", g_failed);
  return g_failed ? 1 : 0;
}
