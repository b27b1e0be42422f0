// woolly_hip.hpp -- C++17 host-side mirror of woolly's quantization API, over
// the C ABI of libwoolly_hip (woolly_hip.h).  Header-only.
//
// Names, argument meaning and errors follow the Rust reference so code (and
// tests) written against it read the same:
//   woolly::tensor::quantization   crates/woolly-tensor/src/quantization.rs
//     BlockQ4_0 / BlockQ4_1 / BlockQ5_0 / BlockQ5_1 / BlockQ8_0   :98-151
//     QuantizationError{UnsupportedScheme, InvalidParameters}   :8-26
//     QuantizedStorage (Q4_0 / Q4_1 / Q8_0)           :154-170
//     dequantize_q4_0 / dequantize_q4_1 / dequantize_q8_0       :466, 490, 576
//     simd::quantized_matvec(weights, input, output, m, k)      :869-909
//     optimized::dequantize_blocks(storage)           :1171-1210
//   woolly::gguf                   crates/woolly-gguf/src
//     GGMLType ids                                     tensor_info.rs:15-30
//     dequantize(data, ggml_type, nelements)           dequantize.rs:189-205
//     Error::{BufferTooSmall{needed, available}, InvalidTensorType}  error.rs:11-64
//     GGUFLoader (from_path, tensor_info, tensor_names, tensor_data, metadata
//       getters, alignment, file_size, total_tensor_size)   loader.rs:111-490
// Every call runs the HIP kernels (synchronous host-memory entry points);
// there is no CPU implementation in this header.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <utility>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

#include "woolly_hip.h"

namespace woolly {

// f16 bit pattern helper (half::f16 is a 16-bit IEEE binary16 value).
struct f16 {
  uint16_t bits = 0;
  static f16 from_bits(uint16_t b) { return f16{b}; }
  // Round-to-nearest-even conversion (half::f16::from_f32).
  static f16 from_f32(float v) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (exp == 0xFFu) return f16{static_cast<uint16_t>(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u))};
    const int e = static_cast<int>(exp) - 112;
    if (e >= 31) return f16{static_cast<uint16_t>(sign | 0x7C00u)};
    if (e <= 0) {
      if (e < -10) return f16{static_cast<uint16_t>(sign)};
      const uint32_t m = man | 0x800000u;
      const int shift = 14 - e;
      uint32_t h = m >> shift;
      const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
      if (rem > half || (rem == half && (h & 1u))) h++;
      return f16{static_cast<uint16_t>(sign | h)};
    }
    uint32_t h = sign | (static_cast<uint32_t>(e) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return f16{static_cast<uint16_t>(h)};
  }
};

namespace tensor {
namespace quantization {

#pragma pack(push, 1)
struct BlockQ4_0 {
  f16 d;
  uint8_t qs[16];
};
struct BlockQ4_1 {
  f16 d;
  f16 m;
  uint8_t qs[16];
};
struct BlockQ5_0 {
  f16 d;
  uint8_t qh[4];
  uint8_t qs[16];
};
struct BlockQ5_1 {
  f16 d;
  f16 m;
  uint8_t qh[4];
  uint8_t qs[16];
};
struct BlockQ8_0 {
  f16 d;
  int8_t qs[32];
};
#pragma pack(pop)
static_assert(sizeof(BlockQ4_0) == 18 && sizeof(BlockQ4_1) == 20 && sizeof(BlockQ8_0) == 34,
              "GGUF block sizes");
static_assert(sizeof(BlockQ5_0) == 22 && sizeof(BlockQ5_1) == 24, "GGUF block sizes");

// QuantizationError (quantization.rs:8-26); thrown, as Result::Err would be returned.
struct QuantizationError : std::runtime_error {
  enum class Kind { UnsupportedScheme, InvalidParameters, Backend };
  Kind kind;
  QuantizationError(Kind k, const std::string& msg) : std::runtime_error(msg), kind(k) {}
};

inline void check_status(int st) {
  if (st == WH_OK) return;
  const std::string msg = wh_last_error();
  if (st == WH_ERR_UNSUPPORTED_TYPE)
    throw QuantizationError(QuantizationError::Kind::UnsupportedScheme, msg);
  if (st == WH_ERR_INVALID_SHAPE || st == WH_ERR_BUFFER_TOO_SMALL || st == WH_ERR_INVALID_ARGUMENT)
    throw QuantizationError(QuantizationError::Kind::InvalidParameters, msg);
  throw QuantizationError(QuantizationError::Kind::Backend, msg);
}

// QuantizedStorage (quantization.rs:154-170), restricted to the 32-element block formats.
struct QuantizedStorage {
  std::variant<std::vector<BlockQ4_0>, std::vector<BlockQ4_1>, std::vector<BlockQ8_0>, std::vector<BlockQ5_0>,
               std::vector<BlockQ5_1>>
      blocks;
  static QuantizedStorage Q4_0(std::vector<BlockQ4_0> b) { return {std::move(b)}; }
  static QuantizedStorage Q4_1(std::vector<BlockQ4_1> b) { return {std::move(b)}; }
  static QuantizedStorage Q8_0(std::vector<BlockQ8_0> b) { return {std::move(b)}; }
  static QuantizedStorage Q5_0(std::vector<BlockQ5_0> b) { return {std::move(b)}; }
  static QuantizedStorage Q5_1(std::vector<BlockQ5_1> b) { return {std::move(b)}; }
  int ggml_type() const {
    static const int ids[5] = {WH_TYPE_Q4_0, WH_TYPE_Q4_1, WH_TYPE_Q8_0, WH_TYPE_Q5_0, WH_TYPE_Q5_1};
    return ids[blocks.index()];
  }
  const void* data() const {
    return std::visit([](const auto& v) { return static_cast<const void*>(v.data()); }, blocks);
  }
  size_t nbytes() const {
    return std::visit([](const auto& v) { return v.size() * sizeof(v[0]); }, blocks);
  }
  size_t nblocks() const {
    return std::visit([](const auto& v) { return v.size(); }, blocks);
  }
};

namespace detail {
inline std::vector<float> dequantize(int type, const void* data, size_t nbytes, size_t nblocks) {
  std::vector<float> out(nblocks * 32);
  if (!out.empty()) check_status(wh_dequantize_host(type, data, nbytes, out.size(), out.data()));
  return out;
}
}  // namespace detail

inline std::vector<float> dequantize_q4_0(const std::vector<BlockQ4_0>& blocks) {
  return detail::dequantize(WH_TYPE_Q4_0, blocks.data(), blocks.size() * sizeof(BlockQ4_0), blocks.size());
}
inline std::vector<float> dequantize_q4_1(const std::vector<BlockQ4_1>& blocks) {
  return detail::dequantize(WH_TYPE_Q4_1, blocks.data(), blocks.size() * sizeof(BlockQ4_1), blocks.size());
}
inline std::vector<float> dequantize_q8_0(const std::vector<BlockQ8_0>& blocks) {
  return detail::dequantize(WH_TYPE_Q8_0, blocks.data(), blocks.size() * sizeof(BlockQ8_0), blocks.size());
}
// dequantize_q5_0 / dequantize_q5_1 (quantization.rs:515-575)
inline std::vector<float> dequantize_q5_0(const std::vector<BlockQ5_0>& blocks) {
  return detail::dequantize(WH_TYPE_Q5_0, blocks.data(), blocks.size() * sizeof(BlockQ5_0), blocks.size());
}
inline std::vector<float> dequantize_q5_1(const std::vector<BlockQ5_1>& blocks) {
  return detail::dequantize(WH_TYPE_Q5_1, blocks.data(), blocks.size() * sizeof(BlockQ5_1), blocks.size());
}

namespace simd {
// simd::quantized_matvec (quantization.rs:869-909), Q4_0 / Q8_0 like the
// reference and Q4_1 in addition (Q5 storage: UnsupportedScheme, as there).
// output[r] = sum_k W[r, k] * input[k].
inline void quantized_matvec(const QuantizedStorage& weights, const std::vector<float>& input,
                             std::vector<float>& output, size_t m, size_t k) {
  if (input.size() < k || output.size() < m)
    throw QuantizationError(QuantizationError::Kind::InvalidParameters, "input/output shorter than k/m");
  check_status(wh_quantized_matvec_host(weights.ggml_type(), weights.data(), weights.nbytes(),
                                        input.data(), output.data(), m, k));
}
inline std::vector<float> dequantize_q4_0_batch(const std::vector<BlockQ4_0>& b) { return dequantize_q4_0(b); }
inline std::vector<float> dequantize_q4_1_batch(const std::vector<BlockQ4_1>& b) { return dequantize_q4_1(b); }
inline std::vector<float> dequantize_q8_0_batch(const std::vector<BlockQ8_0>& b) { return dequantize_q8_0(b); }
inline std::vector<float> dequantize_q5_0_batch(const std::vector<BlockQ5_0>& b) { return dequantize_q5_0(b); }
inline std::vector<float> dequantize_q5_1_batch(const std::vector<BlockQ5_1>& b) { return dequantize_q5_1(b); }
}  // namespace simd

namespace optimized {
// optimized::dequantize_blocks (quantization.rs:1171-1210).
inline std::vector<float> dequantize_blocks(const QuantizedStorage& storage) {
  return detail::dequantize(storage.ggml_type(), storage.data(), storage.nbytes(), storage.nblocks());
}
}  // namespace optimized

}  // namespace quantization
}  // namespace tensor

namespace gguf {

// Type ids of tensor_info.rs:14-60 (the subset a quantized Llama file carries).
enum class GGMLType : uint32_t {
  F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9,
  Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15
};

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct BufferTooSmall : Error {
  size_t needed, available;
  BufferTooSmall(size_t n, size_t a)
      : Error("Buffer too small: needed " + std::to_string(n) + ", available " + std::to_string(a)),
        needed(n), available(a) {}
};
struct InvalidTensorType : Error {
  uint32_t type_id;
  explicit InvalidTensorType(uint32_t t) : Error("Invalid tensor type: " + std::to_string(t)), type_id(t) {}
};
struct InvalidTensorInfo : Error {
  using Error::Error;
};

// woolly_gguf::dequantize(data, ggml_type, nelements) (dequantize.rs:189-205).
// Q5_0 / Q5_1 decode as dequantize_q5_0 / _q5_1 (quantization.rs:515-575); the
// reference's gguf-level Q5 functions (dequantize.rs:538-550) return zeros.
inline std::vector<float> dequantize(const std::vector<uint8_t>& data, GGMLType type, size_t nelements) {
  std::vector<float> out(nelements);
  const int st = wh_dequantize_host(static_cast<int>(type), data.data(), data.size(), nelements,
                                    nelements ? out.data() : nullptr);
  if (st == WH_ERR_BUFFER_TOO_SMALL) {
    const size_t ts = wh_type_size(static_cast<int>(type));
    const size_t bs = wh_block_size(static_cast<int>(type));
    const size_t needed = bs > 1 ? (nelements + bs - 1) / bs * ts : nelements * ts;
    throw BufferTooSmall(needed, data.size());
  }
  if (st == WH_ERR_UNSUPPORTED_TYPE) throw InvalidTensorType(static_cast<uint32_t>(type));
  // short K-quant data (dequantize.rs:416-418, 472-474)
  if (st == WH_ERR_INVALID_METADATA) throw InvalidTensorInfo(wh_last_error());
  if (st != WH_OK) throw Error(wh_last_error());
  return out;
}

// Elements per block (tensor_info.rs:127-140): 32 for the legacy block
// formats, 256 for the K-quants (super-blocks), 1 for plain types.  The formats
// the library computes on are answered by the library itself.
inline size_t get_block_size(GGMLType t) {
  const size_t bs = wh_block_size(static_cast<int>(t));
  if (bs) return bs;
  const uint32_t id = static_cast<uint32_t>(t);
  if (id >= 10 && id <= 15) return 256;
  if (id >= 6 && id <= 9) return 32;
  return 1;
}
// Bytes per block for the formats the library computes on; 0 otherwise.
inline size_t get_type_size(GGMLType t) { return wh_type_size(static_cast<int>(t)); }

struct Io : Error {
  using Error::Error;
};
struct InvalidMagic : Error {
  using Error::Error;
};
struct UnsupportedVersion : Error {
  uint32_t version;
  UnsupportedVersion(uint32_t v, const std::string& m) : Error(m), version(v) {}
};
struct InvalidMetadata : Error {
  using Error::Error;
};
struct TensorNotFound : Error {
  using Error::Error;
};

// TensorInfo (tensor_info.rs:187-258).
struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t ggml_type = 0;
  uint64_t offset = 0, n_elements = 0, data_size = 0;
  const std::vector<uint64_t>& shape() const { return dims; }
};

// GGUFLoader (loader.rs:111-490) over the library's native parser: the file
// stays memory-mapped, tensor_data() is a zero-copy view, upload() moves a
// tensor to the GPU straight from the mapping.
class GGUFLoader {
 public:
  static GGUFLoader from_path(const std::string& path) {
    wh_gguf* g = nullptr;
    check(wh_gguf_open(path.c_str(), &g), path);
    return GGUFLoader(g);
  }
  GGUFLoader(GGUFLoader&& o) noexcept : g_(o.g_), h_(o.h_) { o.g_ = nullptr; }
  GGUFLoader(const GGUFLoader&) = delete;
  GGUFLoader& operator=(const GGUFLoader&) = delete;
  ~GGUFLoader() {
    if (g_) wh_gguf_close(g_);
  }

  uint32_t version() const { return h_.version; }
  uint64_t tensor_count() const { return h_.tensor_count; }
  uint64_t metadata_kv_count() const { return h_.metadata_kv_count; }
  uint32_t alignment() const { return h_.alignment; }
  uint64_t data_start_offset() const { return h_.data_offset; }
  size_t file_size() const { return static_cast<size_t>(h_.file_size); }
  uint64_t total_tensor_size() const { return h_.total_tensor_size; }

  // tensor_info(name): empty when absent (the reference's None).
  bool tensor_info(const std::string& name, TensorInfo* out) const {
    uint64_t i;
    if (wh_gguf_find_tensor(g_, name.c_str(), &i) != WH_OK) return false;
    *out = info_at(i);
    return true;
  }
  std::vector<std::string> tensor_names() const {
    std::vector<std::string> v;
    for (uint64_t i = 0; i < h_.tensor_count; i++) v.push_back(info_at(i).name);
    return v;
  }
  // tensor_data(name) without the copy: pointer into the mapping + size.
  std::pair<const uint8_t*, size_t> tensor_data(const std::string& name) const {
    const void* p = nullptr;
    size_t n = 0;
    check(wh_gguf_tensor_data(g_, index(name), &p, &n), name);
    return {static_cast<const uint8_t*>(p), n};
  }
  // Device-resident weight straight from the mapping (release with wh_weight_free).
  wh_weight* upload(const std::string& name) const {
    wh_weight* w = nullptr;
    check(wh_gguf_upload(g_, index(name), &w), name);
    return w;
  }
  // GGUFMetadata getters (metadata.rs:186-233): false when absent or of another type.
  bool get_u32(const std::string& key, uint32_t* v) const { return wh_gguf_get_u32(g_, key.c_str(), v) == WH_OK; }
  bool get_u64(const std::string& key, uint64_t* v) const { return wh_gguf_get_u64(g_, key.c_str(), v) == WH_OK; }
  bool get_i32(const std::string& key, int32_t* v) const { return wh_gguf_get_i32(g_, key.c_str(), v) == WH_OK; }
  bool get_f32(const std::string& key, float* v) const { return wh_gguf_get_f32(g_, key.c_str(), v) == WH_OK; }
  bool get_bool(const std::string& key, bool* v) const {
    int b;
    if (wh_gguf_get_bool(g_, key.c_str(), &b) != WH_OK) return false;
    *v = b != 0;
    return true;
  }
  bool get_string(const std::string& key, std::string* v) const {
    const char* p;
    size_t n;
    if (wh_gguf_get_string(g_, key.c_str(), &p, &n) != WH_OK) return false;
    v->assign(p, n);
    return true;
  }
  std::string architecture() const {
    std::string s;
    get_string("general.architecture", &s);
    return s;
  }

 private:
  explicit GGUFLoader(wh_gguf* g) : g_(g) { wh_gguf_get_header(g_, &h_); }
  static void check(int st, const std::string& what) {
    if (st == WH_OK) return;
    const std::string m = wh_last_error();
    switch (st) {
      case WH_ERR_IO: throw Io(m);
      case WH_ERR_INVALID_MAGIC: throw InvalidMagic(m);
      case WH_ERR_UNSUPPORTED_VERSION: {
        const size_t p = m.rfind(' ');
        throw UnsupportedVersion(static_cast<uint32_t>(std::strtoul(m.c_str() + p + 1, nullptr, 10)), m);
      }
      case WH_ERR_INVALID_METADATA: throw InvalidMetadata(m);
      case WH_ERR_NOT_FOUND: throw TensorNotFound("Tensor not found: " + what);
      case WH_ERR_UNSUPPORTED_TYPE: throw Error(m);
      default: throw Error(m);
    }
  }
  uint64_t index(const std::string& name) const {
    uint64_t i = 0;
    check(wh_gguf_find_tensor(g_, name.c_str(), &i), name);
    return i;
  }
  TensorInfo info_at(uint64_t i) const {
    wh_gguf_tensor t;
    check(wh_gguf_tensor_at(g_, i, &t), "");
    TensorInfo r;
    r.name = t.name;
    r.dims.assign(t.dims, t.dims + t.n_dims);
    r.ggml_type = static_cast<uint32_t>(t.ggml_type);
    r.offset = t.offset;
    r.n_elements = t.n_elements;
    r.data_size = t.data_size;
    return r;
  }
  wh_gguf* g_ = nullptr;
  wh_gguf_header h_{};
};

}  // namespace gguf
}  // namespace woolly
