// gguf.hip -- GGUF file parsing over a read-only memory map, and weight upload
// straight from the mapping (host code only; no kernels).
//
// Reference: woolly-gguf (crates/woolly-gguf/src): GGUFHeader::read_from
// (format.rs:74-103), GGUFMetadata::read_from / MetadataValue::read_from
// (metadata.rs:86-124, 153-178), TensorInfo::read_from / n_elements /
// data_size (tensor_info.rs:203-255), GGUFLoader::from_mmap_with_config,
// tensor_data, align_offset (loader.rs:141-200, 230-295, 662-667).
//
// Differences from the reference, all on malformed input only: a tensor with
// more than WH_GGUF_MAX_DIMS dimensions, an element count or data size that
// overflows 64 bits, and an array whose declared length exceeds the bytes left
// in the file are rejected (InvalidTensorInfo / InvalidMetadata / end of file)
// before anything is allocated for them.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "wh_common.hpp"

namespace {

constexpr uint32_t kDefaultAlignment = 32;  // GGUF_DEFAULT_ALIGNMENT, format.rs:15

struct KV {
  std::string key;
  uint32_t type = 0;
  uint64_t off = 0;        // first byte of the value
  uint32_t elem_type = 0;  // arrays
  uint64_t count = 0;      // arrays
  std::vector<uint64_t> str_off;  // string arrays: offset of each element's u64 length
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[WH_GGUF_MAX_DIMS] = {};
  uint32_t type = 0;
  uint64_t offset = 0;
  uint64_t n_elements = 1;
  uint64_t nbytes = 0;
};

// GGMLType traits (tensor_info.rs:75-183).  bs = elements per block (1 for
// plain types), ts = bytes per block / element.  Ids 4 and 5 do not exist.
bool ggml_traits(uint32_t t, uint64_t* bs, uint64_t* ts, bool* quant) {
  struct Tr { int16_t bs; int16_t ts; };
  static const Tr tab[31] = {
      {1, 4},    {1, 2},    {32, 18},  {32, 20},  {0, 0},    {0, 0},    {32, 22},  {32, 24},
      {32, 34},  {32, 36},  {256, 82}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},
      {256, 66}, {256, 74}, {256, 98}, {256, 50}, {256, 130}, {256, 110}, {256, 82}, {256, 136},
      {1, 1},    {1, 2},    {1, 4},    {1, 8},    {1, 8},    {256, 56}, {1, 2}};
  if (t > 30 || tab[t].bs == 0) return false;
  *bs = static_cast<uint64_t>(tab[t].bs);
  *ts = static_cast<uint64_t>(tab[t].ts);
  // plain types: F32, F16, I8, I16, I32, I64, F64, BF16 (is_quantized, tensor_info.rs:180-182)
  *quant = !(t <= 1 || (t >= 24 && t <= 28) || t == 30);
  return true;
}

// Strict UTF-8 check with the rules of std::str::from_utf8: no overlong forms,
// no surrogates, nothing above U+10FFFF.
bool valid_utf8(const uint8_t* s, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    if (c < 0x80) {
      i++;
      continue;
    }
    int len;
    uint32_t cp;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
      cp = c & 0x1F;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      cp = c & 0x0F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      cp = c & 0x07;
    } else {
      return false;
    }
    if (n - i < static_cast<uint64_t>(len)) return false;
    for (int k = 1; k < len; k++) {
      const uint8_t cc = s[i + k];
      if ((cc & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (cc & 0x3F);
    }
    if ((len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) || cp > 0x10FFFF ||
        (cp >= 0xD800 && cp <= 0xDFFF))
      return false;
    i += static_cast<uint64_t>(len);
  }
  return true;
}

// Bounds-checked little-endian reader over the mapping.  Every failure records
// the error message and returns the status.
struct Reader {
  const uint8_t* p;
  uint64_t size;
  uint64_t pos = 0;

  int eof(uint64_t need) const {
    return wh::set_error(WH_ERR_IO,
                         "gguf: unexpected end of file: %llu bytes needed at offset %llu, file has %llu",
                         static_cast<unsigned long long>(need), static_cast<unsigned long long>(pos),
                         static_cast<unsigned long long>(size));
  }
  int skip(uint64_t n) {
    if (n > size - pos) return eof(n);
    pos += n;
    return WH_OK;
  }
  template <typename T>
  int get(T* v) {
    if (sizeof(T) > size - pos) return eof(sizeof(T));
    std::memcpy(v, p + pos, sizeof(T));
    pos += sizeof(T);
    return WH_OK;
  }
  // u64 length + UTF-8 bytes
  int str(std::string* out, const char* what) {
    uint64_t n;
    int st = get(&n);
    if (st) return st;
    if (n > size - pos) return eof(n);
    if (!valid_utf8(p + pos, n))
      return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: invalid UTF-8 in %s at offset %llu", what,
                           static_cast<unsigned long long>(pos));
    if (out) out->assign(reinterpret_cast<const char*>(p + pos), n);
    pos += n;
    return WH_OK;
  }
};

int scalar_size(uint32_t t) {
  switch (t) {
    case WH_GGUF_U8: case WH_GGUF_I8: case WH_GGUF_BOOL: return 1;
    case WH_GGUF_U16: case WH_GGUF_I16: return 2;
    case WH_GGUF_U32: case WH_GGUF_I32: case WH_GGUF_F32: return 4;
    case WH_GGUF_U64: case WH_GGUF_I64: case WH_GGUF_F64: return 8;
    default: return 0;
  }
}

int bad_type(const Reader& r, const char* what, uint32_t t) {
  return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: invalid %s type %u at offset %llu", what, t,
                       static_cast<unsigned long long>(r.pos));
}

// Skips one value of type t (MetadataValue::read_from), recording string
// element offsets when `kv` is given (top-level arrays of strings).
int skip_value(Reader& r, uint32_t t, KV* kv, int depth) {
  const int ss = scalar_size(t);
  if (ss) return r.skip(static_cast<uint64_t>(ss));
  if (t == WH_GGUF_STRING) return r.str(nullptr, "string value");
  if (t != WH_GGUF_ARRAY) return bad_type(r, "value", t);
  if (depth > 64) return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: arrays nested too deeply");
  uint32_t et;
  uint64_t n;
  int st = r.get(&et);
  if (st) return st;
  if (et > WH_GGUF_F64) return bad_type(r, "array element", et);
  st = r.get(&n);
  if (st) return st;
  if (kv) {
    kv->elem_type = et;
    kv->count = n;
    kv->off = r.pos;
  }
  const int es = scalar_size(et);
  if (es) {
    if (n > (r.size - r.pos) / static_cast<uint64_t>(es)) return r.eof(n * static_cast<uint64_t>(es));
    return r.skip(n * static_cast<uint64_t>(es));
  }
  // strings take >= 8 bytes, arrays >= 12: a length beyond that is truncated
  const uint64_t min_el = et == WH_GGUF_STRING ? 8 : 12;
  if (n > (r.size - r.pos) / min_el) return r.eof(n * min_el);
  if (kv && et == WH_GGUF_STRING) kv->str_off.reserve(n);
  for (uint64_t j = 0; j < n; j++) {
    if (kv && et == WH_GGUF_STRING) kv->str_off.push_back(r.pos);
    st = skip_value(r, et, nullptr, depth + 1);
    if (st) return st;
  }
  return WH_OK;
}

}  // namespace

struct wh_gguf {
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  bool mapped = false;
  uint32_t version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  uint32_t alignment = kDefaultAlignment;
  uint64_t data_offset = 0;
  uint64_t total_tensor_size = 0;
  std::vector<KV> kvs;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, uint64_t> kv_index, tensor_index;

  ~wh_gguf() {
    if (mapped && base && size) munmap(const_cast<uint8_t*>(base), size);
  }

  int parse() {
    Reader r{base, size};
    // header (format.rs:74-103)
    uint8_t magic[4];
    if (size < 4) return r.eof(4);
    std::memcpy(magic, base, 4);
    r.pos = 4;
    if (std::memcmp(magic, "GGUF", 4) != 0)
      return wh::set_error(WH_ERR_INVALID_MAGIC,
                           "gguf: invalid magic: expected 'GGUF', found [%u, %u, %u, %u]", magic[0],
                           magic[1], magic[2], magic[3]);
    int st = r.get(&version);
    if (st) return st;
    if (version < 1 || version > 3)
      return wh::set_error(WH_ERR_UNSUPPORTED_VERSION, "gguf: unsupported version %u", version);
    if ((st = r.get(&n_tensors)) || (st = r.get(&n_kv))) return st;
    // metadata (metadata.rs:153-178); each entry is at least 12 bytes
    if (n_kv > (size - r.pos) / 12) return r.eof(n_kv * 12);
    kvs.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
      KV kv;
      if ((st = r.str(&kv.key, "metadata key")) || (st = r.get(&kv.type))) return st;
      if (kv.type > WH_GGUF_F64) return bad_type(r, "metadata value", kv.type);
      kv.off = r.pos;
      st = skip_value(r, kv.type, kv.type == WH_GGUF_ARRAY ? &kv : nullptr, 0);
      if (st) return st;
      kv_index[kv.key] = kvs.size();
      kvs.push_back(std::move(kv));
    }
    // general.alignment when it is a u32 (loader.rs:148-151)
    auto it = kv_index.find("general.alignment");
    if (it != kv_index.end() && kvs[it->second].type == WH_GGUF_U32)
      std::memcpy(&alignment, base + kvs[it->second].off, 4);
    // tensor table (tensor_info.rs:203-238); each entry is at least 24 bytes
    if (n_tensors > (size - r.pos) / 24) return r.eof(n_tensors * 24);
    tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
      Tensor t;
      if ((st = r.str(&t.name, "tensor name")) || (st = r.get(&t.n_dims))) return st;
      if (t.n_dims > WH_GGUF_MAX_DIMS)
        return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: tensor '%s' has %u dimensions (max %d)",
                             t.name.c_str(), t.n_dims, WH_GGUF_MAX_DIMS);
      for (uint32_t d = 0; d < t.n_dims; d++) {
        if ((st = r.get(&t.dims[d]))) return st;
        if (t.dims[d] != 0 && t.n_elements > UINT64_MAX / t.dims[d])
          return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: tensor '%s' element count overflows",
                               t.name.c_str());
        t.n_elements *= t.dims[d];
      }
      if ((st = r.get(&t.type))) return st;
      uint64_t bs, ts;
      bool q;
      if (!ggml_traits(t.type, &bs, &ts, &q))
        return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "gguf: invalid tensor type %u (tensor '%s')",
                             t.type, t.name.c_str());
      if ((st = r.get(&t.offset))) return st;
      // data_size (tensor_info.rs:246-258): whole blocks for quantized types
      const uint64_t units = q ? t.n_elements / bs + (t.n_elements % bs != 0) : t.n_elements;
      if (units > UINT64_MAX / ts)
        return wh::set_error(WH_ERR_INVALID_METADATA, "gguf: tensor '%s' data size overflows",
                             t.name.c_str());
      t.nbytes = units * ts;
      tensor_index[t.name] = tensors.size();
      tensors.push_back(std::move(t));
    }
    // align_offset (loader.rs:662-667), the reference's formula as written
    const uint64_t a = alignment;
    data_offset = a == 0 ? r.pos : (r.pos + a - 1) & ~(a - 1);
    // total_tensor_size over distinct names (the reference sums its HashMap)
    total_tensor_size = 0;
    for (const auto& kv : tensor_index) total_tensor_size += tensors[kv.second].nbytes;
    return WH_OK;
  }
};

namespace {

int null_arg(const char* fn) { return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: null argument", fn); }

int open_common(wh_gguf* g, wh_gguf** out) {
  const int st = g->parse();
  if (st) {
    delete g;
    return st;
  }
  *out = g;
  return WH_OK;
}

const KV* kv_by_key(const wh_gguf* g, const char* key, int* st) {
  auto it = g->kv_index.find(key);
  if (it == g->kv_index.end()) {
    *st = wh::set_error(WH_ERR_NOT_FOUND, "gguf: metadata key '%s' not found", key);
    return nullptr;
  }
  *st = WH_OK;
  return &g->kvs[it->second];
}

template <typename T>
int get_typed(const wh_gguf* g, const char* key, uint32_t type, T* out, const char* fn) {
  if (!g || !key || !out) return null_arg(fn);
  int st;
  const KV* kv = kv_by_key(g, key, &st);
  if (!kv) return st;
  if (kv->type != type)
    return wh::set_error(WH_ERR_TYPE_MISMATCH, "%s: '%s' has value type %u, not %u", fn, key, kv->type,
                         type);
  std::memcpy(out, g->base + kv->off, sizeof(T));
  return WH_OK;
}

int kv_checked(const wh_gguf* g, uint64_t i, const char* fn, const KV** kv) {
  if (!g) return null_arg(fn);
  if (i >= g->kvs.size())
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: index %llu out of range (%zu key/values)", fn,
                         static_cast<unsigned long long>(i), g->kvs.size());
  *kv = &g->kvs[i];
  return WH_OK;
}

void string_at(const wh_gguf* g, uint64_t len_off, const char** data, size_t* len) {
  uint64_t n;
  std::memcpy(&n, g->base + len_off, 8);
  *data = reinterpret_cast<const char*>(g->base + len_off + 8);
  *len = static_cast<size_t>(n);
}

}  // namespace

WH_API int wh_gguf_open(const char* path, wh_gguf** out) {
  if (!path || !out) return null_arg("gguf_open");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return wh::set_error(WH_ERR_IO, "gguf: cannot open '%s': %s", path, std::strerror(errno));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    const int e = errno;
    close(fd);
    return wh::set_error(WH_ERR_IO, "gguf: cannot stat '%s': %s", path, std::strerror(e));
  }
  wh_gguf* g = new (std::nothrow) wh_gguf();
  if (!g) {
    close(fd);
    return wh::set_error(WH_ERR_OOM, "gguf: host allocation failed");
  }
  g->size = static_cast<uint64_t>(sb.st_size);
  if (g->size > 0) {
    void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      const int e = errno;
      close(fd);
      delete g;
      return wh::set_error(WH_ERR_IO, "gguf: cannot map '%s': %s", path, std::strerror(e));
    }
    g->base = static_cast<const uint8_t*>(p);
    g->mapped = true;
  }
  close(fd);  // the mapping keeps the file
  return open_common(g, out);
}

WH_API int wh_gguf_open_buffer(const void* data, size_t nbytes, wh_gguf** out) {
  if (!out || (!data && nbytes)) return null_arg("gguf_open_buffer");
  *out = nullptr;
  wh_gguf* g = new (std::nothrow) wh_gguf();
  if (!g) return wh::set_error(WH_ERR_OOM, "gguf: host allocation failed");
  g->base = static_cast<const uint8_t*>(data);
  g->size = nbytes;
  return open_common(g, out);
}

WH_API int wh_gguf_close(wh_gguf* g) {
  delete g;
  return WH_OK;
}

WH_API int wh_gguf_get_header(const wh_gguf* g, wh_gguf_header* out) {
  if (!g || !out) return null_arg("gguf_get_header");
  out->version = g->version;
  out->tensor_count = g->n_tensors;
  out->metadata_kv_count = g->n_kv;
  out->alignment = g->alignment;
  out->data_offset = g->data_offset;
  out->file_size = g->size;
  out->total_tensor_size = g->total_tensor_size;
  return WH_OK;
}

WH_API int wh_gguf_tensor_at(const wh_gguf* g, uint64_t i, wh_gguf_tensor* out) {
  if (!g || !out) return null_arg("gguf_tensor_at");
  if (i >= g->tensors.size())
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "gguf_tensor_at: index %llu out of range (%zu tensors)",
                         static_cast<unsigned long long>(i), g->tensors.size());
  const Tensor& t = g->tensors[i];
  out->name = t.name.c_str();
  out->n_dims = t.n_dims;
  for (int d = 0; d < WH_GGUF_MAX_DIMS; d++) out->dims[d] = t.dims[d];
  out->ggml_type = static_cast<int>(t.type);
  out->offset = t.offset;
  out->n_elements = t.n_elements;
  out->data_size = t.nbytes;
  return WH_OK;
}

WH_API int wh_gguf_find_tensor(const wh_gguf* g, const char* name, uint64_t* index) {
  if (!g || !name || !index) return null_arg("gguf_find_tensor");
  auto it = g->tensor_index.find(name);
  if (it == g->tensor_index.end())
    return wh::set_error(WH_ERR_NOT_FOUND, "gguf: tensor not found: %s", name);
  *index = it->second;
  return WH_OK;
}

WH_API int wh_gguf_tensor_data(const wh_gguf* g, uint64_t i, const void** data, size_t* nbytes) {
  if (!g || !data || !nbytes) return null_arg("gguf_tensor_data");
  if (i >= g->tensors.size())
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "gguf_tensor_data: index %llu out of range",
                         static_cast<unsigned long long>(i));
  const Tensor& t = g->tensors[i];
  // loader.rs:273-282: absolute offset + size must lie inside the file
  const uint64_t abs = g->data_offset + t.offset;
  const bool wraps = abs < g->data_offset || abs + t.nbytes < abs;
  if (wraps || abs + t.nbytes > g->size)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL, "gguf: buffer too small: needed %llu bytes, available %llu",
                         wraps ? static_cast<unsigned long long>(UINT64_MAX)
                               : static_cast<unsigned long long>(abs + t.nbytes),
                         static_cast<unsigned long long>(g->size));
  *data = g->base + abs;
  *nbytes = static_cast<size_t>(t.nbytes);
  return WH_OK;
}

WH_API int wh_gguf_upload(const wh_gguf* g, uint64_t i, wh_weight** out) {
  if (!g || !out) return null_arg("gguf_upload");
  *out = nullptr;
  const void* data;
  size_t nbytes;
  int st = wh_gguf_tensor_data(g, i, &data, &nbytes);
  if (st) return st;
  const Tensor& t = g->tensors[i];
  const uint64_t k = t.n_dims ? t.dims[0] : 1;
  const uint64_t rows = k ? t.n_elements / k : 0;
  return wh_weight_upload(static_cast<int>(t.type), static_cast<size_t>(rows), static_cast<size_t>(k),
                          data, nbytes, out);
}

WH_API int wh_gguf_kv_at(const wh_gguf* g, uint64_t i, const char** key, int* value_type) {
  const KV* kv;
  int st = kv_checked(g, i, "gguf_kv_at", &kv);
  if (st) return st;
  if (key) *key = kv->key.c_str();
  if (value_type) *value_type = static_cast<int>(kv->type);
  return WH_OK;
}

WH_API int wh_gguf_find_kv(const wh_gguf* g, const char* key, uint64_t* index) {
  if (!g || !key || !index) return null_arg("gguf_find_kv");
  auto it = g->kv_index.find(key);
  if (it == g->kv_index.end()) return wh::set_error(WH_ERR_NOT_FOUND, "gguf: metadata key '%s' not found", key);
  *index = it->second;
  return WH_OK;
}

WH_API int wh_gguf_get_u32(const wh_gguf* g, const char* key, uint32_t* out) {
  return get_typed(g, key, WH_GGUF_U32, out, "gguf_get_u32");
}
WH_API int wh_gguf_get_u64(const wh_gguf* g, const char* key, uint64_t* out) {
  return get_typed(g, key, WH_GGUF_U64, out, "gguf_get_u64");
}
WH_API int wh_gguf_get_i32(const wh_gguf* g, const char* key, int32_t* out) {
  return get_typed(g, key, WH_GGUF_I32, out, "gguf_get_i32");
}
WH_API int wh_gguf_get_f32(const wh_gguf* g, const char* key, float* out) {
  return get_typed(g, key, WH_GGUF_F32, out, "gguf_get_f32");
}
WH_API int wh_gguf_get_bool(const wh_gguf* g, const char* key, int* out) {
  uint8_t b;
  const int st = get_typed(g, key, WH_GGUF_BOOL, &b, "gguf_get_bool");
  if (st == WH_OK) *out = b != 0;  // metadata.rs:94: any non-zero byte is true
  return st;
}
WH_API int wh_gguf_get_string(const wh_gguf* g, const char* key, const char** data, size_t* len) {
  if (!g || !key || !data || !len) return null_arg("gguf_get_string");
  int st;
  const KV* kv = kv_by_key(g, key, &st);
  if (!kv) return st;
  if (kv->type != WH_GGUF_STRING)
    return wh::set_error(WH_ERR_TYPE_MISMATCH, "gguf_get_string: '%s' has value type %u", key, kv->type);
  string_at(g, kv->off, data, len);
  return WH_OK;
}

WH_API int wh_gguf_kv_scalar(const wh_gguf* g, uint64_t i, int* value_type, void* out8) {
  const KV* kv;
  int st = kv_checked(g, i, "gguf_kv_scalar", &kv);
  if (st) return st;
  if (!out8) return null_arg("gguf_kv_scalar");
  const int ss = scalar_size(kv->type);
  if (!ss) return wh::set_error(WH_ERR_TYPE_MISMATCH, "gguf_kv_scalar: '%s' is not a scalar", kv->key.c_str());
  std::memset(out8, 0, 8);
  std::memcpy(out8, g->base + kv->off, static_cast<size_t>(ss));
  if (kv->type == WH_GGUF_BOOL) *static_cast<uint8_t*>(out8) = *static_cast<uint8_t*>(out8) != 0;
  if (value_type) *value_type = static_cast<int>(kv->type);
  return WH_OK;
}

WH_API int wh_gguf_kv_array(const wh_gguf* g, uint64_t i, int* elem_type, uint64_t* count,
                            const void** data) {
  const KV* kv;
  int st = kv_checked(g, i, "gguf_kv_array", &kv);
  if (st) return st;
  if (kv->type != WH_GGUF_ARRAY)
    return wh::set_error(WH_ERR_TYPE_MISMATCH, "gguf_kv_array: '%s' is not an array", kv->key.c_str());
  if (elem_type) *elem_type = static_cast<int>(kv->elem_type);
  if (count) *count = kv->count;
  if (data) *data = scalar_size(kv->elem_type) ? g->base + kv->off : nullptr;
  return WH_OK;
}

WH_API int wh_gguf_kv_array_string(const wh_gguf* g, uint64_t i, uint64_t j, const char** data,
                                   size_t* len) {
  const KV* kv;
  int st = kv_checked(g, i, "gguf_kv_array_string", &kv);
  if (st) return st;
  if (!data || !len) return null_arg("gguf_kv_array_string");
  if (kv->type != WH_GGUF_ARRAY || kv->elem_type != WH_GGUF_STRING)
    return wh::set_error(WH_ERR_TYPE_MISMATCH, "gguf_kv_array_string: '%s' is not an array of strings",
                         kv->key.c_str());
  if (j >= kv->str_off.size())
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "gguf_kv_array_string: element %llu out of range",
                         static_cast<unsigned long long>(j));
  string_at(g, kv->str_off[j], data, len);
  return WH_OK;
}

WH_API int wh_gguf_kv_string(const wh_gguf* g, uint64_t i, const char** data, size_t* len) {
  const KV* kv;
  int st = kv_checked(g, i, "gguf_kv_string", &kv);
  if (st) return st;
  if (!data || !len) return null_arg("gguf_kv_string");
  if (kv->type != WH_GGUF_STRING)
    return wh::set_error(WH_ERR_TYPE_MISMATCH, "gguf_kv_string: '%s' is not a string", kv->key.c_str());
  string_at(g, kv->off, data, len);
  return WH_OK;
}

WH_API int wh_ggml_type_traits(int ggml_type, size_t* block_size, size_t* type_size, int* is_quantized) {
  uint64_t bs, ts;
  bool q;
  if (ggml_type < 0 || !ggml_traits(static_cast<uint32_t>(ggml_type), &bs, &ts, &q))
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "invalid tensor type %d", ggml_type);
  if (block_size) *block_size = static_cast<size_t>(bs);
  if (type_size) *type_size = static_cast<size_t>(ts);
  if (is_quantized) *is_quantized = q ? 1 : 0;
  return WH_OK;
}
