// api.hip -- the C ABI of libwoolly_hip (include/woolly_hip.h): argument
// validation with the reference's error semantics, device/stream plumbing,
// weight handles and the synchronous host-pointer variants.  Kernels live in
// dequant.hip, gemv.hip, gemm.hip and elementwise.hip.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "wh_common.hpp"

struct wh_weight {
  int type;
  size_t n_rows;
  size_t k;
  size_t nbytes;
  void* data;
  int device;
  void* prefill = nullptr;    // wh_weight_prepare_prefill's copy (K-quants)
  size_t prefill_bytes = 0;
};

namespace {

thread_local char g_last_error[512] = "";

hipStream_t hs(wh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// per-device caches of device attributes (0: not yet queried)
std::atomic<int> g_cu_count[wh::kMaxDevices];
std::atomic<int> g_max_lds[wh::kMaxDevices];

// A device attribute of the current device, queried once and cached in c.
int cached_attribute(std::atomic<int>* c, hipDeviceAttribute_t attr, int fallback) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= wh::kMaxDevices) return fallback;
  int v = c[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, attr, dev) != hipSuccess || v <= 0) v = fallback;
  c[dev].store(v, std::memory_order_relaxed);
  return v;
}

int check_block_args(const char* fn, int type, size_t k) {
  if (!wh::is_block_type(type))
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE,
                         "%s: unsupported quantization scheme (ggml type %d); supported: "
                         "Q4_0 (2), Q4_1 (3), Q8_0 (8)",
                         fn, type);
  if (k % 32 != 0)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: k = %zu is not a multiple of the block size 32",
                         fn, k);
  return WH_OK;
}

// The GEMV also takes the 256-element K-quant blocks.
int check_gemv_args(const char* fn, int type, size_t k) {
  if (!wh::is_kquant(type)) return check_block_args(fn, type, k);
  if (k % 256 != 0)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: k = %zu is not a multiple of the block size 256",
                         fn, k);
  return WH_OK;
}

int check_weight_bytes(const char* fn, int type, size_t rows, size_t k, size_t have) {
  const size_t ts = wh::type_size(type);
  const size_t nb = k / wh::block_elems(type);
  if (rows != 0 && nb != 0 && (rows > SIZE_MAX / nb || rows * nb > SIZE_MAX / ts))
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: %zu x %zu weight size overflows", fn, rows, k);
  const size_t need = rows * nb * ts;
  if (have < need)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "%s: buffer too small: needed %zu bytes, available %zu", fn, need, have);
  return WH_OK;
}

int check_ptr(const char* fn, const char* what, const void* p, size_t align) {
  if (p == nullptr)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: %s is a null pointer", fn, what);
  if (!wh::aligned(p, align))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: %s is not %zu-byte aligned", fn, what, align);
  return WH_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Handles with a prepared prefill copy, by their data pointer.  Allocated once
// and never destroyed (no destructor runs after the HIP runtime at exit).
struct PreparedRegistry {
  std::mutex mu;
  std::map<const void*, const wh_weight*> by_data;
};
PreparedRegistry& prepared_registry() {
  static PreparedRegistry* r = new PreparedRegistry();
  return *r;
}

}  // namespace

namespace wh {

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_error(hipError_t err, const char* what) {
  const int st = (err == hipErrorOutOfMemory) ? WH_ERR_OOM : WH_ERR_HIP;
  return set_error(st, "%s failed: %s (%d)", what, hipGetErrorString(err), static_cast<int>(err));
}

int cu_count() { return cached_attribute(g_cu_count, hipDeviceAttributeMultiprocessorCount, 256); }

size_t max_lds_per_block() {
  return static_cast<size_t>(cached_attribute(g_max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, 65536));
}

const void* prepared_kquant(const void* w, int type, size_t n_rows, size_t k) {
  PreparedRegistry& r = prepared_registry();
  std::lock_guard<std::mutex> lk(r.mu);
  auto it = r.by_data.find(w);
  if (it == r.by_data.end()) return nullptr;
  const wh_weight* h = it->second;
  return (h->type == type && h->n_rows == n_rows && h->k == k) ? h->prefill : nullptr;
}

int ensure_dynamic_lds(LdsLimit& lim, const void* fn, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = -1;
  const int want = static_cast<int>(bytes);
  if (dev >= 0 && lim.set[dev].load(std::memory_order_relaxed) >= want) return WH_OK;
  WH_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, want));
  if (dev >= 0) {
    int cur = lim.set[dev].load(std::memory_order_relaxed);
    while (cur < want && !lim.set[dev].compare_exchange_weak(cur, want, std::memory_order_relaxed)) {
    }
  }
  return WH_OK;
}

}  // namespace wh

extern "C" {

WH_API const char* wh_status_string(int status) {
  switch (status) {
    case WH_OK: return "WH_OK";
    case WH_ERR_UNSUPPORTED_TYPE: return "WH_ERR_UNSUPPORTED_TYPE";
    case WH_ERR_INVALID_SHAPE: return "WH_ERR_INVALID_SHAPE";
    case WH_ERR_BUFFER_TOO_SMALL: return "WH_ERR_BUFFER_TOO_SMALL";
    case WH_ERR_INVALID_ARGUMENT: return "WH_ERR_INVALID_ARGUMENT";
    case WH_ERR_HIP: return "WH_ERR_HIP";
    case WH_ERR_OOM: return "WH_ERR_OOM";
    case WH_ERR_NO_DEVICE: return "WH_ERR_NO_DEVICE";
    case WH_ERR_IO: return "WH_ERR_IO";
    case WH_ERR_INVALID_MAGIC: return "WH_ERR_INVALID_MAGIC";
    case WH_ERR_UNSUPPORTED_VERSION: return "WH_ERR_UNSUPPORTED_VERSION";
    case WH_ERR_INVALID_METADATA: return "WH_ERR_INVALID_METADATA";
    case WH_ERR_NOT_FOUND: return "WH_ERR_NOT_FOUND";
    case WH_ERR_TYPE_MISMATCH: return "WH_ERR_TYPE_MISMATCH";
    default: return "WH_ERR_UNKNOWN";
  }
}

WH_API const char* wh_last_error(void) { return g_last_error; }

WH_API int wh_version(void) { return 1; }

WH_API int wh_gemv_select(int mode, int* previous) {
  if (mode != WH_GEMV_AUTO && mode != WH_GEMV_STREAM)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "gemv_select: unknown mode %d", mode);
  const int prev = wh::gemv_mode_exchange(mode);
  if (previous) *previous = prev;
  return WH_OK;
}

// ------------------------------------------------------------- device/memory
WH_API int wh_device_count(int* count) {
  if (!count) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_device_count: null count");
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return wh::set_error(WH_ERR_NO_DEVICE, "hipGetDeviceCount failed: %s", hipGetErrorString(e));
  }
  *count = n;
  return WH_OK;
}

WH_API int wh_init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return wh::set_error(WH_ERR_NO_DEVICE, "wh_init: no HIP device is visible");
  if (device < 0 || device >= n)
    return wh::set_error(WH_ERR_NO_DEVICE, "wh_init: device %d out of range (%d visible)", device, n);
  WH_HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  WH_HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return wh::set_error(WH_ERR_NO_DEVICE, "wh_init: device %d is %s; this library is built for gfx950",
                         device, prop.gcnArchName);
  (void)wh::cu_count();
  return wh::init_step_scratch();
}

WH_API int wh_device_name(char* buf, size_t len) {
  if (!buf || len == 0) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_device_name: bad buffer");
  int dev = 0;
  WH_HIP_TRY(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  WH_HIP_TRY(hipGetDeviceProperties(&prop, dev));
  std::snprintf(buf, len, "%s (%s, %d CUs, %zu KiB LDS/block, %d MHz)", prop.name, prop.gcnArchName,
                prop.multiProcessorCount, wh::max_lds_per_block() / 1024, prop.clockRate / 1000);
  return WH_OK;
}

WH_API int wh_malloc(void** dptr, size_t nbytes) {
  if (!dptr) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_malloc: null output pointer");
  *dptr = nullptr;
  if (nbytes == 0) return WH_OK;
  WH_HIP_TRY(hipMalloc(dptr, nbytes));
  return WH_OK;
}

WH_API int wh_free(void* dptr) {
  if (dptr) WH_HIP_TRY(hipFree(dptr));
  return WH_OK;
}

WH_API int wh_memcpy_h2d(void* dst, const void* src, size_t nbytes, wh_stream_t stream) {
  if (nbytes == 0) return WH_OK;
  if (!dst || !src) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_memcpy_h2d: null pointer");
  WH_HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, hs(stream)));
  return WH_OK;
}

WH_API int wh_memcpy_d2h(void* dst, const void* src, size_t nbytes, wh_stream_t stream) {
  if (nbytes == 0) return WH_OK;
  if (!dst || !src) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_memcpy_d2h: null pointer");
  WH_HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, hs(stream)));
  return WH_OK;
}

WH_API int wh_memcpy_d2d(void* dst, const void* src, size_t nbytes, wh_stream_t stream) {
  if (nbytes == 0) return WH_OK;
  if (!dst || !src) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_memcpy_d2d: null pointer");
  WH_HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, hs(stream)));
  return WH_OK;
}

WH_API int wh_fill_bytes(void* dst, int value, size_t nbytes, wh_stream_t stream) {
  if (nbytes == 0) return WH_OK;
  if (!dst) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_fill_bytes: null pointer");
  return wh::launch_fill_bytes(dst, value, nbytes, hs(stream));
}

WH_API int wh_stream_create(wh_stream_t* out) {
  if (!out) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_stream_create: null output");
  hipStream_t s;
  WH_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = reinterpret_cast<wh_stream_t>(s);
  return WH_OK;
}

WH_API int wh_stream_destroy(wh_stream_t stream) {
  if (stream) WH_HIP_TRY(hipStreamDestroy(hs(stream)));
  return WH_OK;
}

WH_API int wh_stream_synchronize(wh_stream_t stream) {
  WH_HIP_TRY(hipStreamSynchronize(hs(stream)));
  return WH_OK;
}

WH_API int wh_device_synchronize(void) {
  WH_HIP_TRY(hipDeviceSynchronize());
  return WH_OK;
}

WH_API int wh_event_create(wh_event_t* out) {
  if (!out) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_event_create: null output");
  hipEvent_t e;
  WH_HIP_TRY(hipEventCreate(&e));
  *out = reinterpret_cast<wh_event_t>(e);
  return WH_OK;
}

WH_API int wh_event_destroy(wh_event_t event) {
  if (event) WH_HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return WH_OK;
}

WH_API int wh_event_record(wh_event_t event, wh_stream_t stream) {
  if (!event) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_event_record: null event");
  WH_HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), hs(stream)));
  return WH_OK;
}

WH_API int wh_event_synchronize(wh_event_t event) {
  if (!event) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_event_synchronize: null event");
  WH_HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
  return WH_OK;
}

WH_API int wh_event_elapsed_ms(float* ms, wh_event_t start, wh_event_t end) {
  if (!ms || !start || !end)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_event_elapsed_ms: null argument");
  WH_HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                 reinterpret_cast<hipEvent_t>(end)));
  return WH_OK;
}

// -------------------------------------------------------------------- graphs
WH_API int wh_graph_begin_capture(wh_stream_t stream) {
  if (!stream)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "graph capture needs a non-null stream");
  WH_HIP_TRY(hipStreamBeginCapture(hs(stream), hipStreamCaptureModeThreadLocal));
  return WH_OK;
}

WH_API int wh_graph_end_capture(wh_stream_t stream, wh_graph_t* out) {
  if (!stream || !out)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_graph_end_capture: null argument");
  *out = nullptr;
  hipGraph_t g = nullptr;
  WH_HIP_TRY(hipStreamEndCapture(hs(stream), &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return wh::hip_error(e, "hipGraphInstantiate");
  *out = reinterpret_cast<wh_graph_t>(exec);
  return WH_OK;
}

WH_API int wh_graph_launch(wh_graph_t graph, wh_stream_t stream) {
  if (!graph) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_graph_launch: null graph");
  WH_HIP_TRY(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), hs(stream)));
  return WH_OK;
}

WH_API int wh_graph_destroy(wh_graph_t graph) {
  if (graph) WH_HIP_TRY(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)));
  return WH_OK;
}

// -------------------------------------------------------------------- format
WH_API size_t wh_block_size(int type) { return wh::block_elems(type); }

WH_API size_t wh_type_size(int type) { return wh::type_size(type); }

WH_API int wh_tensor_nbytes(int type, uint64_t nelements, uint64_t* nbytes) {
  if (!nbytes) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_tensor_nbytes: null output");
  const uint64_t bs = wh_block_size(type), ts = wh::type_size(type);
  if (bs == 0) return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "wh_tensor_nbytes: unsupported type %d", type);
  *nbytes = (nelements + bs - 1) / bs * ts;
  return WH_OK;
}

// ---------------------------------------------------------- dequantization
WH_API int wh_dequantize(int type, const void* data, size_t nbytes, size_t nelements, float* out,
                         wh_stream_t stream) {
  const size_t ts = wh::type_size(type);
  if (ts == 0)
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "dequantize: invalid tensor type %d", type);
  if (type == WH_TYPE_F32 || type == WH_TYPE_F16) {
    if (nbytes != nelements * ts)
      return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                           "dequantize: buffer too small: needed %zu bytes, available %zu",
                           nelements * ts, nbytes);
  } else {
    const size_t bs = wh::block_elems(type);
    const size_t need = (nelements / bs + (nelements % bs != 0)) * ts;
    // The K-quant decoders report a short block as invalid tensor info
    // (dequantize.rs:416-418, 472-474), the others as BufferTooSmall.
    if (nbytes < need && wh::is_kquant(type))
      return wh::set_error(WH_ERR_INVALID_METADATA,
                           "dequantize: insufficient data for K-quant block: needed %zu bytes, available %zu",
                           need, nbytes);
    if (nbytes < need)
      return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                           "dequantize: buffer too small: needed %zu bytes, available %zu", need,
                           nbytes);
  }
  if (nelements == 0) return WH_OK;
  int st = check_ptr("dequantize", "data", data, 1);
  if (st) return st;
  st = check_ptr("dequantize", "out", out, 4);
  if (st) return st;
  return wh::launch_dequantize(type, data, nelements, out, hs(stream));
}

// -------------------------------------------------------------------- GEMV
WH_API int wh_quantized_matvec(int type, const void* weights, size_t weight_nbytes,
                               const float* input, float* output, size_t m, size_t k,
                               wh_stream_t stream) {
  int st = check_gemv_args("quantized_matvec", type, k);
  if (st) return st;
  st = check_weight_bytes("quantized_matvec", type, m, k, weight_nbytes);
  if (st) return st;
  if (m == 0) return WH_OK;
  st = check_ptr("quantized_matvec", "output", output, 4);
  if (st) return st;
  if (k == 0) return wh::launch_fill_bytes(output, 0, m * sizeof(float), hs(stream));
  st = check_ptr("quantized_matvec", "weights", weights, 1);
  if (st) return st;
  st = check_ptr("quantized_matvec", "input", input, 4);
  if (st) return st;
  return wh::launch_gemv(type, weights, input, output, m, k, hs(stream));
}

// -------------------------------------------------------------------- GEMM
WH_API size_t wh_quantized_matmul_workspace_bytes(int type, size_t n_rows, size_t k,
                                                  size_t n_tokens) {
  if (!(wh::is_block_type(type) || wh::is_kquant(type)) || n_tokens <= wh::kGemvTokenLimit || k == 0) return 0;
  return wh::gemm_workspace_bytes_for(type, n_rows, n_tokens, k);
}

WH_API int wh_quantized_matmul(int type, const void* weights, size_t weight_nbytes, size_t n_rows,
                               size_t k, const float* x, size_t n_tokens, float* y, void* workspace,
                               size_t workspace_bytes, wh_stream_t stream) {
  int st = check_gemv_args("quantized_matmul", type, k);
  if (st) return st;
  st = check_weight_bytes("quantized_matmul", type, n_rows, k, weight_nbytes);
  if (st) return st;
  if (n_rows == 0 || n_tokens == 0) return WH_OK;
  st = check_ptr("quantized_matmul", "y", y, 4);
  if (st) return st;
  if (k == 0) return wh::launch_fill_bytes(y, 0, n_rows * n_tokens * sizeof(float), hs(stream));
  st = check_ptr("quantized_matmul", "weights", weights, 1);
  if (st) return st;
  st = check_ptr("quantized_matmul", "x", x, 4);
  if (st) return st;
  if (workspace && !wh::aligned(workspace, 256))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "quantized_matmul: workspace is not 256-byte aligned");
  return wh::launch_gemm(type, weights, n_rows, k, x, n_tokens, y, workspace, workspace_bytes,
                         hs(stream));
}

WH_API size_t wh_quantized_matmul_x_workspace_bytes(int type, size_t n_rows, size_t k, size_t n_tokens,
                                                    int x_dtype) {
  if (x_dtype != WH_TYPE_BF16) return wh_quantized_matmul_workspace_bytes(type, n_rows, k, n_tokens);
  if (!(wh::is_block_type(type) || wh::is_kquant(type)) || k == 0) return 0;
  // the widened activations, then the f32 product's workspace (the tiled
  // kernel reads bf16 directly and needs only the latter)
  return align_up(n_tokens * k * sizeof(float), 256) + wh_quantized_matmul_workspace_bytes(type, n_rows, k, n_tokens);
}

WH_API int wh_quantized_matmul_x(int type, const void* weights, size_t weight_nbytes, size_t n_rows, size_t k,
                                 const void* x, int x_dtype, size_t n_tokens, float* y, void* workspace,
                                 size_t workspace_bytes, wh_stream_t stream) {
  if (x_dtype == WH_TYPE_F32)
    return wh_quantized_matmul(type, weights, weight_nbytes, n_rows, k, static_cast<const float*>(x), n_tokens, y,
                               workspace, workspace_bytes, stream);
  if (x_dtype != WH_TYPE_BF16)
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "quantized_matmul_x: activation type %d (f32 = 0 or bf16 = 30)",
                         x_dtype);
  int st = check_gemv_args("quantized_matmul_x", type, k);
  if (st) return st;
  st = check_weight_bytes("quantized_matmul_x", type, n_rows, k, weight_nbytes);
  if (st) return st;
  if (n_rows == 0 || n_tokens == 0) return WH_OK;
  st = check_ptr("quantized_matmul_x", "y", y, 4);
  if (st) return st;
  hipStream_t s = hs(stream);
  if (k == 0) return wh::launch_fill_bytes(y, 0, n_rows * n_tokens * sizeof(float), s);
  if ((st = check_ptr("quantized_matmul_x", "weights", weights, 1)) || (st = check_ptr("quantized_matmul_x", "x", x, 8)))
    return st;
  const size_t need = wh_quantized_matmul_x_workspace_bytes(type, n_rows, k, n_tokens, x_dtype);
  if (!workspace || workspace_bytes < need)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "quantized_matmul_x: workspace too small: needed %zu bytes, available %zu", need,
                         workspace ? workspace_bytes : static_cast<size_t>(0));
  if (!wh::aligned(workspace, 256))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "quantized_matmul_x: workspace is not 256-byte aligned");
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  // many tokens: the tiled kernel's packing reads bf16 itself
  if (n_tokens > 16 && wh::is_block_type(type) &&
      wh::gemm_tiled_ok(type, weights, static_cast<const float*>(x), n_rows, k, n_tokens))
    return wh::launch_gemm_tiled_bf16(type, weights, n_rows, k, xb, n_tokens, y, workspace, s);
  // otherwise widen into the workspace and run the f32 product
  float* xf = static_cast<float*>(workspace);
  const size_t head = align_up(n_tokens * k * sizeof(float), 256);
  if ((st = wh::launch_bf16_to_f32(xb, n_tokens * k, xf, s))) return st;
  return wh::launch_gemm(type, weights, n_rows, k, xf, n_tokens, y, static_cast<char*>(workspace) + head,
                         workspace_bytes - head, s);
}

// --------------------------------------------------------------- elementwise
WH_API int wh_rms_norm(const float* x, const float* weight, float eps, size_t tokens, size_t hidden,
                       float* out, wh_stream_t stream) {
  if (tokens == 0 || hidden == 0) return WH_OK;
  int st = check_ptr("rms_norm", "x", x, 4);
  if (st) return st;
  st = check_ptr("rms_norm", "weight", weight, 4);
  if (st) return st;
  st = check_ptr("rms_norm", "out", out, 4);
  if (st) return st;
  return wh::launch_rms_norm(x, weight, eps, tokens, hidden, out, hs(stream));
}

WH_API int wh_swiglu(const float* gate, const float* up, size_t n, float* out, wh_stream_t stream) {
  if (n == 0) return WH_OK;
  int st = check_ptr("swiglu", "gate", gate, 4);
  if (st) return st;
  st = check_ptr("swiglu", "up", up, 4);
  if (st) return st;
  st = check_ptr("swiglu", "out", out, 4);
  if (st) return st;
  return wh::launch_swiglu(gate, up, n, out, hs(stream));
}

// ------------------------------------------------------------------- FFN
WH_API size_t wh_ffn_workspace_bytes_for_type(int type, size_t hidden, size_t n_ff, size_t m) {
  size_t gemm_ws = 0;
  if (m > wh::kGemvTokenLimit) {
    if (wh::is_kquant(type)) {
      gemm_ws = wh::ffn_kquant_workspace_bytes(type, hidden, n_ff, m);
    } else {
      const size_t g1 = wh::gemm_workspace_bytes_for(type, n_ff, m, hidden);
      const size_t g2 = wh::gemm_workspace_bytes_for(type, hidden, m, n_ff);
      gemm_ws = g1 > g2 ? g1 : g2;
    }
  }
  return align_up(m * hidden * sizeof(float), 256) + 3 * align_up(m * n_ff * sizeof(float), 256) +
         gemm_ws;
}

// Enough for each of Q4_0, Q4_1 and Q8_0.
WH_API size_t wh_ffn_workspace_bytes(size_t hidden, size_t n_ff, size_t m) {
  size_t need = 0;
  for (int type : {WH_TYPE_Q4_0, WH_TYPE_Q4_1, WH_TYPE_Q8_0}) {
    const size_t b = wh_ffn_workspace_bytes_for_type(type, hidden, n_ff, m);
    if (b > need) need = b;
  }
  return need;
}

WH_API int wh_ffn_swiglu(const wh_ffn_weights* w, const float* gamma, float eps, const float* x,
                         size_t m, float* out, void* workspace, size_t workspace_bytes,
                         wh_stream_t stream) {
  if (!w) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "ffn_swiglu: null weights");
  int st = check_gemv_args("ffn_swiglu", w->type, w->hidden);
  if (st) return st;
  st = check_gemv_args("ffn_swiglu", w->type, w->n_ff);
  if (st) return st;
  if (m == 0 || w->hidden == 0) return WH_OK;
  const size_t need = wh_ffn_workspace_bytes_for_type(w->type, w->hidden, w->n_ff, m);
  if (workspace_bytes < need)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "ffn_swiglu: workspace too small: needed %zu bytes, available %zu", need,
                         workspace_bytes);
  if ((st = check_ptr("ffn_swiglu", "gate", w->gate, 1)) || (st = check_ptr("ffn_swiglu", "up", w->up, 1)) ||
      (st = check_ptr("ffn_swiglu", "down", w->down, 1)) ||
      (st = check_ptr("ffn_swiglu", "gamma", gamma, 4)) || (st = check_ptr("ffn_swiglu", "x", x, 4)) ||
      (st = check_ptr("ffn_swiglu", "out", out, 4)) ||
      (st = check_ptr("ffn_swiglu", "workspace", workspace, 256)))
    return st;
  const size_t H = w->hidden, F = w->n_ff;
  char* ws = static_cast<char*>(workspace);
  float* xh = reinterpret_cast<float*>(ws);
  ws += align_up(m * H * sizeof(float), 256);
  float* g = reinterpret_cast<float*>(ws);
  ws += align_up(m * F * sizeof(float), 256);
  float* u = reinterpret_cast<float*>(ws);
  ws += align_up(m * F * sizeof(float), 256);
  float* h = reinterpret_cast<float*>(ws);
  ws += align_up(m * F * sizeof(float), 256);
  void* gemm_ws = ws;
  const size_t gemm_bytes = need - static_cast<size_t>(ws - static_cast<char*>(workspace));
  hipStream_t s = hs(stream);
  if (F == 0) return wh::launch_fill_bytes(out, 0, m * H * sizeof(float), s);
  if (m >= 2 && m <= 16 && wh::mt_allowed(F, H)) {
    // a few tokens: RMSNorm, gate, up and SwiGLU for all of them in one pass
    // of the gate / up weights, then the down projection
    const void* gu[2] = {w->gate, w->up};
    st = wh::launch_gemv_mt(w->type, gu, true, x, m, gamma, eps, h, F, F, H, s);
    if (st == WH_OK) return wh::launch_gemm(w->type, w->down, H, F, h, m, out, gemm_ws, gemm_bytes, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  if (m <= wh::kGemvTokenLimit) {
    // decode: RMSNorm, gate, up and SwiGLU in one streaming kernel per token,
    // then the down GEMV; the unfused sequence below when the layout does not fit
    bool fused = true;
    for (size_t t = 0; t < m && fused; t++) {
      st = wh::launch_ffn_gate_up(w->type, w->gate, w->up, x + t * H, gamma, eps, h + t * F, F, H, s);
      if (st == WH_ERR_INVALID_SHAPE) fused = false;
      else if (st) return st;
    }
    if (fused) return wh::launch_gemm(w->type, w->down, H, F, h, m, out, gemm_ws, gemm_bytes, s);
  }
  if (m > wh::kGemvTokenLimit) {
    // prefill: the tiled MFMA kernel with RMSNorm and SwiGLU in its packing
    st = wh::launch_ffn_tiled(w->type, w->gate, w->up, w->down, H, F, x, gamma, eps, m, g, u, out, gemm_ws,
                              gemm_bytes, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  if ((st = wh::launch_rms_norm(x, gamma, eps, m, H, xh, s))) return st;
  if ((st = wh::launch_gemm(w->type, w->gate, F, H, xh, m, g, gemm_ws, gemm_bytes, s))) return st;
  if ((st = wh::launch_gemm(w->type, w->up, F, H, xh, m, u, gemm_ws, gemm_bytes, s))) return st;
  if ((st = wh::launch_swiglu(g, u, m * F, h, s))) return st;
  return wh::launch_gemm(w->type, w->down, H, F, h, m, out, gemm_ws, gemm_bytes, s);
}

// ------------------------------------------------------------ weight handles
WH_API int wh_weight_upload(int type, size_t n_rows, size_t k, const void* host_bytes,
                            size_t nbytes, wh_weight** out) {
  if (!out) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "weight_upload: null output");
  *out = nullptr;
  size_t need;
  if (type == WH_TYPE_F32 || type == WH_TYPE_F16) {
    // plain tensors (norm weights, f16 embeddings): n_rows x k elements
    const size_t es = wh::type_size(type);
    if (k != 0 && (n_rows > SIZE_MAX / k || n_rows * k > SIZE_MAX / es))
      return wh::set_error(WH_ERR_INVALID_SHAPE, "weight_upload: %zu x %zu tensor size overflows", n_rows, k);
    need = n_rows * k * es;
    if (nbytes < need)
      return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                           "weight_upload: buffer too small: needed %zu bytes, available %zu", need, nbytes);
  } else {
    int st = check_gemv_args("weight_upload", type, k);
    if (st) return st;
    st = check_weight_bytes("weight_upload", type, n_rows, k, nbytes);
    if (st) return st;
    need = n_rows * (k / wh::block_elems(type)) * wh::type_size(type);
  }
  if (need > 0 && !host_bytes)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "weight_upload: null host bytes");
  wh_weight* wt = new (std::nothrow) wh_weight();
  if (!wt) return wh::set_error(WH_ERR_OOM, "weight_upload: host allocation failed");
  wt->type = type;
  wt->n_rows = n_rows;
  wt->k = k;
  wt->nbytes = need;
  wt->data = nullptr;
  if (hipGetDevice(&wt->device) != hipSuccess) wt->device = -1;
  if (need > 0) {
    hipError_t e = hipMalloc(&wt->data, need);
    if (e != hipSuccess) {
      delete wt;
      return wh::hip_error(e, "weight_upload: hipMalloc");
    }
    e = hipMemcpy(wt->data, host_bytes, need, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(wt->data);
      delete wt;
      return wh::hip_error(e, "weight_upload: hipMemcpy");
    }
  }
  *out = wt;
  return WH_OK;
}

WH_API int wh_weight_prepare_prefill(wh_weight* weight, wh_stream_t stream, size_t* prepared_bytes) {
  if (!weight) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "weight_prepare_prefill: null handle");
  if (prepared_bytes) *prepared_bytes = weight->prefill_bytes;
  if (!wh::is_kquant(weight->type) || weight->prefill || weight->n_rows == 0 || weight->k == 0) return WH_OK;
  if (!wh::aligned(weight->data, 16))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "weight_prepare_prefill: data is not 16-byte aligned");
  const size_t bytes = wh::kquant_repacked_bytes(weight->type, weight->n_rows, weight->k);
  void* copy = nullptr;
  WH_HIP_TRY(hipMalloc(&copy, bytes));
  const int st = wh::launch_repack_kquant(weight->type, weight->data, weight->n_rows, weight->k, copy, hs(stream));
  if (st) {
    (void)hipFree(copy);
    return st;
  }
  weight->prefill = copy;
  weight->prefill_bytes = bytes;
  {
    PreparedRegistry& r = prepared_registry();
    std::lock_guard<std::mutex> lk(r.mu);
    r.by_data[weight->data] = weight;
  }
  if (prepared_bytes) *prepared_bytes = bytes;
  return WH_OK;
}

WH_API int wh_weight_free(wh_weight* weight) {
  if (!weight) return WH_OK;
  if (weight->prefill) {
    {
      PreparedRegistry& r = prepared_registry();
      std::lock_guard<std::mutex> lk(r.mu);
      r.by_data.erase(weight->data);
    }
    (void)hipFree(weight->prefill);
    weight->prefill = nullptr;
  }
  if (weight->data) {
    const hipError_t e = hipFree(weight->data);
    delete weight;
    if (e != hipSuccess) return wh::hip_error(e, "weight_free: hipFree");
    return WH_OK;
  }
  delete weight;
  return WH_OK;
}

WH_API const void* wh_weight_data(const wh_weight* weight) { return weight ? weight->data : nullptr; }

WH_API int wh_weight_info(const wh_weight* weight, int* type, size_t* n_rows, size_t* k,
                          size_t* nbytes) {
  if (!weight) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "weight_info: null handle");
  if (type) *type = weight->type;
  if (n_rows) *n_rows = weight->n_rows;
  if (k) *k = weight->k;
  if (nbytes) *nbytes = weight->nbytes;
  return WH_OK;
}

}  // extern "C"

// -------------------------------------------------- synchronous host variants
namespace {
// One device copy of host block bytes; freed with the last reference.
struct DevBlocks {
  void* dev = nullptr;
  size_t nbytes = 0;
  DevBlocks() = default;
  DevBlocks(const DevBlocks&) = delete;
  DevBlocks& operator=(const DevBlocks&) = delete;
  ~DevBlocks() {
    if (dev) (void)hipFree(dev);
  }
};

// A pooled device buffer of at least `cap` bytes for a call's activations and outputs.
struct PoolBuf {
  int dev = -1;
  size_t cap = 0;
  void* p = nullptr;
};

// The host-weight cache (wh_host_cache_*): entries keyed by (device, host
// address, byte count) with a last-use tick for LRU eviction, and a per-device
// pool of small buffers.  Allocated once and never destroyed, so no hipFree
// runs while the HIP runtime shuts down at process exit.
struct HostCache {
  struct Key {
    int dev;
    uintptr_t host;
    size_t nbytes;
    bool operator<(const Key& o) const {
      if (dev != o.dev) return dev < o.dev;
      if (host != o.host) return host < o.host;
      return nbytes < o.nbytes;
    }
  };
  struct Slot {
    std::shared_ptr<DevBlocks> blocks;
    uint64_t last_use;
  };
  std::mutex mu;
  std::map<Key, Slot> entries;
  std::vector<PoolBuf> pool;
  size_t max_bytes = 0, bytes = 0;
  uint64_t hits = 0, misses = 0, evictions = 0, tick = 0;

  // drops entries, least recently used first, until the budget holds (mu held)
  void trim() {
    while (bytes > max_bytes && !entries.empty()) {
      auto lru = entries.begin();
      for (auto it = entries.begin(); it != entries.end(); ++it)
        if (it->second.last_use < lru->second.last_use) lru = it;
      bytes -= lru->second.blocks->nbytes;
      entries.erase(lru);
      evictions++;
    }
  }
};

HostCache& host_cache() {
  static HostCache* c = new HostCache();
  return *c;
}

// Uploads `nbytes` of host blocks into a fresh device buffer.
int upload_blocks(const void* host, size_t nbytes, std::shared_ptr<DevBlocks>* out) {
  auto b = std::make_shared<DevBlocks>();
  WH_HIP_TRY(hipMalloc(&b->dev, nbytes));
  b->nbytes = nbytes;
  WH_HIP_TRY(hipMemcpy(b->dev, host, nbytes, hipMemcpyHostToDevice));
  *out = std::move(b);
  return WH_OK;
}

// The device copy of a call's block input: from the cache when it is on,
// otherwise (or when the input exceeds the budget) a copy owned by the call.
int blocks_on_device(const void* host, size_t nbytes, std::shared_ptr<DevBlocks>* out) {
  int dev = 0;
  WH_HIP_TRY(hipGetDevice(&dev));
  HostCache& c = host_cache();
  const HostCache::Key key{dev, reinterpret_cast<uintptr_t>(host), nbytes};
  {
    std::lock_guard<std::mutex> lk(c.mu);
    if (c.max_bytes > 0) {
      auto it = c.entries.find(key);
      if (it != c.entries.end()) {
        it->second.last_use = ++c.tick;
        c.hits++;
        *out = it->second.blocks;
        return WH_OK;
      }
    }
    c.misses++;
    if (c.max_bytes == 0 || nbytes > c.max_bytes) {
      // uncached: the call owns the copy
      return upload_blocks(host, nbytes, out);
    }
  }
  // upload outside the lock; a concurrent call for the same key may have
  // inserted meanwhile, and then its copy is used
  std::shared_ptr<DevBlocks> b;
  int st = upload_blocks(host, nbytes, &b);
  if (st) return st;
  std::lock_guard<std::mutex> lk(c.mu);
  if (c.max_bytes == 0 || nbytes > c.max_bytes) {  // reconfigured during the upload
    *out = std::move(b);
    return WH_OK;
  }
  auto ins = c.entries.emplace(key, HostCache::Slot{b, ++c.tick});
  if (ins.second) {
    c.bytes += nbytes;
    c.trim();
  } else {
    ins.first->second.last_use = c.tick;
  }
  *out = ins.first->second.blocks;
  return WH_OK;
}

// A pooled buffer of at least `bytes` on the current device (returned with pool_put).
int pool_get(size_t bytes, PoolBuf* out) {
  int dev = 0;
  WH_HIP_TRY(hipGetDevice(&dev));
  HostCache& c = host_cache();
  {
    std::lock_guard<std::mutex> lk(c.mu);
    for (size_t i = 0; i < c.pool.size(); i++) {
      if (c.pool[i].dev == dev && c.pool[i].cap >= bytes) {
        *out = c.pool[i];
        c.pool.erase(c.pool.begin() + static_cast<std::ptrdiff_t>(i));
        return WH_OK;
      }
    }
  }
  PoolBuf b;
  b.dev = dev;
  b.cap = align_up(bytes < 4096 ? 4096 : bytes, 4096);
  WH_HIP_TRY(hipMalloc(&b.p, b.cap));
  *out = b;
  return WH_OK;
}

// Returns a buffer to the pool while the cache is on, frees it otherwise.
void pool_put(PoolBuf& b) {
  if (!b.p) return;
  HostCache& c = host_cache();
  {
    std::lock_guard<std::mutex> lk(c.mu);
    if (c.max_bytes > 0 && c.pool.size() < 64) {
      c.pool.push_back(b);
      b.p = nullptr;
      return;
    }
  }
  (void)hipFree(b.p);
  b.p = nullptr;
}

// A pooled buffer that goes back to the pool (or is freed) when the call returns.
struct ScopedPoolBuf {
  PoolBuf b;
  ~ScopedPoolBuf() { pool_put(b); }
};
}  // namespace

extern "C" {

WH_API int wh_host_cache_configure(size_t max_bytes) {
  HostCache& c = host_cache();
  std::vector<PoolBuf> freed;
  {
    std::lock_guard<std::mutex> lk(c.mu);
    c.max_bytes = max_bytes;
    c.trim();
    if (max_bytes == 0) freed.swap(c.pool);
  }
  for (PoolBuf& b : freed) (void)hipFree(b.p);
  return WH_OK;
}

WH_API int wh_host_cache_evict(const void* host_ptr, size_t nbytes, size_t* evicted) {
  HostCache& c = host_cache();
  const uintptr_t lo = reinterpret_cast<uintptr_t>(host_ptr);
  size_t n = 0;
  {
    std::lock_guard<std::mutex> lk(c.mu);
    for (auto it = c.entries.begin(); it != c.entries.end();) {
      const uintptr_t elo = it->first.host, ehi = elo + it->first.nbytes;
      const bool hit = nbytes == 0 ? elo == lo : (elo < lo + nbytes && lo < ehi);
      if (hit) {
        c.bytes -= it->second.blocks->nbytes;
        it = c.entries.erase(it);
        n++;
      } else {
        ++it;
      }
    }
    c.evictions += n;
  }
  if (evicted) *evicted = n;
  return WH_OK;
}

WH_API int wh_host_cache_clear(void) {
  HostCache& c = host_cache();
  std::vector<PoolBuf> freed;
  {
    std::lock_guard<std::mutex> lk(c.mu);
    c.evictions += c.entries.size();
    c.entries.clear();
    c.bytes = 0;
    freed.swap(c.pool);
  }
  for (PoolBuf& b : freed) (void)hipFree(b.p);
  return WH_OK;
}

WH_API int wh_host_cache_get_stats(wh_host_cache_stats* out) {
  if (!out) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "wh_host_cache_get_stats: null output");
  HostCache& c = host_cache();
  std::lock_guard<std::mutex> lk(c.mu);
  out->hits = c.hits;
  out->misses = c.misses;
  out->evictions = c.evictions;
  out->entries = c.entries.size();
  out->bytes = c.bytes;
  out->max_bytes = c.max_bytes;
  return WH_OK;
}

WH_API int wh_dequantize_host(int type, const void* data, size_t nbytes, size_t nelements, float* out) {
  const size_t ts = wh::type_size(type);
  if (ts == 0)
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "dequantize: invalid tensor type %d", type);
  // Validate first with a null stream call that performs no work on failure.
  if (nelements == 0) return wh_dequantize(type, data, nbytes, 0, out, nullptr);
  if (!data || !out) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "dequantize_host: null pointer");
  const size_t in_bytes =
      (type == WH_TYPE_F32 || type == WH_TYPE_F16)
          ? nelements * ts
          : (nelements / wh::block_elems(type) + (nelements % wh::block_elems(type) != 0)) * ts;
  if (nbytes < in_bytes || ((type == WH_TYPE_F32 || type == WH_TYPE_F16) && nbytes != in_bytes))
    return wh_dequantize(type, data, nbytes, nelements, out, nullptr);
  std::shared_ptr<DevBlocks> din;
  int st = blocks_on_device(data, in_bytes, &din);
  if (st) return st;
  ScopedPoolBuf dout;
  if ((st = pool_get(nelements * sizeof(float), &dout.b))) return st;
  st = wh_dequantize(type, din->dev, in_bytes, nelements, static_cast<float*>(dout.b.p), nullptr);
  if (st) return st;
  WH_HIP_TRY(hipMemcpy(out, dout.b.p, nelements * sizeof(float), hipMemcpyDeviceToHost));
  return WH_OK;
}

WH_API int wh_quantized_matvec_host(int type, const void* weights, size_t weight_nbytes,
                                    const float* input, float* output, size_t m, size_t k) {
  int st = check_gemv_args("quantized_matvec", type, k);
  if (st) return st;
  st = check_weight_bytes("quantized_matvec", type, m, k, weight_nbytes);
  if (st) return st;
  if (m == 0) return WH_OK;
  if (!output || (k > 0 && (!weights || !input)))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "quantized_matvec_host: null pointer");
  const size_t wbytes = m * (k / wh::block_elems(type)) * wh::type_size(type);
  std::shared_ptr<DevBlocks> dw;
  if (wbytes && (st = blocks_on_device(weights, wbytes, &dw))) return st;
  // x and y in one pooled buffer: x at 0, y at the next 256-byte boundary
  const size_t xoff = align_up(k * sizeof(float), 256);
  ScopedPoolBuf io;
  if ((st = pool_get(xoff + m * sizeof(float), &io.b))) return st;
  float* dx = static_cast<float*>(io.b.p);
  float* dy = reinterpret_cast<float*>(static_cast<char*>(io.b.p) + xoff);
  if (k) WH_HIP_TRY(hipMemcpy(dx, input, k * sizeof(float), hipMemcpyHostToDevice));
  st = wh_quantized_matvec(type, dw ? dw->dev : nullptr, wbytes, dx, dy, m, k, nullptr);
  if (st) return st;
  WH_HIP_TRY(hipMemcpy(output, dy, m * sizeof(float), hipMemcpyDeviceToHost));
  return WH_OK;
}

}  // extern "C"
