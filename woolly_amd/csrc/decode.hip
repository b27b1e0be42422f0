// decode.hip -- the single-token decode step: C ABI of the fused attention
// projections, the attention, the residual projections, one layer and the
// whole step (host code; the kernels live in gemv.hip and attention.hip).
//
// One layer for one token (LazyTransformer::process_layer,
// crates/woolly-core/src/model/lazy_transformer.rs:98-258) is six launches:
//   1. qkv = [Wq; Wk; Wv] rms_norm(x, attn_norm)      gemv, 3 stacked matrices + RMSNorm
//   2-3. attention partials + combine (RoPE, KV store) attention.hip
//   4. x = x + Wo attn                                gemv + residual
//   5. h = silu(Wg x_hat) (Wu x_hat), x_hat = rms_norm(x, ffn_norm)
//                                                     fused gate/up gemv
//   6. x = x + Wd h                                   gemv + residual
// and the step ends with logits = Wout rms_norm(x, output_norm) (gemv +
// RMSNorm).  Nothing here allocates or synchronises, so a caller can capture
// the step into a HIP graph.
#include <cmath>
#include <cstdio>
#include <mutex>

#include "wh_common.hpp"

namespace {

// Scratch of wh_llama_decode_step_noalloc: the step's workspace (q/k/v, the
// attention output and partials, the FFN hidden vector) for callers that
// cannot allocate.  One copy per device, held until the process ends; every
// call on a device shares it, so calls that overlap on one device race.  No
// kernel of the step needs any of it zeroed: each one writes what it reads
// later in the same step.  In host code `scratch` only names the symbol; the
// device address of each device's copy comes from hipGetSymbolAddress.
constexpr size_t kStepScratchBytes = WH_LLAMA_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kStepScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};

// The current device's copy of `scratch`, looked up once per device.
int step_scratch(void** out) {
  *out = nullptr;
  int dev = 0;
  WH_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices)
    return wh::set_error(WH_ERR_NO_DEVICE, "decode step scratch: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return wh::hip_error(e, "hipGetSymbolAddress(decode step scratch)");
    if (!p) return wh::set_error(WH_ERR_HIP, "hipGetSymbolAddress(decode step scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WH_OK;
}

hipStream_t hs(wh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

size_t al256(size_t v) { return (v + 255) / 256 * 256; }

// A matrix of `type` with rows of k elements: the 32-element formats, or the
// K-quants with k a multiple of 256.
int check_type(const char* fn, int type, size_t k) {
  if (!wh::is_block_type(type) && !wh::is_kquant(type))
    return wh::set_error(WH_ERR_UNSUPPORTED_TYPE,
                         "%s: unsupported quantization scheme (ggml type %d); supported: Q4_0 (2), Q4_1 (3), "
                         "Q8_0 (8), Q4_K (12), Q6_K (14)",
                         fn, type);
  const size_t be = wh::block_elems(type);
  if (k % be != 0)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: k = %zu is not a multiple of the block size %zu", fn, k, be);
  return WH_OK;
}

// The block types of a layer's matrices, q k v o gate up down (0: the model's type).
struct LayerTypes {
  int q, k, v, o, g, u, d;
};
LayerTypes layer_types(const wh_llama_model* m, const wh_llama_layer& L) {
  auto t = [&](int v) { return v ? v : m->type; };
  return {t(L.wq_type), t(L.wk_type), t(L.wv_type), t(L.wo_type), t(L.w_gate_type), t(L.w_up_type),
          t(L.w_down_type)};
}

// Fused GEMV with the RMSNorm done separately when the fused kernel does not
// take the shape: x_hat into `scratch` (k floats), then the same call without
// gamma.
int gemv_fused_or_split(int type, const void* const* mats, const size_t* rows, int n_mats, const float* x,
                        const float* gamma, float eps, const float* residual, float* y, size_t k, float* scratch,
                        hipStream_t s) {
  int st = wh::launch_gemv_fused(type, mats, rows, n_mats, x, gamma, eps, residual, y, k, s);
  if (st != WH_ERR_INVALID_SHAPE || !gamma) return st;
  if (!scratch) return wh::set_error(WH_ERR_BUFFER_TOO_SMALL, "fused gemv: workspace needed for this shape");
  st = wh::launch_rms_norm(x, gamma, eps, 1, k, scratch, s);
  if (st) return st;
  return wh::launch_gemv_fused(type, mats, rows, n_mats, scratch, nullptr, 0.f, residual, y, k, s);
}

// Workspace of the decode step (all offsets 256-byte aligned).
struct StepWs {
  float* qkv;     // (n_heads + 2 n_kv_heads) * head_dim
  float* attn;    // n_heads * head_dim
  float* h;       // n_ff
  float* u;       // n_ff (unfused FFN only)
  float* xn;      // hidden (RMSNorm scratch for shapes the fused kernels do not take)
  float* part;    // attention partials
  size_t bytes;
};

StepWs step_layout(const wh_llama_model* m, void* base) {
  StepWs w{};
  char* p = static_cast<char*>(base);
  size_t off = 0;
  const size_t qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
  auto take = [&](size_t bytes) {
    float* r = p ? reinterpret_cast<float*>(p + off) : nullptr;
    off += al256(bytes);
    return r;
  };
  w.qkv = take(4 * (qd + 2 * kvd));
  w.attn = take(4 * qd);
  w.h = take(4 * m->n_ff);
  w.u = take(4 * m->n_ff);
  w.xn = take(4 * (m->hidden > m->n_ff ? m->hidden : m->n_ff));
  w.part = take(wh::attention_workspace_bytes(m->n_heads, m->head_dim, m->max_ctx, m->n_kv_heads));
  w.bytes = off;
  return w;
}

int check_model(const char* fn, const wh_llama_model* m) {
  if (!m || !m->layers || !m->rope_inv_freq)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: null model, layers or rope_inv_freq", fn);
  if (m->hidden == 0 || m->hidden % 32 != 0 || m->n_ff % 32 != 0 || (m->n_heads * m->head_dim) % 32 != 0)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: hidden, n_ff and n_heads * head_dim must be multiples of 32",
                         fn);
  if (!wh::attention_shape_ok(m->n_heads, m->n_kv_heads, m->head_dim))
    return wh::set_error(WH_ERR_INVALID_SHAPE,
                         "%s: attention shape not supported (head_dim 64 or 128, n_heads a multiple of "
                         "n_kv_heads, at most 8 query heads per KV head)",
                         fn);
  if (m->max_ctx == 0) return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: max_ctx is 0", fn);
  for (size_t l = 0; l < m->n_layers; l++) {
    const wh_llama_layer& L = m->layers[l];
    if (!L.k_cache || !L.v_cache || !wh::aligned(L.k_cache, 16) || !wh::aligned(L.v_cache, 16))
      return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: layer %zu KV caches must be non-null and 16-byte aligned",
                           fn, l);
    const void* ptrs[9] = {L.attn_norm, L.wq, L.wk, L.wv, L.wo, L.ffn_norm, L.w_gate, L.w_up, L.w_down};
    static const char* const names[9] = {"attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down"};
    for (int i = 0; i < 9; i++)
      if (!ptrs[i]) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: layer %zu %s is a null pointer", fn, l, names[i]);
    if (!wh::aligned(L.attn_norm, 4) || !wh::aligned(L.ffn_norm, 4))
      return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: layer %zu norm weights must be 4-byte aligned", fn, l);
    const LayerTypes t = layer_types(m, L);
    const size_t qd = m->n_heads * m->head_dim;
    const int types[7] = {t.q, t.k, t.v, t.o, t.g, t.u, t.d};
    const size_t ks[7] = {m->hidden, m->hidden, m->hidden, qd, m->hidden, m->hidden, m->n_ff};
    for (int i = 0; i < 7; i++) {
      const int st = check_type(fn, types[i], ks[i]);
      if (st) return st;
    }
  }
  return WH_OK;
}

// The output head of a step that writes logits: its type, pointers and vocab.
int check_head(const char* fn, const wh_llama_model* m) {
  char what[96];
  std::snprintf(what, sizeof(what), "%s (output head)", fn);
  const int st = check_type(what, m->output_type, m->hidden);
  if (st) return st;
  if (!m->output || !m->output_norm)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: null output head or output_norm", fn);
  if (m->vocab == 0 || m->vocab >= (static_cast<size_t>(1) << 30))
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: vocab = %zu out of range", fn, m->vocab);
  return WH_OK;
}

// A status of INVALID_SHAPE from the kernels' layout checks, reported with the
// entry point's name when no kernel takes the model's shapes.
int shape_status(const char* fn, int st) {
  if (st != WH_ERR_INVALID_SHAPE) return st;
  char detail[256];
  std::snprintf(detail, sizeof(detail), "%s", wh_last_error());
  return wh::set_error(st, "%s: no kernel takes this layer shape (%s)", fn, detail);
}

int layer_step(const wh_llama_model* m, const wh_llama_layer& L, size_t pos, float* x, const StepWs& w,
               hipStream_t s) {
  const size_t D = m->head_dim, qd = m->n_heads * D, kvd = m->n_kv_heads * D;
  const LayerTypes t = layer_types(m, L);
  // 1. qkv: consecutive matrices of one type stacked into one GEMV with the
  // RMSNorm fused (all three for a single-type model; q + k, then v, for
  // Q4_K_M's Q6_K attn_v)
  int st = WH_OK;
  {
    const void* mats[3] = {L.wq, L.wk, L.wv};
    const size_t rows[3] = {qd, kvd, kvd};
    const int ty[3] = {t.q, t.k, t.v};
    // exactly two groups of different types (Q4_K_M): one launch when a kernel takes the pair
    int n0 = 1;
    while (n0 < 3 && ty[n0] == ty[0]) n0++;
    bool done = false;
    if (n0 < 3 && (n0 == 2 || ty[1] == ty[2])) {
      size_t off_b = 0;
      for (int j = 0; j < n0; j++) off_b += rows[j];
      st = wh::launch_gemv_mfma2(ty[0], mats, rows, n0, ty[n0], mats + n0, rows + n0, 3 - n0, x, L.attn_norm,
                                 m->eps, w.qkv, w.qkv + off_b, m->hidden, s);
      if (st == WH_OK) done = true;
      else if (st != WH_ERR_INVALID_SHAPE) return st;
      st = WH_OK;
    }
    size_t off = 0;
    for (int i = 0; i < 3 && !st && !done;) {
      int n = 1;
      while (i + n < 3 && ty[i + n] == ty[i]) n++;
      st = gemv_fused_or_split(ty[i], mats + i, rows + i, n, x, L.attn_norm, m->eps, nullptr, w.qkv + off, m->hidden,
                               w.xn, s);
      for (int j = 0; j < n; j++) off += rows[i + j];
      i += n;
    }
  }
  if (st) return st;
  // 2-3. attention
  st = wh::launch_attention_decode(w.qkv, L.k_cache, L.v_cache, pos, m->n_heads, m->n_kv_heads, D,
                                   m->rope_inv_freq, w.attn, w.part, s);
  if (st) return st;
  // 4. x += Wo attn
  const void* wo[1] = {L.wo};
  const size_t hr[1] = {m->hidden};
  st = wh::launch_gemv_fused(t.o, wo, hr, 1, w.attn, nullptr, 0.f, x, x, qd, s);
  if (st) return st;
  // 5. h = silu(gate) * up of rms_norm(x)
  st = t.g == t.u ? wh::launch_ffn_gate_up(t.g, L.w_gate, L.w_up, x, L.ffn_norm, m->eps, w.h, m->n_ff, m->hidden, s)
                  : WH_ERR_INVALID_SHAPE;
  if (st == WH_ERR_INVALID_SHAPE) {
    // unfused: rms_norm -> gate, up -> swiglu
    st = wh::launch_rms_norm(x, L.ffn_norm, m->eps, 1, m->hidden, w.xn, s);
    if (!st) st = wh::launch_gemv(t.g, L.w_gate, w.xn, w.h, m->n_ff, m->hidden, s);
    if (!st) st = wh::launch_gemv(t.u, L.w_up, w.xn, w.u, m->n_ff, m->hidden, s);
    if (!st) st = wh::launch_swiglu(w.h, w.u, m->n_ff, w.h, s);
  }
  if (st) return st;
  // 6. x += Wd h
  const void* wd[1] = {L.w_down};
  return wh::launch_gemv_fused(t.d, wd, hr, 1, w.h, nullptr, 0.f, x, x, m->n_ff, s);
}

}  // namespace

WH_API int wh_rope_inv_freq(float base, size_t head_dim, float* out_host) {
  if (!out_host) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "rope_inv_freq: null output");
  if (head_dim == 0 || head_dim % 2 != 0)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "rope_inv_freq: head_dim %zu must be even", head_dim);
  // ops/mod.rs:490-494, in f32: freqs[i] = 1.0 / base.powf(2.0 * i / head_dim)
  for (size_t i = 0; i < head_dim / 2; i++) {
    const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(head_dim);
    out_host[i] = 1.0f / powf(base, e);
  }
  return WH_OK;
}

WH_API size_t wh_attention_qkv_workspace_bytes(size_t hidden) { return 4 * hidden; }

WH_API int wh_attention_qkv(int type, const void* wq, const void* wk, const void* wv, size_t q_rows,
                            size_t kv_rows, size_t hidden, const float* gamma, float eps, const float* x,
                            float* qkv, void* workspace, size_t workspace_bytes, wh_stream_t stream) {
  int st = check_type("attention_qkv", type, hidden);
  if (st) return st;
  if (!wq || !wk || !wv || !gamma || !x || !qkv)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "attention_qkv: null pointer");
  if (q_rows + 2 * kv_rows == 0) return WH_OK;
  float* scratch = workspace_bytes >= 4 * hidden ? static_cast<float*>(workspace) : nullptr;
  const void* mats[3] = {wq, wk, wv};
  const size_t rows[3] = {q_rows, kv_rows, kv_rows};
  return gemv_fused_or_split(type, mats, rows, 3, x, gamma, eps, nullptr, qkv, hidden, scratch, hs(stream));
}

WH_API size_t wh_attention_workspace_bytes(size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_ctx) {
  return wh::attention_workspace_bytes(n_heads, head_dim, max_ctx, n_kv_heads);
}

WH_API int wh_attention_decode(const float* qkv, void* k_cache, void* v_cache, size_t pos, size_t n_heads,
                               size_t n_kv_heads, size_t head_dim, const float* inv_freq, float* out,
                               void* workspace, size_t workspace_bytes, wh_stream_t stream) {
  if (!qkv || !k_cache || !v_cache || !inv_freq || !out || !workspace)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "attention_decode: null pointer");
  if (!wh::attention_shape_ok(n_heads, n_kv_heads, head_dim))
    return wh::set_error(WH_ERR_INVALID_SHAPE,
                         "attention_decode: head_dim %zu, %zu heads, %zu KV heads not supported", head_dim,
                         n_heads, n_kv_heads);
  if (!wh::aligned(k_cache, 16) || !wh::aligned(v_cache, 16))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "attention_decode: caches must be 16-byte aligned");
  const size_t need = wh::attention_workspace_bytes(n_heads, head_dim, pos + 1, n_kv_heads);
  if (workspace_bytes < need)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "attention_decode: workspace too small: needed %zu bytes, available %zu", need,
                         workspace_bytes);
  return wh::launch_attention_decode(qkv, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim, inv_freq, out,
                                     workspace, hs(stream));
}

WH_API int wh_quantized_matvec_residual(int type, const void* weights, size_t weight_nbytes, const float* input,
                                        const float* residual, float* output, size_t m, size_t k,
                                        wh_stream_t stream) {
  int st = check_type("quantized_matvec_residual", type, k);
  if (st) return st;
  const size_t need = m * (k / wh::block_elems(type)) * wh::type_size(type);
  if (weight_nbytes < need)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "quantized_matvec_residual: buffer too small: needed %zu bytes, available %zu", need,
                         weight_nbytes);
  if (m == 0) return WH_OK;
  if (!weights || !input || !residual || !output)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "quantized_matvec_residual: null pointer");
  if (m >= (static_cast<size_t>(1) << 31))
    return wh::set_error(WH_ERR_INVALID_SHAPE, "quantized_matvec_residual: %zu rows exceed 2^31", m);
  const void* mats[1] = {weights};
  const size_t rows[1] = {m};
  return wh::launch_gemv_fused(type, mats, rows, 1, input, nullptr, 0.f, residual, output, k, hs(stream));
}

WH_API size_t wh_llama_decode_workspace_bytes(const wh_llama_model* model) {
  if (!model) return 0;
  return step_layout(model, nullptr).bytes;
}

WH_API int wh_llama_layer_decode(const wh_llama_model* model, size_t layer, size_t pos, float* x, void* workspace,
                                 size_t workspace_bytes, wh_stream_t stream) {
  int st = check_model("llama_layer_decode", model);
  if (st) return st;
  if (layer >= model->n_layers)
    return wh::set_error(WH_ERR_INVALID_ARGUMENT, "llama_layer_decode: layer %zu of %zu", layer, model->n_layers);
  if (pos >= model->max_ctx)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "llama_layer_decode: position %zu beyond max_ctx %zu", pos,
                         model->max_ctx);
  const StepWs w = step_layout(model, workspace);
  if (!workspace || workspace_bytes < w.bytes)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "llama_layer_decode: workspace too small: needed %zu bytes, available %zu", w.bytes,
                         workspace ? workspace_bytes : static_cast<size_t>(0));
  if (!x) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "llama_layer_decode: null x");
  return shape_status("llama_layer_decode", layer_step(model, model->layers[layer], pos, x, w, hs(stream)));
}

namespace {

// Checks and launches of one step (x already holds the token's embedding).
// Every argument check runs before the first launch, so a call those checks
// reject changes neither x nor the caches.  A failure reported by a launch
// inside the layers (a HIP error, or a kernel layout rejected as
// INVALID_SHAPE) stops the step there: x and the earlier layers' cache rows
// at pos may then already be written.
int decode_step(const char* fn, const wh_llama_model* model, const uint32_t* token, size_t pos, float* x,
                float* logits, void* workspace, size_t workspace_bytes, hipStream_t s) {
  int st = check_model(fn, model);
  if (st) return st;
  if (pos >= model->max_ctx)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: position %zu beyond max_ctx %zu", fn, pos, model->max_ctx);
  const StepWs w = step_layout(model, workspace);
  if (!workspace || workspace_bytes < w.bytes)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL, "%s: workspace too small: needed %zu bytes, available %zu", fn,
                         w.bytes, workspace ? workspace_bytes : static_cast<size_t>(0));
  if (!x) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: null x", fn);
  if (logits && (st = check_head(fn, model))) return st;
  if (token) {
    if (!model->token_embd)
      return wh::set_error(WH_ERR_INVALID_ARGUMENT, "%s: the model has no token_embd table", fn);
    if ((st = wh::check_embedding_args(fn, model->token_embd_type, model->token_embd, model->vocab, model->hidden,
                                       token, x)))
      return st;
    if ((st = wh::launch_embedding_lookup(model->token_embd_type, model->token_embd, model->vocab, model->hidden,
                                          token, 1, x, s)))
      return st;
  }
  for (size_t l = 0; l < model->n_layers; l++) {
    st = layer_step(model, model->layers[l], pos, x, w, s);
    if (st) return shape_status(fn, st);
  }
  if (!logits) return WH_OK;
  const void* head[1] = {model->output};
  const size_t rows[1] = {model->vocab};
  return shape_status(fn, gemv_fused_or_split(model->output_type, head, rows, 1, x, model->output_norm, model->eps,
                                               nullptr, logits, model->hidden, w.xn, s));
}

}  // namespace

WH_API int wh_llama_decode_step(const wh_llama_model* model, size_t pos, float* x, float* logits, void* workspace,
                                size_t workspace_bytes, wh_stream_t stream) {
  return decode_step("llama_decode_step", model, nullptr, pos, x, logits, workspace, workspace_bytes, hs(stream));
}

WH_API int wh_llama_forward_token(const wh_llama_model* model, const uint32_t* token, size_t pos, float* x,
                                  float* logits, void* workspace, size_t workspace_bytes, wh_stream_t stream) {
  if (!token) return wh::set_error(WH_ERR_INVALID_ARGUMENT, "llama_forward_token: null token");
  return decode_step("llama_forward_token", model, token, pos, x, logits, workspace, workspace_bytes, hs(stream));
}

namespace wh {

// Called by wh_init with the device current: looks up the device's copy of
// the decode step's static scratch ahead of any call (and of any capture).
int init_step_scratch() {
  void* p = nullptr;
  return step_scratch(&p);
}

}  // namespace wh

WH_API int wh_llama_decode_step_noalloc(const wh_llama_model* model, size_t pos, float* x, float* logits,
                                        wh_stream_t stream) {
  static const char* const fn = "llama_decode_step_noalloc";
  int st = check_model(fn, model);
  if (st) return st;
  if (pos >= model->max_ctx)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "%s: position %zu beyond max_ctx %zu", fn, pos, model->max_ctx);
  // The step attends to positions 0..pos only, so its workspace is laid out
  // for pos + 1 positions (the attention partials come last, every other
  // offset is the same as for max_ctx).
  wh_llama_model sized = *model;
  sized.max_ctx = pos + 1;
  const size_t need = step_layout(&sized, nullptr).bytes;
  if (need > kStepScratchBytes)
    return wh::set_error(WH_ERR_BUFFER_TOO_SMALL,
                         "%s: the step at position %zu needs %zu bytes of scratch; the static scratch holds %zu "
                         "(wh_llama_decode_step takes a workspace of any size)",
                         fn, pos, need, kStepScratchBytes);
  void* ws = nullptr;
  if ((st = step_scratch(&ws))) return st;
  return decode_step(fn, &sized, nullptr, pos, x, logits, ws, need, hs(stream));
}
