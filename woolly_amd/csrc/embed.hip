// embed.hip -- token-embedding rows on the device: out[t, :] = the dequantized
// row ids[t] of a [vocab][hidden] table (GGUF token_embd.weight, dims
// [hidden, vocab] with hidden fastest), for the first step of
// LazyTransformer::forward (crates/woolly-core/src/model/lazy_transformer.rs:1155-1230,
// embedding_lookup in crates/woolly-core/src/tensor_utils.rs:548-590).
//
// The ids live in device memory, so a decode step captured into a HIP graph
// reads whatever token the caller (or a sampler on the device) wrote there
// before each replay.  Rows decode with the same per-quad functions as
// wh_dequantize, so a row is bit-identical to dequantizing the table and
// slicing it.  An id >= vocab, which the reference rejects with
// TENSOR_EMBEDDING_TOKEN_OUT_OF_RANGE, cannot raise an error from inside a
// kernel: its row is written as NaN so that the failure propagates visibly.
#include "wh_blocks.hpp"

namespace {

constexpr int kEmbThreads = 256;

// grid: (ceil(hidden / 4 / 256), n_tokens); thread q of row t writes elements
// 4q .. 4q + 3 of output row t.
template <int TYPE>
__global__ __launch_bounds__(kEmbThreads) void embed_rows_kernel(const uint8_t* __restrict__ table, uint32_t vocab,
                                                                 uint32_t hidden, const uint32_t* __restrict__ ids,
                                                                 float* __restrict__ out) {
  const uint32_t t = blockIdx.y;
  const uint32_t q = blockIdx.x * kEmbThreads + threadIdx.x;
  if (4 * q >= hidden) return;
  const uint32_t id = ids[t];
  float v[4];
  if (id >= vocab) {
    v[0] = v[1] = v[2] = v[3] = __builtin_nanf("");
  } else if constexpr (TYPE == WH_TYPE_F32) {
    const float* row = reinterpret_cast<const float*>(table) + static_cast<size_t>(id) * hidden;
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = row[4 * q + i];
  } else if constexpr (TYPE == WH_TYPE_F16) {
    const uint16_t* row = reinterpret_cast<const uint16_t*>(table) + static_cast<size_t>(id) * hidden;
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = whd::f16_bits_to_f32(row[4 * q + i]);
  } else if constexpr (TYPE == WH_TYPE_Q4_K || TYPE == WH_TYPE_Q6_K) {
    constexpr uint32_t TS = TYPE == WH_TYPE_Q4_K ? 144 : 210;
    const uint8_t* row = table + static_cast<size_t>(id) * (hidden / 256) * TS;
    whd::kq_quad<TYPE>(row + (q >> 6) * TS, static_cast<int>(q & 63), v);
  } else {
    constexpr uint32_t TS = whd::BlockFmt<TYPE>::BYTES;  // Q4_0, Q4_1, Q5_0, Q5_1, Q8_0
    const uint8_t* row = table + static_cast<size_t>(id) * (hidden / 32) * TS;
    whd::decode_quad<TYPE, 2>(row + (q >> 3) * TS, static_cast<int>(q & 7), v);
  }
  *reinterpret_cast<float4*>(out + static_cast<size_t>(t) * hidden + 4 * q) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int TYPE>
int launch_typed(const void* table, size_t vocab, size_t hidden, const uint32_t* ids, size_t n_tokens, float* out,
                 hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((hidden / 4 + kEmbThreads - 1) / kEmbThreads), static_cast<unsigned>(n_tokens));
  embed_rows_kernel<TYPE><<<grid, kEmbThreads, 0, s>>>(static_cast<const uint8_t*>(table),
                                                       static_cast<uint32_t>(vocab), static_cast<uint32_t>(hidden),
                                                       ids, out);
  WH_LAUNCH_CHECK("embedding lookup kernel launch");
  return WH_OK;
}

}  // namespace

namespace wh {

int launch_embedding_lookup(int type, const void* table, size_t vocab, size_t hidden, const uint32_t* ids,
                            size_t n_tokens, float* out, hipStream_t s) {
  switch (type) {
    case WH_TYPE_F32: return launch_typed<WH_TYPE_F32>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_F16: return launch_typed<WH_TYPE_F16>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q4_0: return launch_typed<WH_TYPE_Q4_0>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q4_1: return launch_typed<WH_TYPE_Q4_1>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q5_0: return launch_typed<WH_TYPE_Q5_0>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q5_1: return launch_typed<WH_TYPE_Q5_1>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q8_0: return launch_typed<WH_TYPE_Q8_0>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q4_K: return launch_typed<WH_TYPE_Q4_K>(table, vocab, hidden, ids, n_tokens, out, s);
    case WH_TYPE_Q6_K: return launch_typed<WH_TYPE_Q6_K>(table, vocab, hidden, ids, n_tokens, out, s);
    default:
      return set_error(WH_ERR_UNSUPPORTED_TYPE, "embedding_lookup: unsupported tensor type %d", type);
  }
}

// Checks of wh_embedding_lookup's arguments (shared with the decode entry
// point that starts from a token id).
int check_embedding_args(const char* fn, int type, const void* table, size_t vocab, size_t hidden,
                         const uint32_t* ids, float* out) {
  const size_t be = block_elems(type);
  if (be == 0)
    return set_error(WH_ERR_UNSUPPORTED_TYPE, "%s: unsupported tensor type %d", fn, type);
  if (hidden == 0 || hidden % 4 != 0 || hidden % be != 0)
    return set_error(WH_ERR_INVALID_SHAPE, "%s: hidden = %zu must be a multiple of 4 and of the block size %zu", fn,
                     hidden, be);
  if (vocab == 0 || vocab >= (static_cast<size_t>(1) << 32))
    return set_error(WH_ERR_INVALID_SHAPE, "%s: vocab = %zu out of range", fn, vocab);
  if (!table || !ids || !out) return set_error(WH_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned(out, 16) || !aligned(ids, 4) || !aligned(table, type == WH_TYPE_F32 ? 4 : 2))
    return set_error(WH_ERR_INVALID_ARGUMENT, "%s: out must be 16-byte, ids 4-byte and the table %d-byte aligned",
                     fn, type == WH_TYPE_F32 ? 4 : 2);
  return WH_OK;
}

}  // namespace wh

WH_API int wh_embedding_lookup(int type, const void* table, size_t vocab, size_t hidden, const uint32_t* ids,
                               size_t n_tokens, float* out, wh_stream_t stream) {
  if (n_tokens == 0) return WH_OK;
  if (n_tokens > 65535)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "embedding_lookup: %zu tokens (at most 65535 per call)", n_tokens);
  const int st = wh::check_embedding_args("embedding_lookup", type, table, vocab, hidden, ids, out);
  if (st) return st;
  return wh::launch_embedding_lookup(type, table, vocab, hidden, ids, n_tokens, out,
                                     reinterpret_cast<hipStream_t>(stream));
}
