// dequant.hip -- bit-exact GGUF block dequantization on gfx950.
//
// Semantics (crates/woolly-tensor/src/quantization.rs:466-590 and
// crates/woolly-gguf/src/dequantize.rs:286-378, 553-586):
//   Q4_0  {f16 d; u8 qs[16]}        e[j] = ((qs[j] & 15) - 8) * d, e[j+16] = ((qs[j] >> 4) - 8) * d
//   Q4_1  {f16 d; f16 m; u8 qs[16]} e[j] = (qs[j] & 15) * d + m,   e[j+16] = (qs[j] >> 4) * d + m
//   Q8_0  {f16 d; i8 qs[32]}        e[j] = qs[j] * d
//   Q5_0  {f16 d; u8 qh[4]; u8 qs[16]}        x = nibble | (bit e of qh) << 4, e = (x - 16) * d
//   Q5_1  {f16 d; f16 m; u8 qh[4]; u8 qs[16]} e = x * d + m  (quantization.rs:515-575)
// Every product is exact in f32 (a <=8-bit integer times an 11-bit
// significand), so the results are bit-identical to the CPU whatever the
// rounding of the single Q4_1 / Q5_1 addition (fused or not, it is one rounding).
//
// Work mapping: the output dominates the traffic (128 B written per 18-34 B
// read), so each thread produces one quad of 4 consecutive floats with one
// 128-bit store; a wavefront writes 1 KiB contiguously.  Eight threads share
// a block and read its scale and 4 quant bytes with 16-bit loads (blocks are
// only 2-byte aligned in the stream); the repeated scale reads hit L1.
#include "wh_blocks.hpp"

namespace {

template <int TYPE, int ALIGN, bool OUT16>
__global__ __launch_bounds__(256) void dequant_blocks_kernel(const uint8_t* __restrict__ data,
                                                             float* __restrict__ out,
                                                             size_t nelements) {
  constexpr int TS = TYPE == WH_TYPE_Q4_0   ? 18
                     : TYPE == WH_TYPE_Q4_1 ? 20
                     : TYPE == WH_TYPE_Q5_0 ? 22
                     : TYPE == WH_TYPE_Q5_1 ? 24
                                            : 34;
  const size_t nquads = (nelements + 3) / 4;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t q = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < nquads;
       q += stride) {
    const size_t b = q >> 3;
    const int c = static_cast<int>(q & 7);
    float v[4];
    whd::decode_quad<TYPE, ALIGN>(data + b * TS, c, v);
    const size_t e = q * 4;
    if (OUT16 && e + 4 <= nelements) {
      *reinterpret_cast<float4*>(out + e) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (e + i < nelements) out[e + i] = v[i];
    }
  }
}

// F16 -> F32 widening and F32 copy (the non-block types woolly_gguf::dequantize accepts).
__global__ __launch_bounds__(256) void dequant_f16_kernel(const uint8_t* __restrict__ data,
                                                          float* __restrict__ out, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t h = static_cast<uint32_t>(data[2 * i]) | (static_cast<uint32_t>(data[2 * i + 1]) << 8);
    out[i] = whd::f16_bits_to_f32(h);
  }
}

__global__ __launch_bounds__(256) void dequant_f32_kernel(const uint8_t* __restrict__ data,
                                                          float* __restrict__ out, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint8_t* p = data + 4 * i;
    const uint32_t u = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
                       (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
    out[i] = __builtin_bit_cast(float, u);
  }
}

__global__ __launch_bounds__(256) void fill_bytes_kernel(uint8_t* __restrict__ dst, uint8_t value,
                                                         size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = value;
}

// bfloat16 -> f32: the 16 bits become the high half of the f32 (exact).
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ x, size_t n,
                                                          float* __restrict__ out) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = __builtin_bit_cast(float, static_cast<uint32_t>(x[i]) << 16);
}

unsigned grid_for(size_t items, unsigned per_block, unsigned cap) {
  size_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

template <int TYPE>
void launch_blocks(const uint8_t* data, size_t n, float* out, hipStream_t s, unsigned grid) {
  const bool o16 = wh::aligned(out, 16);
  const int a = wh::aligned(data, 4) ? 4 : (wh::aligned(data, 2) ? 2 : 1);
  if (a == 4) {
    if (o16) dequant_blocks_kernel<TYPE, 4, true><<<grid, 256, 0, s>>>(data, out, n);
    else dequant_blocks_kernel<TYPE, 4, false><<<grid, 256, 0, s>>>(data, out, n);
  } else if (a == 2) {
    if (o16) dequant_blocks_kernel<TYPE, 2, true><<<grid, 256, 0, s>>>(data, out, n);
    else dequant_blocks_kernel<TYPE, 2, false><<<grid, 256, 0, s>>>(data, out, n);
  } else {
    if (o16) dequant_blocks_kernel<TYPE, 1, true><<<grid, 256, 0, s>>>(data, out, n);
    else dequant_blocks_kernel<TYPE, 1, false><<<grid, 256, 0, s>>>(data, out, n);
  }
}

}  // namespace

namespace wh {

int launch_dequantize(int type, const void* data, size_t n, float* out, hipStream_t s) {
  if (n == 0) return WH_OK;
  const uint8_t* p = static_cast<const uint8_t*>(data);
  const unsigned cap = static_cast<unsigned>(cu_count()) * 8u;
  switch (type) {
    case WH_TYPE_F32:
      dequant_f32_kernel<<<grid_for(n, 256, cap), 256, 0, s>>>(p, out, n);
      break;
    case WH_TYPE_F16:
      dequant_f16_kernel<<<grid_for(n, 256, cap), 256, 0, s>>>(p, out, n);
      break;
    case WH_TYPE_Q4_0:
      launch_blocks<WH_TYPE_Q4_0>(p, n, out, s, grid_for((n + 3) / 4, 256, cap));
      break;
    case WH_TYPE_Q4_1:
      launch_blocks<WH_TYPE_Q4_1>(p, n, out, s, grid_for((n + 3) / 4, 256, cap));
      break;
    case WH_TYPE_Q8_0:
      launch_blocks<WH_TYPE_Q8_0>(p, n, out, s, grid_for((n + 3) / 4, 256, cap));
      break;
    case WH_TYPE_Q5_0:
      launch_blocks<WH_TYPE_Q5_0>(p, n, out, s, grid_for((n + 3) / 4, 256, cap));
      break;
    case WH_TYPE_Q5_1:
      launch_blocks<WH_TYPE_Q5_1>(p, n, out, s, grid_for((n + 3) / 4, 256, cap));
      break;
    case WH_TYPE_Q4_K:
    case WH_TYPE_Q6_K:
      return launch_dequantize_kquant(type, data, n, out, s);
    default:
      return set_error(WH_ERR_UNSUPPORTED_TYPE, "dequantize: unsupported type %d", type);
  }
  WH_LAUNCH_CHECK("dequantize kernel launch");
  return WH_OK;
}

int launch_bf16_to_f32(const uint16_t* x, size_t n, float* out, hipStream_t s) {
  if (n == 0) return WH_OK;
  const unsigned cap = static_cast<unsigned>(cu_count()) * 8u;
  bf16_to_f32_kernel<<<grid_for(n, 256, cap), 256, 0, s>>>(x, n, out);
  WH_LAUNCH_CHECK("bf16 conversion kernel launch");
  return WH_OK;
}

int launch_fill_bytes(void* dst, int value, size_t nbytes, hipStream_t s) {
  if (nbytes == 0) return WH_OK;
  const unsigned cap = static_cast<unsigned>(cu_count()) * 8u;
  fill_bytes_kernel<<<grid_for(nbytes, 256, cap), 256, 0, s>>>(static_cast<uint8_t*>(dst),
                                                               static_cast<uint8_t>(value), nbytes);
  WH_LAUNCH_CHECK("fill kernel launch");
  return WH_OK;
}

}  // namespace wh
