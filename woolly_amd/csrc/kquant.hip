// kquant.hip -- the 256-element K-quant blocks (Q4_K, Q6_K) as woolly-gguf
// decodes them, on gfx950: bit-exact dequantization and a GEMV defined as that
// dequantization followed by the f32 dot product.
//
// Reference: woolly_gguf::dequantize (crates/woolly-gguf/src/dequantize.rs:189-205)
// with dequantize_q4_k_scalar (:404-458, the x86 path) and dequantize_q6_k
// (:460-536).  woolly reads these blocks its own way (not ggml's layout):
//   Q4_K (144 B): bytes 0..11 pack eight 6-bit scales, scale i from byte
//     src = 3i/2: even i -> b[src] & 63, odd i -> ((b[src] >> 6) |
//     ((b[src+1] & 15) << 2)) & 63; f16 d at 12..13, f16 dmin at 14..15,
//     quants at 16..143: element i is the low nibble of qs[i/2] for even i, the
//     high nibble for odd i; value d * scale[i/32] * q + dmin.
//   Q6_K (210 B): ql = 0..127, qh = 128..191, u8 scales = 192..207, f16 d at
//     208..209; element i takes 4 bits from ql[64(i/128) + 32((i%128)/64) +
//     16((i%64)/32) + i%16] (low nibble below 128, high nibble from 128 on) and
//     2 bits from qh[32(i/128) + 16((i%128)/64) + 8((i%64)/32) + (i%32)/4]
//     at shift 2((i%32)%4) (+2 for the upper half; at shift 6 that pair is the
//     low bits of the next qh byte, 0 past the last one); value
//     ((d * scale[i/16]) * (q - 32)) / 64.
// Every product and sum is rounded in the reference's order with unfused
// operations, so the results are bit-identical to the CPU.
#include "wh_blocks.hpp"

namespace {

using whd::b16;
using whd::kq_quad;
using whd::q4k_scale;
using whd::q6k_quant;

template <int TYPE>
constexpr int kq_bytes() { return TYPE == WH_TYPE_Q4_K ? 144 : 210; }

// One thread per quad of 4 consecutive outputs (64 quads per block), grid-stride.
template <int TYPE>
__global__ __launch_bounds__(256) void kq_dequant_kernel(const uint8_t* __restrict__ data, float* __restrict__ out,
                                                         size_t n) {
  const size_t nquads = (n + 3) / 4;
  for (size_t qd = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; qd < nquads;
       qd += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t blk = qd >> 6;
    const int c = static_cast<int>(qd & 63);
    float v[4];
    kq_quad<TYPE>(data + blk * kq_bytes<TYPE>(), c, v);
    const size_t e = 4 * qd;
    if (e + 4 <= n && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
      *reinterpret_cast<float4*>(out + e) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int t = 0; t < 4 && e + t < n; t++) out[e + t] = v[t];
    }
  }
}

// y[row] = sum_k dequant(W)[row, k] * x[k] (+ residual[row]): one wave per row
// (grid-stride), lane l takes quad l (elements 4l..4l+3) of every block of the
// row.  y may be the residual itself (each row is read, then written, by one lane).
template <int TYPE>
__global__ __launch_bounds__(256) void kq_gemv_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                      const float* residual, float* y, size_t n_rows, size_t nb) {
  const int lane = threadIdx.x & 63;
  const size_t waves = static_cast<size_t>(gridDim.x) * (blockDim.x >> 6);
  for (size_t row = static_cast<size_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6); row < n_rows;
       row += waves) {
    const uint8_t* rp = w + row * nb * kq_bytes<TYPE>();
    float acc = 0.f;
    for (size_t b = 0; b < nb; b++) {
      float v[4];
      kq_quad<TYPE>(rp + b * kq_bytes<TYPE>(), lane, v);
      const float* xb = x + 256 * b + 4 * lane;
#pragma unroll
      for (int t = 0; t < 4; t++) acc = __builtin_fmaf(v[t], xb[t], acc);
    }
    acc = whd::wave_sum(acc);
    if (lane == 0) y[row] = residual ? residual[row] + acc : acc;
  }
}

// ------------------------------------------------------ prefill repacking
// The tiled prefill GEMM takes 32-element blocks with one scale each, so a
// K-quant matrix is rewritten once per call (same row order, same element
// order within a row) into:
//   Q4_K -> {f32 d * scale_j; u8 qs[16]} per 32 elements j (quants in Q4_0's
//     nibble order: byte i holds element i low, element i + 16 high), and the
//     super-block's dmin (its fp16 bits) in an [n_rows][q4f_dmin_stride(k)]
//     table after the blocks, zero past the row's k / 256 super-blocks; the
//     value (d * scale_j) * q + dmin is then the GEMM's d * q plus dmin times
//     the super-block's activation sum;
//   Q6_K -> {f32 (d * scale_j) / 64; i8 q[16] = q - 32} per 16 elements j
//     (the GEMM pads each to a 32-element block, upper half zero).
// The scale products are exact in f32 (11-bit times 6- or 8-bit integers).
// Every thread writes one output block; 16-byte aligned input.
__global__ __launch_bounds__(256) void kq_repack_q4k_kernel(const uint8_t* __restrict__ w, size_t n_groups,
                                                            size_t groups_per_row, size_t n_rows,
                                                            uint32_t* __restrict__ out, uint16_t* __restrict__ dmin_t,
                                                            size_t dmin_stride) {
  for (size_t gi = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; gi < n_groups;
       gi += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint8_t* b = w + (gi >> 3) * 144;
    const int j = static_cast<int>(gi & 7);
    const float d = whd::f16_bits_to_f32(b16(b + 12));
    const uint4 q = *reinterpret_cast<const uint4*>(b + 16 + 16 * j);  // elements 32j .. 32j + 31
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[5];
    o[0] = __float_as_uint(__fmul_rn(d, static_cast<float>(q4k_scale(b, j))));
    // element e is nibble e & 1 of byte e >> 1; output byte 2m = lo(byte m) |
    // lo(byte m + 8) << 4, byte 2m + 1 = hi(byte m) | hi(byte m + 8) << 4
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t v = 0;
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int m = 2 * c + t;
        const uint32_t lo = (qw[m >> 2] >> (8 * (m & 3))) & 0xFFu;
        const uint32_t hi = (qw[(m + 8) >> 2] >> (8 * ((m + 8) & 3))) & 0xFFu;
        const uint32_t b0 = (lo & 15u) | ((hi & 15u) << 4);
        const uint32_t b1 = (lo >> 4) | (hi & 0xF0u);
        v |= (b0 | (b1 << 8)) << (16 * t);
      }
      o[1 + c] = v;
    }
    uint32_t* dst = out + gi * 5;
#pragma unroll
    for (int c = 0; c < 5; c++) dst[c] = o[c];
    if (j == 0) {
      const size_t row = gi / groups_per_row, sb = (gi % groups_per_row) >> 3, nsb = groups_per_row >> 3;
      uint16_t* tr = dmin_t + row * dmin_stride;
      tr[sb] = b16(b + 14);
      if (sb + 1 == nsb)  // the row's last super-block clears the padding
        for (size_t z = nsb; z < dmin_stride; z++) tr[z] = 0;
    }
  }
}

// Q6_K: a workgroup stages 32 consecutive blocks (6720 B, a 16-byte aligned
// run) in LDS with coalesced 16-byte loads, then each thread rewrites halves.
constexpr int kQ6Blocks = 32;
__global__ __launch_bounds__(256) void kq_repack_q6k_kernel(const uint8_t* __restrict__ w, size_t n_blocks,
                                                            uint32_t* __restrict__ out) {
  __shared__ uint4 stage[kQ6Blocks * 210 / 16];
  uint8_t* sb = reinterpret_cast<uint8_t*>(stage);
  for (size_t b0 = static_cast<size_t>(blockIdx.x) * kQ6Blocks; b0 < n_blocks;
       b0 += static_cast<size_t>(gridDim.x) * kQ6Blocks) {
    const int nblk = static_cast<int>(n_blocks - b0 < kQ6Blocks ? n_blocks - b0 : kQ6Blocks);
    const int bytes = nblk * 210;
    const uint8_t* src = w + b0 * 210;
    for (int i = threadIdx.x; i < bytes / 16; i += blockDim.x) stage[i] = reinterpret_cast<const uint4*>(src)[i];
    for (int i = bytes / 16 * 16 + threadIdx.x; i < bytes; i += blockDim.x) sb[i] = src[i];
    __syncthreads();
    for (int h = threadIdx.x; h < nblk * 16; h += blockDim.x) {
      const uint8_t* b = sb + (h >> 4) * 210;
      const int j = h & 15;
      const float d = whd::f16_bits_to_f32(b16(b + 208));
      uint32_t o[5];
      o[0] = __float_as_uint(__fmul_rn(__fmul_rn(d, static_cast<float>(b[192 + j])), 0.015625f));
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) v |= ((q6k_quant(b, 16 * j + 4 * c + t) - 32u) & 0xFFu) << (8 * t);
        o[1 + c] = v;
      }
      uint32_t* dst = out + (b0 * 16 + static_cast<size_t>(h)) * 5;
#pragma unroll
      for (int c = 0; c < 5; c++) dst[c] = o[c];
    }
    __syncthreads();
  }
}

unsigned kq_grid(size_t work, unsigned per_block) {
  size_t g = (work + per_block - 1) / per_block;
  const size_t cap = static_cast<size_t>(wh::cu_count()) * 16;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace

namespace wh {

int launch_dequantize_kquant(int type, const void* data, size_t n, float* out, hipStream_t s) {
  if (n == 0) return WH_OK;
  const uint8_t* p = static_cast<const uint8_t*>(data);
  const unsigned grid = kq_grid((n + 3) / 4, 256);
  if (type == WH_TYPE_Q4_K) kq_dequant_kernel<WH_TYPE_Q4_K><<<grid, 256, 0, s>>>(p, out, n);
  else kq_dequant_kernel<WH_TYPE_Q6_K><<<grid, 256, 0, s>>>(p, out, n);
  WH_LAUNCH_CHECK("dequantize (k-quant) kernel launch");
  return WH_OK;
}

int launch_gemv_kquant(int type, const void* w, const float* x, float* y, size_t n_rows, size_t k, hipStream_t s,
                       const float* residual) {
  if (n_rows == 0) return WH_OK;
  const uint8_t* p = static_cast<const uint8_t*>(w);
  const unsigned grid = kq_grid(n_rows, 4);
  if (type == WH_TYPE_Q4_K) kq_gemv_kernel<WH_TYPE_Q4_K><<<grid, 256, 0, s>>>(p, x, residual, y, n_rows, k / 256);
  else kq_gemv_kernel<WH_TYPE_Q6_K><<<grid, 256, 0, s>>>(p, x, residual, y, n_rows, k / 256);
  WH_LAUNCH_CHECK("gemv (k-quant) kernel launch");
  return WH_OK;
}

int launch_repack_kquant(int type, const void* w, size_t n_rows, size_t k, void* out, hipStream_t s) {
  if (n_rows == 0 || k == 0) return WH_OK;
  const uint8_t* p = static_cast<const uint8_t*>(w);
  uint32_t* o = static_cast<uint32_t*>(out);
  if (type == WH_TYPE_Q4_K) {
    const size_t n = n_rows * (k / 32);
    uint16_t* dmin_t = reinterpret_cast<uint16_t*>(static_cast<char*>(out) + n * 20);
    kq_repack_q4k_kernel<<<kq_grid(n, 256), 256, 0, s>>>(p, n, k / 32, n_rows, o, dmin_t, q4f_dmin_stride(k));
  } else {
    const size_t n = n_rows * (k / 256);
    kq_repack_q6k_kernel<<<kq_grid(n, kQ6Blocks), 256, 0, s>>>(p, n, o);
  }
  WH_LAUNCH_CHECK("k-quant repack kernel launch");
  return WH_OK;
}

}  // namespace wh
