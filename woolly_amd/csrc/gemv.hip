// gemv.hip -- quantized matrix-vector product y = W x on gfx950.
//
// Reference: simd::quantized_matvec (crates/woolly-tensor/src/quantization.rs:869-909)
// and its scalar kernels quantized_matvec_q4_0_scalar / _q8_0_scalar
// (quantization.rs:1100-1163).  W is N rows x K/32 blocks in the GGUF block
// layout; Q4_1 is supported as dequantize_q4_1 composed with the f32 dot.
//
// Fast path ("pair" kernel).  Two consecutive blocks form a pair of 36 B
// (Q4_0), 40 B (Q4_1) or 68 B (Q8_0): always a whole number of dwords and,
// when a row has an even number of blocks, 4-byte aligned.  Lane l of a wave
// owns pair l of the wave's K-slice in every row it visits, so its 64
// activations stay in VGPRs for the whole kernel and each weight byte is
// loaded exactly once with dword-granular vector loads (9/10/17 dwords per
// lane, consecutive lanes reading consecutive 36/40/68-byte spans, so every
// cache line fetched is consumed completely by the same instruction group).
// Nibbles are unpacked in registers (one AND, one SHIFT+AND per dword, then
// v_cvt_f32_ubyte{0..3}); the f32 products accumulate per block and the block
// scale is applied once per block.  Q4_0's "-8" is folded as
// d * (sum q*x - 8 * sum x), with the per-block activation sums computed once.
// Rows are reduced across the 64 lanes; when K needs more than one wave
// (more than 64 pairs, e.g. K = 14336), the WG's waves split K and combine
// their partial sums through LDS in a fixed order (deterministic).
//
// Generic path: one wave per row, lanes stride over blocks with byte loads;
// used for odd block counts, unaligned pointers and K > 16384.
#include "wh_blocks.hpp"

namespace {

template <int TYPE>
struct PairFmt;
template <>
struct PairFmt<WH_TYPE_Q4_0> {
  static constexpr int DW = 9;
  static constexpr int BYTES = 36;
};
template <>
struct PairFmt<WH_TYPE_Q4_1> {
  static constexpr int DW = 10;
  static constexpr int BYTES = 40;
};
template <>
struct PairFmt<WH_TYPE_Q8_0> {
  static constexpr int DW = 17;
  static constexpr int BYTES = 68;
};

// Accumulates the 4-bit quants of dword u, bytes [K0, K1), where byte k holds
// qs[J0 + k]: low nibble -> element J0+k, high nibble -> element J0+k+16.
template <int K0, int K1, int J0>
__device__ __forceinline__ float nib_dot(uint32_t u, const float* xv, float s) {
  uint32_t lo = u & 0x0F0F0F0Fu;
  uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;
  // Hide the mask from the optimizer: otherwise it folds (lo >> 8k) & 0xFF
  // into a 4-bit field extract and loses v_cvt_f32_ubyte{k} (2 ops instead of 1).
  asm("" : "+v"(lo));
  asm("" : "+v"(hi));
#pragma unroll
  for (int k = K0; k < K1; k++) {
    s = __builtin_fmaf(static_cast<float>((lo >> (8 * k)) & 0xFFu), xv[J0 + k], s);
    s = __builtin_fmaf(static_cast<float>((hi >> (8 * k)) & 0xFFu), xv[J0 + k + 16], s);
  }
  return s;
}

// Accumulates the int8 quants of dword u, bytes [K0, K1), byte k = element J0+k.
template <int K0, int K1, int J0>
__device__ __forceinline__ float i8_dot(uint32_t u, const float* xv, float s) {
#pragma unroll
  for (int k = K0; k < K1; k++) {
    const int q = static_cast<int>(static_cast<int8_t>((u >> (8 * k)) & 0xFFu));
    s = __builtin_fmaf(static_cast<float>(q), xv[J0 + k], s);
  }
  return s;
}

// Dot product of one pair (two blocks, 64 elements) with the lane's
// activations xv[0..64); xa / xb are the sums of xv over each block.
template <int TYPE>
__device__ __forceinline__ float pair_dot(const uint32_t* w, const float* xv, float xa, float xb);

template <>
__device__ __forceinline__ float pair_dot<WH_TYPE_Q4_0>(const uint32_t* w, const float* xv,
                                                        float xa, float xb) {
  // dwords: [dA|q0 q1] [q2..5] [q6..9] [q10..13] [q14 q15|dB] [B q0..3] .. [B q12..15]
  const float da = whd::f16_bits_to_f32(w[0] & 0xFFFFu);
  const float db = whd::f16_bits_to_f32(w[4] >> 16);
  float sa = 0.f, sb = 0.f;
  sa = nib_dot<2, 4, -2>(w[0], xv, sa);
  sa = nib_dot<0, 4, 2>(w[1], xv, sa);
  sa = nib_dot<0, 4, 6>(w[2], xv, sa);
  sa = nib_dot<0, 4, 10>(w[3], xv, sa);
  sa = nib_dot<0, 2, 14>(w[4], xv, sa);
  sb = nib_dot<0, 4, 32>(w[5], xv, sb);
  sb = nib_dot<0, 4, 36>(w[6], xv, sb);
  sb = nib_dot<0, 4, 40>(w[7], xv, sb);
  sb = nib_dot<0, 4, 44>(w[8], xv, sb);
  return da * __builtin_fmaf(-8.f, xa, sa) + db * __builtin_fmaf(-8.f, xb, sb);
}

template <>
__device__ __forceinline__ float pair_dot<WH_TYPE_Q4_1>(const uint32_t* w, const float* xv,
                                                        float xa, float xb) {
  // dwords: [dA|mA] [A q0..3] .. [A q12..15] [dB|mB] [B q0..3] .. [B q12..15]
  const float da = whd::f16_bits_to_f32(w[0] & 0xFFFFu);
  const float ma = whd::f16_bits_to_f32(w[0] >> 16);
  const float db = whd::f16_bits_to_f32(w[5] & 0xFFFFu);
  const float mb = whd::f16_bits_to_f32(w[5] >> 16);
  float sa = 0.f, sb = 0.f;
  sa = nib_dot<0, 4, 0>(w[1], xv, sa);
  sa = nib_dot<0, 4, 4>(w[2], xv, sa);
  sa = nib_dot<0, 4, 8>(w[3], xv, sa);
  sa = nib_dot<0, 4, 12>(w[4], xv, sa);
  sb = nib_dot<0, 4, 32>(w[6], xv, sb);
  sb = nib_dot<0, 4, 36>(w[7], xv, sb);
  sb = nib_dot<0, 4, 40>(w[8], xv, sb);
  sb = nib_dot<0, 4, 44>(w[9], xv, sb);
  return __builtin_fmaf(da, sa, ma * xa) + __builtin_fmaf(db, sb, mb * xb);
}

template <>
__device__ __forceinline__ float pair_dot<WH_TYPE_Q8_0>(const uint32_t* w, const float* xv,
                                                        float, float) {
  // dwords: [dA|q0 q1] [q2..5] .. [q26..29] [q30 q31|dB] [B q0..3] .. [B q28..31]
  const float da = whd::f16_bits_to_f32(w[0] & 0xFFFFu);
  const float db = whd::f16_bits_to_f32(w[8] >> 16);
  float sa = 0.f, sb = 0.f;
  sa = i8_dot<2, 4, -2>(w[0], xv, sa);
  sa = i8_dot<0, 4, 2>(w[1], xv, sa);
  sa = i8_dot<0, 4, 6>(w[2], xv, sa);
  sa = i8_dot<0, 4, 10>(w[3], xv, sa);
  sa = i8_dot<0, 4, 14>(w[4], xv, sa);
  sa = i8_dot<0, 4, 18>(w[5], xv, sa);
  sa = i8_dot<0, 4, 22>(w[6], xv, sa);
  sa = i8_dot<0, 4, 26>(w[7], xv, sa);
  sa = i8_dot<0, 2, 30>(w[8], xv, sa);
  sb = i8_dot<0, 4, 32>(w[9], xv, sb);
  sb = i8_dot<0, 4, 36>(w[10], xv, sb);
  sb = i8_dot<0, 4, 40>(w[11], xv, sb);
  sb = i8_dot<0, 4, 44>(w[12], xv, sb);
  sb = i8_dot<0, 4, 48>(w[13], xv, sb);
  sb = i8_dot<0, 4, 52>(w[14], xv, sb);
  sb = i8_dot<0, 4, 56>(w[15], xv, sb);
  sb = i8_dot<0, 4, 60>(w[16], xv, sb);
  return da * sa + db * sb;
}

// Exact per-element form of pair_dot for activations that are not all finite:
// w = (q - 8) * d (Q4_0) or q * d + m (Q4_1) as in dequantize_q4_0/q4_1, then
// w * x accumulated, so inf/NaN propagate exactly as in the reference's
// (x0 * d) * input[j] (quantization.rs:1121-1124).  Q8_0's pair_dot already
// has this form.
template <int TYPE>
__device__ __forceinline__ float pair_dot_exact(const uint32_t* w, const float* xv) {
  float acc = 0.f;
#pragma unroll
  for (int blk = 0; blk < 2; blk++) {
    float d, m = 0.f;
    uint8_t qs[16];
    if constexpr (TYPE == WH_TYPE_Q4_0) {
      // byte offset of block blk inside the 36-byte pair: 18 * blk
      const int base = 18 * blk;
      auto byte_at = [&](int off) -> uint32_t { return (w[off >> 2] >> (8 * (off & 3))) & 0xFFu; };
      d = whd::f16_bits_to_f32(byte_at(base) | (byte_at(base + 1) << 8));
#pragma unroll
      for (int j = 0; j < 16; j++) qs[j] = static_cast<uint8_t>(byte_at(base + 2 + j));
    } else {
      const uint32_t dm = w[5 * blk];
      d = whd::f16_bits_to_f32(dm & 0xFFFFu);
      m = whd::f16_bits_to_f32(dm >> 16);
#pragma unroll
      for (int j = 0; j < 16; j++) qs[j] = static_cast<uint8_t>((w[5 * blk + 1 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      float w0, w1;
      if constexpr (TYPE == WH_TYPE_Q4_0) {
        w0 = static_cast<float>(static_cast<int>(qs[j] & 15) - 8) * d;
        w1 = static_cast<float>(static_cast<int>(qs[j] >> 4) - 8) * d;
      } else {
        w0 = __fadd_rn(__fmul_rn(static_cast<float>(qs[j] & 15), d), m);
        w1 = __fadd_rn(__fmul_rn(static_cast<float>(qs[j] >> 4), d), m);
      }
      s = __builtin_fmaf(w0, xv[32 * blk + j], s);
      s = __builtin_fmaf(w1, xv[32 * blk + j + 16], s);
    }
    acc += s;
  }
  return acc;
}

constexpr int kWaves = 4;  // waves per workgroup of the pair kernel

// ks: waves splitting one row's K (1, 2 or 4); ps: pairs per K-slice (<= 64);
// n_sets: number of R-row sets.  Workgroup w handles sets (it*rg + g) for
// it = w, w + gridDim.x, ... where g = wave / ks and rg = kWaves / ks.
template <int TYPE, int R>
__global__ __launch_bounds__(256) void gemv_pairs_kernel(const uint8_t* __restrict__ W,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int n_rows,
                                                         int pairs_per_row, int ks, int ps,
                                                         int n_sets) {
  constexpr int DW = PairFmt<TYPE>::DW;
  constexpr int PB = PairFmt<TYPE>::BYTES;
  __shared__ float red[kWaves][R];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int s = wave % ks;
  const int g = wave / ks;
  const int rg = kWaves / ks;
  const int p = s * ps + lane;
  const bool active = lane < ps && p < pairs_per_row;
  const size_t row_bytes = static_cast<size_t>(pairs_per_row) * PB;

  float xv[64];
  if (active) {
    const float4* xp = reinterpret_cast<const float4*>(x + 64 * static_cast<size_t>(p));
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 t = xp[i];
      xv[4 * i + 0] = t.x;
      xv[4 * i + 1] = t.y;
      xv[4 * i + 2] = t.z;
      xv[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; i++) xv[i] = 0.f;
  }
  float xa = 0.f, xb = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    xa += xv[i];
    xb += xv[32 + i];
  }
  // Folding the Q4_0 offset / Q4_1 minimum into the block sums xa, xb is exact
  // only for finite activations; a wave whose activations (or their block
  // sums) are not finite uses the per-element form instead.
  bool exact = false;
  if constexpr (TYPE != WH_TYPE_Q8_0) exact = __any(!(__builtin_isfinite(xa) && __builtin_isfinite(xb)));

  for (int it = blockIdx.x; it * rg < n_sets; it += gridDim.x) {
    const int set = it * rg + g;
    const int row0 = set * R;
    uint32_t wv[R][DW];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r;
      if (active && set < n_sets && row < n_rows) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(
            W + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(p) * PB);
#pragma unroll
        for (int j = 0; j < DW; j++) wv[r][j] = __builtin_nontemporal_load(src + j);
      } else {
#pragma unroll
        for (int j = 0; j < DW; j++) wv[r][j] = 0u;
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      float part;
      if constexpr (TYPE == WH_TYPE_Q8_0) {
        part = pair_dot<TYPE>(wv[r], xv, xa, xb);
      } else {
        part = exact ? pair_dot_exact<TYPE>(wv[r], xv) : pair_dot<TYPE>(wv[r], xv, xa, xb);
      }
      acc[r] = whd::wave_sum(part);
    }

    if (ks == 1) {
      if (lane == 0 && set < n_sets) {
#pragma unroll
        for (int r = 0; r < R; r++)
          if (row0 + r < n_rows) y[row0 + r] = acc[r];
      }
    } else {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) red[wave][r] = acc[r];
      }
      __syncthreads();
      if (s == 0 && lane < R && set < n_sets && row0 + lane < n_rows) {
        float t = 0.f;
        for (int s2 = 0; s2 < ks; s2++) t += red[g * ks + s2][lane];
        y[row0 + lane] = t;
      }
      __syncthreads();
    }
  }
}

template <int TYPE>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t* __restrict__ W,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, size_t n_rows,
                                                           size_t nb) {
  constexpr int TS = whd::BlockFmt<TYPE>::BYTES;
  const int lane = threadIdx.x & 63;
  const size_t stride = static_cast<size_t>(gridDim.x) * (blockDim.x >> 6);
  for (size_t row = static_cast<size_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
       row < n_rows; row += stride) {
    float acc = 0.f;
    for (size_t b = lane; b < nb; b += 64) {
      float v[32];
      whd::decode_block_bytes<TYPE>(W + (row * nb + b) * TS, v);
      const float* xb = x + b * 32;
#pragma unroll
      for (int j = 0; j < 32; j++) acc = __builtin_fmaf(v[j], xb[j], acc);
    }
    acc = whd::wave_sum(acc);
    if (lane == 0) y[row] = acc;
  }
}

template <int TYPE>
int launch_typed(const uint8_t* w, const float* x, float* y, size_t n_rows, size_t k,
                 hipStream_t s) {
  constexpr int R = 4;
  const size_t nb = k / 32;
  const int cus = wh::cu_count();
  const bool fast = (nb % 2 == 0) && nb > 0 && nb / 2 <= 256 && wh::aligned(w, 4) &&
                    wh::aligned(x, 16) && n_rows < (1u << 30);
  if (fast) {
    const int P = static_cast<int>(nb / 2);
    int ks = (P + 63) / 64;
    if (ks == 3) ks = 4;
    const int ps = (P + ks - 1) / ks;
    const int rg = kWaves / ks;
    const int n_sets = static_cast<int>((n_rows + R - 1) / R);
    int grid = (n_sets + rg - 1) / rg;
    const int cap = cus * 4;
    if (grid > cap) grid = cap;
    gemv_pairs_kernel<TYPE, R><<<grid, 256, 0, s>>>(w, x, y, static_cast<int>(n_rows), P, ks, ps,
                                                     n_sets);
  } else {
    size_t grid = (n_rows + 3) / 4;
    const size_t cap = static_cast<size_t>(cus) * 16;
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    gemv_generic_kernel<TYPE><<<static_cast<unsigned>(grid), 256, 0, s>>>(w, x, y, n_rows, nb);
  }
  WH_LAUNCH_CHECK("gemv kernel launch");
  return WH_OK;
}

}  // namespace

namespace wh {

int launch_gemv(int type, const void* w, const float* x, float* y, size_t n_rows, size_t k,
                hipStream_t s) {
  if (n_rows == 0) return WH_OK;
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  switch (type) {
    case WH_TYPE_Q4_0: return launch_typed<WH_TYPE_Q4_0>(wp, x, y, n_rows, k, s);
    case WH_TYPE_Q4_1: return launch_typed<WH_TYPE_Q4_1>(wp, x, y, n_rows, k, s);
    case WH_TYPE_Q8_0: return launch_typed<WH_TYPE_Q8_0>(wp, x, y, n_rows, k, s);
    default: return set_error(WH_ERR_UNSUPPORTED_TYPE, "gemv: unsupported type %d", type);
  }
}

}  // namespace wh
