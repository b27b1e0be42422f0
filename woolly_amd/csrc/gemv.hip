// gemv.hip -- quantized matrix-vector product y = W x on gfx950.
//
// Reference: simd::quantized_matvec (crates/woolly-tensor/src/quantization.rs:869-909)
// and its scalar kernels quantized_matvec_q4_0_scalar / _q8_0_scalar
// (quantization.rs:1100-1163).  W is N rows x K/32 blocks in the GGUF block
// layout; Q4_1 is supported as dequantize_q4_1 composed with the f32 dot.
//
// Fast path (gemv_stream_kernel, below): two consecutive blocks form a pair
// of 36 B (Q4_0), 40 B (Q4_1) or 68 B (Q8_0), a whole number of dwords and,
// when a row has an even number of blocks, 4-byte aligned.  Lane l owns pair l
// of its K-slice in every row, so its 64 activations stay in VGPRs; weights
// arrive through coalesced 32/64/96-bit loads and a per-wave LDS transpose.
// Nibbles are unpacked in registers (one AND, one SHIFT+AND per dword, then
// v_cvt_f32_ubyte{0..3}); the f32 products accumulate per block and the block
// scale is applied once per block.  Q4_0's "-8" is folded as
// d * (sum q*x - 8 * sum x), with the per-block activation sums computed once.
//
// Generic path: one wave per row, lanes stride over blocks with byte loads;
// used for odd block counts, unaligned pointers and K > 16384.
#include <algorithm>
#include <atomic>

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
// Four independent accumulators a[0..3] keep the FMA chains short.
template <int K0, int K1, int J0>
__device__ __forceinline__ void nib_dot(uint32_t u, const float* xv, float* a) {
  uint32_t lo = u & 0x0F0F0F0Fu;
  uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;
  // Hide the mask from the optimizer: otherwise it folds (lo >> 8k) & 0xFF
  // into a 4-bit field extract and loses v_cvt_f32_ubyte{k} (2 ops instead of 1).
  asm("" : "+v"(lo));
  asm("" : "+v"(hi));
#pragma unroll
  for (int k = K0; k < K1; k++) {
    a[k & 1] = __builtin_fmaf(static_cast<float>((lo >> (8 * k)) & 0xFFu), xv[J0 + k], a[k & 1]);
    a[2 + (k & 1)] =
        __builtin_fmaf(static_cast<float>((hi >> (8 * k)) & 0xFFu), xv[J0 + k + 16], a[2 + (k & 1)]);
  }
}

// Accumulates the int8 quants of dword u, bytes [K0, K1), byte k = element J0+k.
template <int K0, int K1, int J0>
__device__ __forceinline__ void i8_dot(uint32_t u, const float* xv, float* a) {
#pragma unroll
  for (int k = K0; k < K1; k++) {
    const int q = static_cast<int>(static_cast<int8_t>((u >> (8 * k)) & 0xFFu));
    a[k & 3] = __builtin_fmaf(static_cast<float>(q), xv[J0 + k], a[k & 3]);
  }
}

__device__ __forceinline__ float sum4(const float* a) { return (a[0] + a[1]) + (a[2] + a[3]); }

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
  float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
  nib_dot<2, 4, -2>(w[0], xv, a);
  nib_dot<0, 4, 32>(w[5], xv, b);
  nib_dot<0, 4, 2>(w[1], xv, a);
  nib_dot<0, 4, 36>(w[6], xv, b);
  nib_dot<0, 4, 6>(w[2], xv, a);
  nib_dot<0, 4, 40>(w[7], xv, b);
  nib_dot<0, 4, 10>(w[3], xv, a);
  nib_dot<0, 4, 44>(w[8], xv, b);
  nib_dot<0, 2, 14>(w[4], xv, a);
  return da * __builtin_fmaf(-8.f, xa, sum4(a)) + db * __builtin_fmaf(-8.f, xb, sum4(b));
}

template <>
__device__ __forceinline__ float pair_dot<WH_TYPE_Q4_1>(const uint32_t* w, const float* xv,
                                                        float xa, float xb) {
  // dwords: [dA|mA] [A q0..3] .. [A q12..15] [dB|mB] [B q0..3] .. [B q12..15]
  const float da = whd::f16_bits_to_f32(w[0] & 0xFFFFu);
  const float ma = whd::f16_bits_to_f32(w[0] >> 16);
  const float db = whd::f16_bits_to_f32(w[5] & 0xFFFFu);
  const float mb = whd::f16_bits_to_f32(w[5] >> 16);
  float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
  nib_dot<0, 4, 0>(w[1], xv, a);
  nib_dot<0, 4, 32>(w[6], xv, b);
  nib_dot<0, 4, 4>(w[2], xv, a);
  nib_dot<0, 4, 36>(w[7], xv, b);
  nib_dot<0, 4, 8>(w[3], xv, a);
  nib_dot<0, 4, 40>(w[8], xv, b);
  nib_dot<0, 4, 12>(w[4], xv, a);
  nib_dot<0, 4, 44>(w[9], xv, b);
  return __builtin_fmaf(da, sum4(a), ma * xa) + __builtin_fmaf(db, sum4(b), mb * xb);
}

template <>
__device__ __forceinline__ float pair_dot<WH_TYPE_Q8_0>(const uint32_t* w, const float* xv,
                                                        float, float) {
  // dwords: [dA|q0 q1] [q2..5] .. [q26..29] [q30 q31|dB] [B q0..3] .. [B q28..31]
  const float da = whd::f16_bits_to_f32(w[0] & 0xFFFFu);
  const float db = whd::f16_bits_to_f32(w[8] >> 16);
  float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
  i8_dot<2, 4, -2>(w[0], xv, a);
  i8_dot<0, 4, 32>(w[9], xv, b);
  i8_dot<0, 4, 2>(w[1], xv, a);
  i8_dot<0, 4, 36>(w[10], xv, b);
  i8_dot<0, 4, 6>(w[2], xv, a);
  i8_dot<0, 4, 40>(w[11], xv, b);
  i8_dot<0, 4, 10>(w[3], xv, a);
  i8_dot<0, 4, 44>(w[12], xv, b);
  i8_dot<0, 4, 14>(w[4], xv, a);
  i8_dot<0, 4, 48>(w[13], xv, b);
  i8_dot<0, 4, 18>(w[5], xv, a);
  i8_dot<0, 4, 52>(w[14], xv, b);
  i8_dot<0, 4, 22>(w[6], xv, a);
  i8_dot<0, 4, 56>(w[15], xv, b);
  i8_dot<0, 4, 26>(w[7], xv, a);
  i8_dot<0, 4, 60>(w[16], xv, b);
  i8_dot<0, 2, 30>(w[8], xv, a);
  return da * sum4(a) + db * sum4(b);
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

// ---------------------------------------------------------------------------
// Streaming kernel.
//
// One persistent workgroup per CU, kWaves waves.  The row's pairs are split
// into K-slices of at most 64 pairs (4096 elements); `ks` waves (1, 2 or 4)
// cover one row and the workgroup's kWaves / ks row groups walk its contiguous
// row range.  Lane l of a slice-s wave owns pair 64*s + l in every row, so its
// 64 activations are read once (from an LDS copy of x staged by the whole
// workgroup) and kept in VGPRs.  Each row slice is fetched with coalesced
// V-dword loads (96-bit for Q4_0, 64-bit for Q4_1, 32-bit for Q8_0: a slice of
// 64 pairs is exactly 3 / 5 / 17 such loads per lane), prefetched kPrefetch
// rows ahead in registers, transposed through a wave-private LDS slab so that
// each lane gets its own 36/40/68-byte pair, and reduced across lanes with
// DPP.  With ks > 1 the slices' partial sums meet in LDS in a fixed order.
constexpr int kWaves = 8;
constexpr int kPrefetch = 2;
constexpr int kMaxSlices = 4;  // K <= 4 * 4096

template <int TYPE>
struct LoadFmt;  // V: dwords per vector load; NV: loads per full 64-pair slice
template <>
struct LoadFmt<WH_TYPE_Q4_0> {
  static constexpr int V = 3, NV = 3;
};
template <>
struct LoadFmt<WH_TYPE_Q4_1> {
  static constexpr int V = 2, NV = 5;
};
template <>
struct LoadFmt<WH_TYPE_Q8_0> {
  static constexpr int V = 1, NV = 17;
};

// Sum over the wavefront; the total lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_mov<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_mov<0x140, 0xF>(v);  // row_mirror
  v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15
  v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31
  return v;
}

template <int V>
__device__ __forceinline__ void load_vec(const uint32_t* __restrict__ src, bool ok, uint32_t* dst) {
#pragma unroll
  for (int c = 0; c < V; c++) dst[c] = ok ? __builtin_nontemporal_load(src + c) : 0u;
}

// Arguments of the streaming kernels.  Plain mode (FFN = false): the output
// rows are stacked from up to three matrices with the same K, rows [0, n0)
// from W, [n0, n0 + n1) from W2, the rest from W3 (a single matrix has
// n0 = n_rows); this is how the Q, K and V projections of one token run as one
// launch.  FFN mode: W (gate) and W2 (up) are streamed side by side.  With
// gamma set, x is RMS-normalised while staged (rms = sqrt(sum x^2 / K + eps),
// x_hat = (x / rms) * gamma, tensor_utils.rs:446-480); with residual set,
// y[row] = residual[row] + result (the residual adds of process_layer,
// lazy_transformer.rs:98-258).
struct GemvArgs {
  const uint8_t* W;
  const uint8_t* W2;
  const uint8_t* W3;
  int n0, n1;
  const float* x;
  const float* gamma;
  float eps;
  const float* residual;
  float* y;
  int n_rows, pairs_per_row, ks, rows_per_wg;
};

// Compile-time variants of the streaming kernels (MODE bit set): RMSNorm of
// x while staged, residual add at the store, rows stacked from up to three
// matrices.  The plain GEMV (MODE 0) carries none of their code.
constexpr int kNorm = 1, kResid = 2, kStack = 4;

// Matrix and local row of output row `row` in plain (stacked) mode.
__device__ __forceinline__ const uint8_t* stacked_row(const GemvArgs& a, int row, int* local) {
  int r = row;
  const uint8_t* b = a.W;
  if (r >= a.n0) {
    r -= a.n0;
    b = a.W2;
    if (r >= a.n1) {
      r -= a.n1;
      b = a.W3;
    }
  }
  *local = r;
  return b;
}

// RMSNorm of the x staged in LDS (padded layout, 4 floats per 64), in place;
// red holds kWaves partial sums.  Fixed-shape reduction: deterministic.
__device__ __forceinline__ void norm_staged_x(float* xs, float* red, int K, const float* gamma, float eps,
                                              int wave, int lane);

// FFN = true: the FFN's first half for one token (the decode step): x is
// RMS-normalised with gamma while staged (rms = sqrt(sum x^2 / K + eps),
// x_hat = (x / rms) * gamma, tensor_utils.rs:446-480), the gate row (W) and
// the up row (W2) of every output index are streamed side by side, and
// y = silu(gate . x_hat) * (up . x_hat) (tensor_utils.rs:512-532).
template <int TYPE, bool FFN, int MODE>
__global__ __launch_bounds__(kWaves * 64) void gemv_stream_kernel(const GemvArgs a) {
  const int n_rows = a.n_rows, pairs_per_row = a.pairs_per_row, ks = a.ks, rows_per_wg = a.rows_per_wg;
  const float* __restrict__ x = a.x;
  float* __restrict__ y = a.y;
  constexpr int DW = PairFmt<TYPE>::DW;
  constexpr int PB = PairFmt<TYPE>::BYTES;
  constexpr int V = LoadFmt<TYPE>::V;
  constexpr int NV = LoadFmt<TYPE>::NV;
  constexpr int SLAB = DW * 64 + 4;
  constexpr int NM = FFN ? 2 : 1;                           // weight matrices streamed
  extern __shared__ __align__(16) uint32_t lds[];
  const int K = pairs_per_row * 64;
  float* xs = reinterpret_cast<float*>(lds);                // x, 4 floats of padding per 64
  uint32_t* slabs = lds + K + K / 16;                       // kWaves * NM slabs of SLAB dwords
  float* red = reinterpret_cast<float*>(slabs + kWaves * NM * SLAB);  // NM * kWaves partials

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar address math
  const int lane = threadIdx.x & 63;
  const int s = wave % ks;
  const int g = wave / ks;
  const int groups = kWaves / ks;
  const int ps = min(64, pairs_per_row - 64 * s);           // pairs in this slice (> 0)
  const int nd = DW * ps;                                   // dwords in one row slice
  const bool active = lane < ps;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(n_rows, r0 + rows_per_wg);
  const int nk = (r1 - r0 + groups - 1) / groups;           // row steps (uniform in the WG)
  const size_t row_bytes = static_cast<size_t>(pairs_per_row) * PB;
  const size_t slice_off = static_cast<size_t>(64 * s) * PB;

  // Prefetch the first rows before anything else.
  uint32_t buf[kPrefetch][NM][DW];
  auto fetch = [&](uint32_t (*dst)[DW], int k) {
    const int row = r0 + g + k * groups;
    const bool rok = k < nk && row < r1;
    int local = row;
    const uint8_t* base0 = a.W;
    if constexpr ((MODE & kStack) != 0) base0 = stacked_row(a, rok ? row : r0, &local);
#pragma unroll
    for (int mtx = 0; mtx < NM; mtx++) {
      const uint8_t* base = mtx ? a.W2 : base0;
      const uint32_t* src = reinterpret_cast<const uint32_t*>(base + slice_off + static_cast<size_t>(local) * row_bytes);
#pragma unroll
      for (int i = 0; i < NV; i++) {
        const int e = V * (64 * i + lane);
        load_vec<V>(src + e, rok && e < nd, dst[mtx] + V * i);
      }
    }
  };
#pragma unroll
  for (int d = 0; d < kPrefetch; d++) fetch(buf[d], d);

  // Stage x in LDS once for the workgroup, then each lane copies its 64 values.
  for (int i = threadIdx.x; i < K / 4; i += kWaves * 64) {
    const float4 t = reinterpret_cast<const float4*>(x)[i];
    const int e = 4 * i;
    *reinterpret_cast<float4*>(xs + e + (e >> 6) * 4) = t;
  }
  __syncthreads();
  if constexpr ((MODE & kNorm) != 0) norm_staged_x(xs, red, K, a.gamma, a.eps, wave, lane);
  float xv[64];
  {
    const int p = 64 * s + (active ? lane : 0);
    const float* xp = xs + 68 * p;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 t = *reinterpret_cast<const float4*>(xp + 4 * i);
      xv[4 * i + 0] = active ? t.x : 0.f;
      xv[4 * i + 1] = active ? t.y : 0.f;
      xv[4 * i + 2] = active ? t.z : 0.f;
      xv[4 * i + 3] = active ? t.w : 0.f;
    }
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

  uint32_t* slab = slabs + wave * NM * SLAB;
  // y = silu(g) * u, the SiLU in the reference's form g * (1 / (1 + exp(-g)))
  auto combine = [](float gv, float uv) { return FFN ? (gv * (1.0f / (1.0f + expf(-gv)))) * uv : gv; };
  for (int kb = 0; kb < nk; kb += kPrefetch) {
#pragma unroll
    for (int d = 0; d < kPrefetch; d++) {
      const int k = kb + d;
      if (k >= nk) break;
      const int row = r0 + g + k * groups;
      // this row's slice(s) -> LDS slab(s) (dword e of a slice at slab[e])
#pragma unroll
      for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
        for (int i = 0; i < NV; i++)
#pragma unroll
          for (int c = 0; c < V; c++) slab[mtx * SLAB + V * (64 * i + lane) + c] = buf[d][mtx][V * i + c];
      fetch(buf[d], k + kPrefetch);
      __builtin_amdgcn_wave_barrier();
      float tot[NM];
#pragma unroll
      for (int mtx = 0; mtx < NM; mtx++) {
        uint32_t w[DW];
#pragma unroll
        for (int j = 0; j < DW; j++) w[j] = slab[mtx * SLAB + DW * lane + j];
        float part = 0.f;
        if (active) {
          if constexpr (TYPE == WH_TYPE_Q8_0) {
            part = pair_dot<TYPE>(w, xv, xa, xb);
          } else {
            part = exact ? pair_dot_exact<TYPE>(w, xv) : pair_dot<TYPE>(w, xv, xa, xb);
          }
        }
        tot[mtx] = wave_sum_to_lane63(part);
      }
      __builtin_amdgcn_wave_barrier();
      if (ks == 1) {
        if (lane == 63 && row < r1) y[row] = ((MODE & kResid) != 0 ? a.residual[row] : 0.f) + combine(tot[0], tot[NM - 1]);
      } else {
        if (lane == 63) {
#pragma unroll
          for (int mtx = 0; mtx < NM; mtx++) red[mtx * kWaves + wave] = tot[mtx];
        }
        __syncthreads();
        if (s == 0 && lane == 63 && row < r1) {
          float t[NM];
#pragma unroll
          for (int mtx = 0; mtx < NM; mtx++) {
            t[mtx] = red[mtx * kWaves + g * ks];
            for (int s2 = 1; s2 < ks; s2++) t[mtx] += red[mtx * kWaves + g * ks + s2];
          }
          y[row] = ((MODE & kResid) != 0 ? a.residual[row] : 0.f) + combine(t[0], t[NM - 1]);
        }
        __syncthreads();
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Ring kernel: same work split and arithmetic as gemv_stream_kernel, but each
// wave's row slices are copied global -> LDS with global_load_lds_dwordx4
// (lane l's 16 bytes land at slot + 16 l) into a wave-private ring of RD
// slots, RD - 1 rows ahead of the row being computed.  No VGPRs hold the
// prefetched rows and no LDS stores are issued for them.  The copies are
// issued through inline asm (the compiler would otherwise wait for every copy
// in flight before each LDS read); every wave issues exactly NI copies per
// matrix per row, so completion is tracked with a constant vmcnt.
// `base` and `lds` are wave-uniform; readfirstlane puts them in SGPRs.  The
// builtin returns a signed int: each half is taken back to uint32_t before
// the halves are joined (a sign-extended low half would corrupt the pointer).
__device__ __forceinline__ void ring_copy16(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint64_t ub = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  // M0 (reserved by the compiler) is saved in an SGPR, set for the copy after
  // one wait state, and restored
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(reinterpret_cast<const void*>(ub)), "s"(m0)
      : "memory");
}
template <int N>
__device__ __forceinline__ void ring_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return static_cast<uint32_t>((uintptr_t)((const __attribute__((address_space(3))) uint8_t*)p));
}

template <int TYPE>
constexpr int ring_ni() { return (PairFmt<TYPE>::DW * 64 * 4 + 1023) / 1024; }  // copies per full slice

template <int TYPE, bool FFN, int RD, int MODE>
__global__ __launch_bounds__(kWaves * 64) void gemv_ring_kernel(const GemvArgs a) {
  const int n_rows = a.n_rows, pairs_per_row = a.pairs_per_row, ks = a.ks, rows_per_wg = a.rows_per_wg;
  const float* __restrict__ x = a.x;
  float* __restrict__ y = a.y;
  constexpr int DW = PairFmt<TYPE>::DW;
  constexpr int PB = PairFmt<TYPE>::BYTES;
  constexpr int NM = FFN ? 2 : 1;
  constexpr int NI = ring_ni<TYPE>();
  constexpr int SLOT = DW * 64 * 4;                         // bytes per slot (a full slice)
  extern __shared__ __align__(16) uint32_t lds[];
  const int K = pairs_per_row * 64;
  float* xs = reinterpret_cast<float*>(lds);
  uint8_t* ring = reinterpret_cast<uint8_t*>(lds + K + K / 16);      // kWaves * NM * RD slots
  float* red = reinterpret_cast<float*>(ring + kWaves * NM * RD * SLOT);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar address math
  const int lane = threadIdx.x & 63;
  const int s = wave % ks;
  const int g = wave / ks;
  const int groups = kWaves / ks;
  const int ps = min(64, pairs_per_row - 64 * s);
  const int nbytes = PB * ps;                               // bytes of one row slice (multiple of 16)
  const bool active = lane < ps;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(n_rows, r0 + rows_per_wg);
  const int nk = (r1 - r0 + groups - 1) / groups;
  const uint32_t row_bytes = static_cast<uint32_t>(pairs_per_row) * PB;
  const uint32_t slice_off = static_cast<uint32_t>(64 * s) * PB;
  uint8_t* my_ring = ring + wave * NM * RD * SLOT;
  const uint32_t ring_lds = lds_u32(my_ring);

  // Copies of row step k into slot k % RD.  Rows past the range re-read the
  // range's last row; lanes past the slice are masked off, and copy
  // instructions wholly past it are replaced by lane 0 re-copying the last
  // chunk onto itself, so every wave issues the same number of copies.
  const int nchunks = nbytes / 16;
  auto issue = [&](int k) {
    const int row = min(r0 + g + k * groups, r1 - 1);
    int local = row;
    const uint8_t* base0 = a.W;
    if constexpr ((MODE & kStack) != 0) base0 = stacked_row(a, row, &local);
    const uint32_t base_off = static_cast<uint32_t>(local) * row_bytes + slice_off;
#pragma unroll
    for (int mtx = 0; mtx < NM; mtx++) {
      const uint32_t slot = ring_lds + static_cast<uint32_t>((mtx * RD + (k % RD)) * SLOT);
      const void* base = mtx ? static_cast<const void*>(a.W2) : static_cast<const void*>(base0);
#pragma unroll
      for (int i = 0; i < NI; i++) {
        if (64 * i < nchunks) {
          const int c = 64 * i + lane;
          if (c < nchunks) ring_copy16(base, base_off + 16u * static_cast<uint32_t>(c), slot + 1024u * i);
        } else if (lane == 0) {
          // padding copy (constant copy count): the slice's last chunk onto itself
          const uint32_t last = 16u * static_cast<uint32_t>(nchunks - 1);
          ring_copy16(base, base_off + last, slot + last);
        }
      }
    }
  };
#pragma unroll
  for (int d = 0; d < RD - 1; d++)
    if (d < nk) issue(d);

  // Stage x in LDS once for the workgroup, then each lane copies its 64 values.
  for (int i = threadIdx.x; i < K / 4; i += kWaves * 64) {
    const float4 t = reinterpret_cast<const float4*>(x)[i];
    const int e = 4 * i;
    *reinterpret_cast<float4*>(xs + e + (e >> 6) * 4) = t;
  }
  __syncthreads();
  if constexpr ((MODE & kNorm) != 0) norm_staged_x(xs, red, K, a.gamma, a.eps, wave, lane);
  float xv[64];
  {
    const int p = 64 * s + (active ? lane : 0);
    const float* xp = xs + 68 * p;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 t = *reinterpret_cast<const float4*>(xp + 4 * i);
      xv[4 * i + 0] = active ? t.x : 0.f;
      xv[4 * i + 1] = active ? t.y : 0.f;
      xv[4 * i + 2] = active ? t.z : 0.f;
      xv[4 * i + 3] = active ? t.w : 0.f;
    }
  }
  float xa = 0.f, xb = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    xa += xv[i];
    xb += xv[32 + i];
  }
  bool exact = false;
  if constexpr (TYPE != WH_TYPE_Q8_0) exact = __any(!(__builtin_isfinite(xa) && __builtin_isfinite(xb)));

  auto combine = [](float gv, float uv) { return FFN ? (gv * (1.0f / (1.0f + expf(-gv)))) * uv : gv; };
  for (int k = 0; k < nk; k++) {
    const int row = r0 + g + k * groups;
    if (k + RD - 1 < nk) {
      issue(k + RD - 1);                   // into the slot of step k - 1, already consumed
      ring_wait<(RD - 1) * NM * NI>();     // the copies of steps k + 1 .. k + RD - 1 may be in flight
    } else {
      ring_wait<0>();
    }
    float tot[NM];
#pragma unroll
    for (int mtx = 0; mtx < NM; mtx++) {
      const uint32_t* slot = reinterpret_cast<const uint32_t*>(my_ring + (mtx * RD + (k % RD)) * SLOT);
      uint32_t w[DW];
#pragma unroll
      for (int j = 0; j < DW; j++) w[j] = slot[DW * (active ? lane : 0) + j];
      float part = 0.f;
      if (active) {
        if constexpr (TYPE == WH_TYPE_Q8_0) {
          part = pair_dot<TYPE>(w, xv, xa, xb);
        } else {
          part = exact ? pair_dot_exact<TYPE>(w, xv) : pair_dot<TYPE>(w, xv, xa, xb);
        }
      }
      tot[mtx] = wave_sum_to_lane63(part);
    }
    if (ks == 1) {
      if (lane == 63 && row < r1) y[row] = ((MODE & kResid) != 0 ? a.residual[row] : 0.f) + combine(tot[0], tot[NM - 1]);
    } else {
      if (lane == 63) {
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++) red[mtx * kWaves + wave] = tot[mtx];
      }
      // LDS-only barrier: a __syncthreads() here would also wait for the
      // weight copies in flight
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (s == 0 && lane == 63 && row < r1) {
        float t[NM];
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++) {
          t[mtx] = red[mtx * kWaves + g * ks];
          for (int s2 = 1; s2 < ks; s2++) t[mtx] += red[mtx * kWaves + g * ks + s2];
        }
        y[row] = ((MODE & kResid) != 0 ? a.residual[row] : 0.f) + combine(t[0], t[NM - 1]);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
  }
  ring_wait<0>();  // no copy may land in LDS after the workgroup has exited
}

__device__ __forceinline__ void norm_staged_x(float* xs, float* red, int K, const float* gamma, float eps,
                                              int wave, int lane) {
  float ss = 0.f;
  for (int i = threadIdx.x; i < K; i += kWaves * 64) {
    const float v = xs[i + (i >> 6) * 4];
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = whd::wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; w++) total += red[w];
  const float rms = sqrtf(total / static_cast<float>(K) + eps);
  for (int i = threadIdx.x; i < K; i += kWaves * 64) {
    float* p = xs + i + (i >> 6) * 4;
    *p = (*p / rms) * gamma[i];
  }
  __syncthreads();
}

size_t ring_lds_bytes(int type, int K, int nm, int rd) {
  const int dw = type == WH_TYPE_Q4_0 ? 9 : (type == WH_TYPE_Q4_1 ? 10 : 17);
  return 4u * static_cast<size_t>(K + K / 16) + static_cast<size_t>(kWaves) * nm * rd * dw * 64 * 4 +
         4u * nm * kWaves;
}

size_t stream_lds_bytes(int type, int K, int nm) {
  const int dw = type == WH_TYPE_Q4_0 ? 9 : (type == WH_TYPE_Q4_1 ? 10 : 17);
  return 4u * static_cast<size_t>(K + K / 16 + nm * kWaves * (dw * 64 + 4) + nm * kWaves);
}

// One wave per output row, lanes stride over blocks with byte loads.  Rows
// are stacked from up to three matrices and the residual is added as in the
// streaming kernels (a.n_rows rows, K = 32 nb; no RMSNorm: the caller
// normalises x first).
template <int TYPE>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const GemvArgs a, size_t nb) {
  constexpr int TS = whd::BlockFmt<TYPE>::BYTES;
  const int lane = threadIdx.x & 63;
  const size_t n_rows = static_cast<size_t>(a.n_rows);
  const size_t stride = static_cast<size_t>(gridDim.x) * (blockDim.x >> 6);
  for (size_t row = static_cast<size_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
       row < n_rows; row += stride) {
    int local;
    const uint8_t* W = stacked_row(a, static_cast<int>(row), &local);
    float acc = 0.f;
    for (size_t b = lane; b < nb; b += 64) {
      float v[32];
      whd::decode_block_bytes<TYPE>(W + (static_cast<size_t>(local) * nb + b) * TS, v);
      const float* xb = a.x + b * 32;
#pragma unroll
      for (int j = 0; j < 32; j++) acc = __builtin_fmaf(v[j], xb[j], acc);
    }
    acc = whd::wave_sum(acc);
    if (lane == 0) a.y[row] = (a.residual ? a.residual[row] : 0.f) + acc;
  }
}

template <int TYPE>
int launch_generic(const GemvArgs& a, size_t k, hipStream_t s) {
  size_t grid = (static_cast<size_t>(a.n_rows) + 3) / 4;
  const size_t cap = static_cast<size_t>(wh::cu_count()) * 16;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  gemv_generic_kernel<TYPE><<<static_cast<unsigned>(grid), 256, 0, s>>>(a, k / 32);
  WH_LAUNCH_CHECK("gemv kernel launch");
  return WH_OK;
}

// Chooses the streaming kernel when its layout conditions hold (an even
// number of blocks per row, at most 4 K-slices, 4-byte aligned weights,
// 16-byte aligned x, LDS within the device limit).
template <int TYPE, bool FFN>
bool stream_ok(const GemvArgs& a, size_t k) {
  const size_t nb = k / 32;
  const size_t lds = stream_lds_bytes(TYPE, static_cast<int>(k), FFN ? 2 : 1);
  const bool w2_used = FFN || a.n1 > 0;
  const bool w3_used = !FFN && a.n_rows > a.n0 + a.n1;
  return (nb % 2 == 0) && nb > 0 && nb / 2 <= 64 * kMaxSlices && wh::aligned(a.W, 4) &&
         (!w2_used || wh::aligned(a.W2, 4)) && (!w3_used || wh::aligned(a.W3, 4)) && wh::aligned(a.x, 16) &&
         a.n_rows >= 0 && lds <= wh::max_lds_per_block();
}

#ifndef WH_GEMV_RING
#define WH_GEMV_RING 1
#endif

template <int TYPE, bool FFN, int RD, int MODE>
int launch_ring(const GemvArgs& a, int grid, size_t lds, hipStream_t s) {
  WH_ENSURE_LDS(lds, &gemv_ring_kernel<TYPE, FFN, RD, MODE>);
  gemv_ring_kernel<TYPE, FFN, RD, MODE><<<grid, kWaves * 64, lds, s>>>(a);
  WH_LAUNCH_CHECK(FFN ? "ffn gate/up kernel launch" : "gemv kernel launch");
  return WH_OK;
}

// Fills the work split of `a` (K-slices per row, workgroups, rows per
// workgroup) and launches the ring or the register-staged kernel variant MODE.
template <int TYPE, bool FFN, int MODE>
int launch_stream(GemvArgs a, size_t k, hipStream_t s) {
  const int cus = wh::cu_count();
  const size_t n_rows = static_cast<size_t>(a.n_rows);
  const size_t lds = stream_lds_bytes(TYPE, static_cast<int>(k), FFN ? 2 : 1);
  const int P = static_cast<int>(k / 64);
  int ks = (P + 63) / 64;
  if (ks == 3) ks = 4;
  const int groups = kWaves / ks;
  const size_t max_wg = (n_rows + groups - 1) / groups;
  const int grid = static_cast<int>(max_wg < static_cast<size_t>(cus) ? max_wg : cus);
  a.pairs_per_row = P;
  a.ks = ks;
  a.rows_per_wg = static_cast<int>((n_rows + grid - 1) / grid);
  // Ring kernel: every K-slice a whole number of 16-byte chunks, 32-bit byte
  // offsets within each matrix, and a ring of at least two slots per wave
  // within the LDS limit.
  const int tail = P % 64;
  const bool chunks_ok = (PairFmt<TYPE>::BYTES * 64) % 16 == 0 && (PairFmt<TYPE>::BYTES * tail) % 16 == 0;
  const size_t max_mrows = FFN ? n_rows
                               : std::max({static_cast<size_t>(a.n0), static_cast<size_t>(a.n1),
                                           n_rows - std::min(n_rows, static_cast<size_t>(a.n0 + a.n1))});
  // Measured on MI355X (14336 x 4096 and 4096 x 14336): the ring wins for
  // Q8_0 (more bytes per row) and for the FFN's two matrices; the 4-bit
  // single-matrix GEMV is bound by its unpacking arithmetic and keeps the
  // register-staged kernel.
  const bool ring_pays = TYPE == WH_TYPE_Q8_0 || FFN;
  if (WH_GEMV_RING && ring_pays && chunks_ok &&
      max_mrows * (k / 64) * PairFmt<TYPE>::BYTES < (static_cast<size_t>(1) << 32)) {
    const int nm = FFN ? 2 : 1;
    const size_t maxl = wh::max_lds_per_block();
    const int K = static_cast<int>(k);
    if (ring_lds_bytes(TYPE, K, nm, 4) <= maxl)
      return launch_ring<TYPE, FFN, 4, MODE>(a, grid, ring_lds_bytes(TYPE, K, nm, 4), s);
    if (ring_lds_bytes(TYPE, K, nm, 3) <= maxl)
      return launch_ring<TYPE, FFN, 3, MODE>(a, grid, ring_lds_bytes(TYPE, K, nm, 3), s);
    if (ring_lds_bytes(TYPE, K, nm, 2) <= maxl)
      return launch_ring<TYPE, FFN, 2, MODE>(a, grid, ring_lds_bytes(TYPE, K, nm, 2), s);
  }
  if (lds > 65536) WH_ENSURE_LDS(lds, &gemv_stream_kernel<TYPE, FFN, MODE>);
  gemv_stream_kernel<TYPE, FFN, MODE><<<grid, kWaves * 64, lds, s>>>(a);
  WH_LAUNCH_CHECK(FFN ? "ffn gate/up kernel launch" : "gemv kernel launch");
  return WH_OK;
}

// The variants the decode step uses get their own code: Q/K/V (norm +
// stacked), the output head (norm), the residual projections; any other
// combination runs the variant with every feature on.
template <int TYPE>
int launch_fused_mode(const GemvArgs& a, size_t k, int mode, hipStream_t s) {
  switch (mode) {
    case 0: return launch_stream<TYPE, false, 0>(a, k, s);
    case kNorm: return launch_stream<TYPE, false, kNorm>(a, k, s);
    case kResid: return launch_stream<TYPE, false, kResid>(a, k, s);
    case kNorm | kStack: return launch_stream<TYPE, false, kNorm | kStack>(a, k, s);
    default: return launch_stream<TYPE, false, kNorm | kResid | kStack>(a, k, s);
  }
}

GemvArgs plain_args(const uint8_t* w, const float* x, float* y, size_t n_rows) {
  GemvArgs a{};
  a.W = a.W2 = a.W3 = w;
  a.n0 = static_cast<int>(n_rows);
  a.n1 = 0;
  a.x = x;
  a.y = y;
  a.n_rows = static_cast<int>(n_rows);
  return a;
}

// wh_gemv_select's setting, per calling thread (like wh_last_error): a switch
// on one thread never changes what another thread launches or captures.
thread_local int t_gemv_mode = WH_GEMV_AUTO;

// The matrix-core kernel pays for its activation preparation and its 16-row
// steps on short rows and few rows; below these sizes the streaming kernels
// are used.
bool use_mfma(int type, size_t n_rows, size_t k) {
  return t_gemv_mode == WH_GEMV_AUTO && k >= 1024 && n_rows >= 64 &&
         wh::gemv_mfma_ok(type, n_rows, k);
}

template <int TYPE>
int launch_typed(const uint8_t* w, const float* x, float* y, size_t n_rows, size_t k,
                 hipStream_t s) {
  if (n_rows >= (1u << 31)) return wh::set_error(WH_ERR_INVALID_SHAPE, "gemv: %zu rows exceed 2^31", n_rows);
  if (use_mfma(TYPE, n_rows, k)) {
    const void* mats[1] = {w};
    const size_t rows[1] = {n_rows};
    const int st = wh::launch_gemv_mfma(TYPE, mats, rows, 1, false, x, nullptr, 0.f, nullptr, y, n_rows, k, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  const GemvArgs a = plain_args(w, x, y, n_rows);
  if (n_rows < (1u << 30) && stream_ok<TYPE, false>(a, k)) return launch_stream<TYPE, false, 0>(a, k, s);
  return launch_generic<TYPE>(a, k, s);
}

}  // namespace

namespace wh {

// The FFN's first half for one token, fused (see gemv_stream_kernel<., true>):
// h = silu(W_gate x_hat) * (W_up x_hat), x_hat = rms_norm(x, gamma, eps).
// Returns WH_ERR_INVALID_SHAPE without launching when the fused kernel's
// layout conditions do not hold; the caller then runs the unfused sequence.
bool mt_allowed(size_t n_rows, size_t k) { return t_gemv_mode == WH_GEMV_AUTO && k >= 1024 && n_rows >= 64; }

int gemv_mode_exchange(int mode) {
  const int prev = t_gemv_mode;
  t_gemv_mode = mode;
  return prev;
}

int launch_ffn_gate_up(int type, const void* gate, const void* up, const float* x, const float* gamma,
                       float eps, float* h, size_t n_ff, size_t hidden, hipStream_t s) {
  if (n_ff == 0) return WH_OK;
  if (n_ff >= (1u << 30) || !gamma)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "ffn gate/up: %zu rows (at most 2^30) or no RMSNorm weight", n_ff);
  if (use_mfma(type, n_ff, hidden)) {
    const void* mats[2] = {gate, up};
    const size_t rows[2] = {n_ff, n_ff};
    const int st = launch_gemv_mfma(type, mats, rows, 2, true, x, gamma, eps, nullptr, h, n_ff, hidden, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  GemvArgs a = plain_args(static_cast<const uint8_t*>(gate), x, h, n_ff);
  a.W2 = static_cast<const uint8_t*>(up);
  a.gamma = gamma;
  a.eps = eps;
  switch (type) {
    case WH_TYPE_Q4_0:
      if (!stream_ok<WH_TYPE_Q4_0, true>(a, hidden))
        return wh::set_error(WH_ERR_INVALID_SHAPE, "ffn gate/up: layout not fused (hidden = %zu)", hidden);
      return launch_stream<WH_TYPE_Q4_0, true, kNorm>(a, hidden, s);
    case WH_TYPE_Q4_1:
      if (!stream_ok<WH_TYPE_Q4_1, true>(a, hidden))
        return wh::set_error(WH_ERR_INVALID_SHAPE, "ffn gate/up: layout not fused (hidden = %zu)", hidden);
      return launch_stream<WH_TYPE_Q4_1, true, kNorm>(a, hidden, s);
    case WH_TYPE_Q8_0:
      if (!stream_ok<WH_TYPE_Q8_0, true>(a, hidden))
        return wh::set_error(WH_ERR_INVALID_SHAPE, "ffn gate/up: layout not fused (hidden = %zu)", hidden);
      return launch_stream<WH_TYPE_Q8_0, true, kNorm>(a, hidden, s);
    default:
      return wh::set_error(WH_ERR_INVALID_SHAPE, "ffn gate/up: type %d not fused", type);
  }
}

// Fused single-token GEMV: up to three matrices with the same K stacked by
// rows (rows[i] rows of mats[i]), optional RMSNorm of x (gamma, eps) and
// optional residual add (y may alias residual: each row is read and written
// by one lane).  With gamma set and a layout the streaming kernels do not
// take, WH_ERR_INVALID_SHAPE without launching (the caller normalises x and
// calls again without gamma).
int launch_gemv_fused(int type, const void* const* mats, const size_t* rows, int n_mats, const float* x,
                      const float* gamma, float eps, const float* residual, float* y, size_t k,
                      hipStream_t s) {
  size_t n = 0;
  for (int i = 0; i < n_mats; i++) n += rows[i];
  if (n == 0) return WH_OK;
  if (n >= (1u << 30) || n_mats < 1 || n_mats > 3)
    return wh::set_error(WH_ERR_INVALID_SHAPE, "fused gemv: %zu rows (at most 2^30) over %d matrices (1 to 3)", n,
                         n_mats);
  GemvArgs a = plain_args(static_cast<const uint8_t*>(mats[0]), x, y, n);
  a.n0 = static_cast<int>(rows[0]);
  a.n1 = n_mats > 1 ? static_cast<int>(rows[1]) : 0;
  a.W2 = n_mats > 1 ? static_cast<const uint8_t*>(mats[1]) : a.W;
  a.W3 = n_mats > 2 ? static_cast<const uint8_t*>(mats[2]) : a.W2;
  a.gamma = gamma;
  a.eps = eps;
  a.residual = residual;
  if (use_mfma(type, n, k)) {
    const int st = launch_gemv_mfma(type, mats, rows, n_mats, false, x, gamma, eps, residual, y, n, k, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  if (is_kquant(type)) {
    // the dequantize-then-dot kernel per matrix (the caller normalises x first)
    if (gamma)
      return wh::set_error(WH_ERR_INVALID_SHAPE, "fused gemv: RMSNorm not fused for this K-quant shape (k = %zu)", k);
    size_t off = 0;
    for (int i = 0; i < n_mats; i++) {
      const int st = launch_gemv_kquant(type, mats[i], x, y + off, rows[i], k, s, residual ? residual + off : nullptr);
      if (st) return st;
      off += rows[i];
    }
    return WH_OK;
  }
  // Without the normalisation the generic kernel takes every shape; with it,
  // the caller normalises x first when the streaming kernels do not apply.
  const int mode = (gamma ? kNorm : 0) | (residual ? kResid : 0) | (n_mats > 1 ? kStack : 0);
  switch (type) {
    case WH_TYPE_Q4_0:
      if (stream_ok<WH_TYPE_Q4_0, false>(a, k)) return launch_fused_mode<WH_TYPE_Q4_0>(a, k, mode, s);
      return gamma ? wh::set_error(WH_ERR_INVALID_SHAPE, "fused gemv: RMSNorm not fused for this shape (k = %zu)", k)
                   : launch_generic<WH_TYPE_Q4_0>(a, k, s);
    case WH_TYPE_Q4_1:
      if (stream_ok<WH_TYPE_Q4_1, false>(a, k)) return launch_fused_mode<WH_TYPE_Q4_1>(a, k, mode, s);
      return gamma ? wh::set_error(WH_ERR_INVALID_SHAPE, "fused gemv: RMSNorm not fused for this shape (k = %zu)", k)
                   : launch_generic<WH_TYPE_Q4_1>(a, k, s);
    case WH_TYPE_Q8_0:
      if (stream_ok<WH_TYPE_Q8_0, false>(a, k)) return launch_fused_mode<WH_TYPE_Q8_0>(a, k, mode, s);
      return gamma ? wh::set_error(WH_ERR_INVALID_SHAPE, "fused gemv: RMSNorm not fused for this shape (k = %zu)", k)
                   : launch_generic<WH_TYPE_Q8_0>(a, k, s);
    default:
      return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "gemv: unsupported type %d", type);
  }
}

int launch_gemv(int type, const void* w, const float* x, float* y, size_t n_rows, size_t k,
                hipStream_t s) {
  if (n_rows == 0) return WH_OK;
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  switch (type) {
    case WH_TYPE_Q4_0: return launch_typed<WH_TYPE_Q4_0>(wp, x, y, n_rows, k, s);
    case WH_TYPE_Q4_1: return launch_typed<WH_TYPE_Q4_1>(wp, x, y, n_rows, k, s);
    case WH_TYPE_Q8_0: return launch_typed<WH_TYPE_Q8_0>(wp, x, y, n_rows, k, s);
    case WH_TYPE_Q4_K:
    case WH_TYPE_Q6_K:
      if (use_mfma(type, n_rows, k)) {
        const void* mats[1] = {w};
        const size_t rows[1] = {n_rows};
        const int st = launch_gemv_mfma(type, mats, rows, 1, false, x, nullptr, 0.f, nullptr, y, n_rows, k, s);
        if (st != WH_ERR_INVALID_SHAPE) return st;
      }
      return launch_gemv_kquant(type, w, x, y, n_rows, k, s);
    default: return wh::set_error(WH_ERR_UNSUPPORTED_TYPE, "gemv: unsupported type %d", type);
  }
}

}  // namespace wh
