// gemv_mfma_dev.hpp -- device helpers, formats and launch arguments shared by
// the matrix-core GEMV kernels: the single-token kernels (gemv_mfma.hip) and the
// several-token kernels (gemv_mt.hpp, one translation unit per block type so
// that they compile in parallel).  The arithmetic and data flow are described
// at the top of gemv_mfma.hip.
#pragma once
#include "wh_blocks.hpp"

namespace wh {
// Output rows [0, n_out).  Plain mode: row r is row r of the matrices W0, W1,
// W2 stacked (n0 rows of W0, n1 of W1, the rest of W2).  FFN mode: W0 = gate,
// W1 = up, y[r] = silu(gate_r . x_hat) * (up_r . x_hat).  gamma set: x is
// RMS-normalised first; residual set: y[r] = residual[r] + (W x)[r].
struct MgArgs {
  const uint8_t* W0;
  const uint8_t* W1;
  const uint8_t* W2;
  int n0, n1;
  const float* x;
  const float* gamma;
  float eps;
  const float* residual;
  float* y;
  int n_out, ppr, seg_pairs, rows_per_wg;
  int m, ldy;  // several-token kernel: tokens (rows of x, K apart) and the row stride of y
};
}  // namespace wh

typedef int mg_v4i __attribute__((ext_vector_type(4)));

// raw buffer load of 16 bytes (llvm.amdgcn.raw.buffer.load.v4i32)
__device__ mg_v4i mg_buffer_load_x4(mg_v4i rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

namespace {

// Every argument is requested at once, in one burst of scalar loads.  Left to
// itself the compiler reads each field where a branch first needs it, which
// makes the kernel-argument reads a chain of dependent round trips (each a
// load and a wait) ahead of the first weight load.  The empty asm statement
// takes every field as an input, so all of them are loaded before it; it
// modifies none, so the compiler may still keep or re-read each as it likes.
__device__ __forceinline__ void mg_args_now(const wh::MgArgs& a) {
  asm volatile("" ::"s"(a.W0), "s"(a.W1), "s"(a.W2), "s"(a.x), "s"(a.gamma), "s"(a.residual), "s"(a.y));
  asm volatile("" ::"s"(a.n0), "s"(a.n1), "s"(a.eps), "s"(a.n_out), "s"(a.ppr), "s"(a.seg_pairs),
               "s"(a.rows_per_wg), "s"(a.m), "s"(a.ldy));
}

// A weight pointer held in scalar registers for the whole kernel: a choice
// between the argument's pointers (W0 / W1 / W2 by row) is otherwise compiled
// as a kernel-argument load at a computed offset, one more round trip before
// the first weight load.  Returned as a generic pointer made from a global one,
// so the loads through it stay global loads.
__device__ __forceinline__ const uint8_t* mg_ptr_now(const uint8_t* p) {
  const uint64_t w = reinterpret_cast<uint64_t>(p);
  uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(w));
  uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(w >> 32));
  asm volatile("" : "+s"(lo), "+s"(hi));
  using G = __attribute__((address_space(1))) const uint8_t;
  return (const uint8_t*)(G*)((static_cast<uint64_t>(hi) << 32) | lo);
}

// Buffer resource of a raw byte range: loads at offsets >= nbytes return 0
// without a memory access.
__device__ __forceinline__ mg_v4i mg_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  mg_v4i r;
  r[0] = static_cast<int>(static_cast<uint32_t>(a));
  r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xFFFFu);  // stride 0
  r[2] = static_cast<int>(nbytes);
  r[3] = 0x00020000;  // 32-bit data format, raw access
  return r;
}

constexpr int kMgWaves = 16;                   // waves per workgroup
constexpr int kMgSegMax = 16 * 64 * 4;        // bytes of one row segment (at most 4 loads)
// LDS row stride of a ring slot: the segment (and its lead room) rounded up
// to an odd number of 16-byte units, so that the 16 rows of a step start in
// 16 different bank quads.  Callers include 16 bytes of overflow room in
// lead_room: lanes whose 16-byte piece lies past the segment store it there
// (it is zeros: the buffer range ends at the segment), so that the copy into
// LDS needs no branch.
__host__ __device__ constexpr uint32_t mg_row_stride(uint32_t seg_bytes, uint32_t lead_room) {
  return ((seg_bytes + 15u) & ~15u) + lead_room + (((((seg_bytes + 15u) & ~15u) + lead_room) >> 4) & 1u ? 0u : 16u);
}
constexpr int kMgLimbBytes = 4 * 32;            // four limbs of one block
// limb staging bytes per chunk: the limbs, then the limb sums of each
// 32-element block
constexpr int mg_stage_bytes(int type) { return 8 * kMgLimbBytes + (type == WH_TYPE_Q6_K ? 0 : 8 * 16); }
// several-token kernel: the limbs of one chunk, or of both tokens' chunks in
// the two-token layout
constexpr int mt_stage_bytes(int type, int mt) { return mt == 2 ? 16 * kMgLimbBytes : mg_stage_bytes(type); }
constexpr int kMgNt = 2;                       // streaming (non-temporal) loads
constexpr int kMgNorm = 1, kMgFfn = 2;         // kernel variants
constexpr int kMgDepth1 = 1;                   // steps in flight for one-segment rows

template <int TYPE>
struct MgFmt;
template <>
struct MgFmt<WH_TYPE_Q4_0> {
  static constexpr int PB = 36;  // bytes of two blocks
};
template <>
struct MgFmt<WH_TYPE_Q4_1> {
  static constexpr int PB = 40;
};
template <>
struct MgFmt<WH_TYPE_Q8_0> {
  static constexpr int PB = 68;
};
template <>
struct MgFmt<WH_TYPE_Q4_K> {
  static constexpr int PB = 0;  // not used: one 144-byte block per chunk
};
template <>
struct MgFmt<WH_TYPE_Q6_K> {
  static constexpr int PB = 0;  // not used: one 210-byte block per chunk
};

// bytes of one 256-weight chunk of a format the kernel takes; 0 otherwise
constexpr int mg_chunk_bytes(int type) {
  return type == WH_TYPE_Q4_0 ? 144
         : type == WH_TYPE_Q4_1 ? 160
         : type == WH_TYPE_Q8_0 ? 272
         : type == WH_TYPE_Q4_K ? 144
         : type == WH_TYPE_Q6_K ? 210
                                : 0;
}

using wh::MgArgs;

// k-slot (0..7) of lane group g that element el (0..31) of a block feeds:
// Q4: slots 0..3 = low nibbles of quant bytes 4g..4g+3 (elements 4g..4g+3),
// slots 4..7 = their high nibbles (elements 16+4g..); Q8_0 and Q6_K: element
// 8g + slot.
// Q4_K: quant byte 4g + b of a group holds elements 8g + 2b (low nibble, slot
// b) and 8g + 2b + 1 (high nibble, slot 4 + b).
template <int TYPE>
__device__ __forceinline__ int mg_slot_offset(int el) {
  if constexpr (TYPE == WH_TYPE_Q8_0 || TYPE == WH_TYPE_Q6_K) return el;
  if constexpr (TYPE == WH_TYPE_Q4_K) return 8 * (el >> 3) + ((el & 1) ? 4 : 0) + ((el & 7) >> 1);
  return 8 * ((el & 15) >> 2) + (el & 3) + (el >= 16 ? 4 : 0);
}

// B operand of lane group g for the two blocks of the pair at pw (LDS).
template <int TYPE>
__device__ __forceinline__ void mg_quants(const uint32_t* pw, int g, long& qa, long& qb) {
  auto split = [](uint32_t u) -> long {
    return static_cast<long>(u & 0x0F0F0F0Fu) | (static_cast<long>((u >> 4) & 0x0F0F0F0Fu) << 32);
  };
  if constexpr (TYPE == WH_TYPE_Q4_0) {
    // [dA|q0 q1] [q2..5] .. [q14 q15|dB] [B q0..3] ..: quant bytes 4g..4g+3 of block A
    // start at byte 2 + 4g
    qa = split(__builtin_amdgcn_alignbit(pw[g + 1], pw[g], 16));
    qb = split(pw[5 + g]);
  } else if constexpr (TYPE == WH_TYPE_Q4_1) {
    // [dA|mA] [A q0..3] .. [A q12..15] [dB|mB] [B q0..3] ..
    qa = split(pw[1 + g]);
    qb = split(pw[6 + g]);
  } else {
    // [dA|q0 q1] [q2..5] .. [q30 q31|dB] [B q0..3] ..: quant bytes 8g..8g+7 of block A
    // start at byte 2 + 8g
    const uint32_t w0 = pw[2 * g], w1 = pw[2 * g + 1], w2 = pw[2 * g + 2];
    const uint32_t lo = __builtin_amdgcn_alignbit(w1, w0, 16);
    const uint32_t hi = __builtin_amdgcn_alignbit(w2, w1, 16);
    qa = static_cast<long>(lo) | (static_cast<long>(hi) << 32);
    qb = static_cast<long>(pw[9 + 2 * g]) | (static_cast<long>(pw[10 + 2 * g]) << 32);
  }
}

// Per-element dot product of one pair (64 weights at byte pointer p, in LDS)
// with 64 activations (already RMS-normalised in the norm modes), xs(jj)
// giving elements 4 jj .. 4 jj + 3: w = (q - 8) * d, q * d + m or q * d as in
// dequantize_q4_0 / _q4_1 / _q8_0, then w * x accumulated in element order.
// Used for chunks with non-finite activations.
template <int TYPE, typename XS>
__device__ float mg_pair_exact(const uint8_t* p, XS xs) {
  constexpr int BB = whd::BlockFmt<TYPE>::BYTES;
  float s = 0.f;
#pragma unroll 1
  for (int blk = 0; blk < 2; blk++) {
    const uint8_t* b = p + blk * BB;
    const float d = whd::f16_bits_to_f32(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
    float m = 0.f;
    if constexpr (TYPE == WH_TYPE_Q4_1)
      m = whd::f16_bits_to_f32(static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8));
#pragma unroll 1
    for (int jj = 0; jj < 8; jj++) {
      const float4 xq = xs(8 * blk + jj);
      const float xa[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
      for (int c = 0; c < 4; c++) {
      const int el = 4 * jj + c;
      float w;
      if constexpr (TYPE == WH_TYPE_Q4_0) {
        const uint32_t q = b[2 + (el & 15)];
        w = static_cast<float>(static_cast<int>(el < 16 ? (q & 15u) : (q >> 4)) - 8) * d;
      } else if constexpr (TYPE == WH_TYPE_Q4_1) {
        const uint32_t q = b[4 + (el & 15)];
        w = __fadd_rn(__fmul_rn(static_cast<float>(el < 16 ? (q & 15u) : (q >> 4)), d), m);
      } else {
        w = static_cast<float>(static_cast<int8_t>(b[2 + el])) * d;
      }
      s = __builtin_fmaf(w, xa[c], s);
      }
    }
  }
  return s;
}

// 6-bit scale j (0..7) of a Q4_K block (dequantize.rs:423-431): src = 3j/2,
// even j: b[src] & 63, odd j: ((b[src] >> 6) | ((b[src + 1] & 15) << 2)) & 63.
__device__ __forceinline__ uint32_t mg_q4k_scale(const uint8_t* b, int j) {
  const int src = (3 * j) >> 1;
  return (j & 1) ? (((static_cast<uint32_t>(b[src]) >> 6) | ((static_cast<uint32_t>(b[src + 1]) & 15u) << 2)) & 63u)
                 : (static_cast<uint32_t>(b[src]) & 63u);
}

// Q4_K counterpart of mg_pair_exact: elements 64 g .. 64 g + 63 of the block at
// blk, w = ((d * s) * q) + dmin as dequantize_q4_k_scalar evaluates it.
template <typename XS>
__device__ float mg_q4k_exact(const uint8_t* blk, int g, XS xs) {
  const float d = whd::f16_bits_to_f32(static_cast<uint32_t>(blk[12]) | (static_cast<uint32_t>(blk[13]) << 8));
  const float dmin = whd::f16_bits_to_f32(static_cast<uint32_t>(blk[14]) | (static_cast<uint32_t>(blk[15]) << 8));
  float s = 0.f;
#pragma unroll 1
  for (int jj = 0; jj < 16; jj++) {
    const float4 xq = xs(jj);
    const float xa[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
    const int el = 4 * jj + c;
    const int i = 64 * g + el;
    const float ds = __fmul_rn(d, static_cast<float>(mg_q4k_scale(blk, i >> 5)));
    const uint32_t qb = blk[16 + (i >> 1)];
    const float w = __fadd_rn(__fmul_rn(ds, static_cast<float>((i & 1) ? (qb >> 4) : (qb & 15u))), dmin);
    s = __builtin_fmaf(w, xa[c], s);
    }
  }
  return s;
}

// Q6_K counterpart of mg_pair_exact: elements 64 g .. 64 g + 63 of the block
// at blk, w = ((d * s) * (q - 32)) / 64 as dequantize_q6_k evaluates it.
template <typename XS>
__device__ float mg_q6k_exact(const uint8_t* blk, int g, XS xs) {
  const float d = whd::f16_bits_to_f32(static_cast<uint32_t>(blk[208]) | (static_cast<uint32_t>(blk[209]) << 8));
  float s = 0.f;
#pragma unroll 1
  for (int jj = 0; jj < 16; jj++) {
    const float4 xq = xs(jj);
    const float xa[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
    const int el = 4 * jj + c;
    const int i = 64 * g + el;
    const int ql_idx = 64 * (i >> 7) + 32 * ((i & 127) >> 6) + 16 * ((i & 63) >> 5) + (i & 15);
    const int qh_idx = 32 * (i >> 7) + 16 * ((i & 127) >> 6) + 8 * ((i & 63) >> 5) + ((i & 31) >> 2);
    const int sh = 2 * (i & 3);
    const uint32_t qhv = blk[128 + qh_idx];
    uint32_t q;
    if (i < 128) {
      q = (blk[ql_idx] & 15u) | (((qhv >> sh) & 3u) << 4);
    } else {
      const uint32_t e2 = sh < 6 ? ((qhv >> (sh + 2)) & 3u) : (qh_idx + 1 < 64 ? (blk[129 + qh_idx] & 3u) : 0u);
      q = (static_cast<uint32_t>(blk[ql_idx]) >> 4) | (e2 << 4);
    }
    const float w = __fmul_rn(__fmul_rn(__fmul_rn(d, static_cast<float>(blk[192 + (i >> 4)])),
                                        static_cast<float>(static_cast<int>(q) - 32)),
                              0.015625f);
    s = __builtin_fmaf(w, xa[c], s);
    }
  }
  return s;
}

// Two dwords of LDS bytes at p, which lies mis (0 or 2) bytes past a dword
// boundary.  Pointer arithmetic only: an integer round trip would turn the
// LDS reads into flat loads, which wait behind the global loads in flight.
__device__ __forceinline__ void mg_lds_u64(const uint8_t* p, int mis, uint32_t& lo, uint32_t& hi) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(p - mis);
  const uint32_t sh = static_cast<uint32_t>(mis) * 8u;
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
  lo = __builtin_amdgcn_alignbit(w1, w0, sh);
  hi = __builtin_amdgcn_alignbit(w2, w1, sh);
}

// Cross-lane moves on the VALU (DPP) instead of ds_bpermute shuffles, which
// go through the LDS pipe.
template <int CTRL>
__device__ __forceinline__ int mg_dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E;  // quad_perm [1,0,3,2], [2,3,0,1]
constexpr int kDppHalfMirror = 0x141, kDppMirror = 0x140;  // lane i <-> 7 - i (of 8), 15 - i (of 16)

// Maximum of an unsigned integer over the 64 lanes, uniform: one DPP max per
// step within rows of 16 lanes, then the four rows' maxima on the scalar unit.
__device__ __forceinline__ uint32_t mg_wave_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(mg_dpp<kDppXor1>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(mg_dpp<kDppXor2>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(mg_dpp<kDppHalfMirror>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(mg_dpp<kDppMirror>(static_cast<int>(v))));
  const int vi = static_cast<int>(v);
  const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(vi, 0));
  const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(vi, 16));
  const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(vi, 32));
  const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(vi, 48));
  return max(max(r0, r1), max(r2, r3));
}

// f32 -> i32 as v_cvt_i32_f32 converts (NaN -> 0, out of range -> clamped),
// with no C++ undefined behaviour for such inputs: the limbs of a chunk that
// takes the exact path are converted too (without a branch) and never read.
__device__ __forceinline__ int mg_cvt_i32(float v) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// Sum over the four lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48) in every
// lane, as (v[l] + v[l ^ 16]) + (v[l ^ 32] + v[l ^ 48]), with gfx950's
// v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip).  Inline asm
// with explicit wait states around each swap: the builtins' code returned one
// register for both swapped halves.
__device__ __forceinline__ float mg_sum_lane_groups(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  v = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  a = b = __builtin_bit_cast(uint32_t, v);
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// The four limb sums of one block as one f32, 2^24 C0 + 2^16 C1 + 2^8 C2 + C3:
// the halves 2^8 C0 + C1 and 2^8 C2 + C3 in int32 (exact and without overflow:
// |C| < 2^20: each sum covers one 32-element block), converted (exactly for the 4-bit
// formats, whose halves stay below 2^24) and combined with one fma.
__device__ __forceinline__ float mg_limbs(const mg_v4i& C) {
  const int hi = C[0] * 256 + C[1];
  const int lo = C[2] * 256 + C[3];
  return __builtin_fmaf(static_cast<float>(hi), 65536.f, static_cast<float>(lo));
}

// Bits 2t .. 2t + 1 of v (t = 0..3) moved to bits 4..5 of byte t.
__device__ __forceinline__ uint32_t mg_spread2(uint32_t v) {
  return ((v << 4) | (v << 10) | (v << 16) | (v << 22)) & 0x30303030u;
}


// ---------------------------------------------------------------- several tokens
// The matrix-core GEMV for 2..16 tokens: Y[t] = W X[t] (plain mode) or the FFN
// gate/up pair with each token's RMSNorm prologue and the SwiGLU epilogue (FFN
// mode), in the data flow of gemv_mfma_kernel.  The A operand of one MFMA
// carries the limbs of four tokens for ONE 32-element block (rows 4 t + limb,
// t = token within its group of four), so each block's weights, unpacked
// once, meet one MFMA per group of four tokens and stream from HBM once for
// all tokens; lane group g of the result holds token 4 tg + g's four limb sums
// of the block.  The A operands of every segment stay in registers
// (TG * NSEG <= 4).  Per format:
//   Q4_0: the -8 goes into the B operand: nibble ^ 8 read as a signed 4-bit
//         number is q - 8, kept in the high half of each byte (16 (q - 8), an
//         exact int8), and the block scale enters as d / 16;
//   Q8_0: the quants as they are, scale d;
//   Q4_1: the nibbles q, scale d, and the minimum as m * (block sum of x);
//   Q4_K: the eight 32-element scale groups of the 256-element block take the
//         place of blocks, scale d * s_j (exact), and dmin * (sum of x over
//         the block);
//   Q6_K: one 32-element K-step j of the block per MFMA pair: the B operand
//         holds q - 32 as a signed byte (a byte-permute lookup of the two high
//         bits), and the per-16 scales take two MFMAs whose B operands keep
//         only the lanes of one half (k-slots 16 h .. 16 h + 15), scale
//         d * s / 64 (exact).
// The block sums of x (Q4_1 per block, Q4_K per block of 256) are limb sums
// formed once per chunk by MFMAs of the A operands against a B operand of
// ones, kept per wave in LDS.
// MS = 2 (two tokens, 32-element formats and Q4_K): rows 8 (b & 1) + 4 t +
// limb, so blocks 2p and 2p + 1 share one accumulator and lane group g holds
// token g & 1 of block 2p + (g >> 1), half the accumulator conversions of the
// four-token layout.
template <int TYPE>
constexpr bool mt_type_ok() {
  return TYPE == WH_TYPE_Q4_0 || TYPE == WH_TYPE_Q4_1 || TYPE == WH_TYPE_Q8_0 || TYPE == WH_TYPE_Q4_K ||
         TYPE == WH_TYPE_Q6_K;
}
// formats whose minimum needs the sums of x: Q4_1 per block, Q4_K per block of 256
constexpr bool mt_xsum(int type) { return type == WH_TYPE_Q4_1 || type == WH_TYPE_Q4_K; }
// bytes of one wave's block sums of x: [segment][token][8 blocks] floats
constexpr int mt_xsum_bytes(int type, int nseg, int mt) { return mt_xsum(type) ? nseg * mt * 8 * 4 : 0; }

}  // namespace

namespace wh {
// The several-token launches of one block type (gemv_mt_<type>.hip): plain
// (mats = {W}) or FFN (mats = {gate, up}) mode, the segments, token groups,
// grid and LDS bytes chosen by launch_gemv_mt.
int launch_gemv_mt_q4_0(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s);
int launch_gemv_mt_q4_1(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s);
int launch_gemv_mt_q8_0(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s);
int launch_gemv_mt_q4_k(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s);
int launch_gemv_mt_q6_k(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s);
}  // namespace wh
