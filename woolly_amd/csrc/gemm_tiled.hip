// gemm_tiled.hip -- quantized prefill GEMM Y = X W^T on gfx950, 16x16x32 MFMA.
//
// Replaces the projections woolly computes on fully dequantized f32 weights
// (simd_matmul_optimized -> Gemm::compute, tensor_utils_simd.rs:855-914,
// ops/matmul.rs:83-259, called from simd_ffn_forward tensor_utils_simd.rs:605-754):
//   Y[t, r] = sum_k X[t, k] * W[r, k],  W in GGUF Q4_0 / Q4_1 / Q8_0 blocks.
//
// Numerics (same contract as the 32x32 kernel in gemm.hip).  Each activation
// row is scaled by a power of two (largest magnitude in [2^13, 2^14)) and
// split into fp16 hi and lo halves; weight quants are exact fp16 integers
// (q - 8, q, or the int8 value).  One v_mfma_f32_16x16x32_f16 covers exactly
// one 32-element block: the hi and lo products accumulate into a fresh f32
// tile and the block scale is applied in f32,
//   acc += d * (q . hi + q . lo)                 (Q4_0, Q8_0)
//   acc += d * (q . hi + q . lo) + m * sum(x)    (Q4_1)
//
// Data flow.
//   pack_a_kernel writes the activations pre-swizzled into MFMA fragment order:
//     fragment (token tile T, block b, 16-token group i, limb) = 16 tokens x
//     4 k-groups x 8 halves = 1 KiB, token-major (a token's 64 bytes are
//     contiguous, so a packing workgroup writes whole segments); the copy into
//     LDS reads them in MFMA lane order (lane l: token 16i + l%16, k-group
//     l/16).  The k-slots follow the order in which a weight lane unpacks its
//     nibbles, so the copied fragment feeds the MFMA directly.
//   gemm_tiled_kernel: 512 threads, a BM-token x 256-row tile (BM = 16, 32,
//     64 or 128 from the token count, so small batches do not multiply
//     padding), two waves per SIMD.  Stages of two blocks are copied
//     global -> LDS with global_load_lds (activation fragments as 16-byte
//     lanes, raw weight bytes as 4-byte lanes); NSTAGE stages rotate so that
//     NSTAGE - 1 are in flight while one is computed.  Each lane unpacks its
//     weight quants from LDS into fp16 with bit operations (magic-number
//     conversion, exact), multiplies, and applies the block scale.
//   Tiles are numbered so that the tiles resident on one XCD share a token
//     tile, whose activation fragments then stay in that XCD's L2.
#include "wh_blocks.hpp"

#include <atomic>

// raw buffer load / store of 16 bytes (llvm.amdgcn.raw.buffer.{load,store}.v4f32)
__device__ float __attribute__((ext_vector_type(4))) gt_buffer_load_x4(int __attribute__((ext_vector_type(4))) rsrc,
                                                                       int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4f32");
__device__ void gt_buffer_store_x4(float __attribute__((ext_vector_type(4))) v, int __attribute__((ext_vector_type(4))) rsrc,
                                   int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.store.v4f32");

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int TBN = 256;              // weight rows per tile
constexpr int TWAVES = 8;             // 2 per SIMD
constexpr int SB = 2;                 // blocks per stage
constexpr int FRAG = 1024;            // bytes per activation fragment (16 tokens x 32 k, one limb)

// Wave grid per token-tile height BM: WGM x WGN waves, each a (BM / WGM) x
// (TBN / WGN) tile of 16 x 16 MFMA tiles.
template <int BM>
struct TCfg {
  static constexpr int WGM = BM == 128 ? 2 : 1;
  static constexpr int WGN = TWAVES / WGM;
  static constexpr int WTM = BM / WGM, WTN = TBN / WGN;
  static constexpr int IT = WTM / 16, NT = WTN / 16;
  static constexpr int FPB = BM / 8;                       // fragments per block (groups x limbs)
  static constexpr int A_STAGE = SB * FPB * FRAG;
};

template <int TYPE>
struct TFmt;
template <>
struct TFmt<WH_TYPE_Q4_0> {
  static constexpr int TS = 18, QOFF = 2;
};
template <>
struct TFmt<WH_TYPE_Q4_1> {
  static constexpr int TS = 20, QOFF = 4;
};
template <>
struct TFmt<WH_TYPE_Q8_0> {
  static constexpr int TS = 34, QOFF = 2;
};
// the repacked K-quant formats (f32 scale)
template <>
struct TFmt<wh::kGemmQ4F> {
  static constexpr int TS = 20, QOFF = 4;
};
template <>
struct TFmt<wh::kGemmQ8H> {
  static constexpr int TS = 20, QOFF = 4;
};
// block value d q + m (Q4_1): the m of each block are collected, as the
// stages stream past, into the B operand of products against the
// activations' block sums, over windows of 32 blocks
template <int TYPE>
constexpr bool has_min() { return TYPE == WH_TYPE_Q4_1; }
// int8 quants in natural element order (else 4-bit quants in nibble order)
template <int TYPE>
constexpr bool q8_like() { return TYPE == WH_TYPE_Q8_0 || TYPE == wh::kGemmQ8H; }
// f32 block scale (else f16)
template <int TYPE>
constexpr bool f32_scale() { return TYPE == wh::kGemmQ4F || TYPE == wh::kGemmQ8H; }
// the packing writes the activations' sums over each unit of the minimum
// term (Q4_1: 32-element block; kGemmQ4F: 256-element super-block) as two
// fp16 limbs, rows of units rounded up to 8
inline bool needs_bsum(int type) { return type == WH_TYPE_Q4_1 || type == wh::kGemmQ4F; }
// units per token row in the sums' layout (4 bytes each: two fp16 limbs)
inline size_t bsum_groups(int type, size_t k) {
  return type == wh::kGemmQ4F ? wh::q4f_dmin_stride(k) : (k / 32 + 7) / 8 * 8;
}
// dwords per weight row per stage (SB whole blocks)
template <int TYPE>
constexpr int dwb() { return SB * TFmt<TYPE>::TS / 4; }
static_assert(SB * 18 % 4 == 0 && SB * 34 % 4 == 0, "stage rows must be whole dwords");

// raw weight dwords per stage, rounded up to whole copy instructions
template <int TYPE>
constexpr int b_dma_per_wave() { return (TBN * dwb<TYPE>() + TWAVES * 64 - 1) / (TWAVES * 64); }
template <int TYPE>
constexpr int b_stage_bytes() { return b_dma_per_wave<TYPE>() * TWAVES * 64 * 4; }
template <int TYPE, int BM>
constexpr int stage_bytes() { return TCfg<BM>::A_STAGE + b_stage_bytes<TYPE>(); }
// Copy instructions per wave per stage (the vmcnt of one stage): activation
// fragments, raw weight dwords.
template <int TYPE, int BM>
constexpr int per_stage() {
  return (SB * TCfg<BM>::FPB + TWAVES - 1) / TWAVES + b_dma_per_wave<TYPE>();
}
// Ring depth: as many stages as 160 KiB of LDS holds, 3 to 8 (a deeper ring
// keeps more weight bytes in flight where a stage is small), with the copies
// of the stages in flight behind the one awaited countable by vmcnt (< 64).
template <int TYPE, int BM>
constexpr int nstage() {
  constexpr int n = 160 * 1024 / stage_bytes<TYPE, BM>();
  constexpr int v = 2 + 63 / per_stage<TYPE, BM>();
  constexpr int m = n < v ? n : v;
  return m < 3 ? 3 : (m > 8 ? 8 : m);
}
template <int TYPE, int BM>
constexpr size_t tiled_lds_bytes() { return static_cast<size_t>(nstage<TYPE, BM>()) * stage_bytes<TYPE, BM>(); }

// K-slot order of an MFMA operand: k-slot s (0..7) of k-group g (0..3) holds
// block element 8g + s for the int8 formats, and for the 4-bit formats element
// (s < 4 ? 0 : 16) + 4g + {0, 2, 1, 3}[s % 4], the order unpack_q4 below
// produces the quants in.

// ---------------------------------------------------------------- packing
// One workgroup per token row t of the padded tile grid (token tiles of bm
// rows).  Rows t >= n_tokens are written as zeros.  rscale[t] = 2^e with
// max|x_t| * 2^-e in [2^13, 2^14); bsum = the sums S of hi + lo over each
// unit of the minimum term (Q4_1: 32-element block; kGemmQ4F: 256-element
// super-block) as the A operand of its products: fp16 limbs
// hi = fp16(S 2^-10), lo = fp16(S 2^-10 - hi) (|S| < 2^22, so no overflow),
// laid out [t][limb][units rounded up to 8], zero past the row's units.
// Thread p of a chunk owns the (block, k-group) pairs p, p + NTH, ... (NTH =
// blockDim.x, 256 .. 1024 by the row length): the 8 elements of a pair are
// two float4 loads (slot_elem order), all issued before the first use; a row
// of up to NTH * PPT pairs is read once and packed from registers, longer
// rows are read again per pass.
// MODE: the row packed is x itself (kPackPlain); the RMSNorm of x,
// (x / sqrt(sum x^2 / k + eps)) * gamma as rms_norm computes it
// (tensor_utils.rs:446-480; kPackNorm); or the SwiGLU of two rows,
// (g * (1 / (1 + exp(-g)))) * u with g = x, u = x2 (tensor_utils.rs:512-532;
// kPackSwiglu).  The FFN's elementwise steps thereby never go through HBM.
// Rows of x are kx long; k is the packed length: kx, or 2 kx for kGemmQ8H,
// whose 32-element blocks hold 16 elements of x and 16 zeros.
constexpr int PPT = 2;
constexpr int kPackMaxThreads = 1024;
constexpr int kPackPlain = 0, kPackNorm = 1, kPackSwiglu = 2;
// XB: x holds bfloat16 values (plain mode), widened exactly to f32 on load.
template <int MODE, bool XB = false>
__global__ __launch_bounds__(kPackMaxThreads) void pack_a_kernel(const float* __restrict__ x, const float* __restrict__ x2,
                                                     const float* __restrict__ gamma, float eps, int n_tokens,
                                                     int k, int kx, int type, int bm, _Float16* __restrict__ frag,
                                                     float* __restrict__ rscale, float* __restrict__ bsum,
                                                     uint32_t* __restrict__ sk_flags, int sk_n) {
  // the stream-K flags of the GEMMs that read this packing start cleared
  if (blockIdx.x == 0)
    for (int i = static_cast<int>(threadIdx.x); i < sk_n; i += static_cast<int>(blockDim.x)) sk_flags[i] = 0u;
  __shared__ float red[kPackMaxThreads / 64];
  __shared__ float red2[kPackMaxThreads / 64];
  const int NTH = static_cast<int>(blockDim.x), nw = NTH >> 6;
  const int t = blockIdx.x;
  const bool live = t < n_tokens;
  const float* xr = x + static_cast<size_t>(live ? t : 0) * kx;
  const float* ur = MODE == kPackSwiglu ? x2 + static_cast<size_t>(live ? t : 0) * kx : nullptr;
  const int nb = k / 32, npairs = nb * 4;
  const int nchunks = (npairs + NTH * PPT - 1) / (NTH * PPT);
  const bool q8 = type == WH_TYPE_Q8_0 || type == wh::kGemmQ8H;
  const bool pad = type == wh::kGemmQ8H;
  // offset in the row of x of pair (b, g)'s first element, -1 for padding
  auto elem_off = [&](int b, int g) { return pad ? (g < 2 ? 16 * b + 8 * g : -1) : 32 * b + (q8 ? 8 * g : 4 * g); };
  float4 va[PPT], vb[PPT];
  auto load = [&](int c) {
#pragma unroll
    for (int i = 0; i < PPT; i++) {
      const int p = c * NTH * PPT + NTH * i + static_cast<int>(threadIdx.x);
      va[i] = vb[i] = float4{0.f, 0.f, 0.f, 0.f};
      const int off = p < npairs ? elem_off(p >> 2, p & 3) : -1;
      if (live && off >= 0) {
        const float* src = xr + off;
        if constexpr (XB) {
          // row t of bf16 x: element e at byte 2 (t kx + e)
          const uint16_t* xb = reinterpret_cast<const uint16_t*>(x) + static_cast<size_t>(t) * kx + off;
          auto widen = [](uint2 u) {
            return float4{__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xFFFF0000u),
                          __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xFFFF0000u)};
          };
          va[i] = widen(*reinterpret_cast<const uint2*>(xb));
          vb[i] = widen(*reinterpret_cast<const uint2*>(xb + (q8 ? 4 : 16)));
        } else {
        va[i] = *reinterpret_cast<const float4*>(src);
        vb[i] = *reinterpret_cast<const float4*>(src + (q8 ? 4 : 16));
        }
        if constexpr (MODE == kPackSwiglu) {
          const float* us = ur + (src - xr);
          const float4 ua = *reinterpret_cast<const float4*>(us);
          const float4 ub = *reinterpret_cast<const float4*>(us + (q8 ? 4 : 16));
          auto h = [](float g, float u) { return (g * (1.0f / (1.0f + expf(-g)))) * u; };
          va[i] = float4{h(va[i].x, ua.x), h(va[i].y, ua.y), h(va[i].z, ua.z), h(va[i].w, ua.w)};
          vb[i] = float4{h(vb[i].x, ub.x), h(vb[i].y, ub.y), h(vb[i].z, ub.z), h(vb[i].w, ub.w)};
        }
      }
    }
  };
  // RMSNorm: the row's rms first, then x_hat = (x / rms) * gamma in place of x
  float rms = 1.f;
  auto normalise = [&](int c) {
    if constexpr (MODE == kPackNorm) {
#pragma unroll
      for (int i = 0; i < PPT; i++) {
        const int p = c * NTH * PPT + NTH * i + static_cast<int>(threadIdx.x);
        const int off = p < npairs ? elem_off(p >> 2, p & 3) : -1;
        if (!live || off < 0) continue;
        const float* gs = gamma + off;
        const float4 ga = *reinterpret_cast<const float4*>(gs);
        const float4 gb = *reinterpret_cast<const float4*>(gs + (q8 ? 4 : 16));
        va[i] = float4{(va[i].x / rms) * ga.x, (va[i].y / rms) * ga.y, (va[i].z / rms) * ga.z, (va[i].w / rms) * ga.w};
        vb[i] = float4{(vb[i].x / rms) * gb.x, (vb[i].y / rms) * gb.y, (vb[i].z / rms) * gb.z, (vb[i].w / rms) * gb.w};
      }
    }
  };
  if constexpr (MODE == kPackNorm) {
    float ss = 0.f;
    for (int c = 0; c < nchunks; c++) {
      load(c);
#pragma unroll
      for (int i = 0; i < PPT; i++) {
        ss = __builtin_fmaf(va[i].x, va[i].x, ss); ss = __builtin_fmaf(va[i].y, va[i].y, ss);
        ss = __builtin_fmaf(va[i].z, va[i].z, ss); ss = __builtin_fmaf(va[i].w, va[i].w, ss);
        ss = __builtin_fmaf(vb[i].x, vb[i].x, ss); ss = __builtin_fmaf(vb[i].y, vb[i].y, ss);
        ss = __builtin_fmaf(vb[i].z, vb[i].z, ss); ss = __builtin_fmaf(vb[i].w, vb[i].w, ss);
      }
    }
    ss = whd::wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red2[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < nw; w++) tot += red2[w];
    rms = sqrtf(tot / static_cast<float>(kx) + eps);
  }
  float mx = 0.f;
  for (int c = 0; c < nchunks; c++) {
    if (MODE != kPackNorm || nchunks > 1) load(c);  // one chunk: still in registers
    normalise(c);
#pragma unroll
    for (int i = 0; i < PPT; i++)
      mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(va[i].x), fabsf(va[i].y)), fmaxf(fabsf(va[i].z), fabsf(va[i].w))),
                           fmaxf(fmaxf(fabsf(vb[i].x), fabsf(vb[i].y)), fmaxf(fabsf(vb[i].z), fabsf(vb[i].w)))));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = 0.f;
  for (int w = 0; w < nw; w++) mx = fmaxf(mx, red[w]);
  int e = 0;
  if (mx > 0.f && mx <= 3.4e38f) {
    int ex;
    frexpf(mx, &ex);          // mx = f * 2^ex, f in [0.5, 1)
    e = ex - 14;              // mx * 2^-e in [2^13, 2^14)
    if (e < -100) e = -100;
  }
  const float down = ldexpf(1.f, -e);
  if (threadIdx.x == 0) rscale[t] = ldexpf(1.f, e);
  const int T = t / bm, i16 = (t % bm) / 16, tl = t % 16, fpb = bm / 8;
  for (int c = 0; c < nchunks; c++) {
    if (nchunks > 1) {   // one chunk: its values are still in registers
      load(c);
      normalise(c);
    }
#pragma unroll
    for (int i = 0; i < PPT; i++) {
      const int p = c * NTH * PPT + NTH * i + static_cast<int>(threadIdx.x);
      if (p >= npairs) break;   // uniform across the four lanes of a block
      const int b = p >> 2, g = p & 3;
      // slot order: 4-bit formats {0, 2, 1, 3} within each half, Q8_0 natural
      float v[8];
      if (q8) {
        v[0] = va[i].x; v[1] = va[i].y; v[2] = va[i].z; v[3] = va[i].w;
        v[4] = vb[i].x; v[5] = vb[i].y; v[6] = vb[i].z; v[7] = vb[i].w;
      } else {
        v[0] = va[i].x; v[1] = va[i].z; v[2] = va[i].y; v[3] = va[i].w;
        v[4] = vb[i].x; v[5] = vb[i].z; v[6] = vb[i].y; v[7] = vb[i].w;
      }
      half8 hv, lv;
      float part = 0.f;
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const float sv = v[s] * down;  // exact scaling
        const _Float16 h = static_cast<_Float16>(sv);
        const _Float16 l = static_cast<_Float16>(sv - static_cast<float>(h));
        hv[s] = h;
        lv[s] = l;
        part += static_cast<float>(h) + static_cast<float>(l);
      }
      // token-major inside a fragment: token tl's four k-groups are 64
      // contiguous bytes (the copy into LDS puts them in MFMA lane order)
      const size_t base = ((static_cast<size_t>(T) * nb + b) * fpb + 2 * i16) * 512 + 8 * (4 * tl + g);
      *reinterpret_cast<half8*>(frag + base) = hv;          // limb 0 (hi)
      *reinterpret_cast<half8*>(frag + base + 512) = lv;    // limb 1 (lo)
      if (bsum) {
        // the unit's lanes: the four k-groups of a block are adjacent lanes
        // (p = 4 b + g); a super-block's 8 blocks are 32 adjacent lanes
        // (p = 32 sb + ..; rows are whole super-blocks, so all 32 are live)
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        const bool sup = type == wh::kGemmQ4F;
        if (sup) {
          part += __shfl_xor(part, 4, 64);
          part += __shfl_xor(part, 8, 64);
          part += __shfl_xor(part, 16, 64);
        }
        if ((p & (sup ? 31 : 3)) == 0) {
          const int nu = sup ? nb / 8 : nb, nup = (nu + 7) & ~7, u = sup ? b >> 3 : b;
          _Float16* sr = reinterpret_cast<_Float16*>(bsum) + static_cast<size_t>(t) * 2 * nup;
          const float sv = part * 0x1p-10f;  // exact
          const _Float16 h = static_cast<_Float16>(sv);
          sr[u] = h;
          sr[nup + u] = static_cast<_Float16>(sv - static_cast<float>(h));
          if (u == nu - 1)  // the row's last unit clears the padding
            for (int z = nu; z < nup; z++) sr[z] = sr[nup + z] = static_cast<_Float16>(0.f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- weights
// Unpacks the quants a weight lane of k-group g needs for one block into the
// MFMA B operand (8 fp16 integers in slot_elem order).
// 4-bit: one quant dword u = qs[4g .. 4g+3]; (u & 0x000F000F) | 0x6400 per
// half is 1024 + q exactly, (u & 0x00F000F0) | 0x6400 is 1024 + 16 q; a
// packed fp16 add / fma then yields q - 8 (Q4_0) or q (Q4_1) exactly.
template <int TYPE>
__device__ __forceinline__ half8 unpack_q4(uint32_t u) {
  constexpr float OFF_LO = TYPE == WH_TYPE_Q4_0 ? -1032.f : -1024.f;
  constexpr float OFF_HI = TYPE == WH_TYPE_Q4_0 ? -72.f : -64.f;
  const uint32_t t8 = u >> 8;
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const half2v lo_a = __builtin_bit_cast(half2v, (u & 0x000F000Fu) | 0x64006400u);
  const half2v lo_b = __builtin_bit_cast(half2v, (t8 & 0x000F000Fu) | 0x64006400u);
  const half2v hi_a = __builtin_bit_cast(half2v, (u & 0x00F000F0u) | 0x64006400u);
  const half2v hi_b = __builtin_bit_cast(half2v, (t8 & 0x00F000F0u) | 0x64006400u);
  const half2v off_lo = {static_cast<_Float16>(OFF_LO), static_cast<_Float16>(OFF_LO)};
  const half2v off_hi = {static_cast<_Float16>(OFF_HI), static_cast<_Float16>(OFF_HI)};
  const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
  const half2v r0 = lo_a + off_lo;                       // exact: integers below 2048
  const half2v r1 = lo_b + off_lo;
  const half2v r2 = __builtin_elementwise_fma(hi_a, sixteenth, off_hi);  // (1024 + 16q)/16 exact
  const half2v r3 = __builtin_elementwise_fma(hi_b, sixteenth, off_hi);
  half8 out;
  out[0] = r0[0]; out[1] = r0[1]; out[2] = r1[0]; out[3] = r1[1];
  out[4] = r2[0]; out[5] = r2[1]; out[6] = r3[0]; out[7] = r3[1];
  return out;
}

// int8 quants q[8g .. 8g+7] (two dwords) -> fp16: bytes moved into the low
// half of each 16-bit lane with v_perm, (b ^ 0x80) | 0x6400 = 1024 + q + 128,
// minus 1152.
__device__ __forceinline__ half8 unpack_q8(uint32_t u0, uint32_t u1) {
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const half2v off = {static_cast<_Float16>(-1152.f), static_cast<_Float16>(-1152.f)};
  half8 out;
  const uint32_t w[2] = {u0, u1};
#pragma unroll
  for (int i = 0; i < 2; i++) {
    // selector bytes: 0x0c gives 0x00
    const uint32_t p0 = __builtin_amdgcn_perm(0u, w[i], 0x0c010c00u) ^ 0x64806480u;  // bytes 0, 1
    const uint32_t p1 = __builtin_amdgcn_perm(0u, w[i], 0x0c030c02u) ^ 0x64806480u;  // bytes 2, 3
    const half2v a = __builtin_bit_cast(half2v, p0) + off;
    const half2v b = __builtin_bit_cast(half2v, p1) + off;
    out[4 * i + 0] = a[0]; out[4 * i + 1] = a[1]; out[4 * i + 2] = b[0]; out[4 * i + 3] = b[1];
  }
  return out;
}

// (u & mask) | magic in one instruction: gfx950's three-input v_bitop3_b32
// (truth table 0xEA over (u, mask, magic)).  As a builtin, not inline asm,
// so that the compiler's hazard tracking sees the instruction and adds no
// wait states after it (it padded every inline-asm v_and_or_b32 that fed an
// MFMA with an s_nop); left to itself it emits a separate and and or.
__device__ __forceinline__ uint32_t and_or(uint32_t u, uint32_t mask, uint32_t magic) {
  return __builtin_amdgcn_bitop3_b32(u, mask, magic, 0xEA);
}

// Part p (0..3) of the B operand of one weight lane, i.e. its fp16 slots
// 2p, 2p + 1, in the slot order of unpack_q4 / unpack_q8; the four parts can
// be computed at different points of the schedule.
template <int TYPE>
__device__ __forceinline__ void unpack_part(int p, uint32_t u0, uint32_t u1, uint32_t magic, half8& out) {
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  half2v r;
  if constexpr (q8_like<TYPE>()) {
    const half2v off = {static_cast<_Float16>(-1152.f), static_cast<_Float16>(-1152.f)};
    const uint32_t w = p < 2 ? u0 : u1;
    const uint32_t sel = (p & 1) ? 0x0c030c02u : 0x0c010c00u;
    r = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0u, w, sel) ^ 0x64806480u) + off;
  } else {
    constexpr float OFF_LO = TYPE == WH_TYPE_Q4_0 ? -1032.f : -1024.f;
    constexpr float OFF_HI = TYPE == WH_TYPE_Q4_0 ? -72.f : -64.f;
    const uint32_t w = (p & 1) ? (u0 >> 8) : u0;
    if (p < 2) {
      const half2v off_lo = {static_cast<_Float16>(OFF_LO), static_cast<_Float16>(OFF_LO)};
      r = __builtin_bit_cast(half2v, and_or(w, 0x000F000Fu, magic)) + off_lo;
    } else {
      const half2v off_hi = {static_cast<_Float16>(OFF_HI), static_cast<_Float16>(OFF_HI)};
      const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
      r = __builtin_elementwise_fma(__builtin_bit_cast(half2v, and_or(w, 0x00F000F0u, magic)), sixteenth, off_hi);
    }
  }
  out[2 * p] = r[0];
  out[2 * p + 1] = r[1];
}

// Global -> LDS copies (global_load_lds): lane l's 16 (or 4) bytes at
// base + voff land at LDS address lds + 16 l (4 l).  Issued through inline asm
// so that the compiler does not treat them as pending LDS writes (it would
// otherwise wait for every copy in flight before each LDS read); completion
// is tracked explicitly with wait_vmcnt.  The copy reads its LDS address from
// M0, a register the compiler reserves: the statement saves M0 in an SGPR of
// its own, sets it (one wait state before the copy reads it, as GFX9-family
// parts require after an SALU write of M0) and restores it, so M0 holds the
// compiler's value again after every copy.
__device__ __forceinline__ void copy16_to_lds(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);  // wave-uniform by construction
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(base), "s"(m0)
      : "memory");
}
__device__ __forceinline__ void copy4_to_lds(const void* base, uint32_t voff, uint32_t lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(base), "s"(m0)
      : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  // generic -> LDS address space (an address-space cast), then its 32-bit address
  return static_cast<uint32_t>((uintptr_t)((const __attribute__((address_space(3))) uint8_t*)p));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Stream-K partial tiles: a buffer resource over one slot (128 KB or less)
// and the cache policy of the slot's loads and stores, sc1 (bit 4 of the
// buffer instructions' cache-policy operand on gfx950): the policy the memory
// model gives agent-scope atomic loads and stores, coherent across the XCDs'
// L2s without a cache-wide writeback or invalidate.
constexpr int kSkCoherent = 16;
__device__ __forceinline__ int __attribute__((ext_vector_type(4))) sk_rsrc(const float* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  int __attribute__((ext_vector_type(4))) r;
  r[0] = static_cast<int>(static_cast<uint32_t>(a));
  r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xFFFFu);
  r[2] = 1 << 20;  // 1 MB of records: every slot offset is in range
  r[3] = 0x00020000;
  return r;
}

// ---------------------------------------------------------------- GEMM
// Waits until at most min(n, J) stages of N copies each are in flight.
template <int N, int J>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (J == 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= J) wait_vmcnt<J * N>();
    else wait_stages<N, J - 1>(n);
  }
}

// Y (or split-K partial plane blockIdx.y) for one BM x 256 tile over blocks
// [kb0, kb1).  Grid: x = tiles (XCD-grouped order), y = K splits.
// SK (stream-K; one workgroup per CU, used when the tiles do not fill the CUs
// evenly): the work is the sequence of (tile, stage) units in tile order, and
// workgroup v (XCD-grouped numbering) takes units [v upw, (v + 1) upw), so a
// tile can be shared by consecutive workgroups.  A workgroup whose range
// starts inside a tile computes that part first, stores its raw accumulators
// in its slot of sk_part and raises its flag (sk_sub + 1; the packing kernel
// cleared the flags); the workgroup holding the tile's first stage adds the
// other owners' slots in owner order, then scales and stores, so the result
// does not depend on timing.  Its wait is bounded (sk_wait ticks of the
// 100 MHz clock, wh_set_stream_k_wait): if a flag has not come, it computes
// the rest of the tile itself.
// FFNP (the FFN's gate and up in one pass, no split-K): a tile's 256 weight
// rows are 128 rows of W (gate) and the same 128 rows of W2 (up); every wave
// holds gate and up tiles of the same rows side by side (row groups 2m and
// 2m + 1), and the epilogue writes y = silu(gate x) * (up x) for n_rows
// output columns (tensor_utils.rs:512-532), so neither product reaches HBM.
// LO = false (activations given as bfloat16): a bf16 value carries 8
// significant bits, so its scaled copy (the row's largest in [2^13, 2^14)) is
// an fp16 exactly and its lo limb zero, unless it lies below 2^-17, where fp16
// subnormals round it; the lo products, below 2^-39 of the row's largest term
// each, are left out and the kernel issues half the MFMAs.
template <int TYPE, int BM, bool FFNP = false, bool SK = false, bool LO = true>
__global__ __launch_bounds__(TWAVES * 64, 1) void gemm_tiled_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ W2, const _Float16* __restrict__ frag,
    const float* __restrict__ rscale, const float* __restrict__ bsum, const float* __restrict__ dmin,
    float* __restrict__ y, int n_tokens, int n_rows, int nb, int blocks_per_split, int tiles_n, int n_tiles,
    uint32_t* __restrict__ sk_flags, float* __restrict__ sk_part, int sk_upw, int sk_sub, uint32_t sk_wait) {
  using C = TCfg<BM>;
  constexpr int IT = C::IT, NT = C::NT, FPB = C::FPB, NSTAGE = nstage<TYPE, BM>();
  constexpr int A_STAGE = C::A_STAGE;
  constexpr int TS = TFmt<TYPE>::TS, QOFF = TFmt<TYPE>::QOFF, DWB = dwb<TYPE>();
  constexpr int BSTAGE = b_stage_bytes<TYPE>();
  constexpr int STAGE = stage_bytes<TYPE, BM>();
  constexpr int A_FR = SB * FPB;                                    // fragments per stage
  constexpr int A_DMA = (A_FR + TWAVES - 1) / TWAVES;               // copies per wave (wrapping)
  constexpr int B_DMA = b_dma_per_wave<TYPE>();
  constexpr int PER_STAGE = A_DMA + B_DMA;                          // vmcnt per stage
  static_assert(PER_STAGE == per_stage<TYPE, BM>(), "copy count");
  static_assert((NSTAGE - 2) * PER_STAGE < 64, "vmcnt range");
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  // wave-uniform (an SGPR): the copies' LDS addresses and every other
  // per-wave offset are then scalar arithmetic, not VALU + v_readfirstlane
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = (wave / C::WGN) * C::WTM;   // token offset of the wave tile
  const int wn = (wave % C::WGN) * C::WTN;   // row offset of the wave tile

  const int bid = blockIdx.x;
  constexpr int HALF = TBN / 2;  // FFNP: rows of each matrix per tile
  const size_t row_bytes = static_cast<size_t>(nb) * TS;
  const int tile_st = nb / SB;   // stages of a whole tile
  // units [u, u_end) of this workgroup; without SK one segment: a tile (tiles
  // resident on one XCD, workgroup id mod 8, are consecutive) and the stages
  // of split blockIdx.y
  int u = 0, u_end = 1, v = 0;
  if constexpr (SK) {
    v = (bid % 8) * static_cast<int>(gridDim.x / 8) + bid / 8;
    u = v * sk_upw;
    u_end = min(n_tiles * tile_st, u + sk_upw);
  }
  __shared__ int sk_ok;
  for (bool first = true; u < u_end; first = false) {
  int L, st_a, st_b;
  if constexpr (SK) {
    L = u / tile_st;
    st_a = u % tile_st;
    st_b = min(tile_st, st_a + (u_end - u));
    u += st_b - st_a;
  } else {
    const int q = n_tiles / 8, rem = n_tiles % 8;
    const int xcd = bid % 8, local = bid / 8;
    L = xcd * q + min(xcd, rem) + local;
    const int kbs = blockIdx.y * blocks_per_split;
    st_a = kbs / SB;
    st_b = min(nb, kbs + blocks_per_split) / SB;
    if (st_b < st_a) st_b = st_a;
    u = u_end;
  }
  const int T = L / tiles_n, R = L % tiles_n;
  const int t0 = T * BM, r0 = R * (FFNP ? HALF : TBN);
  // every wave is done with the ring of the previous segment before it is refilled
  if (!first) __syncthreads();

  // Byte offset (from W) of each raw weight dword this lane copies per stage:
  // dword gi of the stage's [row][DWB] chunk; rows past the end re-read the
  // last row, and copies past the chunk (gi >= TBN * DWB, the rounding of the
  // last instruction) land in the slot's tail, which is never read.  Offsets
  // fit 32 bits (checked by the launcher).
  // FFNP: chunk rows [0, 128) are gate rows r0.., [128, 256) the same up rows;
  // the boundary (128 DWB dwords) is a multiple of 64, so each wave's copy
  // instruction reads from one matrix.
  static_assert(!FFNP || (HALF * DWB) % 64 == 0, "gate / up halves of the stage chunk in whole copy instructions");
  uint32_t b_off[B_DMA];
#pragma unroll
  for (int c = 0; c < B_DMA; c++) {
    const int gi = min(static_cast<int>(threadIdx.x) + TWAVES * 64 * c, TBN * DWB - 1);
    const int row = min(r0 + (FFNP ? (gi / DWB) % HALF : gi / DWB), n_rows - 1);
    b_off[c] = static_cast<uint32_t>(static_cast<size_t>(row) * row_bytes) + 4u * static_cast<uint32_t>(gi % DWB);
  }
  const uint32_t smem_base = lds_addr(smem);
  // MFMA lane l (k-group l / 16, token l % 16) of a fragment, stored token-major
  const uint32_t frag_lane_off = 16u * (4u * (lane & 15) + (lane >> 4));

  // the stages of the current pass: [kb0, kb0 + SB n_stages) in blocks
  int kb0 = st_a * SB, n_stages = st_b - st_a;
  auto issue = [&](int st) {
    if (st >= n_stages) return;
    const uint32_t slot = smem_base + (st % NSTAGE) * STAGE;
    const int kb = kb0 + st * SB;
    // activation fragments (block j = fi / FPB); when a stage has fewer
    // fragments than A_DMA * TWAVES, some are copied twice (same data, same place)
#pragma unroll
    for (int f = 0; f < A_DMA; f++) {
      const int fi = (wave * A_DMA + f) % A_FR;
      const int j = fi / FPB;
      // the wave-uniform part of the source in the scalar base, the lane's in the offset
      const size_t off = ((static_cast<size_t>(T) * nb + kb + j) * FPB + fi % FPB) * FRAG;
      copy16_to_lds(reinterpret_cast<const uint8_t*>(frag) + off, frag_lane_off, slot + fi * FRAG);
    }
    const uint32_t bslot = slot + A_STAGE;
    const uint32_t kboff = static_cast<uint32_t>(kb) * TS;
#pragma unroll
    for (int c = 0; c < B_DMA; c++) {
      const uint8_t* wb = W;
      if constexpr (FFNP)  // this wave's copy c lies in the up half (a wave-uniform choice: the base is an SGPR pair)
        if (TWAVES * 64 * c + 64 * __builtin_amdgcn_readfirstlane(wave) >= HALF * DWB) wb = W2;
      copy4_to_lds(wb + kboff, b_off[c], bslot + 4 * (TWAVES * 64 * c + 64 * wave));
    }
  };

  float4v acc[IT][NT];
#pragma unroll
  for (int i = 0; i < IT; i++)
#pragma unroll
    for (int n = 0; n < NT; n++) acc[i][n] = float4v{0.f, 0.f, 0.f, 0.f};

  const int g = lane >> 4;       // k-group
  const int ln = lane & 15;      // token (A) / weight row (B) within a 16-tile

  // Software pipeline over pairs of row groups (NT is even).  Per pair of a
  // block: the hi MFMAs of both groups, then their lo MFMAs (a lo MFMA comes
  // 2 IT MFMAs after the hi MFMA it depends on), with the block-scale FMAs of
  // the previous pair (pending: possibly of the previous block or stage) and
  // the unpacking of the next pair's weights spread over the 4 IT MFMA slots;
  // scheduling fences keep that order, so the matrix pipe and the VALU work
  // side by side within a wave.  The pending scales start as 0 * 0 (no-ops)
  // and are flushed after the last stage.
  static_assert(NT % 2 == 0 && (SB * (NT / 2)) % 2 == 0, "pairs of row groups alternate buffers");
  float4v cc[2][2][IT];  // [current / pending pair][group of the pair][token group]
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int i = 0; i < IT; i++) cc[b][h][i] = float4v{0.f, 0.f, 0.f, 0.f};
  float pd[2] = {0.f, 0.f};  // pending block scales
  // Q4_1: the m of the current window's blocks as MFMA B operands, lane group
  // g holding blocks 8g .. 8g + 7 of the window (blocks of other parts zero)
  u32x4 mfr[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) mfr[n] = u32x4{0u, 0u, 0u, 0u};
  const uint32_t magic = 0x64006400u;  // fp16 1024 in both halves (held in a VGPR)

  // acc[i][N] += pd[h] * cc[B][h][i]; constants after unrolling
  auto scale_one = [&](int N, int B, int h, int i) {
#pragma unroll
    for (int r = 0; r < 4; r++) acc[i][N][r] = __builtin_fmaf(pd[h], cc[B][h][i][r], acc[i][N][r]);
  };
  // Q4_1: acc += 2^10 (S 2^-10 . m) over the window starting at block w0: the
  // A operands (the packing's fp16 limbs of the block sums S) from memory,
  // two MFMAs per 16 x 16 outputs; then the window's m start again at zero
  auto flush_min = [&](int w0) {
    const int nbp = (nb + 7) & ~7;
    const int s0 = w0 + 8 * g;
    const bool in = s0 < nbp;
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(bsum);
    u32x4 sh[IT], sl[IT];
#pragma unroll
    for (int i = 0; i < IT; i++) {
      const uint32_t off = static_cast<uint32_t>((t0 + wm + 16 * i + ln) * 2 * nbp + s0);
      sh[i] = in ? *reinterpret_cast<const u32x4*>(s16 + off) : u32x4{0u, 0u, 0u, 0u};
      sl[i] = in ? *reinterpret_cast<const u32x4*>(s16 + off + nbp) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < IT; i++)
#pragma unroll
      for (int n = 0; n < NT; n++) {
        float4v t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, sh[i]), __builtin_bit_cast(half8, mfr[n]),
                                                           float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, sl[i]), __builtin_bit_cast(half8, mfr[n]), t, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][n][r] = __builtin_fmaf(1024.f, t[r], acc[i][n][r]);
      }
#pragma unroll
    for (int n = 0; n < NT; n++) mfr[n] = u32x4{0u, 0u, 0u, 0u};
  };

  // A head part (SK) that does not get every other owner's slot in time runs
  // a second pass over the rest of the tile, into the same accumulators.
  for (int pass = 0; pass < 2; pass++) {
  if (pass > 0) {
    __syncthreads();  // the ring of the first pass is no longer read
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < IT; i++) cc[b][h][i] = float4v{0.f, 0.f, 0.f, 0.f};
    pd[0] = pd[1] = 0.f;
  }
#pragma unroll
  for (int st = 0; st < NSTAGE - 1; st++) issue(st);
  for (int st = 0; st < n_stages; st++) {
    // stage st landed (this wave's copies); later issued stages may be in flight
    wait_stages<PER_STAGE, NSTAGE - 2>(n_stages - 1 - st);
    __builtin_amdgcn_s_barrier();   // every wave's copies of stage st are in LDS
    issue(st + NSTAGE - 1);         // into the slot of stage st - 1, which all waves finished
    const uint8_t* slot = smem + (st % NSTAGE) * STAGE;
    const uint8_t* bslot = slot + A_STAGE;
    // every LDS operand of the stage, read up front
    half8 ah[SB][IT], al[SB][IT];
    uint32_t wq0[SB][NT], wq1[SB][NT], wdm[SB][NT];
    auto load_a = [&](int j) {
#pragma unroll
      for (int i = 0; i < IT; i++) {
        const int grp = (wm >> 4) + i;
        ah[j][i] = *reinterpret_cast<const half8*>(slot + (j * FPB + 2 * grp) * FRAG + 16 * lane);
        if constexpr (LO) al[j][i] = *reinterpret_cast<const half8*>(slot + (j * FPB + 2 * grp + 1) * FRAG + 16 * lane);
      }
    };
#pragma unroll
    for (int j = 0; j < SB; j++) {
      load_a(j);
#pragma unroll
      for (int n = 0; n < NT; n++) {
        // FFNP: group 2m is gate rows wn / 2 + 16 m.., group 2m + 1 the same up rows
        const int row = FFNP ? ((n & 1) ? HALF : 0) + wn / 2 + 16 * (n >> 1) + ln : wn + 16 * n + ln;
        const uint8_t* rb = bslot + row * (DWB * 4) + j * TS;     // this block's bytes
        const uint16_t* r16 = reinterpret_cast<const uint16_t*>(rb);
        if constexpr (TYPE == wh::kGemmQ8H) {
          // 16 quants: k-groups 0, 1; groups 2, 3 are the zero padding
          const uint32_t* q32 = reinterpret_cast<const uint32_t*>(rb + QOFF + 8 * (g & 1));
          wq0[j][n] = g < 2 ? q32[0] : 0u;
          wq1[j][n] = g < 2 ? q32[1] : 0u;
        } else if constexpr (TYPE == WH_TYPE_Q8_0) {
          const uint16_t* q16 = reinterpret_cast<const uint16_t*>(rb + QOFF + 8 * g);
          wq0[j][n] = static_cast<uint32_t>(q16[0]) | (static_cast<uint32_t>(q16[1]) << 16);
          wq1[j][n] = static_cast<uint32_t>(q16[2]) | (static_cast<uint32_t>(q16[3]) << 16);
        } else {
          const uint16_t* q16 = reinterpret_cast<const uint16_t*>(rb + QOFF + 4 * g);
          wq0[j][n] = static_cast<uint32_t>(q16[0]) | (static_cast<uint32_t>(q16[1]) << 16);
          wq1[j][n] = 0u;
        }
        if constexpr (f32_scale<TYPE>()) {
          wdm[j][n] = reinterpret_cast<const uint32_t*>(rb)[0];
        } else {
          wdm[j][n] = TYPE == WH_TYPE_Q4_1 ? (static_cast<uint32_t>(r16[0]) | (static_cast<uint32_t>(r16[1]) << 16))
                                           : static_cast<uint32_t>(r16[0]);
        }
      }
    }
    half8 bw[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int part = 0; part < 4; part++) unpack_part<TYPE>(part, wq0[0][h], wq1[0][h], magic, bw[h]);
#pragma unroll
    for (int j = 0; j < SB; j++) {
#pragma unroll
      for (int np = 0; np < NT / 2; np++) {
        // the pairs of a stage alternate between the two buffers (SB NT / 2 is even)
        const int cur = (j * (NT / 2) + np) & 1, pend = cur ^ 1;
        // the pending pair: groups 2 np - 2, 2 np - 1 of this block, or the last pair of the previous
        const int pn = np == 0 ? NT - 2 : 2 * np - 2;
        // the next pair's weights: pair np + 1 of this block, or pair 0 of the next block
        const bool more = np + 1 < NT / 2 || j + 1 < SB;
        const int jn = np + 1 < NT / 2 ? j : (j + 1 < SB ? j + 1 : j);
        const int nn = np + 1 < NT / 2 ? 2 * np + 2 : 0;
        half8 bn[2] = {bw[0], bw[1]};
        // the pending pair's scales over the first 2 IT MFMA slots, the next
        // pair's unpacking over the last 2 IT
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int i = 0; i < IT; i++) {
            cc[cur][h][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j][i], bw[h], float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            scale_one(pn + h, pend, h, i);
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int i = 0; i < IT; i++) {
            if constexpr (LO) cc[cur][h][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j][i], bw[h], cc[cur][h][i], 0, 0, 0);
            if (more) {
              // 8 parts (2 groups x 4) over 2 IT slots
#pragma unroll
              for (int q = (h * IT + i) * 8 / (2 * IT); q < (h * IT + i + 1) * 8 / (2 * IT); q++)
                unpack_part<TYPE>(q % 4, wq0[jn][nn + q / 4], wq1[jn][nn + q / 4], magic, bn[q / 4]);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        // this pair becomes the pending one
#pragma unroll
        for (int h = 0; h < 2; h++) {
          if constexpr (f32_scale<TYPE>()) {
            pd[h] = __uint_as_float(wdm[j][2 * np + h]);
          } else {
            pd[h] = whd::f16_bits_to_f32(wdm[j][2 * np + h] & 0xFFFFu);
          }
          asm("" : "+v"(pd[h]));  // in a VGPR: the FMAs are then plain v_fmac_f32
        }
        bw[0] = bn[0];
        bw[1] = bn[1];
      }
    }
    if constexpr (has_min<TYPE>()) {
      // the stage's two blocks' m (bits 16..31 of wdm) into dword (kb mod 8) / 2
      // of lane group (kb mod 32) / 8 of the window's B operands
      static_assert(SB == 2, "one B-operand dword per stage");
      const int kb = kb0 + st * SB, pw = kb & 31;
      const bool mine = g == (pw >> 3);
      const int dq = (pw & 7) >> 1;
#pragma unroll
      for (int n = 0; n < NT; n++) {
        const uint32_t val = __builtin_amdgcn_perm(wdm[1][n], wdm[0][n], 0x07060302u);
#pragma unroll
        for (int d = 0; d < 4; d++) mfr[n][d] = (d == dq && mine) ? val : mfr[n][d];
      }
      if (pw == 32 - SB || st == n_stages - 1) flush_min(kb & ~31);
    }
  }
  // flush the pending scales (the last pair of the last block)
#pragma unroll
  for (int h = 0; h < 2; h++)
#pragma unroll
    for (int i = 0; i < IT; i++) scale_one(NT - 2 + h, (SB * (NT / 2) - 1) & 1, h, i);
  wait_vmcnt<0>();  // (no copies remain: every issued stage was consumed)
  if constexpr (!SK) break;
  if (pass > 0 || st_a > 0 || st_b == tile_st) break;  // a tail part, the whole tile, or done here
  // head part: wait for the owners of the rest of the tile (workgroups
  // v + 1 .. w_last), then add their slots in order
  const int w_last = min(static_cast<int>(gridDim.x) - 1, ((L + 1) * tile_st - 1) / sk_upw);
  if (threadIdx.x == 0) {
    int ok = 1;
    const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
    for (int w = v + 1; w <= w_last && ok; w++) {
      while (__hip_atomic_load(sk_flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
             static_cast<uint32_t>(sk_sub + 1)) {
        if (__builtin_amdgcn_s_memrealtime() - t_start > sk_wait) {  // ticks of the 100 MHz clock
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    sk_ok = ok;
  }
  __syncthreads();
  if (sk_ok) {
    for (int w = v + 1; w <= w_last; w++) {
      // the slot through device-coherent loads (sc1: the policy of an
      // agent-scope atomic load), all issued before the first is used
      const i32x4 rs = sk_rsrc(sk_part + static_cast<size_t>(w) * BM * TBN);
#pragma unroll
      for (int i = 0; i < IT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++)
          acc[i][n] += gt_buffer_load_x4(rs, 16 * ((i * NT + n) * (TWAVES * 64) + static_cast<int>(threadIdx.x)), 0,
                                         kSkCoherent);
    }
    break;
  }
  kb0 = st_b * SB;  // the rest of the tile, here
  n_stages = tile_st - st_b;
  }  // pass
  if constexpr (SK) {
    if (st_a > 0) {
      // a tail part: the raw accumulators to this workgroup's slot through
      // device-coherent stores (sc1, write-through), then its flag
      const i32x4 rs = sk_rsrc(sk_part + static_cast<size_t>(v) * BM * TBN);
#pragma unroll
      for (int i = 0; i < IT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++)
          gt_buffer_store_x4(acc[i][n], rs, 16 * ((i * NT + n) * (TWAVES * 64) + static_cast<int>(threadIdx.x)), 0,
                             kSkCoherent);
      // every store of the slot complete before the flag is raised
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0)
        __hip_atomic_store(sk_flags + v, static_cast<uint32_t>(sk_sub + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
  }

  if constexpr (TYPE == wh::kGemmQ4F) {
    // Q4_K's dmin: acc += dmin[row][sb] * S[token][sb] over this split's
    // super-blocks (split bounds are multiples of 8 blocks), S the packing's
    // super-block sums in the same scaled domain as acc.  Under stream-K the
    // workgroup that finishes a tile adds the term of every super-block (the
    // other owners' parts carry none).  As matrix-core products over windows
    // of 32 super-blocks: lane group g holds super-blocks 8g .. 8g + 7 of the
    // window in both operands (B: the fp16 dmin table, those outside
    // [sb_lo, sb_hi) masked to zero; A: S as hi + lo fp16 limbs of S 2^-10),
    // and one fma per output adds 2^10 times the window's sum.
    static_assert(!FFNP, "the gate / up pass has no dmin term");
    const int nsb = nb / 8, nsbp = (nsb + 7) & ~7;
    const int sb_lo = SK ? 0 : st_a * SB / 8, sb_hi = SK ? nsb : st_b * SB / 8;
    const uint16_t* dm16 = reinterpret_cast<const uint16_t*>(dmin);
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(bsum);
    // the lane index opaque here, so that the loads' offsets are formed here
    // and not held in registers through the stage loop; 32-bit offsets (both
    // arrays hold fewer than 2^28 halves: the launcher keeps the weight and
    // fragment bytes below 2^32)
    int lnv = ln;
    asm volatile("" : "+v"(lnv));
    for (int w0 = sb_lo & ~31; w0 < sb_hi; w0 += 32) {
      const int s0 = w0 + 8 * g;                  // this lane's first super-block
      const bool in = s0 < nsbp;                  // inside the table's rows
      uint32_t mk[4];
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const int a = s0 + 2 * d;
        mk[d] = (a >= sb_lo && a < sb_hi ? 0x0000FFFFu : 0u) | (a + 1 >= sb_lo && a + 1 < sb_hi ? 0xFFFF0000u : 0u);
      }
      u32x4 bd[NT];
#pragma unroll
      for (int n = 0; n < NT; n++) {
        const uint32_t off = static_cast<uint32_t>(min(r0 + wn + 16 * n + lnv, n_rows - 1) * nsbp + s0);
        bd[n] = in ? *reinterpret_cast<const u32x4*>(dm16 + off) : u32x4{0u, 0u, 0u, 0u};
      }
      u32x4 sh[IT], sl[IT];
#pragma unroll
      for (int i = 0; i < IT; i++) {
        const uint32_t off = static_cast<uint32_t>((t0 + wm + 16 * i + lnv) * 2 * nsbp + s0);
        sh[i] = in ? *reinterpret_cast<const u32x4*>(s16 + off) : u32x4{0u, 0u, 0u, 0u};
        sl[i] = in ? *reinterpret_cast<const u32x4*>(s16 + off + nsbp) : u32x4{0u, 0u, 0u, 0u};
      }
      __builtin_amdgcn_sched_barrier(0);  // every load issued before the first use
#pragma unroll
      for (int n = 0; n < NT; n++)
#pragma unroll
        for (int d = 0; d < 4; d++) bd[n][d] &= mk[d];
#pragma unroll
      for (int i = 0; i < IT; i++) {
#pragma unroll
        for (int n = 0; n < NT; n++) {
          float4v t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, sh[i]), __builtin_bit_cast(half8, bd[n]),
                                                             float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, sl[i]), __builtin_bit_cast(half8, bd[n]), t, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][n][r] = __builtin_fmaf(1024.f, t[r], acc[i][n][r]);
        }
        __builtin_amdgcn_sched_barrier(0);  // one token group's products at a time
      }
    }
  }

  if constexpr (FFNP) {
    // h = silu(g) * u for the gate / up pairs, as (g * (1 / (1 + e^-g))) * u
#pragma unroll
    for (int i = 0; i < IT; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int t = t0 + wm + 16 * i + 4 * g + r;
        if (t >= n_tokens) continue;
        const float sc = rscale[t];
#pragma unroll
        for (int m = 0; m < NT / 2; m++) {
          const int col = r0 + wn / 2 + 16 * m + ln;
          if (col >= n_rows) continue;
          const float gv = acc[i][2 * m][r] * sc, uv = acc[i][2 * m + 1][r] * sc;
          y[static_cast<size_t>(t) * n_rows + col] = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
        }
      }
    }
    continue;
  }
  // epilogue: undo the row scale; split-K partials go to plane blockIdx.y
  float* out = y + static_cast<size_t>(blockIdx.y) * n_tokens * n_rows;
#pragma unroll
  for (int i = 0; i < IT; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int t = t0 + wm + 16 * i + 4 * g + r;
      if (t >= n_tokens) continue;
      const float sc = rscale[t];
#pragma unroll
      for (int n = 0; n < NT; n++) {
        const int row = r0 + wn + 16 * n + ln;
        if (row < n_rows) out[static_cast<size_t>(t) * n_rows + row] = acc[i][n][r] * sc;
      }
    }
  }
  }  // segment
}

__global__ __launch_bounds__(256) void tiled_splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                                  size_t n, float* __restrict__ y) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = part[i];
    for (int s = 1; s < splits; s++) v += part[static_cast<size_t>(s) * n + i];
    y[i] = v;
  }
}

// Token-tile height for a token count: the smallest of 16, 32, 64, 128 that
// holds it (one tile) or 128 beyond.
int tile_bm(size_t n_tokens) { return n_tokens <= 16 ? 16 : (n_tokens <= 32 ? 32 : (n_tokens <= 64 ? 64 : 128)); }

// Stream-K grid for n_tiles tiles of tile_st stages each: one workgroup per
// CU whenever the tiles do not fill the CUs evenly (a last round with idle
// CUs, or fewer tiles than CUs, where split-K planes and a reduce would
// otherwise be needed) and every workgroup's share is at least 8 stages; 0
// (one workgroup per tile) otherwise.  Every block format of the kernel.
int sk_grid(int type, size_t n_tiles, size_t tile_st) {
  if (type != WH_TYPE_Q4_0 && type != WH_TYPE_Q4_1 && type != WH_TYPE_Q8_0 && type != wh::kGemmQ4F &&
      type != wh::kGemmQ8H)
    return 0;
  const size_t g = static_cast<size_t>(wh::cu_count());
  if (g == 0 || g % 8 != 0 || n_tiles % g == 0) return 0;
  const size_t upw = (n_tiles * tile_st + g - 1) / g;
  return upw >= 8 ? static_cast<int>(g) : 0;
}

// The stream-K state of a launch: flags and partial slots (SkWs::g workgroups).
struct SkWs {
  uint32_t* flags;
  float* part;
  int g;    // stream-K grid, 0 for one workgroup per tile
  int sub;  // which of the GEMMs after one packing this is (its flag value - 1)
};

// Bound of the stream-K hand-off wait, in ticks of the 100 MHz clock read by
// s_memrealtime (default 1 ms); read at every launch (wh_set_stream_k_wait).
std::atomic<uint32_t> g_sk_wait{100000u};

template <int TYPE, int BM, bool LO>
int launch_bm_lo(const uint8_t* w, size_t n_rows, size_t k, size_t n_tokens, const _Float16* frag,
              const float* rs, const float* bs, const float* dmin, float* part, int splits, const SkWs& sk,
              hipStream_t s) {
  const int nb = static_cast<int>(k / 32);
  const int tiles_n = static_cast<int>((n_rows + TBN - 1) / TBN);
  const int tiles_m = static_cast<int>((n_tokens + BM - 1) / BM);
  const int n_tiles = tiles_m * tiles_n;
  const size_t lds = tiled_lds_bytes<TYPE, BM>();
  {
    if (splits == 1 && sk.g > 0 && sk_grid(TYPE, n_tiles, nb / SB) == sk.g) {
      const int upw = (n_tiles * (nb / SB) + sk.g - 1) / sk.g;
      WH_ENSURE_LDS(lds, &gemm_tiled_kernel<TYPE, BM, false, true, LO>);
      gemm_tiled_kernel<TYPE, BM, false, true, LO><<<static_cast<unsigned>(sk.g), TWAVES * 64, lds, s>>>(
          w, nullptr, frag, rs, bs, dmin, part, static_cast<int>(n_tokens), static_cast<int>(n_rows), nb, nb, tiles_n,
          n_tiles, sk.flags, sk.part, upw, sk.sub, g_sk_wait.load(std::memory_order_relaxed));
      WH_LAUNCH_CHECK("tiled gemm kernel launch");
      return WH_OK;
    }
  }
  int bps = (nb + splits - 1) / splits;
  constexpr int ALIGN = TYPE == wh::kGemmQ4F ? 8 : SB;   // kGemmQ4F: whole super-blocks per split
  bps = (bps + ALIGN - 1) / ALIGN * ALIGN;
  WH_ENSURE_LDS(lds, &gemm_tiled_kernel<TYPE, BM, false, false, LO>);
  dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(splits));
  gemm_tiled_kernel<TYPE, BM, false, false, LO><<<grid, TWAVES * 64, lds, s>>>(w, nullptr, frag, rs, bs, dmin, part,
                                                           static_cast<int>(n_tokens), static_cast<int>(n_rows), nb,
                                                           bps, tiles_n, n_tiles, nullptr, nullptr, 0, 0, 0u);
  WH_LAUNCH_CHECK("tiled gemm kernel launch");
  return WH_OK;
}

// lo = false: the activations were bfloat16, so the packed lo limbs are
// (all but) zero and the products of the hi limbs alone are issued (32- to
// 128-token tiles of the 32-element block formats, the bf16 path's shapes).
template <int TYPE, int BM>
int launch_bm(const uint8_t* w, size_t n_rows, size_t k, size_t n_tokens, const _Float16* frag,
              const float* rs, const float* bs, const float* dmin, float* part, int splits, const SkWs& sk,
              hipStream_t s, bool lo) {
  if constexpr ((TYPE == WH_TYPE_Q4_0 || TYPE == WH_TYPE_Q4_1 || TYPE == WH_TYPE_Q8_0) && BM >= 32) {
    if (!lo) return launch_bm_lo<TYPE, BM, false>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s);
  }
  return launch_bm_lo<TYPE, BM, true>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s);
}

// The FFN's gate and up (n_ff rows each) in one pass: h = silu(gate x) * (up x).
template <int TYPE, int BM>
int launch_ffn_bm(const uint8_t* gate, const uint8_t* up, size_t n_ff, size_t k, size_t n_tokens,
                  const _Float16* frag, const float* rs, const float* bs, float* h, const SkWs& sk, hipStream_t s) {
  const int nb = static_cast<int>(k / 32);
  const int tiles_n = static_cast<int>((n_ff + TBN / 2 - 1) / (TBN / 2));
  const int tiles_m = static_cast<int>((n_tokens + BM - 1) / BM);
  const int n_tiles = tiles_m * tiles_n;
  const size_t lds = tiled_lds_bytes<TYPE, BM>();
  if (sk.g > 0 && sk_grid(TYPE, n_tiles, nb / SB) == sk.g) {
    const int upw = (n_tiles * (nb / SB) + sk.g - 1) / sk.g;
    WH_ENSURE_LDS(lds, &gemm_tiled_kernel<TYPE, BM, true, true>);
    gemm_tiled_kernel<TYPE, BM, true, true><<<static_cast<unsigned>(sk.g), TWAVES * 64, lds, s>>>(
        gate, up, frag, rs, bs, nullptr, h, static_cast<int>(n_tokens), static_cast<int>(n_ff), nb, nb, tiles_n,
        n_tiles, sk.flags, sk.part, upw, sk.sub, g_sk_wait.load(std::memory_order_relaxed));
    WH_LAUNCH_CHECK("tiled ffn gate/up kernel launch");
    return WH_OK;
  }
  WH_ENSURE_LDS(lds, &gemm_tiled_kernel<TYPE, BM, true>);
  gemm_tiled_kernel<TYPE, BM, true><<<static_cast<unsigned>(n_tiles), TWAVES * 64, lds, s>>>(
      gate, up, frag, rs, bs, nullptr, h, static_cast<int>(n_tokens), static_cast<int>(n_ff), nb, nb, tiles_n,
      n_tiles, nullptr, nullptr, 0, 0, 0u);
  WH_LAUNCH_CHECK("tiled ffn gate/up kernel launch");
  return WH_OK;
}

template <int TYPE>
int launch_ffn_typed(const uint8_t* gate, const uint8_t* up, size_t n_ff, size_t k, size_t n_tokens,
                     const _Float16* frag, const float* rs, const float* bs, float* h, const SkWs& sk, hipStream_t s) {
  switch (tile_bm(n_tokens)) {
    case 16: return launch_ffn_bm<TYPE, 16>(gate, up, n_ff, k, n_tokens, frag, rs, bs, h, sk, s);
    case 32: return launch_ffn_bm<TYPE, 32>(gate, up, n_ff, k, n_tokens, frag, rs, bs, h, sk, s);
    case 64: return launch_ffn_bm<TYPE, 64>(gate, up, n_ff, k, n_tokens, frag, rs, bs, h, sk, s);
    default: return launch_ffn_bm<TYPE, 128>(gate, up, n_ff, k, n_tokens, frag, rs, bs, h, sk, s);
  }
}

template <int TYPE>
int launch_typed(const uint8_t* w, size_t n_rows, size_t k, size_t n_tokens, const _Float16* frag,
                 const float* rs, const float* bs, const float* dmin, float* part, int splits, const SkWs& sk,
                 hipStream_t s, bool lo) {
  switch (tile_bm(n_tokens)) {
    case 16: return launch_bm<TYPE, 16>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s, lo);
    case 32: return launch_bm<TYPE, 32>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s, lo);
    case 64: return launch_bm<TYPE, 64>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s, lo);
    default: return launch_bm<TYPE, 128>(w, n_rows, k, n_tokens, frag, rs, bs, dmin, part, splits, sk, s, lo);
  }
}

template <int TYPE>
size_t lds_typed(int bm) {
  switch (bm) {
    case 16: return tiled_lds_bytes<TYPE, 16>();
    case 32: return tiled_lds_bytes<TYPE, 32>();
    case 64: return tiled_lds_bytes<TYPE, 64>();
    default: return tiled_lds_bytes<TYPE, 128>();
  }
}

size_t al256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

namespace wh {

// The tiled kernel needs whole stages per row (k a multiple of 32 SB), 4-byte
// aligned rows and weights, 16-byte aligned activations, byte offsets into the weights, the activation
// fragments and the block sums that fit 32 bits, and an LDS budget the device
// provides.
// Bytes per 32-element block of a GEMM format.
static size_t tiled_ts(int type) {
  switch (type) {
    case WH_TYPE_Q4_0: return TFmt<WH_TYPE_Q4_0>::TS;
    case WH_TYPE_Q4_1: return TFmt<WH_TYPE_Q4_1>::TS;
    case WH_TYPE_Q8_0: return TFmt<WH_TYPE_Q8_0>::TS;
    case kGemmQ4F: return TFmt<kGemmQ4F>::TS;
    case kGemmQ8H: return TFmt<kGemmQ8H>::TS;
    default: return 0;
  }
}

bool gemm_tiled_ok(int type, const void* w, const float* x, size_t n_rows, size_t k, size_t n_tokens) {
  const size_t ts = tiled_ts(type);
  if (ts == 0 || k == 0 || k % (32 * SB) != 0 || !aligned(w, 4) || !aligned(x, 16) || ((k / 32) * ts) % 4 != 0) return false;
  const size_t bm = static_cast<size_t>(tile_bm(n_tokens));
  const size_t tm = (n_tokens + bm - 1) / bm * bm;
  const size_t lim = static_cast<size_t>(1) << 32;
  if (n_rows * (k / 32) * ts >= lim || tm * k * 4 >= lim) return false;
  const int b = static_cast<int>(bm);
  size_t lds;
  switch (type) {
    case WH_TYPE_Q4_0: lds = lds_typed<WH_TYPE_Q4_0>(b); break;
    case WH_TYPE_Q4_1: lds = lds_typed<WH_TYPE_Q4_1>(b); break;
    case WH_TYPE_Q8_0: lds = lds_typed<WH_TYPE_Q8_0>(b); break;
    case kGemmQ4F: lds = lds_typed<kGemmQ4F>(b); break;
    default: lds = lds_typed<kGemmQ8H>(b); break;
  }
  return lds <= max_lds_per_block();
}

// Split-K factor: the largest power of two up to 8 that keeps the workgroups
// within one per CU and every split at least 16 blocks deep.
int gemm_tiled_splits(size_t n_rows, size_t n_tokens, size_t k) {
  const size_t bm = static_cast<size_t>(tile_bm(n_tokens));
  const size_t tiles = ((n_rows + TBN - 1) / TBN) * ((n_tokens + bm - 1) / bm);
  const size_t nb = k / 32;
  const size_t cus = static_cast<size_t>(cu_count());
  int s = 1;
  while (s < 8 && tiles * s * 2 <= cus && nb / (2 * s) >= 16) s *= 2;
  return s;
}

// Stream-K workgroups of a workspace laid out for a GEMM over n_rows rows:
// the grid of that GEMM, or of the FFN's gate and up over n_rows rows each in
// one pass (the same packing), whichever uses stream-K; 0 when neither does.
// Token tiles of 16 and 32 keep split-K: their stages are short, and the
// hand-off of a partial tile costs more than the reduce it replaces (M=32,
// 14336 x 4096: 31.9 against 31.3 us).
// The K-quant formats keep split-K too (their FFN at M=512: 462 against 442
// us with stream-K in the down projection); their tiles take stream-K only
// where they would leave CUs idle in a last round.
static int sk_plain(int type, size_t n_rows, size_t n_tokens, size_t k) {
  const size_t bm = static_cast<size_t>(tile_bm(n_tokens));
  if (bm < 64) return 0;
  if ((type == kGemmQ4F || type == kGemmQ8H) && gemm_tiled_splits(n_rows, n_tokens, k) > 1) return 0;
  return sk_grid(type, ((n_tokens + bm - 1) / bm) * ((n_rows + TBN - 1) / TBN), k / 32 / SB);
}
// Split-K factor of the GEMM over n_rows rows: 1 where it runs stream-K.
static int tiled_splits(int type, size_t n_rows, size_t n_tokens, size_t k) {
  return sk_plain(type, n_rows, n_tokens, k) ? 1 : gemm_tiled_splits(n_rows, n_tokens, k);
}
static int sk_slots(int type, size_t n_rows, size_t n_tokens, size_t k) {
  const int g = sk_plain(type, n_rows, n_tokens, k);
  if (g) return g;
  if (gemm_tiled_splits(2 * n_rows, n_tokens, k) == 1 && tile_bm(n_tokens) >= 64) {
    const size_t bm = static_cast<size_t>(tile_bm(n_tokens));
    return sk_grid(type, ((n_tokens + bm - 1) / bm) * ((n_rows + TBN / 2 - 1) / (TBN / 2)), k / 32 / SB);
  }
  return 0;
}

static size_t sk_bytes(int slots, size_t n_tokens) {
  return slots ? al256(static_cast<size_t>(slots) * 4) +
                     static_cast<size_t>(slots) * static_cast<size_t>(tile_bm(n_tokens)) * TBN * 4
               : 0;
}

size_t gemm_tiled_workspace_bytes(int type, size_t n_rows, size_t n_tokens, size_t k) {
  const size_t bm = static_cast<size_t>(tile_bm(n_tokens));
  const size_t tm = (n_tokens + bm - 1) / bm * bm;   // padded tokens
  size_t b = al256(tm * k * 4) + al256(tm * 4);
  if (needs_bsum(type)) b += al256(tm * bsum_groups(type, k) * 4);
  const int splits = tiled_splits(type, n_rows, n_tokens, k);
  if (splits > 1) b += al256(static_cast<size_t>(splits) * n_rows * n_tokens * 4);
  return b + sk_bytes(sk_slots(type, n_rows, n_tokens, k), n_tokens);
}

// Workspace of one tiled GEMM: packed activations, row scales, Q4_1 block
// sums, split-K partial planes, stream-K flags and partial tiles.
struct TiledWs {
  _Float16* frag;
  float* rs;
  float* bs;
  float* part;  // null without split-K
  uint32_t* sk_flags;
  float* sk_part;
  int sk_n;     // stream-K slots (0: none)
  int bm, splits;
  size_t tm;
};

static TiledWs tiled_ws(int type, size_t n_rows, size_t k, size_t n_tokens, void* workspace) {
  TiledWs t{};
  t.bm = tile_bm(n_tokens);
  t.tm = (n_tokens + t.bm - 1) / t.bm * t.bm;
  char* ws = static_cast<char*>(workspace);
  t.frag = reinterpret_cast<_Float16*>(ws);
  ws += al256(t.tm * k * 4);
  t.rs = reinterpret_cast<float*>(ws);
  ws += al256(t.tm * 4);
  if (needs_bsum(type)) {
    t.bs = reinterpret_cast<float*>(ws);
    ws += al256(t.tm * bsum_groups(type, k) * 4);
  }
  t.splits = tiled_splits(type, n_rows, n_tokens, k);
  t.part = t.splits > 1 ? reinterpret_cast<float*>(ws) : nullptr;
  if (t.splits > 1) ws += al256(static_cast<size_t>(t.splits) * n_rows * n_tokens * 4);
  t.sk_n = sk_slots(type, n_rows, n_tokens, k);
  if (t.sk_n) {
    t.sk_flags = reinterpret_cast<uint32_t*>(ws);
    t.sk_part = reinterpret_cast<float*>(ws + al256(static_cast<size_t>(t.sk_n) * 4));
  }
  return t;
}

template <int MODE, bool XB = false>
static int tiled_pack(int type, const TiledWs& t, const float* x, const float* x2, const float* gamma, float eps,
                      size_t n_tokens, size_t k, size_t kx, hipStream_t s) {
  // threads per row: enough for PPT pairs each, 256 .. 1024
  const size_t npairs = k / 8;
  size_t threads = (npairs + PPT - 1) / PPT;
  threads = threads < 256 ? 256 : (threads > kPackMaxThreads ? kPackMaxThreads : (threads + 63) / 64 * 64);
  pack_a_kernel<MODE, XB><<<static_cast<unsigned>(t.tm), static_cast<unsigned>(threads), 0, s>>>(x, x2, gamma, eps, static_cast<int>(n_tokens),
                                                                  static_cast<int>(k), static_cast<int>(kx), type, t.bm,
                                                                  t.frag, t.rs, t.bs, t.sk_flags, t.sk_n);
  WH_LAUNCH_CHECK("pack kernel launch");
  return WH_OK;
}

// The GEMM over packed activations (and the split-K reduce) into y.
// sub: which of the GEMMs that read one packing this is (0, 1), so that their
// stream-K flags differ.
static int tiled_run(int type, const void* w, size_t n_rows, size_t k, size_t n_tokens, const TiledWs& t, float* y,
                     hipStream_t s, const float* dmin = nullptr, int sub = 0, bool lo = true) {
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  float* part = t.splits > 1 ? t.part : y;
  const SkWs sk{t.sk_flags, t.sk_part, t.sk_n, sub};
  int st;
  switch (type) {
    case WH_TYPE_Q4_0: st = launch_typed<WH_TYPE_Q4_0>(wp, n_rows, k, n_tokens, t.frag, t.rs, t.bs, dmin, part, t.splits, sk, s, lo); break;
    case WH_TYPE_Q4_1: st = launch_typed<WH_TYPE_Q4_1>(wp, n_rows, k, n_tokens, t.frag, t.rs, t.bs, dmin, part, t.splits, sk, s, lo); break;
    case WH_TYPE_Q8_0: st = launch_typed<WH_TYPE_Q8_0>(wp, n_rows, k, n_tokens, t.frag, t.rs, t.bs, dmin, part, t.splits, sk, s, lo); break;
    case kGemmQ4F: st = launch_typed<kGemmQ4F>(wp, n_rows, k, n_tokens, t.frag, t.rs, t.bs, dmin, part, t.splits, sk, s, lo); break;
    case kGemmQ8H: st = launch_typed<kGemmQ8H>(wp, n_rows, k, n_tokens, t.frag, t.rs, t.bs, dmin, part, t.splits, sk, s, lo); break;
    default: return set_error(WH_ERR_UNSUPPORTED_TYPE, "gemm: unsupported type %d", type);
  }
  if (st != WH_OK) return st;
  if (t.splits > 1) {
    const size_t n = n_rows * n_tokens;
    size_t gsz = (n + 255) / 256;
    const size_t cap = static_cast<size_t>(cu_count()) * 8;
    if (gsz > cap) gsz = cap;
    tiled_splitk_reduce_kernel<<<static_cast<unsigned>(gsz), 256, 0, s>>>(part, t.splits, n, y);
    WH_LAUNCH_CHECK("split-K reduce launch");
  }
  return WH_OK;
}

int launch_gemm_tiled(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                      float* y, void* workspace, hipStream_t s) {
  const TiledWs t = tiled_ws(type, n_rows, k, n_tokens, workspace);
  int st = tiled_pack<kPackPlain>(type, t, x, nullptr, nullptr, 0.f, n_tokens, k, k, s);
  if (st) return st;
  return tiled_run(type, w, n_rows, k, n_tokens, t, y, s);
}

int launch_gemm_tiled_bf16(int type, const void* w, size_t n_rows, size_t k, const uint16_t* x, size_t n_tokens,
                           float* y, void* workspace, hipStream_t s) {
  const TiledWs t = tiled_ws(type, n_rows, k, n_tokens, workspace);
  int st = tiled_pack<kPackPlain, true>(type, t, reinterpret_cast<const float*>(x), nullptr, nullptr, 0.f, n_tokens,
                                        k, k, s);
  if (st) return st;
  return tiled_run(type, w, n_rows, k, n_tokens, t, y, s, nullptr, 0, /*lo=*/false);
}

// ------------------------------------------------------------- K-quants
// The matrix is repacked (kquant.hip) into the front of the workspace, in the
// GEMM format of kquant_gemm_type with reduction length kquant_gemm_k; the
// packed activations and the rest of the GEMM's workspace follow it.
bool gemm_kquant_ok(int type, const void* w, const float* x, size_t n_rows, size_t k, size_t n_tokens) {
  if (!is_kquant(type) || k % 256 != 0 || !aligned(w, 16)) return false;
  // the repacked matrix is 256-byte aligned; any such address stands for it
  const void* repacked = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
  return gemm_tiled_ok(kquant_gemm_type(type), repacked, x, n_rows, kquant_gemm_k(type, k), n_tokens);
}

// GEMM on a repacked K-quant matrix rp (its GEMM format, rows of k elements)
// over packed activations t; Q4_K's dmin table follows the blocks.
static int kquant_run(int type, const char* rp, size_t n_rows, size_t k, size_t n_tokens, const TiledWs& t,
                      float* y, hipStream_t s, int sub = 0) {
  // (the fp16 table, passed through the kernels' dmin pointer)
  const float* dmin_t =
      type == WH_TYPE_Q4_K ? reinterpret_cast<const float*>(rp + n_rows * (k / 32) * 20) : nullptr;
  return tiled_run(kquant_gemm_type(type), rp, n_rows, kquant_gemm_k(type, k), n_tokens, t, y, s, dmin_t, sub);
}

size_t gemm_kquant_workspace_bytes(int type, size_t n_rows, size_t n_tokens, size_t k) {
  return al256(kquant_repacked_bytes(type, n_rows, k)) +
         gemm_tiled_workspace_bytes(kquant_gemm_type(type), n_rows, n_tokens, kquant_gemm_k(type, k));
}

int launch_gemm_kquant(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                       float* y, void* workspace, hipStream_t s) {
  const int it = kquant_gemm_type(type);
  const size_t kk = kquant_gemm_k(type, k);
  char* rp = static_cast<char*>(workspace);
  const TiledWs t = tiled_ws(it, n_rows, kk, n_tokens, rp + al256(kquant_repacked_bytes(type, n_rows, k)));
  // a handle's copy prepared once (wh_weight_prepare_prefill), else a conversion per call
  const char* src = static_cast<const char*>(prepared_kquant(w, type, n_rows, k));
  int st = src ? WH_OK : launch_repack_kquant(type, w, n_rows, k, rp, s);
  if (!src) src = rp;
  if (!st) st = tiled_pack<kPackPlain>(it, t, x, nullptr, nullptr, 0.f, n_tokens, kk, k, s);
  if (st) return st;
  return kquant_run(type, src, n_rows, k, n_tokens, t, y, s);
}

size_t ffn_kquant_workspace_bytes(int type, size_t hidden, size_t n_ff, size_t n_tokens) {
  const int it = kquant_gemm_type(type);
  const size_t r1 = kquant_repacked_bytes(type, n_ff, hidden), r2 = kquant_repacked_bytes(type, hidden, n_ff);
  const size_t t1 = gemm_tiled_workspace_bytes(it, n_ff, n_tokens, kquant_gemm_k(type, hidden));
  const size_t t2 = gemm_tiled_workspace_bytes(it, hidden, n_tokens, kquant_gemm_k(type, n_ff));
  return al256(r1 > r2 ? r1 : r2) + (t1 > t2 ? t1 : t2);
}

// The FFN for n_tokens rows on the tiled kernel: the RMSNorm of x is packed
// once for both gate and up, the SwiGLU of their outputs is formed while the
// down projection's activations are packed.  g, u: n_tokens x n_ff scratch.
// WH_ERR_INVALID_SHAPE (nothing launched) when a product does not fit.
int launch_ffn_tiled(int type, const void* gate, const void* up, const void* down, size_t hidden, size_t n_ff,
                     const float* x, const float* gamma, float eps, size_t n_tokens, float* g, float* u, float* out,
                     void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (is_kquant(type)) {
    // one repacked matrix at a time in the front of the workspace (stream order
    // keeps a GEMM's reads ahead of the next repack)
    const int it = kquant_gemm_type(type);
    const size_t H2 = kquant_gemm_k(type, hidden), F2 = kquant_gemm_k(type, n_ff);
    const size_t r1 = kquant_repacked_bytes(type, n_ff, hidden), r2 = kquant_repacked_bytes(type, hidden, n_ff);
    char* rp = static_cast<char*>(workspace);
    char* ws = rp + al256(r1 > r2 ? r1 : r2);
    if (!gemm_kquant_ok(type, gate, x, n_ff, hidden, n_tokens) || !aligned(up, 16) || !aligned(down, 16) ||
        !gemm_kquant_ok(type, down, g, hidden, n_ff, n_tokens) || !aligned(gamma, 16) || !aligned(u, 16) ||
        !aligned(workspace, 256) || workspace_bytes < ffn_kquant_workspace_bytes(type, hidden, n_ff, n_tokens))
      return WH_ERR_INVALID_SHAPE;
    // each matrix: its handle's prepared copy, or converted into rp for this call
    auto repacked = [&](const void* w, size_t rows, size_t k, const char** out_rp) -> int {
      const char* pre = static_cast<const char*>(prepared_kquant(w, type, rows, k));
      *out_rp = pre ? pre : rp;
      return pre ? WH_OK : launch_repack_kquant(type, w, rows, k, rp, s);
    };
    const char* src = nullptr;
    const TiledWs t1 = tiled_ws(it, n_ff, H2, n_tokens, ws);
    int st = tiled_pack<kPackNorm>(it, t1, x, nullptr, gamma, eps, n_tokens, H2, hidden, s);
    if (!st) st = repacked(gate, n_ff, hidden, &src);
    if (!st) st = kquant_run(type, src, n_ff, hidden, n_tokens, t1, g, s, 0);
    if (!st) st = repacked(up, n_ff, hidden, &src);
    if (!st) st = kquant_run(type, src, n_ff, hidden, n_tokens, t1, u, s, 1);
    if (st) return st;
    const TiledWs t2 = tiled_ws(it, hidden, F2, n_tokens, ws);
    st = tiled_pack<kPackSwiglu>(it, t2, g, u, nullptr, 0.f, n_tokens, F2, n_ff, s);
    if (!st) st = repacked(down, hidden, n_ff, &src);
    if (st) return st;
    return kquant_run(type, src, hidden, n_ff, n_tokens, t2, out, s);
  }
  if (!gemm_tiled_ok(type, gate, x, n_ff, hidden, n_tokens) || !gemm_tiled_ok(type, up, x, n_ff, hidden, n_tokens) ||
      !gemm_tiled_ok(type, down, g, hidden, n_ff, n_tokens) || !aligned(gamma, 16) || !aligned(u, 16))
    return WH_ERR_INVALID_SHAPE;
  if (workspace_bytes < gemm_tiled_workspace_bytes(type, n_ff, n_tokens, hidden) ||
      workspace_bytes < gemm_tiled_workspace_bytes(type, hidden, n_tokens, n_ff))
    return WH_ERR_INVALID_SHAPE;
  const TiledWs t1 = tiled_ws(type, n_ff, hidden, n_tokens, workspace);
  int st = tiled_pack<kPackNorm>(type, t1, x, nullptr, gamma, eps, n_tokens, hidden, hidden, s);
  if (st) return st;
  const TiledWs t2 = tiled_ws(type, hidden, n_ff, n_tokens, workspace);
  if (gemm_tiled_splits(2 * n_ff, n_tokens, hidden) == 1) {
    // enough tiles without split-K: gate and up in one pass, h = silu(g) * u
    // written by its epilogue (g holds h), then packed for the down projection
    const uint8_t* gp = static_cast<const uint8_t*>(gate);
    const uint8_t* upp = static_cast<const uint8_t*>(up);
    const SkWs sk{t1.sk_flags, t1.sk_part, t1.sk_n, 0};
    switch (type) {
      case WH_TYPE_Q4_0: st = launch_ffn_typed<WH_TYPE_Q4_0>(gp, upp, n_ff, hidden, n_tokens, t1.frag, t1.rs, t1.bs, g, sk, s); break;
      case WH_TYPE_Q4_1: st = launch_ffn_typed<WH_TYPE_Q4_1>(gp, upp, n_ff, hidden, n_tokens, t1.frag, t1.rs, t1.bs, g, sk, s); break;
      default: st = launch_ffn_typed<WH_TYPE_Q8_0>(gp, upp, n_ff, hidden, n_tokens, t1.frag, t1.rs, t1.bs, g, sk, s); break;
    }
    if (!st) st = tiled_pack<kPackPlain>(type, t2, g, nullptr, nullptr, 0.f, n_tokens, n_ff, n_ff, s);
  } else {
    st = tiled_run(type, gate, n_ff, hidden, n_tokens, t1, g, s, nullptr, 0);
    if (!st) st = tiled_run(type, up, n_ff, hidden, n_tokens, t1, u, s, nullptr, 1);
    if (!st) st = tiled_pack<kPackSwiglu>(type, t2, g, u, nullptr, 0.f, n_tokens, n_ff, n_ff, s);
  }
  if (st) return st;
  return tiled_run(type, down, hidden, n_ff, n_tokens, t2, out, s);
}

}  // namespace wh

WH_API int wh_set_stream_k_wait(uint32_t ticks) {
  g_sk_wait.store(ticks, std::memory_order_relaxed);
  return WH_OK;
}
