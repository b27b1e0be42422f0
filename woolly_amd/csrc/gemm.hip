// gemm.hip -- quantized matrix-matrix product Y = X W^T on gfx950 MFMA.
//
// Replaces the projections woolly computes on fully dequantized f32 weights
// (simd_matmul_optimized -> Gemm::compute, tensor_utils_simd.rs:855-914 and
// ops/matmul.rs:83-259, called from simd_ffn_forward tensor_utils_simd.rs:605-754):
//   Y[t, r] = sum_k X[t, k] * W[r, k],  W in GGUF Q4_0 / Q4_1 / Q8_0 blocks.
//
// Numerics.  The weights' integer parts are exact in fp16 (q - 8 in [-8, 7],
// q in [0, 15], int8 in [-127, 127]); each activation row is scaled by a power
// of two so that its largest magnitude lies in [2^13, 2^14) and split into
// hi = fp16(x) and lo = fp16(x - hi) (about 22 significant bits).  For each
// 32-element block the MFMA accumulates both halves in f32 into a fresh
// accumulator, and the block scale d is then applied in f32:
//   acc += d * (sum_k q_k hi_k + sum_k q_k lo_k)         (Q4_0, Q8_0)
//   acc += d * (...) + m * sum_{k in block} x_k          (Q4_1)
// so no weight precision is lost and activations keep f32-level accuracy.
//
// Kernels.
//   split_rows_kernel: one workgroup per token row: row max -> power-of-two
//     scale, hi/lo halves, and (Q4_1) per-block sums of x.
//   gemm_mfma_kernel: 256 threads, a 128 (tokens) x 128 (weight rows) tile,
//     each wave a 64 x 64 sub-tile of 2 x 2 v_mfma_f32_32x32x16_f16.  Two
//     blocks per iteration: activations (hi, lo) and the dequantized weights
//     (q - 8 as fp16) are staged in LDS with a 16-byte row pad (conflict-free
//     128-bit reads), block scales in small LDS arrays; the next iteration's
//     data is fetched into registers while the current MFMAs run.  When the
//     output has fewer tiles than CUs, K is split over blockIdx.z and the
//     partial planes are summed in split order (splitk_reduce_kernel).
#include "wh_blocks.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128;        // token rows per workgroup tile
constexpr int BN = 128;        // weight rows per workgroup tile

// ---------------------------------------------------------------- pre-pass
// Row t of X -> hi/lo fp16 halves of X * 2^-e (e chosen so that
// max|x| * 2^-e is in [2^13, 2^14)), rscale[t] = 2^e; optional per-block sums
// of the scaled row.
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, size_t k,
                                                         _Float16* __restrict__ hi,
                                                         _Float16* __restrict__ lo,
                                                         float* __restrict__ rscale,
                                                         float* __restrict__ bsum) {
  __shared__ float red[4];
  const size_t t = blockIdx.x;
  const float* xr = x + t * k;
  float mx = 0.f;
  for (size_t i = threadIdx.x; i < k; i += 256) mx = fmaxf(mx, fabsf(xr[i]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // Scale every finite, non-zero row so that its largest magnitude lands in
  // [2^13, 2^14): large rows cannot overflow fp16 and small rows keep both
  // halves out of the fp16 subnormal range.
  int e = 0;
  if (mx > 0.f && mx <= 3.4e38f) {
    int ex;
    frexpf(mx, &ex);          // mx = f * 2^ex, f in [0.5, 1)
    e = ex - 14;              // mx * 2^-e in [2^13, 2^14)
    if (e < -100) e = -100;   // keep 2^e a normal float
  }
  const float down = ldexpf(1.f, -e);
  if (threadIdx.x == 0) rscale[t] = ldexpf(1.f, e);
  _Float16* hr = hi + t * k;
  _Float16* lr = lo + t * k;
  for (size_t i = threadIdx.x; i < k; i += 256) {
    const float v = xr[i] * down;  // exact: power-of-two scaling
    const _Float16 h = static_cast<_Float16>(v);
    hr[i] = h;
    lr[i] = static_cast<_Float16>(v - static_cast<float>(h));
  }
  if (bsum) {  // block sums of the scaled row (same units as hi + lo)
    const size_t nb = k / 32;
    for (size_t b = threadIdx.x; b < nb; b += 256) {
      float s = 0.f;
      for (int j = 0; j < 32; j++) s += xr[b * 32 + j] * down;
      bsum[t * nb + b] = s;
    }
  }
}

// ---------------------------------------------------------------- dequant to LDS
// Thread (n, h) of the B stage: weight row n of the tile, half h of the block
// (h = 0: quant bytes 0..7 -> elements 0..7 and 16..23; h = 1: bytes 8..15 ->
// elements 8..15 and 24..31).  Writes 16 fp16 integers to LDS and the scale(s).
template <int TYPE>
__device__ __forceinline__ void stage_b(const uint8_t* __restrict__ blk, bool ok, int h,
                                        _Float16* __restrict__ row_lds, float* __restrict__ d_lds,
                                        float* __restrict__ m_lds) {
  half8 lo8, hi8;
  if (!ok) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      lo8[i] = static_cast<_Float16>(0.f);
      hi8[i] = static_cast<_Float16>(0.f);
    }
    if (h == 0) {
      *d_lds = 0.f;
      if (m_lds) *m_lds = 0.f;
    }
  } else if constexpr (TYPE == WH_TYPE_Q8_0) {
    // h selects elements [16h, 16h + 16): quant bytes 2 + 16h .. (2-byte aligned)
    const uint16_t* q16 = reinterpret_cast<const uint16_t*>(blk + 2 + 16 * h);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t u = q16[i];
      lo8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(u & 0xFFu)));
      lo8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(u >> 8)));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t u = q16[4 + i];
      hi8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(u & 0xFFu)));
      hi8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(u >> 8)));
    }
    if (h == 0) *d_lds = whd::f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk));
  } else {
    constexpr int QOFF = TYPE == WH_TYPE_Q4_0 ? 2 : 4;
    constexpr int BIAS = TYPE == WH_TYPE_Q4_0 ? 8 : 0;
    const uint16_t* q16 = reinterpret_cast<const uint16_t*>(blk + QOFF + 8 * h);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t u = q16[i];
      lo8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int>(u & 15u) - BIAS));
      lo8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 8) & 15u) - BIAS));
      hi8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 4) & 15u) - BIAS));
      hi8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 12) & 15u) - BIAS));
    }
    if (h == 0) {
      const uint16_t* dm = reinterpret_cast<const uint16_t*>(blk);
      *d_lds = whd::f16_bits_to_f32(dm[0]);
      if constexpr (TYPE == WH_TYPE_Q4_1) *m_lds = whd::f16_bits_to_f32(dm[1]);
    }
  }
  if constexpr (TYPE == WH_TYPE_Q8_0) {
    *reinterpret_cast<half8*>(row_lds + 16 * h) = lo8;
    *reinterpret_cast<half8*>(row_lds + 16 * h + 8) = hi8;
  } else {
    *reinterpret_cast<half8*>(row_lds + 8 * h) = lo8;
    *reinterpret_cast<half8*>(row_lds + 16 + 8 * h) = hi8;
  }
}

// Raw bytes of one block for one B-stage thread: the scale word(s) and the 8
// (Q4_x) or 16 (Q8_0) quant bytes of its half, loaded as 16-bit words (blocks
// are only 2-byte aligned).  Dequantized to fp16 integers when staged in LDS.
template <int TYPE>
struct BRaw {
  static constexpr int NQ = TYPE == WH_TYPE_Q8_0 ? 8 : 4;  // 16-bit words of quants
  uint32_t dm;                                             // d | m << 16
  uint32_t q[NQ];
};

template <int TYPE>
__device__ __forceinline__ void load_braw(const uint8_t* __restrict__ blk, bool ok, int h, BRaw<TYPE>& r) {
  constexpr int QOFF = TYPE == WH_TYPE_Q4_1 ? 4 : 2;
  constexpr int HSTEP = TYPE == WH_TYPE_Q8_0 ? 16 : 8;
  const uint16_t* p = reinterpret_cast<const uint16_t*>(blk);
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(blk + QOFF + HSTEP * h);
  r.dm = ok ? (TYPE == WH_TYPE_Q4_1 ? (static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16))
                                    : static_cast<uint32_t>(p[0]))
            : 0u;
#pragma unroll
  for (int i = 0; i < BRaw<TYPE>::NQ; i++) r.q[i] = ok ? q16[i] : 0u;
}

template <int TYPE>
__device__ __forceinline__ void store_braw(const BRaw<TYPE>& r, int h, _Float16* __restrict__ row_lds,
                                           float* __restrict__ d_lds, float* __restrict__ m_lds) {
  half8 lo8, hi8;
  if constexpr (TYPE == WH_TYPE_Q8_0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      lo8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(r.q[i] & 0xFFu)));
      lo8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(r.q[i] >> 8)));
      hi8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(r.q[4 + i] & 0xFFu)));
      hi8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(r.q[4 + i] >> 8)));
    }
    *reinterpret_cast<half8*>(row_lds + 16 * h) = lo8;
    *reinterpret_cast<half8*>(row_lds + 16 * h + 8) = hi8;
  } else {
    constexpr int BIAS = TYPE == WH_TYPE_Q4_0 ? 8 : 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t u = r.q[i];
      lo8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int>(u & 15u) - BIAS));
      lo8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 8) & 15u) - BIAS));
      hi8[2 * i] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 4) & 15u) - BIAS));
      hi8[2 * i + 1] = static_cast<_Float16>(static_cast<float>(static_cast<int>((u >> 12) & 15u) - BIAS));
    }
    *reinterpret_cast<half8*>(row_lds + 8 * h) = lo8;
    *reinterpret_cast<half8*>(row_lds + 16 + 8 * h) = hi8;
  }
  if (h == 0) {
    *d_lds = whd::f16_bits_to_f32(r.dm & 0xFFFFu);
    if constexpr (TYPE == WH_TYPE_Q4_1) *m_lds = whd::f16_bits_to_f32(r.dm >> 16);
  }
}

constexpr int BKB = 2;  // blocks (of 32 k) per main-loop iteration

// Y (or the split-K partial plane blockIdx.z) for tokens [t0, t0 + BM) and
// weight rows [r0, r0 + BN), over blocks [kb0, kb1).  The next iteration's
// activations and raw weight bytes are fetched into registers while the
// current iteration's MFMAs run.
template <int TYPE>
__global__ __launch_bounds__(256, 2) void gemm_mfma_kernel(const uint8_t* __restrict__ W,
                                                        const _Float16* __restrict__ xhi,
                                                        const _Float16* __restrict__ xlo,
                                                        const float* __restrict__ rscale,
                                                        const float* __restrict__ bsum,
                                                        float* __restrict__ y, int n_tokens,
                                                        int n_rows, int k, int blocks_per_split) {
  constexpr int TS = whd::BlockFmt<TYPE>::BYTES;
  constexpr int KS = 32 * BKB;        // k per iteration
  constexpr int STR = KS + 8;         // halves per staged row (pad 16 B)
  __shared__ __align__(16) _Float16 a_lds[2 * BM * STR];  // hi rows, then lo rows
  _Float16* const a_hi = a_lds;
  _Float16* const a_lo = a_lds + BM * STR;
  __shared__ __align__(16) _Float16 b_q[BN * STR];
  __shared__ float b_d[BKB][BN];
  __shared__ float b_m[BKB][BN];
  __shared__ float a_s[BKB][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;
  const int t0 = blockIdx.y * BM;
  const int r0 = blockIdx.x * BN;
  const int nb = k / 32;
  const int kb0 = blockIdx.z * blocks_per_split;
  const int kb1 = min(nb, kb0 + blocks_per_split);
  const size_t row_bytes = static_cast<size_t>(nb) * TS;

  // A staging: 2 limbs x BM rows x KS halves = 2 * BM * KS / 8 chunks of 16 B
  constexpr int ACH = 2 * BM * KS / 8 / 256;  // chunks per thread (8)
  const _Float16* a_src[ACH];
  int a_dst[ACH];
  bool a_ok[ACH];
#pragma unroll
  for (int c = 0; c < ACH; c++) {
    const int chunk = tid + 256 * c;
    const int limb = chunk / (BM * KS / 8);
    const int rem = chunk % (BM * KS / 8);
    const int row = rem / (KS / 8);
    const int q = rem % (KS / 8);
    const int t = t0 + row;
    a_ok[c] = t < n_tokens;
    a_src[c] = (limb ? xlo : xhi) + static_cast<size_t>(a_ok[c] ? t : 0) * k + 8 * q;
    a_dst[c] = (limb ? BM * STR : 0) + row * STR + 8 * q;  // offset into a_lds
  }
  // B staging: (row n, block j of the iteration, half h) = BN * BKB * 2 tasks
  constexpr int BCH = BN * BKB * 2 / 256;  // tasks per thread (2)
  const uint8_t* b_src[BCH];
  int b_n[BCH], b_j[BCH], b_h[BCH];
  bool b_ok[BCH];
#pragma unroll
  for (int c = 0; c < BCH; c++) {
    const int task = tid + 256 * c;
    b_n[c] = task >> 2;
    b_j[c] = (task >> 1) & 1;
    b_h[c] = task & 1;
    b_ok[c] = r0 + b_n[c] < n_rows;
    b_src[c] = W + static_cast<size_t>(b_ok[c] ? r0 + b_n[c] : 0) * row_bytes + b_j[c] * TS;
  }

  half8 a_reg[ACH];
  BRaw<TYPE> b_reg[BCH];
  float s_reg = 0.f;
  auto fetch = [&](int kb) {
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      if (a_ok[c]) {
        a_reg[c] = *reinterpret_cast<const half8*>(a_src[c] + kb * 32);
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) a_reg[c][i] = static_cast<_Float16>(0.f);
      }
    }
#pragma unroll
    for (int c = 0; c < BCH; c++) {
      const bool ok = b_ok[c] && kb + b_j[c] < kb1;
      load_braw<TYPE>(b_src[c] + static_cast<size_t>(kb) * TS, ok, b_h[c], b_reg[c]);
    }
    if constexpr (TYPE == WH_TYPE_Q4_1) {
      if (tid < BM * BKB) {
        const int row = tid % BM, j = tid / BM;
        const int t = t0 + row;
        s_reg = (t < n_tokens && kb + j < kb1) ? bsum[static_cast<size_t>(t) * nb + kb + j] : 0.f;
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int c = 0; c < ACH; c++) *reinterpret_cast<half8*>(a_lds + a_dst[c]) = a_reg[c];
#pragma unroll
    for (int c = 0; c < BCH; c++)
      store_braw<TYPE>(b_reg[c], b_h[c], b_q + b_n[c] * STR + 32 * b_j[c], &b_d[b_j[c]][b_n[c]],
                       TYPE == WH_TYPE_Q4_1 ? &b_m[b_j[c]][b_n[c]] : nullptr);
    if constexpr (TYPE == WH_TYPE_Q4_1) {
      if (tid < BM * BKB) a_s[tid / BM][tid % BM] = s_reg;
    }
  };

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const int mrow = lane & 31;
  const int kg = lane >> 5;
  if (kb0 < kb1) {
    fetch(kb0);
    stash();
  }
  __syncthreads();
  for (int kb = kb0; kb < kb1; kb += BKB) {
    const bool more = kb + BKB < kb1;
    if (more) fetch(kb + BKB);
#pragma unroll
    for (int j = 0; j < BKB; j++) {
      if (kb + j >= kb1) break;
      half8 ah[2][2], al[2][2], bq[2][2];
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
          const int off = (wm + 32 * i + mrow) * STR + 32 * j + 16 * s + 8 * kg;
          ah[i][s] = *reinterpret_cast<const half8*>(a_hi + off);
          al[i][s] = *reinterpret_cast<const half8*>(a_lo + off);
        }
#pragma unroll
      for (int n = 0; n < 2; n++)
#pragma unroll
        for (int s = 0; s < 2; s++)
          bq[n][s] = *reinterpret_cast<const half8*>(b_q + (wn + 32 * n + mrow) * STR + 32 * j + 16 * s + 8 * kg);
#pragma unroll
      for (int n = 0; n < 2; n++) {
        const float d = b_d[j][wn + 32 * n + mrow];
        const float mm = TYPE == WH_TYPE_Q4_1 ? b_m[j][wn + 32 * n + mrow] : 0.f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          float16v t = {};
          t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bq[n][0], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bq[n][1], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], bq[n][0], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], bq[n][1], t, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 16; e++) {
            float v = __builtin_fmaf(d, t[e], acc[i][n][e]);
            if constexpr (TYPE == WH_TYPE_Q4_1) {
              const int m = wm + 32 * i + 8 * (e >> 2) + 4 * kg + (e & 3);
              v = __builtin_fmaf(mm, a_s[j][m], v);
            }
            acc[i][n][e] = v;
          }
        }
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }

  // epilogue: undo the row scale; split-K partials go to plane blockIdx.z
  float* out = y + static_cast<size_t>(blockIdx.z) * n_tokens * n_rows;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int n = 0; n < 2; n++) {
      const int r = r0 + wn + 32 * n + mrow;
      if (r >= n_rows) continue;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int t = t0 + wm + 32 * i + 8 * (e >> 2) + 4 * kg + (e & 3);
        if (t < n_tokens) out[static_cast<size_t>(t) * n_rows + r] = acc[i][n][e] * rscale[t];
      }
    }
}

// y[i] = sum_s part[s][i] in split order (deterministic).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                            size_t n, float* __restrict__ y) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = part[i];
    for (int s = 1; s < splits; s++) v += part[static_cast<size_t>(s) * n + i];
    y[i] = v;
  }
}

}  // namespace

namespace wh {

// Split-K factor: enough workgroups to cover the CUs when the output has few
// tiles (e.g. the FFN down projection, 4096 rows x 512 tokens = 128 tiles).
int gemm_splits(size_t n_rows, size_t n_tokens, size_t k) {
  const size_t tiles = ((n_rows + BN - 1) / BN) * ((n_tokens + BM - 1) / BM);
  const size_t nb = k / 32;
  const size_t cus = static_cast<size_t>(cu_count());
  int s = 1;
  while (s < 8 && tiles * s < cus && nb / (2 * s) >= 16) s *= 2;
  return s;
}

size_t gemm_workspace_bytes(int type, size_t n_tokens, size_t k) {
  // hi, lo halves + row scales (+ block sums for Q4_1), each 256-byte aligned,
  // plus room for split-K partial planes (sized for up to 8 splits of a
  // 4096-row output; callers with other shapes get the exact need below).
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  size_t b = 2 * al(n_tokens * k * 2) + al(n_tokens * 4);
  if (type == WH_TYPE_Q4_1) b += al(n_tokens * (k / 32) * 4);
  return b;
}

static size_t splitk_bytes(size_t n_rows, size_t n_tokens, int splits) {
  return splits > 1 ? (static_cast<size_t>(splits) * n_rows * n_tokens * 4 + 255) / 256 * 256 : 0;
}

size_t gemm_workspace_bytes_for(int type, size_t n_rows, size_t n_tokens, size_t k) {
  if (is_kquant(type)) return gemm_kquant_workspace_bytes(type, n_rows, n_tokens, k);
  // enough for either kernel (the choice also depends on the weights' alignment)
  const size_t a = gemm_workspace_bytes(type, n_tokens, k) +
                   splitk_bytes(n_rows, n_tokens, gemm_splits(n_rows, n_tokens, k));
  const size_t b = gemm_tiled_workspace_bytes(type, n_rows, n_tokens, k);
  return a > b ? a : b;
}

int launch_gemm_mfma(int type, const void* w, size_t n_rows, size_t k, const float* x,
                     size_t n_tokens, float* y, void* workspace, hipStream_t s) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  char* ws = static_cast<char*>(workspace);
  _Float16* hi = reinterpret_cast<_Float16*>(ws);
  ws += al(n_tokens * k * 2);
  _Float16* lo = reinterpret_cast<_Float16*>(ws);
  ws += al(n_tokens * k * 2);
  float* rs = reinterpret_cast<float*>(ws);
  ws += al(n_tokens * 4);
  float* bs = nullptr;
  if (type == WH_TYPE_Q4_1) {
    bs = reinterpret_cast<float*>(ws);
    ws += al(n_tokens * (k / 32) * 4);
  }
  const int splits = gemm_splits(n_rows, n_tokens, k);
  float* part = splits > 1 ? reinterpret_cast<float*>(ws) : y;
  split_rows_kernel<<<static_cast<unsigned>(n_tokens), 256, 0, s>>>(x, k, hi, lo, rs, bs);
  WH_LAUNCH_CHECK("split_rows kernel launch");
  const int nb = static_cast<int>(k / 32);
  int bps = (nb + splits - 1) / splits;
  bps = (bps + BKB - 1) / BKB * BKB;
  dim3 grid(static_cast<unsigned>((n_rows + BN - 1) / BN), static_cast<unsigned>((n_tokens + BM - 1) / BM),
            static_cast<unsigned>(splits));
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  switch (type) {
    case WH_TYPE_Q4_0:
      gemm_mfma_kernel<WH_TYPE_Q4_0><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, part, (int)n_tokens, (int)n_rows, (int)k, bps);
      break;
    case WH_TYPE_Q4_1:
      gemm_mfma_kernel<WH_TYPE_Q4_1><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, part, (int)n_tokens, (int)n_rows, (int)k, bps);
      break;
    case WH_TYPE_Q8_0:
      gemm_mfma_kernel<WH_TYPE_Q8_0><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, part, (int)n_tokens, (int)n_rows, (int)k, bps);
      break;
    default:
      return set_error(WH_ERR_UNSUPPORTED_TYPE, "gemm: unsupported type %d", type);
  }
  WH_LAUNCH_CHECK("gemm kernel launch");
  if (splits > 1) {
    const size_t n = n_rows * n_tokens;
    size_t g = (n + 255) / 256;
    const size_t cap = static_cast<size_t>(cu_count()) * 8;
    if (g > cap) g = cap;
    splitk_reduce_kernel<<<static_cast<unsigned>(g), 256, 0, s>>>(part, splits, n, y);
    WH_LAUNCH_CHECK("split-K reduce launch");
  }
  return WH_OK;
}

// Y[t, r] = sum_k X[t, k] W[r, k].  Few tokens: one streaming GEMV per token;
// otherwise the MFMA kernel (needs the workspace).  Q4_K / Q6_K take the
// tiled kernel after repacking, or one GEMV per token where it does not fit.
int launch_gemm(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                float* y, void* workspace, size_t workspace_bytes, hipStream_t s) {
  const bool kq = is_kquant(type);
  // 2..16 tokens: one pass of the weights on the matrix-core GEMV (Q4_0 and
  // Q8_0 shapes it takes); the workspace stays required as documented
  if (n_tokens >= 2 && n_tokens <= 16 && k > 0 && mt_allowed(n_rows, k) &&
      (n_tokens <= kGemvTokenLimit ||
       (workspace && workspace_bytes >= gemm_workspace_bytes_for(type, n_rows, n_tokens, k)))) {
    const void* mats[1] = {w};
    const int st = launch_gemv_mt(type, mats, false, x, n_tokens, nullptr, 0.f, y, n_rows, n_rows, k, s);
    if (st != WH_ERR_INVALID_SHAPE) return st;
  }
  if (n_tokens <= kGemvTokenLimit || k == 0 || !aligned(w, 2) ||
      (kq && !gemm_kquant_ok(type, w, x, n_rows, k, n_tokens))) {
    for (size_t t = 0; t < n_tokens; t++) {
      int st = launch_gemv(type, w, x + t * k, y + t * n_rows, n_rows, k, s);
      if (st != WH_OK) return st;
    }
    return WH_OK;
  }
  const size_t need = gemm_workspace_bytes_for(type, n_rows, n_tokens, k);
  if (!workspace || workspace_bytes < need)
    return set_error(WH_ERR_BUFFER_TOO_SMALL,
                     "quantized_matmul: workspace too small: needed %zu bytes, available %zu", need,
                     workspace ? workspace_bytes : static_cast<size_t>(0));
  if (kq) return launch_gemm_kquant(type, w, n_rows, k, x, n_tokens, y, workspace, s);
  if (gemm_tiled_ok(type, w, x, n_rows, k, n_tokens)) return launch_gemm_tiled(type, w, n_rows, k, x, n_tokens, y, workspace, s);
  return launch_gemm_mfma(type, w, n_rows, k, x, n_tokens, y, workspace, s);
}

}  // namespace wh
