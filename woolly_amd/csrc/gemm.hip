// gemm.hip -- quantized matrix-matrix product Y = X W^T on gfx950 MFMA.
//
// Replaces the projections woolly computes on fully dequantized f32 weights
// (simd_matmul_optimized -> Gemm::compute, tensor_utils_simd.rs:855-914 and
// ops/matmul.rs:83-259, called from simd_ffn_forward tensor_utils_simd.rs:605-754):
//   Y[t, r] = sum_k X[t, k] * W[r, k],  W in GGUF Q4_0 / Q4_1 / Q8_0 blocks.
//
// Numerics.  The weights' integer parts are exact in fp16 (q - 8 in [-8, 7],
// q in [0, 15], int8 in [-127, 127]); each activation row is scaled by a power
// of two so that its largest magnitude stays below 2^15 and split into
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
//     each wave a 64 x 64 sub-tile of 2 x 2 v_mfma_f32_32x32x16_f16.  Per
//     block: activations (hi, lo) and the dequantized weights (q - 8 as fp16)
//     are staged in LDS with a 16-byte row pad (conflict-free 128-bit reads),
//     block scales in a small LDS array.
#include "wh_blocks.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128;        // token rows per workgroup tile
constexpr int BN = 128;        // weight rows per workgroup tile
constexpr int LDS_STRIDE = 40; // halves per staged row: 32 + 8 pad (80 bytes)

// ---------------------------------------------------------------- pre-pass
// Row t of X -> hi/lo fp16 halves of X * 2^-e (e >= 0 chosen so that
// max|x| * 2^-e < 2^15), rscale[t] = 2^e; optional per-block sums of x.
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
  int e = 0;
  if (mx >= 16384.f && mx <= 3.0e38f) {
    int ex;
    frexpf(mx, &ex);          // mx = f * 2^ex, f in [0.5, 1)
    e = ex - 14;              // mx * 2^-e < 2^14
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

// Y[t, r] for t in [t0, t0 + BM), r in [r0, r0 + BN).  hi/lo: [m_rows][k]
// halves (rows >= n_tokens are never read: their tile rows load zeros).
template <int TYPE>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint8_t* __restrict__ W,
                                                        const _Float16* __restrict__ xhi,
                                                        const _Float16* __restrict__ xlo,
                                                        const float* __restrict__ rscale,
                                                        const float* __restrict__ bsum,
                                                        float* __restrict__ y, int n_tokens,
                                                        int n_rows, int k) {
  constexpr int TS = whd::BlockFmt<TYPE>::BYTES;
  __shared__ __align__(16) _Float16 a_hi[BM * LDS_STRIDE];
  __shared__ __align__(16) _Float16 a_lo[BM * LDS_STRIDE];
  __shared__ __align__(16) _Float16 b_q[BN * LDS_STRIDE];
  __shared__ float b_d[BN];
  __shared__ float b_m[BN];
  __shared__ float a_s[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 64;  // wave's token offset inside the tile
  const int wn = (wave & 1) * 64;   // wave's weight-row offset inside the tile
  const int t0 = blockIdx.y * BM;
  const int r0 = blockIdx.x * BN;
  const int nb = k / 32;
  const size_t row_bytes = static_cast<size_t>(nb) * TS;

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // B staging role of this thread
  const int bn = tid >> 1;
  const int bh = tid & 1;
  const bool b_ok = r0 + bn < n_rows;
  const uint8_t* b_row = W + static_cast<size_t>(b_ok ? r0 + bn : 0) * row_bytes;

  for (int b = 0; b < nb; b++) {
    // ---- stage A: BM rows x 32 halves x (hi, lo); 16-byte chunks
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int chunk = tid + 256 * c;      // 0..1023: limb, row, quarter
      const int limb = chunk >> 9;
      const int row = (chunk >> 2) & (BM - 1);
      const int q = chunk & 3;
      const int t = t0 + row;
      half8 v;
      if (t < n_tokens) {
        const _Float16* src = (limb ? xlo : xhi) + static_cast<size_t>(t) * k + b * 32 + 8 * q;
        v = *reinterpret_cast<const half8*>(src);
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = static_cast<_Float16>(0.f);
      }
      *reinterpret_cast<half8*>((limb ? a_lo : a_hi) + row * LDS_STRIDE + 8 * q) = v;
    }
    if (TYPE == WH_TYPE_Q4_1 && tid < BM) {
      const int t = t0 + tid;
      a_s[tid] = t < n_tokens ? bsum[static_cast<size_t>(t) * nb + b] : 0.f;
    }
    // ---- stage B: dequantize BN weight rows of block b
    stage_b<TYPE>(b_row + static_cast<size_t>(b) * TS, b_ok, bh, b_q + bn * LDS_STRIDE, &b_d[bn],
                  TYPE == WH_TYPE_Q4_1 ? &b_m[bn] : nullptr);
    __syncthreads();

    // ---- MFMA: per 32x32 tile, fresh accumulator over the block, then scale
    const int mrow = lane & 31;
    const int kg = lane >> 5;
    half8 ah[2][2], al[2][2], bq[2][2];  // [tile][kstep]
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const int off = (wm + 32 * i + mrow) * LDS_STRIDE + 16 * s + 8 * kg;
        ah[i][s] = *reinterpret_cast<const half8*>(a_hi + off);
        al[i][s] = *reinterpret_cast<const half8*>(a_lo + off);
      }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int s = 0; s < 2; s++)
        bq[j][s] = *reinterpret_cast<const half8*>(b_q + (wn + 32 * j + mrow) * LDS_STRIDE + 16 * s + 8 * kg);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float d = b_d[wn + 32 * j + mrow];
      const float mm = TYPE == WH_TYPE_Q4_1 ? b_m[wn + 32 * j + mrow] : 0.f;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        float16v t = {};
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bq[j][0], t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bq[j][1], t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], bq[j][0], t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], bq[j][1], t, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; e++) {
          float v = __builtin_fmaf(d, t[e], acc[i][j][e]);
          if constexpr (TYPE == WH_TYPE_Q4_1) {
            // block sum of the token row of C element e (x scale folded in later)
            const int m = wm + 32 * i + 8 * (e >> 2) + 4 * kg + (e & 3);
            v = __builtin_fmaf(mm, a_s[m], v);
          }
          acc[i][j][e] = v;
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: undo the row scale and store
  const int ncol = lane & 31;
  const int kg = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int r = r0 + wn + 32 * j + ncol;
      if (r >= n_rows) continue;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int t = t0 + wm + 32 * i + 8 * (e >> 2) + 4 * kg + (e & 3);
        if (t < n_tokens) {
          y[static_cast<size_t>(t) * n_rows + r] = acc[i][j][e] * rscale[t];
        }
      }
    }
}

}  // namespace

namespace wh {

size_t gemm_workspace_bytes(int type, size_t n_tokens, size_t k) {
  // hi, lo halves + row scales (+ block sums for Q4_1), each 256-byte aligned
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  size_t b = 2 * al(n_tokens * k * 2) + al(n_tokens * 4);
  if (type == WH_TYPE_Q4_1) b += al(n_tokens * (k / 32) * 4);
  return b;
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
  float* bs = type == WH_TYPE_Q4_1 ? reinterpret_cast<float*>(ws) : nullptr;
  split_rows_kernel<<<static_cast<unsigned>(n_tokens), 256, 0, s>>>(x, k, hi, lo, rs, bs);
  WH_LAUNCH_CHECK("split_rows kernel launch");
  dim3 grid(static_cast<unsigned>((n_rows + BN - 1) / BN), static_cast<unsigned>((n_tokens + BM - 1) / BM));
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  switch (type) {
    case WH_TYPE_Q4_0:
      gemm_mfma_kernel<WH_TYPE_Q4_0><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, y, (int)n_tokens, (int)n_rows, (int)k);
      break;
    case WH_TYPE_Q4_1:
      gemm_mfma_kernel<WH_TYPE_Q4_1><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, y, (int)n_tokens, (int)n_rows, (int)k);
      break;
    case WH_TYPE_Q8_0:
      gemm_mfma_kernel<WH_TYPE_Q8_0><<<grid, 256, 0, s>>>(wp, hi, lo, rs, bs, y, (int)n_tokens, (int)n_rows, (int)k);
      break;
    default:
      return set_error(WH_ERR_UNSUPPORTED_TYPE, "gemm: unsupported type %d", type);
  }
  WH_LAUNCH_CHECK("gemm kernel launch");
  return WH_OK;
}

// Y[t, r] = sum_k X[t, k] W[r, k].  Few tokens: one streaming GEMV per token;
// otherwise the MFMA kernel (needs the workspace).
int launch_gemm(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                float* y, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (n_tokens <= kGemvTokenLimit || k == 0 || !aligned(w, 2)) {
    for (size_t t = 0; t < n_tokens; t++) {
      int st = launch_gemv(type, w, x + t * k, y + t * n_rows, n_rows, k, s);
      if (st != WH_OK) return st;
    }
    return WH_OK;
  }
  const size_t need = gemm_workspace_bytes(type, n_tokens, k);
  if (!workspace || workspace_bytes < need)
    return set_error(WH_ERR_BUFFER_TOO_SMALL,
                     "quantized_matmul: workspace too small: needed %zu bytes, available %zu", need,
                     workspace ? workspace_bytes : static_cast<size_t>(0));
  return launch_gemm_mfma(type, w, n_rows, k, x, n_tokens, y, workspace, s);
}

}  // namespace wh
