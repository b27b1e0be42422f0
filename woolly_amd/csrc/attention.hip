// attention.hip -- single-token (decode) grouped-query attention over an f16
// KV cache, with rotary position embedding, on gfx950.
//
// Reference semantics: compute_optimized_gqa_attention
// (crates/woolly-core/src/model/lazy_transformer.rs:261-456) for one new token
// at position pos with a KV cache: query head h attends with KV head
// h / (n_heads / n_kv_heads) (:380-388), scores s_p = (q . k_p) / sqrt(d) for
// p <= pos (:391-400, causal), softmax with the maximum subtracted (:407-420),
// out = sum_p w_p v_p (:423-433); the new token's k and v are appended to the
// cache (:326-345).  RoPE::apply_f32 (crates/woolly-tensor/src/ops/mod.rs:472-530):
// pairs (i, i + d/2) rotate by angle = pos * inv_freq[i],
// inv_freq[i] = 1 / base^(2i/d).  The cache holds f16 ([ctx][n_kv_heads][d]);
// the new k (after RoPE) and v are rounded to f16 when stored and the step
// attends to the stored values.
//
// Work split (flash-decoding): one workgroup per (KV head, chunk of C
// positions); it applies RoPE to its G = n_heads / n_kv_heads query heads and
// writes per query head the chunk's maximum m, sum l = sum exp(s - m) and
// acc = sum exp(s - m) v (the row of position pos comes from the fresh k / v,
// which the workgroup owning pos also writes to the cache).
// attn_combine_kernel merges the chunks of each head.
//
// head_dim 128 (attn_partial_mfma_kernel): each wave owns 16-position tiles of
// the chunk (tiles w, w + 4, ...).  Scores on the matrix cores: one
// v_mfma_f32_16x16x32_f16 per 32 dims with A = the rotated queries (rows 0..G-1,
// each query split exactly enough into f16 hi + lo, two MFMAs) and B = the
// tile's K rows, which lanes load from HBM straight into the operand layout
// (lane (n, g): 16 bytes of row n at 16 g + 64 ks).  Softmax per wave with a
// running maximum (online), P·V on the VALU with V read as one dword (two dims)
// per lane and position (a 256-byte row per load instruction), P broadcast
// through LDS.  The four waves' (m, l, acc) merge through LDS in fixed order.
// head_dim 64 keeps the LDS-staged VALU kernel (attn_partial_kernel).
#include "wh_common.hpp"

typedef _Float16 at_half8 __attribute__((ext_vector_type(8)));
typedef float at_f4 __attribute__((ext_vector_type(4)));
typedef int at_i4 __attribute__((ext_vector_type(4)));

// raw buffer loads of 16 and 4 bytes (llvm.amdgcn.raw.buffer.load.*)
__device__ at_i4 at_buffer_load_x4(at_i4 rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");
__device__ int at_buffer_load_x1(at_i4 rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.i32");

namespace {

constexpr int kAttnThreads = 256;

// Buffer resource of a raw byte range: loads at offsets >= nbytes return 0
// without a memory access.
__device__ __forceinline__ at_i4 at_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  at_i4 r;
  r[0] = static_cast<int>(static_cast<uint32_t>(a));
  r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xFFFFu);
  r[2] = static_cast<int>(nbytes);
  r[3] = 0x00020000;
  return r;
}

template <int CTRL>
__device__ __forceinline__ float at_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Maximum / sum over each row of 16 lanes, in every lane of the row (fixed
// order: quad swaps, then half-row and row mirrors).
__device__ __forceinline__ float at_row_max(float v) {
  v = fmaxf(v, at_dpp<0xB1>(v));
  v = fmaxf(v, at_dpp<0x4E>(v));
  v = fmaxf(v, at_dpp<0x141>(v));
  return fmaxf(v, at_dpp<0x140>(v));
}
__device__ __forceinline__ float at_row_sum(float v) {
  v += at_dpp<0xB1>(v);
  v += at_dpp<0x4E>(v);
  v += at_dpp<0x141>(v);
  return v + at_dpp<0x140>(v);
}

// GMAX: 4 (G <= 4 query heads per KV head) or 8 (G <= 8).
template <int GMAX>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_mfma_kernel(
    const float* __restrict__ qkv, _Float16* __restrict__ k_cache, _Float16* __restrict__ v_cache,
    const float* __restrict__ inv_freq, float* __restrict__ part, int pos, int n_heads, int n_kv_heads,
    int chunk, int n_chunks, float scale) {
  constexpr int D = 128;
  extern __shared__ __align__(16) float sm[];
  const int G = n_heads / n_kv_heads;
  const int kvh = blockIdx.x;
  const int c = blockIdx.y;
  const int p0 = c * chunk;
  const int np = min(chunk, pos + 1 - p0);  // positions of this chunk (>= 1)
  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63, n = lane & 15, g = lane >> 4;
  const bool own = pos < p0 + chunk;  // pos lies in this (the last) chunk
  float* qs = sm;                                          // [GMAX][D] rotated queries
  _Float16* kvnew = reinterpret_cast<_Float16*>(qs + GMAX * D);  // [2][D] new k (rotated), v
  float* pbuf = qs + GMAX * D + D;                         // [4 waves][16][GMAX] softmax weights
  float* mw = pbuf + 4 * 16 * GMAX;                        // [4][GMAX] wave maxima, then sums
  float* lw = mw + 4 * GMAX;
  float* aw = lw + 4 * GMAX;                               // [4][GMAX][D] wave accumulators

  // K / V rows of this head: row r (0-based in the chunk) starts r * RS bytes
  // after row p0; rows from pos on read as zeros (the buffer range ends there),
  // the row of pos is filled in from the fresh k / v below
  const uint32_t RS = static_cast<uint32_t>(n_kv_heads) * D * 2;
  const int nload = own ? pos - p0 : np;
  const uint32_t range = nload > 0 ? static_cast<uint32_t>(nload - 1) * RS + D * 2 : 0u;
  const size_t head0 = (static_cast<size_t>(p0) * n_kv_heads + kvh) * D;
  const at_i4 krs = at_rsrc(k_cache + head0, range);
  const at_i4 vrs = at_rsrc(v_cache + head0, range);
  auto load_k = [&](int tile, at_i4 (&kk)[4]) {
    const int off = static_cast<int>(static_cast<uint32_t>(16 * tile + n) * RS) + 16 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) kk[ks] = at_buffer_load_x4(krs, off + 64 * ks, 0, 0);
  };
  auto load_v = [&](int tile, int (&vv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++)
      vv[i] = at_buffer_load_x1(vrs, static_cast<int>(static_cast<uint32_t>(16 * tile + i) * RS) + 4 * lane, 0, 0);
  };
  // this thread's query pairs (thread -> (head, pair i)) and its share of
  // the new k / v, requested before K and V (loads complete in order and
  // these are needed first).  Every load is unconditional (indices clamped
  // into the buffers): a load under a branch makes the compiler wait for all
  // loads in flight where the branches join.
  constexpr int QI = GMAX * (D / 2) / kAttnThreads;
  const float fpos = static_cast<float>(pos);
  float qx1[QI], qx2[QI], qf[QI];
#pragma unroll
  for (int u = 0; u < QI; u++) {
    const int e = min(t + u * kAttnThreads, G * (D / 2) - 1);
    const int h = e / (D / 2), i = e % (D / 2);
    const float* q = qkv + (kvh * G + h) * D;
    qx1[u] = q[i];
    qx2[u] = q[i + D / 2];
    qf[u] = inv_freq[i];
  }
  const float* kn = qkv + n_heads * D + kvh * D;
  const float* vn = qkv + n_heads * D + n_kv_heads * D + kvh * D;
  const float kx1 = kn[t % (D / 2)], kx2 = kn[t % (D / 2) + D / 2], kf = inv_freq[t % (D / 2)];
  const float vx = vn[t % D];
  __builtin_amdgcn_sched_barrier(0);
  at_i4 kc[4];
  int vc[16];
  int tile = wave;
  load_k(tile, kc);  // rows past the chunk's valid range read as zeros
  load_v(tile, vc);
  __builtin_amdgcn_sched_barrier(0);  // the rotations below wait for the query loads

  // rotated queries into LDS.  No branch: threads past the last pair write
  // the last pair's values again (a branch would let the compiler move the
  // loads above into it, after the K / V loads)
#pragma unroll
  for (int u = 0; u < QI; u++) {
    const int e = min(t + u * kAttnThreads, G * (D / 2) - 1);
    const int h = e / (D / 2), i = e % (D / 2);
    float sn, cs;
    sincosf(fpos * qf[u], &sn, &cs);
    qs[h * D + i] = qx1[u] * cs - qx2[u] * sn;
    qs[h * D + i + D / 2] = qx1[u] * sn + qx2[u] * cs;
  }
  {
    // the new token: rotate k, round k and v to f16; the chunk of pos stores
    // them in the cache
    float sn, cs;
    sincosf(fpos * kf, &sn, &cs);
    const _Float16 a = static_cast<_Float16>(kx1 * cs - kx2 * sn);
    const _Float16 b = static_cast<_Float16>(kx1 * sn + kx2 * cs);
    const _Float16 v = static_cast<_Float16>(vx);
    const size_t off = (static_cast<size_t>(pos) * n_kv_heads + kvh) * D;
    if (own && t < D / 2) {
      kvnew[t] = a;
      kvnew[t + D / 2] = b;
      k_cache[off + t] = a;
      k_cache[off + t + D / 2] = b;
    } else if (own && t >= D && t < 2 * D) {
      const int d = t - D;  // t % D == d: vx is vn[d]
      kvnew[D + d] = v;
      v_cache[off + d] = v;
    }
  }
  // LDS-only barrier: a __syncthreads() would also wait for the K / V loads in flight
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // A operands: row m < G is query head m, split into f16 hi + lo
  at_half8 qh[4], ql[4];
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float x = n < G ? qs[n * D + 32 * ks + 8 * g + j] : 0.f;
      const _Float16 hi = static_cast<_Float16>(x);
      qh[ks][j] = hi;
      ql[ks][j] = static_cast<_Float16>(x - static_cast<float>(hi));
    }
  }

  float m_run[GMAX], l_run[GMAX], acc[GMAX][2];
#pragma unroll
  for (int h = 0; h < GMAX; h++) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
    acc[h][0] = acc[h][1] = 0.f;
  }
  float* pw = pbuf + wave * 16 * GMAX;
  for (; 16 * tile < np; tile += 4) {
    at_i4 kn_[4];
    int vn_[16];
    const bool more = 16 * (tile + 4) < np;
    if (more) {
      load_k(tile + 4, kn_);
      load_v(tile + 4, vn_);
    }
    if (own && tile == (pos - p0) / 16) {
      // the row of pos from the fresh k / v
      const int r = (pos - p0) % 16;
      if (n == r) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) kc[ks] = *reinterpret_cast<const at_i4*>(kvnew + 32 * ks + 8 * g);
      }
      const int vnew = *reinterpret_cast<const int*>(kvnew + D + 2 * lane);
#pragma unroll
      for (int i = 0; i < 16; i++)
        if (i == r) vc[i] = vnew;
    }
    at_f4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const at_half8 kb = __builtin_bit_cast(at_half8, kc[ks]);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], kb, S, 0, 0, 0);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[ks], kb, S, 0, 0, 0);
    }
    // lane (n, g): scores of heads 4 g .. 4 g + 3 at tile position n
    const bool valid = 16 * tile + n < np;
    float s[4], mt[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      s[j] = valid ? S[j] * scale : -INFINITY;
      mt[j] = at_row_max(s[j]);
    }
    float m_new[GMAX], alpha[GMAX];
#pragma unroll
    for (int h = 0; h < GMAX; h++) {
      const float th = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mt[h & 3]), 16 * (h >> 2)));
      m_new[h] = fmaxf(m_run[h], th);  // finite: the tile holds a valid position
      alpha[h] = expf(m_run[h] - m_new[h]);  // 0 while m_run is -inf
    }
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float mn = m_new[j];
      if constexpr (GMAX == 8) mn = g == 1 ? m_new[4 + j] : mn;
      p[j] = valid ? expf(s[j] - mn) : 0.f;
    }
    float lt[4];
#pragma unroll
    for (int j = 0; j < 4; j++) lt[j] = at_row_sum(p[j]);
    if (g < GMAX / 4) *reinterpret_cast<float4*>(pw + n * GMAX + 4 * g) = make_float4(p[0], p[1], p[2], p[3]);
#pragma unroll
    for (int h = 0; h < GMAX; h++) {
      const float th = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lt[h & 3]), 16 * (h >> 2)));
      l_run[h] = __builtin_fmaf(l_run[h], alpha[h], th);
      m_run[h] = m_new[h];
      acc[h][0] *= alpha[h];
      acc[h][1] *= alpha[h];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    // P V: lane -> dims 2 lane, 2 lane + 1, over all 16 positions of the
    // tile (a position past the chunk's last has p = 0 and a V row of zeros
    // from the buffer range, so it adds nothing)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 pa = *reinterpret_cast<const float4*>(pw + i * GMAX);
      float pb[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (GMAX == 8) {
        const float4 q2 = *reinterpret_cast<const float4*>(pw + i * GMAX + 4);
        pb[0] = q2.x, pb[1] = q2.y, pb[2] = q2.z, pb[3] = q2.w;
      }
      const uint32_t w = static_cast<uint32_t>(vc[i]);
      const float v0 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu)));
      const float v1 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
      const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb[0], pb[1], pb[2], pb[3]};
#pragma unroll
      for (int h = 0; h < GMAX; h++) {
        acc[h][0] = __builtin_fmaf(pv[h], v0, acc[h][0]);
        acc[h][1] = __builtin_fmaf(pv[h], v1, acc[h][1]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    if (more) {
#pragma unroll
      for (int ks = 0; ks < 4; ks++) kc[ks] = kn_[ks];
#pragma unroll
      for (int i = 0; i < 16; i++) vc[i] = vn_[i];
    }
  }

  // merge the four waves (fixed order); a wave without positions holds m = -inf
  if (lane < GMAX) {
    float mv = m_run[0], lv = l_run[0];
#pragma unroll
    for (int h = 1; h < GMAX; h++)
      if (lane == h) mv = m_run[h], lv = l_run[h];
    mw[wave * GMAX + lane] = mv;
    lw[wave * GMAX + lane] = lv;
  }
#pragma unroll
  for (int h = 0; h < GMAX; h++)
    *reinterpret_cast<float2*>(aw + (wave * GMAX + h) * D + 2 * lane) = make_float2(acc[h][0], acc[h][1]);
  __syncthreads();
  for (int e = t; e < G * (D / 2); e += kAttnThreads) {
    const int h = e / (D / 2), dp = e % (D / 2);
    float M = mw[h];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, mw[w * GMAX + h]);
    float L = 0.f, A0 = 0.f, A1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float ew = expf(mw[w * GMAX + h] - M);  // 0 for a wave without positions
      const float2 a = *reinterpret_cast<const float2*>(aw + (w * GMAX + h) * D + 2 * dp);
      L = __builtin_fmaf(lw[w * GMAX + h], ew, L);
      A0 = __builtin_fmaf(a.x, ew, A0);
      A1 = __builtin_fmaf(a.y, ew, A1);
    }
    float* o = part + (static_cast<size_t>(kvh * G + h) * n_chunks + c) * (D + 2);
    o[2 + 2 * dp] = A0;
    o[3 + 2 * dp] = A1;
    if (dp == 0) {
      o[0] = M;
      o[1] = L;
    }
  }
}

template <int GMAX>
size_t partial_mfma_lds() {
  return 4u * (GMAX * 128 + 128 + 4 * 16 * GMAX + 2 * 4 * GMAX + 4 * GMAX * 128);
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const float* __restrict__ qkv, _Float16* __restrict__ k_cache, _Float16* __restrict__ v_cache,
    const float* __restrict__ inv_freq, float* __restrict__ part, int pos, int n_heads, int n_kv_heads,
    int chunk, int n_chunks, float scale) {
  constexpr int RS = D / 2 + 1;  // LDS row stride of K and V tiles in dwords (one pad dword)
  extern __shared__ __align__(16) float sm[];
  const int G = n_heads / n_kv_heads;
  const int kvh = blockIdx.x;
  const int c = blockIdx.y;
  const int p0 = c * chunk;
  const int np = min(chunk, pos + 1 - p0);  // positions of this chunk (>= 1)
  const int kv_dim = n_kv_heads * D;
  float* qs = sm;                                  // [G][D]
  uint32_t* ks = reinterpret_cast<uint32_t*>(qs + G * D);   // [chunk][RS] half2
  uint32_t* vs = ks + chunk * RS;                  // [chunk][RS] half2
  float* sc = reinterpret_cast<float*>(vs + chunk * RS);    // [G][chunk]
  const int t = threadIdx.x;
  const float fpos = static_cast<float>(pos);

  // K / V rows of positions [p0, p0 + np) except pos, f16 pairs, as 16-byte
  // pieces, kBatch per thread: every load of a batch is issued before the
  // first LDS store (a load-store loop would wait out the memory latency each
  // time), and the first batch is in flight while q is rotated
  const bool own = pos >= p0 && pos < p0 + chunk;
  const int nrow = own ? np - 1 : np;
  constexpr int kBatch = 8;
  uint4 kk[kBatch], vv[kBatch];
  auto kv_load = [&](int e0) {
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const int e = e0 + b * kAttnThreads + t;
      if (e < nrow * (D / 8)) {
        const int r = e / (D / 8), j = e % (D / 8);
        const size_t off = (static_cast<size_t>(p0 + r) * n_kv_heads + kvh) * D + 8 * j;
        kk[b] = *reinterpret_cast<const uint4*>(k_cache + off);
        vv[b] = *reinterpret_cast<const uint4*>(v_cache + off);
      }
    }
  };
  auto kv_store = [&](int e0) {
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const int e = e0 + b * kAttnThreads + t;
      if (e < nrow * (D / 8)) {
        const int r = e / (D / 8), j = e % (D / 8);
        uint32_t* kd = ks + r * RS + 4 * j;
        uint32_t* vd = vs + r * RS + 4 * j;
        kd[0] = kk[b].x, kd[1] = kk[b].y, kd[2] = kk[b].z, kd[3] = kk[b].w;
        vd[0] = vv[b].x, vd[1] = vv[b].y, vd[2] = vv[b].z, vd[3] = vv[b].w;
      }
    }
  };
  // q heads of this group, rotated: thread -> (head, pair i), at most
  // 8 * D / 2 / 256 pairs per thread.  Their loads go out before the K / V
  // loads (loads complete in order, so waiting for q then leaves K / V in flight).
  constexpr int QI = 8 * D / 2 / kAttnThreads;
  float qx1[QI], qx2[QI], qf[QI];
#pragma unroll
  for (int u = 0; u < QI; u++) {
    const int e = t + u * kAttnThreads;
    if (e < G * D / 2) {
      const int g = e / (D / 2), i = e % (D / 2);
      const float* q = qkv + (kvh * G + g) * D;
      qx1[u] = q[i];
      qx2[u] = q[i + D / 2];
      qf[u] = inv_freq[i];
    }
  }
  kv_load(0);
#pragma unroll
  for (int u = 0; u < QI; u++) {
    const int e = t + u * kAttnThreads;
    if (e < G * D / 2) {
      const int g = e / (D / 2), i = e % (D / 2);
      float sn, cs;
      sincosf(fpos * qf[u], &sn, &cs);
      qs[g * D + i] = qx1[u] * cs - qx2[u] * sn;
      qs[g * D + i + D / 2] = qx1[u] * sn + qx2[u] * cs;
    }
  }
  kv_store(0);
  for (int e0 = kBatch * kAttnThreads; e0 < nrow * (D / 8); e0 += kBatch * kAttnThreads) {
    kv_load(e0);
    kv_store(e0);
  }
  if (own) {
    // the new token: rotate k, round k and v to f16, store them in the cache
    // and in the tile row of pos
    const float* kn = qkv + n_heads * D + kvh * D;
    const float* vn = qkv + n_heads * D + kv_dim + kvh * D;
    const int r = pos - p0;
    _Float16* kt = reinterpret_cast<_Float16*>(ks + r * RS);
    _Float16* vt = reinterpret_cast<_Float16*>(vs + r * RS);
    const size_t off = (static_cast<size_t>(pos) * n_kv_heads + kvh) * D;
    for (int i = t; i < D / 2; i += kAttnThreads) {
      const float ang = fpos * inv_freq[i];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      const float x1 = kn[i], x2 = kn[i + D / 2];
      const _Float16 a = static_cast<_Float16>(x1 * cs - x2 * sn);
      const _Float16 b = static_cast<_Float16>(x1 * sn + x2 * cs);
      kt[i] = a;
      kt[i + D / 2] = b;
      k_cache[off + i] = a;
      k_cache[off + i + D / 2] = b;
    }
    for (int d = t; d < D; d += kAttnThreads) {
      const _Float16 v = static_cast<_Float16>(vn[d]);
      vt[d] = v;
      v_cache[off + d] = v;
    }
  }
  __syncthreads();

  // scores: thread -> position p and a pair of heads, so each K row is read
  // once per pair (q comes from LDS as a broadcast: one address per wave)
  for (int e = t; e < ((G + 1) / 2) * chunk; e += kAttnThreads) {
    const int g0 = 2 * (e / chunk), p = e % chunk;
    const bool two = g0 + 1 < G;
    float s0 = -INFINITY, s1 = -INFINITY;
    if (p < np) {
      const uint32_t* kr = ks + p * RS;
      const float* q0 = qs + g0 * D;
      const float* q1 = qs + (two ? g0 + 1 : g0) * D;
      float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll 8
      for (int j = 0; j < D / 2; j++) {
        const uint32_t w = kr[j];
        const float k0 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu)));
        const float k1 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
        a0 = __builtin_fmaf(q0[2 * j], k0, a0);
        a1 = __builtin_fmaf(q0[2 * j + 1], k1, a1);
        b0 = __builtin_fmaf(q1[2 * j], k0, b0);
        b1 = __builtin_fmaf(q1[2 * j + 1], k1, b1);
      }
      s0 = (a0 + a1) * scale;
      s1 = (b0 + b1) * scale;
    }
    sc[g0 * chunk + p] = s0;
    if (two) sc[(g0 + 1) * chunk + p] = s1;
  }
  __syncthreads();

  // per head: max and sum of exp over the chunk (one wave per head at a time)
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;  // wave scalar
  float* ml = reinterpret_cast<float*>(sc + G * chunk);  // [G][2]
  for (int g = wave; g < G; g += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int p = lane; p < chunk; p += 64) m = fmaxf(m, sc[g * chunk + p]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float l = 0.f;
    for (int p = lane; p < chunk; p += 64) {
      const float ev = p < np ? expf(sc[g * chunk + p] - m) : 0.f;
      sc[g * chunk + p] = ev;
      l += ev;
    }
    l = whd::wave_sum(l);
    if (lane == 0) {
      ml[2 * g] = m;
      ml[2 * g + 1] = l;
    }
  }
  __syncthreads();

  // acc[g][d] = sum_p e[g][p] v[p][d]: thread -> (head, pair of dims), V read
  // as one dword per position (consecutive lanes, consecutive dwords)
  for (int e = t; e < G * (D / 2); e += kAttnThreads) {
    const int g = e / (D / 2), dp = e % (D / 2);
    const float* ev = sc + g * chunk;
    const uint32_t* vcol = vs + dp;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
    for (int p = 0; p < np; p++) {
      const uint32_t w = vcol[p * RS];
      const float e_p = ev[p];
      a0 = __builtin_fmaf(e_p, static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu))), a0);
      a1 = __builtin_fmaf(e_p, static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16))), a1);
    }
    float* o = part + (static_cast<size_t>(kvh * G + g) * n_chunks + c) * (D + 2);
    o[2 + 2 * dp] = a0;
    o[3 + 2 * dp] = a1;
    if (dp == 0) {
      o[0] = ml[2 * g];
      o[1] = ml[2 * g + 1];
    }
  }
}

// out[h][d] = sum_c acc_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M}, M = max_c m_c.
// A workgroup covers 64 dims of one head.  Every wave loads (m, l) of chunks
// lane, lane + 64, ... and this wave's 16 accumulators of the first 64 chunks
// (chunks 4 i + wave, i < 16: one 256-byte row per load) in one burst, forms
// M with a wave maximum, one weight e^{m_c - M} per lane and L with a wave sum
// (fixed order), then sums w_c acc_c[d] over its chunks with the weights read
// across lanes; contexts of more than 64 chunks repeat the accumulation per 64.
// The four waves' sums add in fixed order through LDS.  A chunk whose m is
// -inf gets weight 0; NaN anywhere makes the head NaN, as a softmax over the
// positions does.
constexpr int kCombDims = 64, kCombPer = 16;
__device__ __forceinline__ float at_rl(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Workgroup j -> (head h, 64-dim slice hf).  Workgroups go to the 8 XCDs in
// turn (linear index mod 8), so with a multiple of 8 KV heads every partial
// workgroup of KV head kvh ran on XCD kvh mod 8; the heads of kvh are then
// combined on that XCD, whose L2 holds their partials.  Placement affects
// speed only.
template <int D>
__device__ __forceinline__ void at_combine_slot(int j, int n_kv_heads, int G, int& h, int& hf) {
  constexpr int H = D / kCombDims;
  if (n_kv_heads % 8 == 0) {
    const int x = j & 7, r = j >> 3, per = G * H;
    h = (x + 8 * (r / per)) * G + (r % per) / H;
    hf = r % H;
  } else {
    h = j / H;
    hf = j % H;
  }
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                    float* __restrict__ out, int n_chunks,
                                                                    int n_kv_heads, int G) {
  __shared__ float sacc[kAttnThreads / 64][kCombDims];
  int h, hf;
  at_combine_slot<D>(static_cast<int>(blockIdx.x), n_kv_heads, G, h, hf);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int d = hf * kCombDims + lane;
  constexpr int kStride = (D + 2) * 4;  // bytes per chunk record (m, l, acc[D])
  const at_i4 rs = at_rsrc(part + static_cast<size_t>(h) * n_chunks * (D + 2),
                           static_cast<uint32_t>(n_chunks) * kStride);
  // first 64 chunks: (m, l) of chunk `lane`, then acc[d] of this wave's chunks
  // (offsets past the head's records read 0)
  const float m0 = __builtin_bit_cast(float, at_buffer_load_x1(rs, lane * kStride, 0, 0));
  const float l0 = __builtin_bit_cast(float, at_buffer_load_x1(rs, lane * kStride + 4, 0, 0));
  float av[kCombPer];
#pragma unroll
  for (int i = 0; i < kCombPer; i++)
    av[i] = __builtin_bit_cast(float, at_buffer_load_x1(rs, (4 * i + wave) * kStride + 8 + 4 * d, 0, 0));
  float mx = lane < n_chunks ? m0 : -INFINITY;
  for (int c = lane + 64; c < n_chunks; c += 64)
    mx = fmaxf(mx, __builtin_bit_cast(float, at_buffer_load_x1(rs, c * kStride, 0, 0)));
  mx = at_row_max(mx);
  const float M = fmaxf(fmaxf(at_rl(mx, 0), at_rl(mx, 16)),
                        fmaxf(at_rl(mx, 32), at_rl(mx, 48)));
  float w = lane < n_chunks ? expf(m0 - M) : 0.f;
  float lp = w * l0;
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < kCombPer; i++) a = __builtin_fmaf(at_rl(w, 4 * i + wave), av[i], a);
  for (int c0 = 64; c0 < n_chunks; c0 += 64) {
    const int c = c0 + lane;
    const float mc = __builtin_bit_cast(float, at_buffer_load_x1(rs, c * kStride, 0, 0));
    const float lc = __builtin_bit_cast(float, at_buffer_load_x1(rs, c * kStride + 4, 0, 0));
#pragma unroll
    for (int i = 0; i < kCombPer; i++)
      av[i] = __builtin_bit_cast(float, at_buffer_load_x1(rs, (c0 + 4 * i + wave) * kStride + 8 + 4 * d, 0, 0));
    w = c < n_chunks ? expf(mc - M) : 0.f;
    lp = __builtin_fmaf(w, lc, lp);
#pragma unroll
    for (int i = 0; i < kCombPer; i++) a = __builtin_fmaf(at_rl(w, 4 * i + wave), av[i], a);
  }
  lp = at_row_sum(lp);
  const float L = (at_rl(lp, 0) + at_rl(lp, 16)) +
                  (at_rl(lp, 32) + at_rl(lp, 48));
  sacc[wave][lane] = a;
  __syncthreads();
  if (wave == 0) out[h * D + d] = ((sacc[0][lane] + sacc[1][lane]) + (sacc[2][lane] + sacc[3][lane])) / L;
}

// Positions per workgroup: enough chunks for about two workgroups per CU,
// between 64 and 256 positions (a multiple of 64).
int attn_chunk(size_t ctx, size_t n_kv_heads) {
  const size_t target = 2 * static_cast<size_t>(wh::cu_count());
  size_t per_head = (target + n_kv_heads - 1) / n_kv_heads;
  if (per_head < 1) per_head = 1;
  size_t c = (ctx + per_head - 1) / per_head;
  c = (c + 63) / 64 * 64;
  if (c < 64) c = 64;
  if (c > 256) c = 256;
  return static_cast<int>(c);
}

template <int D>
size_t partial_lds(int G, int chunk) {
  return 4u * (static_cast<size_t>(G) * D + 2u * chunk * (D / 2 + 1) + static_cast<size_t>(G) * chunk + 2 * G);
}

}  // namespace

namespace wh {

// Partials of every chunk: a chunk is at least 64 positions, so a context of
// up to max_ctx positions has at most ceil(max_ctx / 64) chunks.
size_t attention_workspace_bytes(size_t n_heads, size_t head_dim, size_t max_ctx, size_t /*n_kv_heads*/) {
  const size_t n_chunks = (max_ctx + 63) / 64;
  return n_heads * (n_chunks ? n_chunks : 1) * (head_dim + 2) * sizeof(float);
}

bool attention_shape_ok(size_t n_heads, size_t n_kv_heads, size_t head_dim) {
  return (head_dim == 64 || head_dim == 128) && n_kv_heads > 0 && n_heads % n_kv_heads == 0 &&
         n_heads / n_kv_heads <= 8 && n_heads <= 1024;
}

int launch_attention_decode(const float* qkv, void* k_cache, void* v_cache, size_t pos, size_t n_heads,
                            size_t n_kv_heads, size_t head_dim, const float* inv_freq, float* out, void* ws,
                            hipStream_t s) {
  const int chunk = attn_chunk(pos + 1, n_kv_heads);
  const int n_chunks = static_cast<int>((pos + 1 + chunk - 1) / chunk);
  const int G = static_cast<int>(n_heads / n_kv_heads);
  float* part = static_cast<float*>(ws);
  const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const dim3 cgrid(static_cast<unsigned>(n_heads * (head_dim / kCombDims)));
  dim3 grid(static_cast<unsigned>(n_kv_heads), static_cast<unsigned>(n_chunks));
  if (head_dim == 128) {
    if (G <= 4) {
      attn_partial_mfma_kernel<4><<<grid, kAttnThreads, partial_mfma_lds<4>(), s>>>(
          qkv, static_cast<_Float16*>(k_cache), static_cast<_Float16*>(v_cache), inv_freq, part,
          static_cast<int>(pos), static_cast<int>(n_heads), static_cast<int>(n_kv_heads), chunk, n_chunks, scale);
    } else {
      attn_partial_mfma_kernel<8><<<grid, kAttnThreads, partial_mfma_lds<8>(), s>>>(
          qkv, static_cast<_Float16*>(k_cache), static_cast<_Float16*>(v_cache), inv_freq, part,
          static_cast<int>(pos), static_cast<int>(n_heads), static_cast<int>(n_kv_heads), chunk, n_chunks, scale);
    }
    WH_LAUNCH_CHECK("attention kernel launch");
    attn_combine_kernel<128><<<cgrid, kAttnThreads, 0, s>>>(part, out, n_chunks, static_cast<int>(n_kv_heads), G);
  } else {
    const size_t lds = partial_lds<64>(G, chunk);
    WH_ENSURE_LDS(lds, &attn_partial_kernel<64>);
    attn_partial_kernel<64><<<grid, kAttnThreads, lds, s>>>(
        qkv, static_cast<_Float16*>(k_cache), static_cast<_Float16*>(v_cache), inv_freq, part,
        static_cast<int>(pos), static_cast<int>(n_heads), static_cast<int>(n_kv_heads), chunk, n_chunks, scale);
    WH_LAUNCH_CHECK("attention kernel launch");
    attn_combine_kernel<64><<<cgrid, kAttnThreads, 0, s>>>(part, out, n_chunks, static_cast<int>(n_kv_heads), G);
  }
  WH_LAUNCH_CHECK("attention combine launch");
  return WH_OK;
}

}  // namespace wh
