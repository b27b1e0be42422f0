// gemv_mt.hpp -- the several-token matrix-core GEMV kernels (2..16 tokens),
// included by one translation unit per block type (gemv_mt_<type>.hip), which
// instantiates them for that type only.
#pragma once
#include "gemv_mfma_dev.hpp"

namespace {

// Q6_K B operand of lane group g for K-step j of the block at rowp (LDS),
// whose bytes start mis (0 or 2) bytes past a dword boundary: element 8 g + t
// of the step as the signed byte q - 32 (quantization of dequantize.rs:460-536:
// the nibble of ql and two bits of qh).
__device__ __forceinline__ long mt_q6k_quants(const uint8_t* rowp, int mis, int j, int g) {
  uint32_t l0, l1;
  mg_lds_u64(rowp + 16 * j + 8 * (g & 1), mis, l0, l1);
  const uint8_t* hp = rowp + 128 + 8 * j + 2 * g;
  uint32_t w = *reinterpret_cast<const uint16_t*>(hp);  // hp is even
  if (j >= 4) {
    // 8 j + 2 g + 2 == 64 only for j = 7, g = 3 (element 255)
    if (j < 7 || g < 3) w |= static_cast<uint32_t>(hp[2]) << 16;
    w >>= 2;
    l0 >>= 4;
    l1 >>= 4;
  }
  // two-bit fields t = 0..3 of v to bits 0..1 of byte t, then the high nibble
  // of q - 32 (two's complement) looked up: 0 -> 0xE, 1 -> 0xF, 2 -> 0x0, 3 -> 0x1
  auto hi = [](uint32_t v) -> uint32_t {
    const uint32_t sel = (v | (v << 6) | (v << 12) | (v << 18)) & 0x03030303u;
    return __builtin_amdgcn_perm(0u, 0x1000F0E0u, sel);
  };
  const uint32_t b0 = (l0 & 0x0F0F0F0Fu) | hi(w & 0xFFu);
  const uint32_t b1 = (l1 & 0x0F0F0F0Fu) | hi((w >> 8) & 0xFFu);
  return static_cast<long>(b0) | (static_cast<long>(b1) << 32);
}

template <int TYPE, int NSEG, int NL, int MODE, int TG, int MS>
__device__ __forceinline__ void gemv_mt_body(const MgArgs& a, int bid) {
  static_assert(mt_type_ok<TYPE>(), "several-token GEMV: Q4_0, Q4_1, Q8_0, Q4_K, Q6_K");
  static_assert(TG * NSEG <= 4, "A operands of every segment in registers");
  static_assert(MS == 4 || (MS == 2 && TG == 1 && TYPE != WH_TYPE_Q6_K), "two-token layout: one group");
  constexpr bool Q41 = TYPE == WH_TYPE_Q4_1;
  constexpr bool Q4K = TYPE == WH_TYPE_Q4_K;
  constexpr bool Q6K = TYPE == WH_TYPE_Q6_K;
  constexpr bool XSUM = mt_xsum(TYPE);
  constexpr int PB = Q4K ? 32 : MgFmt<TYPE>::PB;  // bytes of two blocks (Q4_K: two groups' quants)
  constexpr int BB = PB / 2;                       // bytes of one block
  constexpr bool FFN = (MODE & kMgFfn) != 0;
  constexpr bool NORM = (MODE & kMgNorm) != 0;
  constexpr int CB = mg_chunk_bytes(TYPE);
  // Segments that do not start on a 16-byte boundary (Q6_K's 210-byte
  // chunks) are loaded from the boundary below, `lead` bytes early, into an
  // LDS row whose data then starts `lead` bytes in.
  constexpr uint32_t kLeadRoom = (CB & 15) ? 16u : 0u;
  constexpr int MT = MS * TG;  // token slots
  constexpr int STG = mt_stage_bytes(TYPE, MT);
  constexpr int XSB = mt_xsum_bytes(TYPE, NSEG, MT);
  constexpr float kScale = TYPE == WH_TYPE_Q4_0 ? 0.0625f : 1.0f;
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int S = a.seg_pairs;
  const int M = a.m;
  const uint32_t seg_bytes = static_cast<uint32_t>(S >> 2) * CB;
  const uint32_t rstr = mg_row_stride(seg_bytes, kLeadRoom + 16u);
  const uint32_t slot_bytes = 16 * rstr;
  const size_t row_bytes = static_cast<size_t>(a.ppr >> 2) * CB;
  const int K = a.ppr * 64;
  const int R = a.rows_per_wg;
  uint8_t* ring = lds;
  uint8_t* stage = lds + 2 * slot_bytes + wave * (STG + XSB);
  float* xsum = reinterpret_cast<float*>(stage + STG);  // [NSEG][MT][8] this wave's block sums of x
  float* part = reinterpret_cast<float*>(lds + 2 * slot_bytes + kMgWaves * (STG + XSB));  // [2][16 waves][MT][16]
  float* misc = part + 2 * kMgWaves * MT * 16;  // [16 waves][MT] norm sums, later [MT][16] gate values
  float* rms_lds = misc + kMgWaves * MT;        // [MT] RMSNorm scale of each token
  float* rows_lds = rms_lds + MT;               // [MT][R] the workgroup's output rows

  const int r0 = bid * R;
  const int r1 = min(a.n_out, r0 + R);
  const int G = (r1 - r0 + 15) >> 4;
  const int GT = FFN ? 2 * G : G;
  const bool owns = wave < (S >> 2);

  auto row_src = [&](int q, const uint8_t** base) -> bool {
    const int gi = FFN ? (q >> 1) : q;
    const int row = r0 + 16 * gi + wave;
    if (q >= GT || row >= r1) return false;
    *base = (FFN && (q & 1) ? a.W1 : a.W0) + static_cast<size_t>(row) * row_bytes;
    return true;
  };
  mg_v4i buf[NL];
  auto load = [&](int q, int seg) {
    const uint8_t* base = a.W0;
    const bool ok = row_src(q, &base);
    const uint32_t lead = (static_cast<uint32_t>(seg) * seg_bytes) & (kLeadRoom ? 15u : 0u);
    const mg_v4i rs = mg_rsrc(base + static_cast<size_t>(seg) * seg_bytes - lead, ok ? seg_bytes + lead : 0u);
#pragma unroll
    for (int i = 0; i < NL; i++) buf[i] = mg_buffer_load_x4(rs, 16 * (64 * i + lane), 0, kMgNt);
  };
  auto xload = [&](int t, int seg) -> float4 {
    if (t >= M || !owns) return make_float4(0.f, 0.f, 0.f, 0.f);
    return *reinterpret_cast<const float4*>(a.x + static_cast<size_t>(t) * K + (seg * S + 4 * wave) * 64 + 4 * lane);
  };
  // The same as a buffer load whose range is empty for a token slot past M or
  // a wave without a chunk (zeros, no memory access): no branch around the
  // load, which would make the compiler wait for every load in flight where
  // the branches join.
  auto xload_nb = [&](int t, int seg) -> float4 {
    const bool ok = t < M && owns;
    const mg_v4i rs = mg_rsrc(a.x + (ok ? static_cast<size_t>(t) * K + (seg * S + 4 * wave) * 64 : static_cast<size_t>(0)),
                              ok ? 1024u : 0u);
    return __builtin_bit_cast(float4, mg_buffer_load_x4(rs, 16 * lane, 0, 0));
  };

  // XPRE (up to 8 chunks per wave, 4 with the longest rows, whose four loads
  // per step leave fewer registers): every chunk's activations are requested
  // first and kept in registers, then the first weights, so that neither the
  // RMSNorm reduction nor the limbs wait for the weights (loads complete in
  // order); with more chunks the activations are read where they are used and
  // the weights are requested after the RMSNorm's barrier.
  constexpr bool XPRE = MT * NSEG * (NL >= 4 ? 2 : 1) <= 8;
  float4 xr[XPRE ? NSEG : 1][XPRE ? MT : 1];
  auto xget = [&](int t, int seg) -> float4 {
    if constexpr (XPRE) return xr[seg][t];
    else return xload(t, seg);
  };
  float4 gv[NSEG];
  if constexpr (NORM) {
#pragma unroll
    for (int seg = 0; seg < NSEG; seg++)
      gv[seg] = owns ? *reinterpret_cast<const float4*>(a.gamma + (seg * S + 4 * wave) * 64 + 4 * lane)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if constexpr (XPRE) {
#pragma unroll
    for (int seg = 0; seg < (XPRE ? NSEG : 0); seg++)
#pragma unroll
      for (int t = 0; t < (XPRE ? MT : 0); t++) xr[seg][t] = xload_nb(t, seg);
    load(0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- RMSNorm (tensor_utils.rs:446-480) as (W (x * gamma)) / rms per token:
  // each wave's share of every token's sum x^2 goes to LDS here; wave 0 forms
  // the tokens' rms after the first step's barrier, and a token's rows are
  // divided by its rms where they are finished (no barrier in the prologue).
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < MT; t++) {
      float ss = 0.f;
#pragma unroll
      for (int seg = 0; seg < NSEG; seg++) {
        const float4 v = xget(t, seg);
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
      }
      ss = whd::wave_sum(ss);
      if (lane == 0) misc[wave * MT + t] = ss;
    }
  }
  for (int i = threadIdx.x; i < MT * R; i += kMgWaves * 64) rows_lds[i] = 0.f;
  if constexpr (!XPRE) load(0, 0);

  // ---- limbs of every (segment, token) chunk -> A operands in registers
  // two-token layout: a lane's rows belong to the even blocks (n < 8) or the
  // odd ones, so one register per block pair holds its nonzero operand
  constexpr int NA = MS == 4 ? 8 : 4;
  long xa[NSEG][TG][NA];
  int ex_u[NSEG][MT];       // chunk exponent (wave-uniform)
  uint32_t exact_u[NSEG];   // bit t: token t's chunk holds inf / NaN (computed per element)
#pragma unroll
  for (int seg = 0; seg < NSEG; seg++)
#pragma unroll
    for (int tg = 0; tg < TG; tg++)
#pragma unroll
      for (int b = 0; b < NA; b++) xa[seg][tg][b] = 0;
  auto xnorm = [&](int t, int seg) -> float4 {
    float4 v = xget(t, seg);
    if constexpr (NORM) {
      v.x *= gv[seg].x;
      v.y *= gv[seg].y;
      v.z *= gv[seg].z;
      v.w *= gv[seg].w;
    }
    return v;
  };
#pragma unroll
  for (int seg = 0; seg < NSEG; seg++) {
    exact_u[seg] = 0u;
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const float4 v = xnorm(t, seg);
      const float xv[4] = {v.x, v.y, v.z, v.w};
      // the largest |x| as the maximum of the bit patterns of |x| (inf / NaN above every finite value)
      uint32_t um = 0u;
#pragma unroll
      for (int i = 0; i < 4; i++) um = max(um, __builtin_bit_cast(uint32_t, xv[i]) & 0x7FFFFFFFu);
      um = mg_wave_max_u32(um);
      const bool exact = um >= 0x7F800000u;
      int e = 0;
      if (um != 0u && !exact) {
        int ee;
        frexpf(__builtin_bit_cast(float, um), &ee);
        e = 30 - ee;
      }
      ex_u[seg][t] = __builtin_amdgcn_readfirstlane(e);
      if (exact) exact_u[seg] |= 1u << t;
      uint32_t z[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int xi = exact ? 0 : static_cast<int>(rintf(ldexpf(xv[i], e)));
        z[i] = static_cast<uint32_t>(xi + 0x808080) ^ 0x808080u;
      }
      const uint32_t pa = __builtin_amdgcn_perm(z[1], z[0], 0x06020703u);
      const uint32_t pb2 = __builtin_amdgcn_perm(z[1], z[0], 0x04000501u);
      const uint32_t pc = __builtin_amdgcn_perm(z[3], z[2], 0x06020703u);
      const uint32_t pd = __builtin_amdgcn_perm(z[3], z[2], 0x04000501u);
      const uint32_t row[4] = {__builtin_amdgcn_perm(pc, pa, 0x05040100u), __builtin_amdgcn_perm(pc, pa, 0x07060302u),
                               __builtin_amdgcn_perm(pd, pb2, 0x05040100u), __builtin_amdgcn_perm(pd, pb2, 0x07060302u)};
      // two-token layout: token t's limbs in the t-th half of the stage
      int8_t* pw = reinterpret_cast<int8_t*>(stage) + (MS == 2 ? t * 8 * kMgLimbBytes : 0) +
                   (lane >> 3) * kMgLimbBytes + mg_slot_offset<TYPE>(4 * (lane & 7));
      if constexpr (Q4K) {
        // elements 0..3 of the lane go to slots +0, +4, +1, +5
#pragma unroll
        for (int r = 0; r < 4; r++) {
          *reinterpret_cast<uint16_t*>(pw + 32 * r) = static_cast<uint16_t>(__builtin_amdgcn_perm(0u, row[r], 0x0c0c0200u));
          *reinterpret_cast<uint16_t*>(pw + 32 * r + 4) = static_cast<uint16_t>(__builtin_amdgcn_perm(0u, row[r], 0x0c0c0301u));
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) *reinterpret_cast<uint32_t*>(pw + 32 * r) = row[r];
      }
      if constexpr (MS == 4) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        // this token's rows of the A operands: rows 4 (t & 3) .. + 3 of token group t / 4
        const int8_t* xs = reinterpret_cast<const int8_t*>(stage) + 32 * (n & 3) + 8 * g;
        if ((n >> 2) == (t & 3)) {
          long v8[8];
#pragma unroll
          for (int b = 0; b < 8; b++) v8[b] = *reinterpret_cast<const long*>(xs + b * kMgLimbBytes);
#pragma unroll
          for (int b = 0; b < 8; b++) xa[seg][t >> 2][b] = v8[b];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
      }
    }
    if constexpr (MS == 2) {
      // two-token layout: rows 8 (b & 1) + 4 t .. + 3 hold token t's limbs of
      // block b, so a lane's rows belong to token (n >> 2) & 1 and to the
      // blocks of parity n >> 3: four reads from that token's half, no branch
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      const int8_t* xs = reinterpret_cast<const int8_t*>(stage) + ((n >> 2) & 1) * 8 * kMgLimbBytes +
                         (n >> 3) * kMgLimbBytes + 32 * (n & 3) + 8 * g;
#pragma unroll
      for (int j = 0; j < 4; j++) xa[seg][0][j] = *reinterpret_cast<const long*>(xs + 2 * j * kMgLimbBytes);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
    }
    if constexpr (XSUM) {
      // block sums of x in units of 2^-e: the limb sums of each block, from
      // MFMAs against a B operand of ones (the same for every weight row);
      // lane group g's accumulator holds those of token 4 tg + g of the block
      // (two-token layout: token g & 1 of block 2j + (g >> 1))
      constexpr long kOnes = static_cast<long>(0x0101010101010101ull);
      auto limbsum = [](const mg_v4i& v) {
        return __builtin_fmaf(static_cast<float>(v[0]), 16777216.f,
                              __builtin_fmaf(static_cast<float>(v[1]), 65536.f,
                                             __builtin_fmaf(static_cast<float>(v[2]), 256.f, static_cast<float>(v[3]))));
      };
#pragma unroll
      for (int tg = 0; tg < TG; tg++) {
#pragma unroll
        for (int b = 0; b < NA; b++) {
          const mg_v4i v = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[seg][tg][b], kOnes, (mg_v4i){0, 0, 0, 0}, 0, 0, 0);
          if (n == 0) {
            const int t = MS == 4 ? 4 * tg + g : (g & 1);
            const int blk = MS == 4 ? b : 2 * b + (g >> 1);
            xsum[(seg * MT + t) * 8 + blk] = limbsum(v);
          }
        }
      }
    }
  }
  // exponent of the token this lane's results belong to (4 tg + g; two-token layout: g & 1)
  int ex_l[NSEG][TG];
#pragma unroll
  for (int seg = 0; seg < NSEG; seg++)
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
      if constexpr (MS == 4) {
        const int* e4 = &ex_u[seg][4 * tg];
        ex_l[seg][tg] = g == 0 ? e4[0] : g == 1 ? e4[1] : g == 2 ? e4[2] : e4[3];
      } else {
        // values, not the elements: a conditional over two lvalues selects an
        // address, and the array would live in scratch memory
        const int e0 = ex_u[seg][0], e1 = ex_u[seg][MT > 1 ? 1 : 0];
        ex_l[seg][tg] = (g & 1) ? e1 : e0;
      }
    }

  // B operands of lane group g for the two blocks (Q4_K: groups) of pair p of
  // the chunk at rowp (LDS)
  auto quants = [&](const uint8_t* rowp, int p, long& qa, long& qb) {
    auto split = [](uint32_t u) -> long {
      return static_cast<long>(u & 0x0F0F0F0Fu) | (static_cast<long>((u >> 4) & 0x0F0F0F0Fu) << 32);
    };
    if constexpr (TYPE == WH_TYPE_Q4_0) {
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp + p * PB);
      auto split8 = [](uint32_t u) -> long {
        const uint32_t v = u ^ 0x88888888u;  // nibble ^ 8: q - 8 as a signed 4-bit number
        return static_cast<long>((v << 4) & 0xF0F0F0F0u) | (static_cast<long>(v & 0xF0F0F0F0u) << 32);
      };
      qa = split8(__builtin_amdgcn_alignbit(pw[g + 1], pw[g], 16));
      qb = split8(pw[5 + g]);
    } else if constexpr (Q41) {
      // [dA|mA] [A q0..3] .. [A q12..15] [dB|mB] [B q0..3] ..
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp + p * PB);
      qa = split(pw[1 + g]);
      qb = split(pw[6 + g]);
    } else if constexpr (Q4K) {
      // quant bytes 16 j + 4 g .. + 3 of group j at byte 16 + 16 j
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp);
      qa = split(pw[4 + 8 * p + g]);
      qb = split(pw[8 + 8 * p + g]);
    } else {
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp + p * PB);
      const uint32_t w0 = pw[2 * g], w1 = pw[2 * g + 1], w2 = pw[2 * g + 2];
      qa = static_cast<long>(__builtin_amdgcn_alignbit(w1, w0, 16)) |
           (static_cast<long>(__builtin_amdgcn_alignbit(w2, w1, 16)) << 32);
      qb = static_cast<long>(pw[9 + 2 * g]) | (static_cast<long>(pw[10 + 2 * g]) << 32);
    }
  };

  // Sum of group q over the 16 waves (fixed order) for every token, then the
  // output rows (to_y: straight to y, for the last group after the loop).
  auto finish = [&](int q, bool to_y) {
    const int gi = FFN ? (q >> 1) : q;
    const int row = r0 + 16 * gi + n;
    if (MS == 2 && g >= 2) return;
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
      const int t = MS * tg + g;
      const float* pp = part + ((q & 1) * kMgWaves * MT + t) * 16 + n;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kMgWaves; w++) v += pp[w * MT * 16];
      if constexpr (NORM) v = v / rms_lds[t];
      if constexpr (FFN) {
        if ((q & 1) == 0) {
          misc[t * 16 + n] = v;  // gate, combined with up one group later
        } else if (row < r1) {
          const float gt = misc[t * 16 + n];
          const float out = (gt * (1.0f / (1.0f + expf(-gt)))) * v;
          if (!to_y) rows_lds[t * R + row - r0] = out;
          else if (t < M) a.y[static_cast<size_t>(t) * a.ldy + row] = out;
        }
      } else if (row < r1) {
        if (!to_y) rows_lds[t * R + row - r0] = v;
        else if (t < M) a.y[static_cast<size_t>(t) * a.ldy + row] = v;
      }
    }
  };

  float acc[TG];
#pragma unroll
  for (int tg = 0; tg < TG; tg++) acc[tg] = 0.f;
  for (int q = 0; q < GT; q++) {
#pragma unroll
    for (int seg = 0; seg < NSEG; seg++) {
      const int s = q * NSEG + seg;
      uint8_t* slot = ring + (s & 1) * slot_bytes;
      const uint32_t lead = (static_cast<uint32_t>(seg) * seg_bytes) & (kLeadRoom ? 15u : 0u);
      {
        // every lane stores (pieces past the segment go to the overflow room)
        uint8_t* dst = slot + wave * rstr;
        const uint32_t end16 = (seg_bytes + lead + 15u) & ~15u;
#pragma unroll
        for (int i = 0; i < NL; i++) {
          const uint32_t o = 16u * (64 * i + lane);
          *reinterpret_cast<mg_v4i*>(dst + (o < end16 ? o : end16)) = buf[i];
        }
      }
      if (seg + 1 < NSEG) load(q, seg + 1);
      else load(q + 1, 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if constexpr (NORM) {
        // every wave's shares of sum x^2 are visible (the step barrier); the
        // first finish, and the first gate value written over them, come after
        // the next barrier
        if (q == 0 && seg == 0 && wave == 0 && lane < MT) {
          float tot = 0.f;
#pragma unroll
          for (int w = 0; w < kMgWaves; w++) tot += misc[w * MT + lane];
          rms_lds[lane] = sqrtf(tot / static_cast<float>(K) + a.eps);
        }
      }
      if (seg == 0 && q > 0 && wave == ((q - 1) & (kMgWaves - 1))) finish(q - 1, false);
      if (owns) {
        const uint8_t* rowp = slot + n * rstr + lead + wave * CB;
        float sacc[TG];
#pragma unroll
        for (int tg = 0; tg < TG; tg++) sacc[tg] = 0.f;
        const mg_v4i zero = {0, 0, 0, 0};
        if constexpr (Q6K) {
          // LDS rows start 16-byte aligned, the chunk `lead + 210 wave` bytes in
          const int mis = static_cast<int>((lead + 2 * (wave & 1)) & 3u);
          uint32_t sc[4];  // the sixteen u8 scales
          mg_lds_u64(rowp + 192, mis, sc[0], sc[1]);
          mg_lds_u64(rowp + 200, mis, sc[2], sc[3]);
          const float d64 = whd::f16_bits_to_f32(static_cast<uint32_t>(rowp[208]) |
                                                 (static_cast<uint32_t>(rowp[209]) << 8)) * 0.015625f;
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const long qj = mt_q6k_quants(rowp, mis, j, g);
            // half h of the step: k-slots 16 h .. 16 h + 15, the lanes of groups 2 h, 2 h + 1
            const long q0 = g < 2 ? qj : 0, q1 = g < 2 ? 0 : qj;
            const uint32_t s2 = sc[j >> 1] >> (16 * (j & 1));
            const float da = d64 * static_cast<float>(s2 & 0xFFu);
            const float db = d64 * static_cast<float>((s2 >> 8) & 0xFFu);
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
              const mg_v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[seg][tg][j], q0, zero, 0, 0, 0);
              const mg_v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[seg][tg][j], q1, zero, 0, 0, 0);
              sacc[tg] = __builtin_fmaf(da, mg_limbs(c0), sacc[tg]);
              sacc[tg] = __builtin_fmaf(db, mg_limbs(c1), sacc[tg]);
              // each step's products are converted where they are made:
              // deferred to the end of the chunk, the results of all eight
              // steps stay live and the kernel runs out of registers
              asm volatile("" : "+v"(sacc[tg]));
            }
          }
        } else {
          float kd = 0.f;        // Q4_K: d
          uint32_t ks[3] = {};   // Q4_K: the twelve bytes of packed 6-bit scales
          if constexpr (Q4K) {
            const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp);
            ks[0] = pw[0], ks[1] = pw[1], ks[2] = pw[2];
            kd = whd::f16_bits_to_f32(pw[3] & 0xFFFFu);
          }
          // 6-bit scale j of the Q4_K block (dequantize.rs:423-431) from the packed bytes
          auto q4k_scale = [&](int j) -> uint32_t {
            const int src = (3 * j) >> 1;
            const uint32_t b0 = (ks[src >> 2] >> (8 * (src & 3))) & 0xFFu;
            if ((j & 1) == 0) return b0 & 63u;
            const uint32_t b1 = (ks[(src + 1) >> 2] >> (8 * ((src + 1) & 3))) & 0xFFu;
            return ((b0 >> 6) | ((b1 & 15u) << 2)) & 63u;
          };
#pragma unroll
          for (int p = 0; p < 4; p++) {
            long qa, qb;
            quants(rowp, p, qa, qb);
            float da, db, ma = 0.f, mb = 0.f;
            if constexpr (Q4K) {
              da = kd * static_cast<float>(q4k_scale(2 * p));
              db = kd * static_cast<float>(q4k_scale(2 * p + 1));
            } else if constexpr (Q41) {
              const uint32_t ha = *reinterpret_cast<const uint32_t*>(rowp + p * PB);
              const uint32_t hb = *reinterpret_cast<const uint32_t*>(rowp + p * PB + BB);
              da = whd::f16_bits_to_f32(ha & 0xFFFFu), ma = whd::f16_bits_to_f32(ha >> 16);
              db = whd::f16_bits_to_f32(hb & 0xFFFFu), mb = whd::f16_bits_to_f32(hb >> 16);
            } else {
              da = whd::f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(rowp + p * PB)) * kScale;
              db = whd::f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(rowp + p * PB + BB)) * kScale;
            }
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
              if constexpr (MS == 4) {
                const mg_v4i ca = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[seg][tg][2 * p], qa, zero, 0, 0, 0);
                const mg_v4i cb = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[seg][tg][2 * p + 1], qb, zero, 0, 0, 0);
                sacc[tg] = __builtin_fmaf(da, mg_limbs(ca), sacc[tg]);
                sacc[tg] = __builtin_fmaf(db, mg_limbs(cb), sacc[tg]);
                if constexpr (Q41) {
                  const float2 xs2 = *reinterpret_cast<const float2*>(xsum + (seg * MT + 4 * tg + g) * 8 + 2 * p);
                  sacc[tg] = __builtin_fmaf(ma, xs2.x, sacc[tg]);
                  sacc[tg] = __builtin_fmaf(mb, xs2.y, sacc[tg]);
                }
              } else {
                const long ae = n < 8 ? xa[seg][tg][p] : 0, ao = n < 8 ? 0 : xa[seg][tg][p];
                mg_v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ae, qa, zero, 0, 0, 0);
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ao, qb, c, 0, 0, 0);
                sacc[tg] = __builtin_fmaf((g >> 1) ? db : da, mg_limbs(c), sacc[tg]);
                if constexpr (Q41)
                  sacc[tg] = __builtin_fmaf((g >> 1) ? mb : ma, xsum[(seg * MT + (g & 1)) * 8 + 2 * p + (g >> 1)], sacc[tg]);
              }
              asm volatile("" : "+v"(sacc[tg]));
            }
          }
          if constexpr (Q4K) {
            // dmin times the sum of x over the block (the eight groups' sums)
            const float dmin = whd::f16_bits_to_f32(reinterpret_cast<const uint32_t*>(rowp)[3] >> 16);
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
              const int t = MS == 4 ? 4 * tg + g : (g & 1);
              const float4 s0 = *reinterpret_cast<const float4*>(xsum + (seg * MT + t) * 8);
              const float4 s1 = *reinterpret_cast<const float4*>(xsum + (seg * MT + t) * 8 + 4);
              // two-token layout: lane groups g and g + 2 hold the same token; one of them adds it
              const float bs = ((s0.x + s0.y) + (s0.z + s0.w)) + ((s1.x + s1.y) + (s1.z + s1.w));
              if (MS == 4 || g < 2) sacc[tg] = __builtin_fmaf(dmin, bs, sacc[tg]);
            }
          }
        }
#pragma unroll
        for (int tg = 0; tg < TG; tg++) acc[tg] += ldexpf(sacc[tg], -ex_l[seg][tg]);
        // tokens whose chunk is not finite: their limbs are zero, the lanes of
        // the token add the chunk per element (the reference's order)
        for (uint32_t em = exact_u[seg]; em != 0u; em &= em - 1u) {
          const int t = __builtin_ctz(em);
          if (g != (MS == 4 ? (t & 3) : t)) continue;
          float sx = 0.f;
#pragma unroll 1
          for (int p = 0; p < 4; p++) {
            auto xs = [&](int jj) {
              const int el = (seg * S + 4 * wave) * 64 + 64 * p + 4 * jj;
              float4 v = *reinterpret_cast<const float4*>(a.x + static_cast<size_t>(t) * K + el);
              if constexpr (NORM) {
                const float4 gm = *reinterpret_cast<const float4*>(a.gamma + el);
                v = make_float4(v.x * gm.x, v.y * gm.y, v.z * gm.z, v.w * gm.w);
              }
              return v;
            };
            if constexpr (Q4K) sx += mg_q4k_exact(rowp, p, xs);
            else if constexpr (Q6K) sx += mg_q6k_exact(rowp, p, xs);
            else sx += mg_pair_exact<TYPE>(rowp + p * PB, xs);
          }
#pragma unroll
          for (int tg = 0; tg < TG; tg++)
            if (t / MS == tg) acc[tg] += sx;
        }
      }
      if (seg == NSEG - 1) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
          if constexpr (MS == 4) {
            part[(((q & 1) * kMgWaves + wave) * MT + 4 * tg + g) * 16 + n] = acc[tg];
          } else {
            // token g & 1: the even blocks' sum (lane group g) + the odd blocks' (g + 2)
            const float v = acc[tg] + __shfl_xor(acc[tg], 32, 64);
            if (g < 2) part[(((q & 1) * kMgWaves + wave) * MT + g) * 16 + n] = v;
          }
          acc[tg] = 0.f;
        }
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // The last row group goes from the wave that finishes it straight to y;
  // every earlier group is complete in rows_lds since the barrier above.
  if (GT > 0 && wave == ((GT - 1) & (kMgWaves - 1))) finish(GT - 1, true);
  const int done_rows = min(16 * (G - 1), r1 - r0);
  for (int i = threadIdx.x; i < M * done_rows; i += kMgWaves * 64) {
    const int t = i / done_rows, r = i - t * done_rows;
    a.y[static_cast<size_t>(t) * a.ldy + r0 + r] = rows_lds[t * R + r];
  }
}

template <int TYPE, int NSEG, int NL, int MODE, int TG, int MS>
__global__ __launch_bounds__(kMgWaves * 64) void gemv_mt_kernel(const MgArgs a) {
  gemv_mt_body<TYPE, NSEG, NL, MODE, TG, MS>(a, static_cast<int>(blockIdx.x));
}


template <int TYPE, int NSEG, int NL, int MODE, int TG, int MS = 4>
int mt_launch(const MgArgs& a, int grid, size_t lds, hipStream_t s) {
  auto* fn = &gemv_mt_kernel<TYPE, NSEG, NL, MODE, TG, MS>;
  WH_ENSURE_LDS(lds, fn);
  fn<<<grid, kMgWaves * 64, lds, s>>>(a);
  WH_LAUNCH_CHECK("gemv (several tokens) kernel launch");
  return WH_OK;
}

template <int TYPE, int NL, int MODE>
int mt_dispatch_nl(const MgArgs& a, int nseg, int tg, int grid, size_t lds, hipStream_t s) {
  if constexpr (TYPE != WH_TYPE_Q6_K) {
    if (a.m == 2) {
      switch (nseg) {
        case 1: return mt_launch<TYPE, 1, NL, MODE, 1, 2>(a, grid, lds, s);
        case 2: return mt_launch<TYPE, 2, NL, MODE, 1, 2>(a, grid, lds, s);
        default: return mt_launch<TYPE, 4, NL, MODE, 1, 2>(a, grid, lds, s);
      }
    }
  }
  if (nseg == 1) {
    switch (tg) {
      case 1: return mt_launch<TYPE, 1, NL, MODE, 1>(a, grid, lds, s);
      case 2: return mt_launch<TYPE, 1, NL, MODE, 2>(a, grid, lds, s);
      case 3: return mt_launch<TYPE, 1, NL, MODE, 3>(a, grid, lds, s);
      default: return mt_launch<TYPE, 1, NL, MODE, 4>(a, grid, lds, s);
    }
  }
  if (nseg == 2) return tg == 1 ? mt_launch<TYPE, 2, NL, MODE, 1>(a, grid, lds, s) : mt_launch<TYPE, 2, NL, MODE, 2>(a, grid, lds, s);
  return mt_launch<TYPE, 4, NL, MODE, 1>(a, grid, lds, s);
}

// bytes one lane group of 64 lanes loads per row: the segment and its lead
template <int TYPE>
constexpr int mt_lead() {
  return (mg_chunk_bytes(TYPE) & 15) ? 15 : 0;
}

template <int TYPE, int MODE>
int mt_dispatch(const MgArgs& a, int nseg, int tg, int grid, size_t lds, hipStream_t s) {
  const int seg_bytes = a.seg_pairs / 4 * mg_chunk_bytes(TYPE) + mt_lead<TYPE>();
  if (nseg == 4 && seg_bytes <= 2048) {
    if constexpr (TYPE != WH_TYPE_Q6_K)
      if (a.m == 2) return mt_launch<TYPE, 4, 2, MODE, 1, 2>(a, grid, lds, s);
    return mt_launch<TYPE, 4, 2, MODE, 1>(a, grid, lds, s);
  }
  // four loads per lane only for formats whose 16-chunk segments pass 3 KB
  if constexpr (16 * mg_chunk_bytes(TYPE) + mt_lead<TYPE>() > 3072)
    if (seg_bytes > 3072) return mt_dispatch_nl<TYPE, 4, MODE>(a, nseg, tg, grid, lds, s);
  return mt_dispatch_nl<TYPE, 3, MODE>(a, nseg, tg, grid, lds, s);
}

template <int TYPE>
int mt_typed(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s) {
  return ffn ? mt_dispatch<TYPE, kMgNorm | kMgFfn>(a, nseg, tg, grid, lds, s) : mt_dispatch<TYPE, 0>(a, nseg, tg, grid, lds, s);
}


}  // namespace

// Defines wh::launch_gemv_mt_<name> for block type TYPE.
#define WH_GEMV_MT_LAUNCHER(name, TYPE)                                                                   \
  namespace wh {                                                                                          \
  int launch_gemv_mt_##name(const MgArgs& a, bool ffn, int nseg, int tg, int grid, size_t lds, hipStream_t s) { \
    return mt_typed<TYPE>(a, ffn, nseg, tg, grid, lds, s);                                                \
  }                                                                                                       \
  }
