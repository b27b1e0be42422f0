// gemv_mfma.hip -- quantized matrix-vector product y = W x on the int8 matrix
// cores of gfx950 (v_mfma_i32_16x16x32_i8).
//
// Reference: simd::quantized_matvec (crates/woolly-tensor/src/quantization.rs:869-909)
// with its scalar kernels quantized_matvec_q4_0_scalar / _q8_0_scalar
// (quantization.rs:1100-1163); Q4_1 as dequantize_q4_1 (:490-511) composed with
// the f32 dot.  The fused variants add the RMSNorm prologue (tensor_utils.rs:446-480),
// the residual adds of process_layer (lazy_transformer.rs:98-258) and the SwiGLU
// epilogue h = silu(gate . x) * (up . x) (tensor_utils.rs:512-532).
//
// Arithmetic.  Every weight of a block is an exact small integer q (Q4_0 and
// Q4_1: the nibble 0..15, Q8_0: the int8 quant) times the block scale d.  The
// activations of one 256-element chunk are written as
//     x = 2^-e * (2^24 l0 + 2^16 l1 + 2^8 l2 + l3),   |l0| <= 65, l1..l3 int8,
// with e chosen per chunk so that max|x| * 2^e lies in [2^29, 2^30): every
// element within 2^-6 of the chunk's largest is represented exactly (its 24
// significant bits fit), the others to 2^-31 of the chunk maximum.  One MFMA
// per block multiplies the four limbs (rows 0..3 of the A operand) with the
// block's quants (the B operand, one weight row per column): the int32
// accumulation is exact.  Four consecutive blocks share one accumulator, their
// limbs placed in rows 4j..4j+3, so lane group j of the result holds block j's
// four limb sums and one FMA per lane applies the four block scales:
// d * (2^24 C0 + 2^16 C1 + 2^8 C2 + C3), the Q4_0 offset -8 entering as
// -8 * (sum of each limb) through the accumulator input, the Q4_1 minimum as
// m * sum(x).
//
// Data flow.  A workgroup of 16 waves owns a contiguous range of output rows;
// a step streams 16 of its rows (one per wave) over one K-segment of at most
// 4 KB with coalesced 16-byte buffer loads, so the workgroup reads a
// contiguous region of the weights per step.  The loads land in registers one
// step ahead, are written into a 2-slot LDS ring (one LDS-only barrier per
// step), and every wave then computes one 4-pair chunk of the segment for all
// 16 rows.  Out-of-range rows are given an empty buffer range: their loads
// return zeros without touching memory.  Row sums are reduced across the 16
// waves in a fixed order (deterministic) one step later by a rotating wave.
//
// Activations that are not finite cannot be written as limbs: a wave whose
// chunk holds inf or NaN computes that chunk per element instead,
// ((q - 8) * d) * x accumulated like the reference, so inf/NaN propagate as in
// quantized_matvec_q4_0_scalar (quantization.rs:1121-1124).
//
// Q4_K (woolly_gguf's layout, dequantize.rs:404-458: 6-bit scales s_j at bytes
// 0..11, f16 d and dmin at 12..15, element 2b / 2b+1 = low / high nibble of
// quant byte b at 16 + b) is one 256-element block per chunk, 144 bytes like
// four Q4_0 pairs: its eight 32-element scale groups take the place of the
// eight blocks, with scale d * s_j (exact in f32) and the minimum entering as
// dmin * sum(x) over the block.
//
// Q6_K (woolly_gguf's indexing, dequantize.rs:460-536) is one 210-byte block
// per chunk.  Element i = 32 j + 8 g + t of K-step j takes the low (j < 4) or
// high (j >= 4) nibble of quant byte 16 j + 8 (g & 1) + t and the two bits
// 2 t + 2 (j >= 4) .. of the 24-bit word qh[8 j + 2 g .. 8 j + 2 g + 2] (the
// byte past the last is 0), so one lane's eight B values are two dwords of
// nibbles or-ed with spread 2-bit fields (q = 0..63); the -32 enters through
// the accumulator input, -32 * (limb sums), the same for every weight row
// and computed once per segment with MFMAs against a B operand of -32s.  Its scales are per
// 16 elements: the limbs of the two halves of a 32-element step sit in
// different A rows (rows 8 (j & 1) + 4 h + limb), so lane group G of
// accumulator t holds the sums of 16-element group 4 t + G, scaled by
// d * s / 64 (exact).
#include "gemv_mfma_dev.hpp"

namespace {

// NL: 16-byte loads per lane per step (row segments of up to 1024 NL bytes).
// DEPTH: steps whose loads are in flight in registers (one-segment rows only).
template <int TYPE, int NSEG, int NL, int MODE, int DEPTH>
__device__ __forceinline__ void gemv_mfma_body(const MgArgs& a, int bid) {
  // The fused modes (RMSNorm, gate + up) read more arguments before their
  // first weight load: they request them in one burst.  The plain mode keeps
  // the compiler's order, which measured faster for it (7.87 against 7.97 us
  // at 14336 x 4096).
  constexpr bool BURST = MODE != 0;
  struct WPtrs {
    const uint8_t *W0, *W1, *W2;
  };
  WPtrs pinned{};
  if constexpr (BURST) {
    mg_args_now(a);
    pinned = WPtrs{mg_ptr_now(a.W0), mg_ptr_now(a.W1), mg_ptr_now(a.W2)};
  }
  // the weight pointers: the pinned copies, or the arguments themselves
  const auto& wsrc = [&]() -> const auto& {
    if constexpr (BURST) return pinned;
    else return a;
  }();
  static_assert(DEPTH >= 1 && (DEPTH == 1 || NSEG == 1), "register prefetch of several steps needs one segment");
  constexpr int PB = MgFmt<TYPE>::PB;
  constexpr bool FFN = (MODE & kMgFfn) != 0;
  constexpr bool NORM = (MODE & kMgNorm) != 0;
  constexpr bool Q41 = TYPE == WH_TYPE_Q4_1;
  constexpr bool Q4K = TYPE == WH_TYPE_Q4_K;
  constexpr bool Q6K = TYPE == WH_TYPE_Q6_K;
  constexpr int CB = mg_chunk_bytes(TYPE);
  constexpr int STG = mg_stage_bytes(TYPE);
  extern __shared__ __align__(16) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int S = a.seg_pairs;
  const uint32_t seg_bytes = static_cast<uint32_t>(S >> 2) * CB;
  // Segments that do not start on a 16-byte boundary (Q6_K's 210-byte chunks)
  // are loaded from the boundary below, `lead` bytes early, into an LDS row
  // whose data then starts `lead` bytes in (the writes stay 16-byte aligned).
  constexpr uint32_t kLeadRoom = (CB & 15) ? 16u : 0u;
  const uint32_t rstr = mg_row_stride(seg_bytes, kLeadRoom + 16u);
  const uint32_t slot_bytes = 16 * rstr;
  const size_t row_bytes = static_cast<size_t>(a.ppr >> 2) * CB;
  const int K = a.ppr * 64;
  uint8_t* ring = lds;
  uint8_t* stage = lds + 2 * slot_bytes + wave * NSEG * STG;  // per segment: limbs, block sums
  float* part = reinterpret_cast<float*>(lds + 2 * slot_bytes + kMgWaves * NSEG * STG);  // [2][16][16]
  float* misc = part + 2 * kMgWaves * 16;                                                    // [16] + [16]
  float* rows_lds = misc + 32;  // the workgroup's output rows (the residual, then += W x)

  const int r0 = bid * a.rows_per_wg;
  const int r1 = min(a.n_out, r0 + a.rows_per_wg);
  const int G = (r1 - r0 + 15) >> 4;
  const int GT = FFN ? 2 * G : G;          // row groups streamed
  const bool owns = wave < (S >> 2);       // computes chunk `wave` of every segment

  // Row (16 q + wave) of streamed group q: its bytes, or an empty range.
  auto row_src = [&](int q, const uint8_t** base) -> bool {
    const int gi = FFN ? (q >> 1) : q;
    const int row = r0 + 16 * gi + wave;
    if (q >= GT || row >= r1) return false;
    int local = row;
    const uint8_t* w = wsrc.W0;
    if constexpr (FFN) {
      const uint8_t* const w0 = wsrc.W0;  // values, not a choice of addresses
      const uint8_t* const w1 = wsrc.W1;
      w = (q & 1) ? w1 : w0;
    } else {
      if (local >= a.n0) {
        local -= a.n0;
        w = wsrc.W1;
        if (local >= a.n1) {
          local -= a.n1;
          w = wsrc.W2;
        }
      }
    }
    *base = w + static_cast<size_t>(local) * row_bytes;
    return true;
  };
  mg_v4i buf[DEPTH][NL];
  auto load = [&](int q, int seg, int d) {
    const uint8_t* base = wsrc.W0;
    const bool ok = row_src(q, &base);
    const uint32_t lead = (static_cast<uint32_t>(seg) * seg_bytes) & (kLeadRoom ? 15u : 0u);
    const mg_v4i rs = mg_rsrc(base + static_cast<size_t>(seg) * seg_bytes - lead, ok ? seg_bytes + lead : 0u);
#pragma unroll
    for (int i = 0; i < NL; i++) buf[d][i] = mg_buffer_load_x4(rs, 16 * (64 * i + lane), 0, kMgNt);
  };

  // The workgroup's output rows are accumulated in LDS and stored to y after
  // the step loop: a global store inside the loop would share the load
  // counter with the weight loads, and the compiler then waits for every load
  // in flight before each step.  They start as the residual (or 0).  Up to one
  // row per thread the residual goes through a register, requested after x
  // and before the weights (loads complete in order, so waiting for it does
  // not wait for them); longer ranges are copied here.
  const bool res_reg = r1 - r0 <= kMgWaves * 64;
  if (!res_reg) {
    for (int i = threadIdx.x; i < r1 - r0; i += kMgWaves * 64)
      rows_lds[i] = (!FFN && a.residual) ? a.residual[r0 + i] : 0.f;
  }
  // ---- activations of this wave's chunks (4 consecutive per lane), then the first weights
  float xv[NSEG][4];
  float gv[NSEG][4];
#pragma unroll
  for (int seg = 0; seg < NSEG; seg++) {
    const int base = (seg * S + 4 * wave) * 64 + 4 * lane;
    float4 xt = make_float4(0.f, 0.f, 0.f, 0.f), gt = xt;
    if (owns) {
      xt = *reinterpret_cast<const float4*>(a.x + base);
      if constexpr (NORM) gt = *reinterpret_cast<const float4*>(a.gamma + base);
    }
    xv[seg][0] = xt.x, xv[seg][1] = xt.y, xv[seg][2] = xt.z, xv[seg][3] = xt.w;
    gv[seg][0] = gt.x, gv[seg][1] = gt.y, gv[seg][2] = gt.z, gv[seg][3] = gt.w;
  }
  float resv = 0.f;
  if (!FFN && a.residual && res_reg && static_cast<int>(threadIdx.x) < r1 - r0) resv = a.residual[r0 + threadIdx.x];
#pragma unroll
  for (int d = 0; d < DEPTH; d++) load(d, 0, d);
  // Nothing that waits for x may be scheduled above the weight loads: the
  // first step's weights must be requested before x's latency is waited out.
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NSEG == 1) {
    // No wave starts the VALU-heavy prologue below before every wave has
    // requested its first weights (a barrier without a memory wait): the
    // oldest-first issue order otherwise lets the prologues of a SIMD's older
    // waves hold back the youngest wave's loads, whose data then lands last.
    // (Rows of several segments request four times the activations first and
    // lose more waiting here than they gain.)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (NORM) {
    // RMSNorm (tensor_utils.rs:446-480): W ((x / rms) * gamma) is formed as
    // (W (x * gamma)) / rms, rms = sqrt(sum x^2 / K + eps).  The limbs are
    // those of x * gamma; each wave's share of sum x^2 goes to LDS, and a
    // row's product is divided by rms where the row is finished, after step
    // barriers that have made every share visible, so the prologue needs no
    // barrier of its own.  (Per element this differs from the reference's
    // (x / rms) * gamma by its roundings only.)
    float ss = 0.f;
#pragma unroll
    for (int seg = 0; seg < NSEG; seg++)
#pragma unroll
      for (int i = 0; i < 4; i++) ss = __builtin_fmaf(xv[seg][i], xv[seg][i], ss);
    ss = whd::wave_sum(ss);
    if (lane == 0) misc[wave] = ss;
#pragma unroll
    for (int seg = 0; seg < NSEG; seg++)
#pragma unroll
      for (int i = 0; i < 4; i++) xv[seg][i] *= gv[seg][i];
  }


  // ---- limbs of each chunk -> this wave's staging area (the MFMA A operands are
  // read from it: the lanes of rows 4j..4j+3 of block j's operand, zeros elsewhere)
  int ex[NSEG];
  bool exact[NSEG];
#pragma unroll
  for (int seg = 0; seg < NSEG; seg++) {
    // the chunk's largest |x| as the maximum of the bit patterns of |x| (they
    // order like the values, and a NaN or an infinity lies above every finite
    // value, which sends the chunk down the exact path)
    uint32_t um = 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) um = max(um, __builtin_bit_cast(uint32_t, xv[seg][i]) & 0x7FFFFFFFu);
    um = mg_wave_max_u32(um);
    exact[seg] = um >= 0x7F800000u;
    int e = 0;
    if (um != 0u && !exact[seg]) {
      int ee;
      frexpf(__builtin_bit_cast(float, um), &ee);
      e = 30 - ee;
    }
    ex[seg] = e;
    int8_t* xop = reinterpret_cast<int8_t*>(stage + seg * STG);
    // Signed base-256 digits of xi = 2^24 l0 + 2^16 l1 + 2^8 l2 + l3 (l1..l3
    // in [-128, 127]): adding 128 to each of the three low digits makes them
    // bytes without carries, so the bytes of (xi + 0x808080) ^ 0x808080 are
    // l3, l2, l1, l0 (|xi| < 2^30 keeps l0 within [-64, 64]).
    uint32_t z[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // |x * 2^e| < 2^30: the conversion is exact for the chunk's larger elements
      const int xi = mg_cvt_i32(rintf(ldexpf(xv[seg][i], e)));
      z[i] = (static_cast<uint32_t>(xi) + 0x808080u) ^ 0x808080u;
    }
    // the lane's four elements feed four consecutive k-slots (all but Q4_K):
    // transpose the 4 x 4 bytes so that row[r] holds limb r of elements 0..3
    uint32_t row[4];
    {
      const uint32_t a = __builtin_amdgcn_perm(z[1], z[0], 0x06020703u);  // z0.b3 z1.b3 z0.b2 z1.b2
      const uint32_t b = __builtin_amdgcn_perm(z[1], z[0], 0x04000501u);  // z0.b1 z1.b1 z0.b0 z1.b0
      const uint32_t c = __builtin_amdgcn_perm(z[3], z[2], 0x06020703u);
      const uint32_t d = __builtin_amdgcn_perm(z[3], z[2], 0x04000501u);
      row[0] = __builtin_amdgcn_perm(c, a, 0x05040100u);
      row[1] = __builtin_amdgcn_perm(c, a, 0x07060302u);
      row[2] = __builtin_amdgcn_perm(d, b, 0x05040100u);
      row[3] = __builtin_amdgcn_perm(d, b, 0x07060302u);
    }
    int8_t* pb = xop + (lane >> 3) * kMgLimbBytes + mg_slot_offset<TYPE>(4 * (lane & 7));
    if constexpr (Q4K) {
      // elements 0..3 of the lane go to slots +0, +4, +1, +5
#pragma unroll
      for (int r = 0; r < 4; r++) {
        *reinterpret_cast<uint16_t*>(pb + 32 * r) = static_cast<uint16_t>(__builtin_amdgcn_perm(0u, row[r], 0x0c0c0200u));
        *reinterpret_cast<uint16_t*>(pb + 32 * r + 4) = static_cast<uint16_t>(__builtin_amdgcn_perm(0u, row[r], 0x0c0c0301u));
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) *reinterpret_cast<uint32_t*>(pb + 32 * r) = row[r];
    }
  }
  if (res_reg && static_cast<int>(threadIdx.x) < r1 - r0) rows_lds[threadIdx.x] = resv;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  // A operands of segment seg: lanes outside rows 4j..4j+3 of block j keep the
  // zeros set here
  long xo[8];
  mg_v4i cin[2];  // Q4_0: -8 * limb sums of block 4t + g (accumulator input)
  mg_v4i cq[Q6K ? 4 : 1];  // Q6_K: -32 * limb sums of 16-element group 4t + g
  float bsum[2];  // Q4_1 / Q4_K: sum of the block's activations, in units of 2^-e
#pragma unroll
  for (int lb = 0; lb < 8; lb++) xo[lb] = 0;
  auto get_x = [&](int seg) {
    const int8_t* xop = reinterpret_cast<const int8_t*>(stage + seg * STG);
#pragma unroll
    for (int lb = 0; lb < 8; lb++) {
      // Q6_K: rows 8 (lb & 1) + 4 h + limb carry half h of block lb (k groups 2h, 2h + 1)
      const bool mine = Q6K ? ((n >> 2) == 2 * (lb & 1) + (g >> 1)) : ((n >> 2) == (lb & 3));
      if (mine) xo[lb] = *reinterpret_cast<const long*>(xop + lb * kMgLimbBytes + 32 * (n & 3) + 8 * g);
    }
    if constexpr (Q6K) {
      // -32 * (limb sums of each 16-element group): the same for every weight
      // row, so one MFMA per K-step against a B operand of -32s
#pragma unroll
      for (int t = 0; t < 4; t++) cq[t] = (mg_v4i){0, 0, 0, 0};
#pragma unroll
      for (int lb = 0; lb < 8; lb++)
        cq[lb >> 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[lb], static_cast<long>(0xE0E0E0E0E0E0E0E0ull), cq[lb >> 1], 0, 0, 0);
      return;
    }
    // Limb sums of each block, the same for every weight row: MFMAs of the
    // blocks' A operands against a B operand of equal bytes, so lane (n, g)'s
    // accumulator t holds (times the byte) the sums of limbs 0..3 of block
    // 4t + g.  Q4_0: -8 times them start its accumulators; Q4_1 / Q4_K: their
    // base-256 combination is the block's activation sum.
#pragma unroll
    for (int t = 0; t < 2; t++) {
      cin[t] = (mg_v4i){0, 0, 0, 0};
      bsum[t] = 0.f;
      if constexpr (TYPE == WH_TYPE_Q4_0) {
#pragma unroll
        for (int lb = 4 * t; lb < 4 * t + 4; lb++)
          cin[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[lb], static_cast<long>(0xF8F8F8F8F8F8F8F8ull), cin[t], 0, 0, 0);
      } else if constexpr (Q41 || Q4K) {
        mg_v4i v = {0, 0, 0, 0};
#pragma unroll
        for (int lb = 4 * t; lb < 4 * t + 4; lb++)
          v = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[lb], static_cast<long>(0x0101010101010101ull), v, 0, 0, 0);
        bsum[t] = __builtin_fmaf(static_cast<float>(v[0]), 16777216.f,
                                 __builtin_fmaf(static_cast<float>(v[1]), 65536.f,
                                                __builtin_fmaf(static_cast<float>(v[2]), 256.f, static_cast<float>(v[3]))));
      }
    }
  };
  if constexpr (NSEG == 1) get_x(0);

  // Elements 64 g + 4 jj .. + 3 of this wave's chunk of segment seg (the
  // activations of the exact path, times gamma like the limbs), read again from
  // x (and gamma) so that no register holds the activations past the limbs.
  auto xquad = [&](int seg, int jj) -> float4 {
    const int el = (seg * S + 4 * wave) * 64 + 64 * g + 4 * jj;
    float4 v = *reinterpret_cast<const float4*>(a.x + el);
    if constexpr (NORM) {
      const float4 gm = *reinterpret_cast<const float4*>(a.gamma + el);
      v = make_float4(v.x * gm.x, v.y * gm.y, v.z * gm.z, v.w * gm.w);
    }
    return v;
  };

  // Sum of group q over the 16 waves (fixed order), then the output row.
  // All 64 lanes: lane (n, g) adds waves 4g .. 4g + 3 of row n, the lane
  // groups are then summed across (a short chain on the finishing wave, which
  // computes its own chunk after this).
  // to_y: the group's rows go straight to y (the last group, after the loop)
  auto finish = [&](int q, bool to_y) {
    const float* pp = part + (q & 1) * kMgWaves * 16 + 64 * g + n;
    const float v0 = pp[0], v1 = pp[16], v2 = pp[32], v3 = pp[48];
    float v = mg_sum_lane_groups((v0 + v1) + (v2 + v3));
    if (lane >= 16) return;
    if constexpr (NORM) {
      // the waves' shares of sum x^2, in fixed order
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kMgWaves; w++) tot += misc[w];
      v = v / sqrtf(tot / static_cast<float>(K) + a.eps);
    }
    const int gi = FFN ? (q >> 1) : q;
    const int row = r0 + 16 * gi + n;
    if constexpr (FFN) {
      if ((q & 1) == 0) {
        misc[16 + n] = v;  // gate, combined with up one group later
        return;
      }
      const float gt = misc[16 + n];
      if (row < r1) {
        const float out = (gt * (1.0f / (1.0f + expf(-gt)))) * v;
        if (to_y) a.y[row] = out;
        else rows_lds[row - r0] = out;
      }
    } else {
      if (row < r1) {
        const float out = rows_lds[row - r0] + v;
        if (to_y) a.y[row] = out;
        else rows_lds[row - r0] = out;
      }
    }
  };

  // With DEPTH > 1 the last pass may run up to DEPTH - 1 steps past GT: they
  // copy (empty-range, so zero) loads and meet the barriers like any step but
  // compute nothing.  No branch skips a load, so the compiler's wait counts
  // stay exact (a skipped load merged into the loop header would make it wait
  // for every load in flight).
  float acc = 0.f;
  for (int q0 = 0; q0 < GT; q0 += DEPTH)
#pragma unroll
  for (int bb = 0; bb < DEPTH; bb++) {
    const int q = q0 + bb;
    const bool live = q < GT;
#pragma unroll
    for (int seg = 0; seg < NSEG; seg++) {
      const int s = q * NSEG + seg;
      uint8_t* slot = ring + (s & 1) * slot_bytes;
      {
        // every lane stores (pieces past the segment go to the overflow room)
        uint8_t* dst = slot + wave * rstr;
        const uint32_t end = seg_bytes + ((static_cast<uint32_t>(seg) * seg_bytes) & (kLeadRoom ? 15u : 0u));
        const uint32_t end16 = (end + 15u) & ~15u;
#pragma unroll
        for (int i = 0; i < NL; i++) {
          const uint32_t o = 16u * (64 * i + lane);
          *reinterpret_cast<mg_v4i*>(dst + (o < end16 ? o : end16)) = buf[bb][i];
        }
      }
      if (seg + 1 < NSEG) load(q, seg + 1, bb);
      else load(q + DEPTH, 0, bb);
      // LDS-only barrier (a __syncthreads() would also wait for the loads in flight)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (seg == 0 && q > 0 && q < GT && wave == ((q - 1) & (kMgWaves - 1))) finish(q - 1, false);
      if (owns && live) {
        if constexpr (NSEG > 1) get_x(seg);
        const uint32_t lead = (static_cast<uint32_t>(seg) * seg_bytes) & (kLeadRoom ? 15u : 0u);
        const uint8_t* rowp = slot + n * rstr + lead + wave * CB;
        if constexpr (Q6K) {
          if (!exact[seg]) {
            mg_v4i C[4];
#pragma unroll
            for (int t = 0; t < 4; t++) C[t] = cq[t];
#pragma unroll
            for (int j = 0; j < 8; j++) {
              uint32_t l0, l1;
              // LDS rows start 16-byte aligned, the chunk `lead + 210 wave` bytes in
              mg_lds_u64(rowp + 16 * j + 8 * (g & 1), static_cast<int>((lead + 2 * (wave & 1)) & 3u), l0, l1);
              const uint8_t* hp = rowp + 128 + 8 * j + 2 * g;
              uint32_t w = *reinterpret_cast<const uint16_t*>(hp);  // hp is even
              if (j >= 4) {
                // 8 j + 2 g + 2 == 64 only for j = 7, g = 3 (element 255)
                if (j < 7 || g < 3) w |= static_cast<uint32_t>(hp[2]) << 16;
                w >>= 2;
                l0 >>= 4;
                l1 >>= 4;
              }
              const uint32_t b0 = (l0 & 0x0F0F0F0Fu) | mg_spread2(w & 0xFFu);
              const uint32_t b1 = (l1 & 0x0F0F0F0Fu) | mg_spread2((w >> 8) & 0xFFu);
              const long qj = static_cast<long>(b0) | (static_cast<long>(b1) << 32);
              C[j >> 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[j], qj, C[j >> 1], 0, 0, 0);
            }
            const float d64 = whd::f16_bits_to_f32(static_cast<uint32_t>(rowp[208]) |
                                                   (static_cast<uint32_t>(rowp[209]) << 8)) * 0.015625f;
            float sacc = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
              const float f = mg_limbs(C[t]);
              sacc = __builtin_fmaf(d64 * static_cast<float>(rowp[192 + 4 * t + g]), f, sacc);
            }
            acc += ldexpf(sacc, -ex[seg]);
          } else {
            // lane group g: elements 64 g .. 64 g + 63 of the block, row n
            acc += mg_q6k_exact(rowp, g, [&](int jj) { return xquad(seg, jj); });
          }
        } else if constexpr (Q4K) {
          if (!exact[seg]) {
            // the chunk is one block: groups j = 0..7 of 32 elements, group
            // 4t + g's limb sums in lane group g of C[t]
            const uint32_t* pw = reinterpret_cast<const uint32_t*>(rowp);
            mg_v4i C[2];
#pragma unroll
            for (int t = 0; t < 2; t++) C[t] = cin[t];
#pragma unroll
            for (int j = 0; j < 8; j++) {
              const uint32_t u = pw[4 + 4 * j + g];
              const long qj = static_cast<long>(u & 0x0F0F0F0Fu) | (static_cast<long>((u >> 4) & 0x0F0F0F0Fu) << 32);
              C[j >> 2] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[j], qj, C[j >> 2], 0, 0, 0);
            }
            const uint32_t dd = pw[3];
            const float d = whd::f16_bits_to_f32(dd & 0xFFFFu);
            const float dmin = whd::f16_bits_to_f32(dd >> 16);
            float sacc = 0.f;
#pragma unroll
            for (int t = 0; t < 2; t++) {
              const float f = mg_limbs(C[t]);
              const float ds = d * static_cast<float>(mg_q4k_scale(rowp, 4 * t + g));
              sacc = __builtin_fmaf(ds, f, sacc);
              sacc = __builtin_fmaf(dmin, bsum[t], sacc);
            }
            acc += ldexpf(sacc, -ex[seg]);
          } else {
            // lane group g: elements 64 g .. 64 g + 63 of the block, row n
            acc += mg_q4k_exact(rowp, g, [&](int jj) { return xquad(seg, jj); });
          }
        } else {
          if (!exact[seg]) {
            // scale (and minimum) of block 4t + g
            uint32_t dm[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
              const int blk = 4 * t + g;
              const uint8_t* bp = rowp + (blk >> 1) * PB + (blk & 1) * (PB / 2);
              if constexpr (Q41) dm[t] = *reinterpret_cast<const uint32_t*>(bp);
              else dm[t] = *reinterpret_cast<const uint16_t*>(bp);
            }
            mg_v4i C[2];
#pragma unroll
            for (int t = 0; t < 2; t++) C[t] = cin[t];
#pragma unroll
            for (int p = 0; p < 4; p++) {
              long qa, qb;
              mg_quants<TYPE>(reinterpret_cast<const uint32_t*>(rowp + p * PB), g, qa, qb);
              C[p >> 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[2 * p], qa, C[p >> 1], 0, 0, 0);
              C[p >> 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo[2 * p + 1], qb, C[p >> 1], 0, 0, 0);
            }
            float sacc = 0.f;
#pragma unroll
            for (int t = 0; t < 2; t++) {
              const float f = mg_limbs(C[t]);
              const float d = whd::f16_bits_to_f32(dm[t] & 0xFFFFu);
              sacc = __builtin_fmaf(d, f, sacc);
              if constexpr (Q41) sacc = __builtin_fmaf(whd::f16_bits_to_f32(dm[t] >> 16), bsum[t], sacc);
            }
            acc += ldexpf(sacc, -ex[seg]);
          } else {
            // lane group g: pair g of the chunk, row n
            acc += mg_pair_exact<TYPE>(rowp + g * PB, [&](int jj) { return xquad(seg, jj); });
          }
        }
      }
      if (seg == NSEG - 1 && live) {
        const float v = mg_sum_lane_groups(acc);
        if (g == 0) part[(q & 1) * kMgWaves * 16 + wave * 16 + n] = v;
        acc = 0.f;
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
  for (int i = threadIdx.x; i < done_rows; i += kMgWaves * 64) a.y[r0 + i] = rows_lds[i];
}

template <int TYPE, int NSEG, int NL, int MODE, int DEPTH>
__global__ __launch_bounds__(kMgWaves * 64) void gemv_mfma_kernel(const MgArgs a) {
  gemv_mfma_body<TYPE, NSEG, NL, MODE, DEPTH>(a, static_cast<int>(blockIdx.x));
}

// Two groups of row-stacked matrices of different block types over the same x
// and RMSNorm in one launch (the decode step's q + k in Q4_K and v in Q6_K of
// Q4_K_M files): workgroups [0, grid_a) run group a, the rest group b, each
// with its own rows, LDS layout and output.  A launch's fixed costs are most
// of a small GEMV's time, so one launch replaces two.
template <int TA, int NLA, int TB, int NLB, int MODE>
__global__ __launch_bounds__(kMgWaves * 64) void gemv_mfma2_kernel(const MgArgs a, const MgArgs b, int grid_a) {
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < grid_a)
    gemv_mfma_body<TA, 1, NLA, MODE, kMgDepth1>(a, bid);
  else
    gemv_mfma_body<TB, 1, NLB, MODE, kMgDepth1>(b, bid - grid_a);
}

size_t mt_lds_bytes(int type, int seg_pairs, int nseg, int mt, int rows_per_wg) {
  const int cb = mg_chunk_bytes(type);
  const size_t seg_bytes = static_cast<size_t>(seg_pairs / 4 * cb);
  const size_t rstr = mg_row_stride(static_cast<uint32_t>(seg_bytes), ((cb & 15) ? 16u : 0u) + 16u);
  return 2u * 16u * rstr + static_cast<size_t>(kMgWaves) * (mt_stage_bytes(type, mt) + mt_xsum_bytes(type, nseg, mt)) +
         4u * (2u * kMgWaves * mt * 16 + static_cast<size_t>(kMgWaves) * mt + mt + static_cast<size_t>(mt) * rows_per_wg);
}

size_t mg_lds_bytes(int type, int seg_pairs, int nseg, int rows_per_wg) {
  const int cb = mg_chunk_bytes(type);
  const size_t seg_bytes = static_cast<size_t>(seg_pairs / 4 * cb);
  const size_t rstr = mg_row_stride(static_cast<uint32_t>(seg_bytes), ((cb & 15) ? 16u : 0u) + 16u);
  return 2u * 16u * rstr +
         static_cast<size_t>(kMgWaves) * nseg * mg_stage_bytes(type) +
         4u * (2 * kMgWaves * 16 + 32 + static_cast<size_t>(rows_per_wg));
}

// Segments: the fewest (1 .. 4) that split the row into whole 4-pair chunks,
// at most 16 chunks and 4 KB per segment (with the up to 15 bytes loaded
// ahead of a segment that does not start on a 16-byte boundary).  Rows must
// be a multiple of 16 bytes (Q6_K: a multiple of 8 blocks), so that a load
// range only ends inside a 16-byte piece in the middle of a row, never at the
// end of the matrix.  0 when none does.
int mg_segments(int type, size_t ppr) {
  const size_t cb = mg_chunk_bytes(type);
  if (cb == 0 || ppr == 0 || ppr % 4 != 0 || (ppr / 4 * cb) % 16 != 0) return 0;
  const size_t lead = (cb & 15) ? 15 : 0;
  for (int ns = 1; ns <= 4; ns++) {
    if (ppr % ns != 0) continue;
    const size_t s = ppr / ns;
    if (s % 4 == 0 && s / 4 <= kMgWaves && s / 4 * cb + lead <= kMgSegMax) return ns;
  }
  return 0;
}

template <int TYPE, int NSEG, int NL, int MODE, int DEPTH = 1>
int mg_launch(const MgArgs& a, int grid, size_t lds, hipStream_t s) {
  auto* fn = &gemv_mfma_kernel<TYPE, NSEG, NL, MODE, DEPTH>;
  WH_ENSURE_LDS(lds, fn);
  fn<<<grid, kMgWaves * 64, lds, s>>>(a);
  WH_LAUNCH_CHECK("gemv (mfma) kernel launch");
  return WH_OK;
}

template <int TYPE, int NL, int MODE>
int mg_dispatch_nl(const MgArgs& a, int nseg, int grid, size_t lds, hipStream_t s) {
  switch (nseg) {
    case 1: return mg_launch<TYPE, 1, NL, MODE, kMgDepth1>(a, grid, lds, s);
    case 2: return mg_launch<TYPE, 2, NL, MODE>(a, grid, lds, s);
    case 3: return mg_launch<TYPE, 3, NL, MODE>(a, grid, lds, s);
    default: return mg_launch<TYPE, 4, NL, MODE>(a, grid, lds, s);
  }
}

template <int TYPE, int MODE>
int mg_dispatch(const MgArgs& a, int nseg, int grid, size_t lds, hipStream_t s) {
  // bytes one lane group of 64 lanes loads per row: the segment and its lead
  const int seg_bytes = a.seg_pairs / 4 * mg_chunk_bytes(TYPE) + ((mg_chunk_bytes(TYPE) & 15) ? 15 : 0);
  if constexpr (TYPE == WH_TYPE_Q4_0 || TYPE == WH_TYPE_Q4_1 || TYPE == WH_TYPE_Q8_0)
    if (nseg == 4 && seg_bytes <= 2048) return mg_launch<TYPE, 4, 2, MODE>(a, grid, lds, s);
  return seg_bytes <= 3072 ? mg_dispatch_nl<TYPE, 3, MODE>(a, nseg, grid, lds, s)
                           : mg_dispatch_nl<TYPE, 4, MODE>(a, nseg, grid, lds, s);
}

template <int TYPE>
int mg_typed(const MgArgs& a, int nseg, int mode, int grid, size_t lds, hipStream_t s) {
  switch (mode) {
    case 0: return mg_dispatch<TYPE, 0>(a, nseg, grid, lds, s);
    case kMgNorm: return mg_dispatch<TYPE, kMgNorm>(a, nseg, grid, lds, s);
    default: return mg_dispatch<TYPE, kMgNorm | kMgFfn>(a, nseg, grid, lds, s);
  }
}

}  // namespace

namespace wh {

bool gemv_mfma_ok(int type, size_t n_out, size_t k) {
  if (mg_chunk_bytes(type) == 0) return false;
  if (n_out == 0 || n_out >= (1u << 30) || k % 64 != 0) return false;
  return mg_segments(type, k / 64) > 0;
}

// mats / rows: up to three row-stacked matrices with the same K (ffn: gate, up
// with n_out rows each).  Returns WH_ERR_INVALID_SHAPE without launching when
// the layout does not fit this kernel.
namespace {
// The arguments, segments, grid and LDS bytes of one single-token launch;
// WH_ERR_INVALID_SHAPE when the layout does not fit the kernel.
int mg_prepare(int type, const void* const* mats, const size_t* rows, int n_mats, bool ffn, const float* x,
               const float* gamma, float eps, const float* residual, float* y, size_t n_out, size_t k, MgArgs* out,
               int* nseg_out, size_t* grid_out, size_t* lds_out) {
  if (!gemv_mfma_ok(type, n_out, k) || n_mats < 1 || n_mats > 3 || (ffn && (n_mats != 2 || !gamma)))
    return WH_ERR_INVALID_SHAPE;
  for (int i = 0; i < n_mats; i++)
    if (!aligned(mats[i], 4)) return WH_ERR_INVALID_SHAPE;
  if (!aligned(x, 16) || (gamma && !aligned(gamma, 16))) return WH_ERR_INVALID_SHAPE;
  const size_t ppr = k / 64;
  const int nseg = mg_segments(type, ppr);
  MgArgs a{};
  a.W0 = static_cast<const uint8_t*>(mats[0]);
  a.W1 = n_mats > 1 ? static_cast<const uint8_t*>(mats[1]) : a.W0;
  a.W2 = n_mats > 2 ? static_cast<const uint8_t*>(mats[2]) : a.W1;
  a.n0 = ffn ? static_cast<int>(n_out) : static_cast<int>(rows[0]);
  a.n1 = (!ffn && n_mats > 1) ? static_cast<int>(rows[1]) : 0;
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.residual = ffn ? nullptr : residual;
  a.y = y;
  a.n_out = static_cast<int>(n_out);
  a.ppr = static_cast<int>(ppr);
  a.seg_pairs = static_cast<int>(ppr / nseg);
  a.m = 1;
  a.ldy = static_cast<int>(n_out);
  // at most one workgroup per CU, each with a whole number of 16-row groups:
  // a half-empty last step costs about as much as a full one, so fewer
  // workgroups with full steps finish sooner (Q4_0 K = 4096: 14336 rows in
  // 224 x 64 take 8.55 us against 8.83 us in 256 x 56)
  const size_t groups = (n_out + 15) / 16;
  const size_t cus = static_cast<size_t>(cu_count());
  const size_t grid0 = groups < cus ? groups : cus;
  a.rows_per_wg = static_cast<int>((groups + grid0 - 1) / grid0 * 16);
  const size_t grid = (n_out + a.rows_per_wg - 1) / a.rows_per_wg;
  const size_t lds = mg_lds_bytes(type, a.seg_pairs, nseg, a.rows_per_wg);
  if (lds > max_lds_per_block()) return WH_ERR_INVALID_SHAPE;
  *out = a;
  *nseg_out = nseg;
  *grid_out = grid;
  *lds_out = lds;
  return WH_OK;
}

// loads per lane per step that mg_dispatch gives a one-segment row
int mg_nl_one_segment(int type, const MgArgs& a) {
  const int seg_bytes = a.seg_pairs / 4 * mg_chunk_bytes(type) + ((mg_chunk_bytes(type) & 15) ? 15 : 0);
  return seg_bytes <= 3072 ? 3 : 4;
}
}  // namespace

int launch_gemv_mfma(int type, const void* const* mats, const size_t* rows, int n_mats, bool ffn, const float* x,
                     const float* gamma, float eps, const float* residual, float* y, size_t n_out, size_t k,
                     hipStream_t s) {
  if (n_out == 0) return WH_OK;
  MgArgs a{};
  int nseg = 0;
  size_t grid = 0, lds = 0;
  const int st = mg_prepare(type, mats, rows, n_mats, ffn, x, gamma, eps, residual, y, n_out, k, &a, &nseg, &grid, &lds);
  if (st) return st;
  const int mode = ffn ? (kMgNorm | kMgFfn) : (gamma ? kMgNorm : 0);
  switch (type) {
    case WH_TYPE_Q4_0: return mg_typed<WH_TYPE_Q4_0>(a, nseg, mode, static_cast<int>(grid), lds, s);
    case WH_TYPE_Q4_1: return mg_typed<WH_TYPE_Q4_1>(a, nseg, mode, static_cast<int>(grid), lds, s);
    case WH_TYPE_Q4_K: return mg_typed<WH_TYPE_Q4_K>(a, nseg, mode, static_cast<int>(grid), lds, s);
    case WH_TYPE_Q6_K: return mg_typed<WH_TYPE_Q6_K>(a, nseg, mode, static_cast<int>(grid), lds, s);
    default: return mg_typed<WH_TYPE_Q8_0>(a, nseg, mode, static_cast<int>(grid), lds, s);
  }
}


int launch_gemv_mfma2(int type_a, const void* const* mats_a, const size_t* rows_a, int n_a, int type_b,
                      const void* const* mats_b, const size_t* rows_b, int n_b, const float* x, const float* gamma,
                      float eps, float* y_a, float* y_b, size_t k, hipStream_t s) {
  if (!gamma || type_a != WH_TYPE_Q4_K || type_b != WH_TYPE_Q6_K || n_a < 1 || n_b < 1 || n_a + n_b > 3)
    return WH_ERR_INVALID_SHAPE;
  size_t out_a = 0, out_b = 0;
  for (int i = 0; i < n_a; i++) out_a += rows_a[i];
  for (int i = 0; i < n_b; i++) out_b += rows_b[i];
  if (out_a == 0 || out_b == 0) return WH_ERR_INVALID_SHAPE;
  MgArgs a{}, b{};
  int nseg_a = 0, nseg_b = 0;
  size_t grid_a = 0, grid_b = 0, lds_a = 0, lds_b = 0;
  if (mg_prepare(type_a, mats_a, rows_a, n_a, false, x, gamma, eps, nullptr, y_a, out_a, k, &a, &nseg_a, &grid_a,
                 &lds_a) ||
      mg_prepare(type_b, mats_b, rows_b, n_b, false, x, gamma, eps, nullptr, y_b, out_b, k, &b, &nseg_b, &grid_b,
                 &lds_b))
    return WH_ERR_INVALID_SHAPE;
  // the one instantiation: one segment each, three loads per step for Q4_K,
  // four for Q6_K (K = 4096, Llama-3-8B)
  if (nseg_a != 1 || nseg_b != 1 || mg_nl_one_segment(type_a, a) != 3 || mg_nl_one_segment(type_b, b) != 4)
    return WH_ERR_INVALID_SHAPE;
  const size_t lds = lds_a > lds_b ? lds_a : lds_b;
  auto* fn = &gemv_mfma2_kernel<WH_TYPE_Q4_K, 3, WH_TYPE_Q6_K, 4, kMgNorm>;
  WH_ENSURE_LDS(lds, fn);
  fn<<<static_cast<unsigned>(grid_a + grid_b), kMgWaves * 64, lds, s>>>(a, b, static_cast<int>(grid_a));
  WH_LAUNCH_CHECK("gemv (mfma, two types) kernel launch");
  return WH_OK;
}

// Several tokens (2..16) on the matrix cores: plain Y[t] = W X[t] (mats =
// {W}) or, with ffn, H[t] = silu(gate x_hat[t]) * (up x_hat[t]) (mats = {gate,
// up}, x_hat the RMS-normalised x[t]).  x: [m][k]; y: row t at y + t * ldy.
// WH_ERR_INVALID_SHAPE without launching when the shape does not fit.
int launch_gemv_mt(int type, const void* const* mats, bool ffn, const float* x, size_t m, const float* gamma,
                   float eps, float* y, size_t ldy, size_t n_out, size_t k, hipStream_t s) {
  if (n_out == 0 || m == 0) return WH_OK;
  if (m < 2 || m > 16 || !gemv_mfma_ok(type, n_out, k) || (ffn && !gamma))
    return WH_ERR_INVALID_SHAPE;
  const size_t ppr = k / 64;
  const int nseg = mg_segments(type, ppr);
  const int tg = static_cast<int>((m + 3) / 4);
  if (nseg == 3 || tg * nseg > 4) return WH_ERR_INVALID_SHAPE;
  for (int i = 0; i < (ffn ? 2 : 1); i++)
    if (!aligned(mats[i], 4)) return WH_ERR_INVALID_SHAPE;
  if (!aligned(x, 16) || (gamma && !aligned(gamma, 16))) return WH_ERR_INVALID_SHAPE;
  MgArgs a{};
  a.W0 = static_cast<const uint8_t*>(mats[0]);
  a.W1 = ffn ? static_cast<const uint8_t*>(mats[1]) : a.W0;
  a.W2 = a.W1;
  a.n0 = static_cast<int>(n_out);
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.y = y;
  a.n_out = static_cast<int>(n_out);
  a.ppr = static_cast<int>(ppr);
  a.seg_pairs = static_cast<int>(ppr / nseg);
  a.m = static_cast<int>(m);
  a.ldy = static_cast<int>(ldy);
  const size_t groups = (n_out + 15) / 16;
  const size_t cus = static_cast<size_t>(cu_count());
  const size_t grid0 = groups < cus ? groups : cus;
  a.rows_per_wg = static_cast<int>((groups + grid0 - 1) / grid0 * 16);
  const size_t grid = (n_out + a.rows_per_wg - 1) / a.rows_per_wg;
  // token slots: two in the two-token layout (not for Q6_K), else four per group
  const int mt = (m == 2 && type != WH_TYPE_Q6_K) ? 2 : 4 * tg;
  const size_t lds = mt_lds_bytes(type, a.seg_pairs, nseg, mt, a.rows_per_wg);
  if (lds > max_lds_per_block()) return WH_ERR_INVALID_SHAPE;
  const int g = static_cast<int>(grid);
  switch (type) {
    case WH_TYPE_Q4_0: return launch_gemv_mt_q4_0(a, ffn, nseg, tg, g, lds, s);
    case WH_TYPE_Q4_1: return launch_gemv_mt_q4_1(a, ffn, nseg, tg, g, lds, s);
    case WH_TYPE_Q8_0: return launch_gemv_mt_q8_0(a, ffn, nseg, tg, g, lds, s);
    case WH_TYPE_Q4_K: return launch_gemv_mt_q4_k(a, ffn, nseg, tg, g, lds, s);
    case WH_TYPE_Q6_K: return launch_gemv_mt_q6_k(a, ffn, nseg, tg, g, lds, s);
    default: return WH_ERR_INVALID_SHAPE;
  }
}

}  // namespace wh
