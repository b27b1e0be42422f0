// probe.hip -- measurement aid, no counterpart in the reference: a read-only
// stream over an n_rows x row_bytes matrix in the geometry of the
// single-token matrix-core GEMV (gemv_mfma.hip).  Workgroups of 16 waves own
// ceil(n_rows / 16 / CUs) 16-row groups each; in step q wave w reads row
// r0 + 16 q + w with 16-byte buffer loads of its 64 lanes (bytes past the row
// read as zeros without a memory access).  Nothing is stored in LDS and
// nothing is computed but an xor of the data, which workgroup b stores in
// out[b] (so that no load can be dropped; one atomic dword shared by all
// workgroups serialised them and took longer than the reads).
//   mode 0: one step in flight per wave, the next step's loads issued when
//           this step's data has arrived (the GEMV's pipelining);
//   mode 1: every step of the wave in flight at once (up to 4 per batch);
//   mode 2: not the GEMV's geometry: the matrix as one flat byte range, split
//           into one contiguous piece per workgroup (one per CU while that
//           keeps at most 16 loads per lane), every lane issuing all of its
//           16-byte loads before it uses any (every load in flight at once).
// bench.py times it beside the GEMV: modes 0 and 1 as the floor of that access
// pattern, mode 2 as the floor of one launch that reads the same bytes.
#include "wh_common.hpp"

typedef int pr_i4 __attribute__((ext_vector_type(4)));
__device__ pr_i4 pr_buffer_load_x4(pr_i4 rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

namespace {

__device__ __forceinline__ pr_i4 pr_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  pr_i4 r;
  r[0] = static_cast<int>(static_cast<uint32_t>(a));
  r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xFFFFu);
  r[2] = static_cast<int>(nbytes);
  r[3] = 0x00020000;
  return r;
}

constexpr int kPrWaves = 16;
constexpr int kPrNt = 2;  // streaming loads, as the GEMV issues them

// NL: 16-byte loads per lane per row (rows of up to 1024 NL bytes).
template <int NL, int MODE>
__global__ __launch_bounds__(kPrWaves * 64) void read_probe_kernel(const uint8_t* __restrict__ src, uint32_t row_bytes,
                                                                  int n_rows, int rows_per_wg, uint32_t* __restrict__ out) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(n_rows, r0 + rows_per_wg);
  const int G = (r1 - r0 + 15) >> 4;
  auto rs = [&](int q) {
    const int row = r0 + 16 * q + wave;
    const bool ok = q < G && row < r1;
    return pr_rsrc(src + static_cast<size_t>(ok ? row : 0) * row_bytes, ok ? row_bytes : 0u);
  };
  pr_i4 x = {0, 0, 0, 0};
  if constexpr (MODE == 0) {
    pr_i4 buf[NL];
    {
      const pr_i4 r = rs(0);
#pragma unroll
      for (int i = 0; i < NL; i++) buf[i] = pr_buffer_load_x4(r, 16 * (64 * i + lane), 0, kPrNt);
    }
    for (int q = 0; q < G; q++) {
#pragma unroll
      for (int i = 0; i < NL; i++) x ^= buf[i];  // waits for step q
      const pr_i4 r = rs(q + 1);
#pragma unroll
      for (int i = 0; i < NL; i++) buf[i] = pr_buffer_load_x4(r, 16 * (64 * i + lane), 0, kPrNt);
    }
#pragma unroll
    for (int i = 0; i < NL; i++) x ^= buf[i];  // the empty-range loads past the last step
  } else {
    constexpr int B = 4;
    for (int q0 = 0; q0 < G; q0 += B) {
      pr_i4 buf[B][NL];
#pragma unroll
      for (int b = 0; b < B; b++) {
        const pr_i4 r = rs(q0 + b);
#pragma unroll
        for (int i = 0; i < NL; i++) buf[b][i] = pr_buffer_load_x4(r, 16 * (64 * i + lane), 0, kPrNt);
      }
#pragma unroll
      for (int b = 0; b < B; b++)
#pragma unroll
        for (int i = 0; i < NL; i++) x ^= buf[b][i];
    }
  }
  uint32_t v = static_cast<uint32_t>(x[0] ^ x[1] ^ x[2] ^ x[3]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64));
  // the waves' checksums meet in LDS; one store per workgroup
  __shared__ uint32_t red[kPrWaves];
  if (lane == 0) red[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kPrWaves; w++) t ^= red[w];
    out[blockIdx.x] = t;
  }
}

// Mode 2: workgroup b reads bytes [b * per_wg, (b + 1) * per_wg) of the flat
// range (the buffer range ends at the matrix), lane l of the workgroup the
// 16-byte pieces l, l + 1024, ... of that piece, all loads issued first.
constexpr int kPrFlatLoads = 16;
__global__ __launch_bounds__(kPrWaves * 64) void read_probe_flat_kernel(const uint8_t* __restrict__ src, size_t total,
                                                                        size_t per_wg, uint32_t* __restrict__ out) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const size_t b0 = blockIdx.x * per_wg;
  const size_t len = b0 < total ? (total - b0 < per_wg ? total - b0 : per_wg) : 0;
  const pr_i4 r = pr_rsrc(src + (len ? b0 : 0), static_cast<uint32_t>(len));
  pr_i4 buf[kPrFlatLoads];
#pragma unroll
  for (int i = 0; i < kPrFlatLoads; i++)
    buf[i] = pr_buffer_load_x4(r, 16 * (kPrWaves * 64 * i + static_cast<int>(threadIdx.x)), 0, kPrNt);
  pr_i4 x = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kPrFlatLoads; i++) x ^= buf[i];
  uint32_t v = static_cast<uint32_t>(x[0] ^ x[1] ^ x[2] ^ x[3]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64));
  __shared__ uint32_t red[kPrWaves];
  if (lane == 0) red[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kPrWaves; w++) t ^= red[w];
    out[blockIdx.x] = t;
  }
}

template <int NL>
void launch_nl(int mode, const uint8_t* src, uint32_t row_bytes, int n_rows, int rows_per_wg, int grid, uint32_t* out,
               hipStream_t s) {
  if (mode == 0)
    read_probe_kernel<NL, 0><<<grid, kPrWaves * 64, 0, s>>>(src, row_bytes, n_rows, rows_per_wg, out);
  else
    read_probe_kernel<NL, 1><<<grid, kPrWaves * 64, 0, s>>>(src, row_bytes, n_rows, rows_per_wg, out);
}

}  // namespace

WH_API int wh_read_probe(const void* src, size_t row_bytes, size_t n_rows, int mode, uint32_t* out,
                         wh_stream_t stream) {
  if (!src || !out || row_bytes == 0 || row_bytes > 4096 || n_rows == 0 || n_rows >= (1u << 30) ||
      mode < 0 || mode > 2 || !wh::aligned(out, 4))
    return wh::set_error(WH_ERR_INVALID_ARGUMENT,
                         "read_probe: non-null source and output, rows of 1 .. 4096 bytes, mode 0, 1 or 2");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (mode == 2) {
    // one workgroup per CU, more when a lane would need more than kPrFlatLoads
    // loads; never more workgroups than out has dwords (ceil(n_rows / 16))
    const size_t total = row_bytes * n_rows;
    const size_t per_wg_max = static_cast<size_t>(kPrWaves) * 64 * 16 * kPrFlatLoads;  // bytes one workgroup reads
    size_t grid = static_cast<size_t>(wh::cu_count());
    if (grid * per_wg_max < total) grid = (total + per_wg_max - 1) / per_wg_max;
    const size_t cap = (n_rows + 15) / 16;
    if (grid > cap) grid = cap;
    size_t per_wg = (total + grid - 1) / grid;
    per_wg = (per_wg + 15) / 16 * 16;
    if (per_wg > per_wg_max || per_wg > 0xFFFFFFFFu)
      return wh::set_error(WH_ERR_INVALID_ARGUMENT, "read_probe: mode 2 takes at most %zu bytes per %zu rows",
                           per_wg_max * cap, n_rows);
    read_probe_flat_kernel<<<static_cast<unsigned>(grid), kPrWaves * 64, 0, s>>>(static_cast<const uint8_t*>(src), total,
                                                                               per_wg, out);
    WH_LAUNCH_CHECK("read probe kernel launch");
    return WH_OK;
  }
  const size_t groups = (n_rows + 15) / 16;
  const size_t cus = static_cast<size_t>(wh::cu_count());
  const size_t grid0 = groups < cus ? groups : cus;
  const int rows_per_wg = static_cast<int>((groups + grid0 - 1) / grid0 * 16);
  const int grid = static_cast<int>((n_rows + rows_per_wg - 1) / rows_per_wg);
  const uint8_t* p = static_cast<const uint8_t*>(src);
  const uint32_t rb = static_cast<uint32_t>(row_bytes);
  const int nr = static_cast<int>(n_rows);
  switch ((row_bytes + 1023) / 1024) {
    case 1: launch_nl<1>(mode, p, rb, nr, rows_per_wg, grid, out, s); break;
    case 2: launch_nl<2>(mode, p, rb, nr, rows_per_wg, grid, out, s); break;
    case 3: launch_nl<3>(mode, p, rb, nr, rows_per_wg, grid, out, s); break;
    default: launch_nl<4>(mode, p, rb, nr, rows_per_wg, grid, out, s); break;
  }
  WH_LAUNCH_CHECK("read probe kernel launch");
  return WH_OK;
}
