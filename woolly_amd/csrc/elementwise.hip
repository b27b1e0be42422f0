// elementwise.hip -- RMSNorm and SwiGLU on gfx950.
//
// rms_norm (crates/woolly-core/src/tensor_utils.rs:446-480):
//   rms = sqrt(sum_i x_i^2 / hidden + eps); out_i = (x_i / rms) * w_i
// swiglu (crates/woolly-core/src/tensor_utils.rs:512-532):
//   out = g * (1 / (1 + exp(-g))) * u      (exact SiLU)
// The sum of squares is a fixed-shape tree reduction (deterministic); the
// division and square root are the correctly rounded IEEE operations.
#include "wh_common.hpp"

namespace {

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w, float eps,
                                                       size_t hidden, float* __restrict__ out) {
  __shared__ float part[4];
  const size_t t = blockIdx.x;
  const float* xt = x + t * hidden;
  float ss = 0.f;
  for (size_t i = threadIdx.x; i < hidden; i += 256) ss = __builtin_fmaf(xt[i], xt[i], ss);
  ss = whd::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float rms = sqrtf(total / static_cast<float>(hidden) + eps);
  float* ot = out + t * hidden;
  for (size_t i = threadIdx.x; i < hidden; i += 256) ot[i] = (xt[i] / rms) * w[i];
}

// Rows of up to kNormVec * 4 * 1024 elements, 16-byte aligned, hidden % 4 == 0:
// one workgroup of 1024 threads per row, the row held in registers between the
// sum of squares and the scaling (one pass over x), float4 loads.
constexpr int kNormVec = 4;
__global__ __launch_bounds__(1024) void rms_norm_vec_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w, float eps,
                                                            size_t hidden, float* __restrict__ out) {
  __shared__ float part[16];
  const size_t t = blockIdx.x;
  const float4* xt = reinterpret_cast<const float4*>(x + t * hidden);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  const int n4 = static_cast<int>(hidden / 4);
  float4 v[kNormVec];
  float ss = 0.f;
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    const int i = static_cast<int>(threadIdx.x) + 1024 * r;
    v[r] = i < n4 ? xt[i] : float4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    ss = __builtin_fmaf(v[r].x, v[r].x, ss);
    ss = __builtin_fmaf(v[r].y, v[r].y, ss);
    ss = __builtin_fmaf(v[r].z, v[r].z, ss);
    ss = __builtin_fmaf(v[r].w, v[r].w, ss);
  }
  ss = whd::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) total += part[i];
  const float rms = sqrtf(total / static_cast<float>(hidden) + eps);
  float4* ot = reinterpret_cast<float4*>(out + t * hidden);
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    const int i = static_cast<int>(threadIdx.x) + 1024 * r;
    if (i < n4) {
      const float4 g = w4[i];
      ot[i] = float4{(v[r].x / rms) * g.x, (v[r].y / rms) * g.y, (v[r].z / rms) * g.z, (v[r].w / rms) * g.w};
    }
  }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g,
                                                     const float* __restrict__ u, size_t n,
                                                     float* __restrict__ out) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gv = g[i];
    const float sig = 1.0f / (1.0f + expf(-gv));
    out[i] = (gv * sig) * u[i];
  }
}

}  // namespace

namespace wh {

int launch_rms_norm(const float* x, const float* weight, float eps, size_t tokens, size_t hidden,
                    float* out, hipStream_t s) {
  if (tokens == 0 || hidden == 0) return WH_OK;
  const bool vec = hidden % 4 == 0 && hidden <= static_cast<size_t>(kNormVec) * 4 * 1024 && aligned(x, 16) &&
                   aligned(weight, 16) && aligned(out, 16);
  for (size_t t0 = 0; t0 < tokens; t0 += 65535u * 16u) {
    const size_t nt = tokens - t0 < 65535u * 16u ? tokens - t0 : 65535u * 16u;
    if (vec)
      rms_norm_vec_kernel<<<static_cast<unsigned>(nt), 1024, 0, s>>>(x + t0 * hidden, weight, eps, hidden,
                                                                     out + t0 * hidden);
    else
      rms_norm_kernel<<<static_cast<unsigned>(nt), 256, 0, s>>>(x + t0 * hidden, weight, eps, hidden,
                                                                out + t0 * hidden);
  }
  WH_LAUNCH_CHECK("rms_norm kernel launch");
  return WH_OK;
}

int launch_swiglu(const float* gate, const float* up, size_t n, float* out, hipStream_t s) {
  if (n == 0) return WH_OK;
  size_t grid = (n + 255) / 256;
  const size_t cap = static_cast<size_t>(cu_count()) * 8;
  if (grid > cap) grid = cap;
  swiglu_kernel<<<static_cast<unsigned>(grid), 256, 0, s>>>(gate, up, n, out);
  WH_LAUNCH_CHECK("swiglu kernel launch");
  return WH_OK;
}

}  // namespace wh
