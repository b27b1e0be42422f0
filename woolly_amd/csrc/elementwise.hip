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
  for (size_t t0 = 0; t0 < tokens; t0 += 65535u * 16u) {
    const size_t nt = tokens - t0 < 65535u * 16u ? tokens - t0 : 65535u * 16u;
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
