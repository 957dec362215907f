// mr_norm.hip -- RMSNorm of the MoE input and the residual add of its output, as
// separate kernels for the multi-kernel decode path of mr_moe_forward_residual
// (the fused decode kernels do both inside their own launch).
//
// rms_norm(h) = (h * inv) * w, inv = 1 / sqrt(mean(h^2) + eps)   (norm.rs:16-37)
// hidden' = h + moe(rms_norm(h))                                  (layer.rs:462-473)
//
// inv is computed by one wave in the same order as the fused kernels' rms_inv
// (lane l sums the squares of elements 4*(l + 64*j) .. +3 for j = 0, 1, ... in order,
// then a butterfly), so both paths see the same bits of the normalised input.
#include "mr_device.h"
#include "mr_internal.h"

namespace mr {

__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ h, const float* __restrict__ w,
                                                  float eps, int H, float* __restrict__ out) {
#pragma clang fp contract(off)
  const float* hr = h + (size_t)blockIdx.x * H;
  float* orow = out + (size_t)blockIdx.x * H;
  __shared__ float inv_s;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float s = 0.f;
    for (int c = lane * 4; c < H; c += 256) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(hr + c);
      s = s + v.x * v.x;
      s = s + v.y * v.y;
      s = s + v.z * v.z;
      s = s + v.w * v.w;
    }
    s = wave_sum(s);
    if (lane == 0) inv_s = 1.f / sqrtf(s / (float)H + eps);
  }
  __syncthreads();
  const float inv = inv_s;
  for (int i = threadIdx.x; i < H; i += 256) orow[i] = (hr[i] * inv) * w[i];
}

__global__ __launch_bounds__(256) void k_residual_add(const float* __restrict__ h, const float* __restrict__ m,
                                                      uint64_t n, float* out) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = h[i] + m[i];  // residual + moe_out
}

hipError_t launch_rms_norm(const Launch& K, const float* h, const float* w, float eps, uint32_t T, uint32_t H,
                           float* out) {
  ProfScope ps(K, "rms_norm");
  hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(256), 0, K.s, h, w, eps, (int)H, out);
  return hipGetLastError();
}

hipError_t launch_residual_add(const Launch& K, const float* h, const float* m, uint64_t n, float* out) {
  ProfScope ps(K, "residual_add");
  hipLaunchKernelGGL(k_residual_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, K.s, h, m, n, out);
  return hipGetLastError();
}

}  // namespace mr
