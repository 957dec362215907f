// mr_probe.hip -- measurement probes for the decode path's ceilings (bench support, not a
// reference interface): a plain streaming read of a buffer, as fast as the memory system
// moves bytes with a given number of workgroups, and an empty kernel, whose launches in a
// graph are the floor of a per-layer kernel boundary.
#include "mr_device.h"
#include "mr_internal.h"

namespace mr {

// Workgroup b reads 16-byte pieces b*256 + tid, then + grid*256 ..., four loads in flight per
// thread, and folds them into one word per workgroup (so no load is dead).
__global__ __launch_bounds__(256) void k_probe_read(const i32x4* __restrict__ src, uint64_t n16,
                                                    uint32_t* __restrict__ sink) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const i32x4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= (uint32_t)(a.x ^ a.y ^ a.z ^ a.w) ^ (uint32_t)(b.x ^ b.y ^ b.z ^ b.w) ^
           (uint32_t)(c.x ^ c.y ^ c.z ^ c.w) ^ (uint32_t)(d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n16; i += stride) {
    const i32x4 a = src[i];
    acc ^= (uint32_t)(a.x ^ a.y ^ a.z ^ a.w);
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int t = 0; t < 256; ++t) r ^= red[t];
    sink[blockIdx.x] = r;
  }
}

__global__ __launch_bounds__(256) void k_probe_empty() {}

hipError_t launch_probe_read(const Launch& K, const void* src, uint64_t nbytes, uint32_t n_wg, uint32_t* sink) {
  ProfScope ps(K, "probe_read");
  hipLaunchKernelGGL(k_probe_read, dim3(n_wg), dim3(256), 0, K.s, static_cast<const i32x4*>(src), nbytes / 16, sink);
  return hipGetLastError();
}

hipError_t launch_probe_empty(const Launch& K, uint32_t n_wg) {
  ProfScope ps(K, "probe_empty");
  hipLaunchKernelGGL(k_probe_empty, dim3(n_wg), dim3(256), 0, K.s);
  return hipGetLastError();
}

}  // namespace mr
