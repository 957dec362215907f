// mr_probe.hip -- measurement probes for the decode path's ceilings (bench support, not a
// reference interface): a plain streaming read of a buffer, as fast as the memory system
// moves bytes with a given number of workgroups and loads in flight, and an empty kernel,
// whose launches in a graph are the floor of a per-layer kernel boundary.
#include "mr_device.h"
#include "mr_internal.h"

#include <algorithm>

namespace mr {

// Workgroup b reads its own contiguous range of the buffer (per16 pieces of 16 bytes), thread
// t the pieces t, t + 256, ... of that range in batches of D: the D loads of a batch are issued
// together, then folded (pieces past the range end re-read the range's last piece, a cache
// hit). The loads are ordinary global loads, so the compiler places every wait for their data.
// Every piece is folded into one word per workgroup, so no load is dead.
template <int D>
__global__ __launch_bounds__(256) void k_probe_read(const i32x4* __restrict__ src, uint64_t n16, uint64_t per16,
                                                    uint32_t* __restrict__ sink) {
  const uint64_t beg = (uint64_t)blockIdx.x * per16;
  const uint64_t end = min(beg + per16, n16);
  uint32_t acc = 0;
  if (beg < end) {
    const uint64_t last = end - 1;
    const auto* g = (const __attribute__((address_space(1))) i32x4*)(src);
    for (uint64_t i = beg + threadIdx.x; i < end; i += (uint64_t)D * 256) {
      i32x4 v[D];
#pragma unroll
      for (int j = 0; j < D; ++j) v[j] = g[min(i + (uint64_t)j * 256, last)];
      __builtin_amdgcn_sched_barrier(0);  // all D loads issue before the first fold
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const uint32_t f = (uint32_t)(v[j].x ^ v[j].y ^ v[j].z ^ v[j].w);
        acc ^= i + (uint64_t)j * 256 < end ? f : 0u;  // a select, not a branch
      }
    }
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

// The fused MXFP4 kernel's gate/up access pattern: the buffer as rows of rb bytes, tiles of 16
// adjacent rows; wave w of workgroup b streams tiles 4 (b + k grid) + w over the row in chunks of
// 204 bytes per row (12 MXFP4 blocks), each chunk as 240-byte 16-byte-aligned row segments, 15
// per row, lane-contiguous: four 16-byte loads per lane per chunk, D chunks in flight (issued
// together, then folded). Tiles past n_tiles are not read.
template <int D>
__global__ __launch_bounds__(256) void k_probe_tiles(const uint8_t* __restrict__ src, uint32_t rb, uint32_t n_tiles,
                                                     uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const auto* g = (const __attribute__((address_space(1))) uint8_t*)(src);
  uint32_t rrb[4], pc16[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int q = it * 64 + lane, row = min(q / 15, 15), pc = min(q - row * 15, 14);
    rrb[it] = (uint32_t)row * rb;
    pc16[it] = 16u * (uint32_t)pc;
  }
  const int nc = (int)((rb + 203u) / 204u);  // chunks per row
  uint32_t acc = 0;
  for (uint32_t t = 4 * blockIdx.x + wave; t < n_tiles; t += 4 * gridDim.x) {
    const uint64_t base = (uint64_t)t * 16u * rb;
    const uint32_t a = (uint32_t)(base & 15u);
    for (int c0 = 0; c0 < nc; c0 += D) {
      i32x4 v[D][4];
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const uint32_t cb = 204u * (uint32_t)min(c0 + d, nc - 1);
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const uint32_t rowa = a + rrb[it];
          const uint32_t lastr = (rowa + rb - 1u) & ~15u;
          const uint32_t off = min(((rowa + cb) & ~15u) + pc16[it], lastr);
          v[d][it] = *(const __attribute__((address_space(1))) i32x4*)(g + (base - a) + off);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // all D chunks issue before the first fold
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int it = 0; it < 4; ++it) acc ^= (uint32_t)(v[d][it].x ^ v[d][it].y ^ v[d][it].z ^ v[d][it].w);
    }
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int k = 0; k < 256; ++k) r ^= red[k];
    sink[blockIdx.x] = r;
  }
}

// The same with longer row segments: chunks of S K steps (68 S bytes per row), fetched as
// 16-byte pieces of npc per row (NL wave loads per chunk), one chunk at a time per wave.
template <int NL>
__global__ __launch_bounds__(256) void k_probe_tiles_seg(const uint8_t* __restrict__ src, uint32_t rb, uint32_t n_tiles,
                                                         uint32_t steps, uint32_t npc, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const auto* g = (const __attribute__((address_space(1))) uint8_t*)(src);
  uint32_t rrb[NL], pc16[NL];
#pragma unroll
  for (int it = 0; it < NL; ++it) {
    const int q = it * 64 + lane, row = min(q / (int)npc, 15), pc = min(q - row * (int)npc, (int)npc - 1);
    rrb[it] = (uint32_t)row * rb;
    pc16[it] = 16u * (uint32_t)pc;
  }
  const uint32_t cbytes = 68u * steps;
  const int nc = (int)((rb + cbytes - 1u) / cbytes);
  uint32_t acc = 0;
  for (uint32_t t = 4 * blockIdx.x + wave; t < n_tiles; t += 4 * gridDim.x) {
    const uint64_t base = (uint64_t)t * 16u * rb;
    const uint32_t a = (uint32_t)(base & 15u);
    for (int c = 0; c < nc; ++c) {
      i32x4 v[NL];
#pragma unroll
      for (int it = 0; it < NL; ++it) {
        const uint32_t rowa = a + rrb[it];
        const uint32_t lastr = (rowa + rb - 1u) & ~15u;
        const uint32_t off = min(((rowa + cbytes * (uint32_t)c) & ~15u) + pc16[it], lastr);
        v[it] = *(const __attribute__((address_space(1))) i32x4*)(g + (base - a) + off);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int it = 0; it < NL; ++it) acc ^= (uint32_t)(v[it].x ^ v[it].y ^ v[it].z ^ v[it].w);
    }
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int k = 0; k < 256; ++k) r ^= red[k];
    sink[blockIdx.x] = r;
  }
}

// A light touch of a buffer: one 4-byte read every `stride` bytes (for example one per page), so
// the address translations of the range are cached while almost none of its bytes are read.
__global__ __launch_bounds__(256) void k_probe_touch(const uint8_t* __restrict__ src, uint64_t nbytes, uint32_t stride,
                                                     uint32_t* __restrict__ sink) {
  const uint64_t n = (nbytes + stride - 1) / stride;
  uint32_t acc = 0;
  for (uint64_t k = (uint64_t)blockIdx.x * 256 + threadIdx.x; k < n; k += (uint64_t)gridDim.x * 256)
    acc ^= *reinterpret_cast<const uint32_t*>(src + k * stride);
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;  // keeps the loads; almost never stores
}

__global__ __launch_bounds__(256) void k_probe_empty() {}

hipError_t launch_probe_read(const Launch& K, const void* src, uint64_t nbytes, uint32_t n_wg, uint32_t depth,
                             uint32_t* sink) {
  ProfScope ps(K, "probe_read");
  const uint64_t n16 = nbytes / 16;
  const uint64_t per16 = ((n16 + n_wg - 1) / n_wg + 255) / 256 * 256;  // whole 4 KiB runs per workgroup
  const auto* s = static_cast<const i32x4*>(src);
  switch (depth) {
    case 4: hipLaunchKernelGGL(k_probe_read<4>, dim3(n_wg), dim3(256), 0, K.s, s, n16, per16, sink); break;
    case 8: hipLaunchKernelGGL(k_probe_read<8>, dim3(n_wg), dim3(256), 0, K.s, s, n16, per16, sink); break;
    case 16: hipLaunchKernelGGL(k_probe_read<16>, dim3(n_wg), dim3(256), 0, K.s, s, n16, per16, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_probe_tiles(const Launch& K, const void* src, uint32_t rb, uint32_t n_tiles, uint32_t n_wg,
                              uint32_t depth, uint32_t* sink) {
  ProfScope ps(K, "probe_tiles");
  const auto* s = static_cast<const uint8_t*>(src);
  switch (depth) {
    case 2: hipLaunchKernelGGL(k_probe_tiles<2>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, sink); break;
    case 4: hipLaunchKernelGGL(k_probe_tiles<4>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, sink); break;
    case 8: hipLaunchKernelGGL(k_probe_tiles<8>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, sink); break;
    // depth 0x100 + S: one chunk of S steps at a time (S = 6, 12, 23)
    case 0x106: hipLaunchKernelGGL(k_probe_tiles_seg<7>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, 6u, 27u, sink); break;
    case 0x10C: hipLaunchKernelGGL(k_probe_tiles_seg<14>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, 12u, 53u, sink); break;
    case 0x117: hipLaunchKernelGGL(k_probe_tiles_seg<25>, dim3(n_wg), dim3(256), 0, K.s, s, rb, n_tiles, 23u, 99u, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_probe_touch(const Launch& K, const void* src, uint64_t nbytes, uint32_t stride, uint32_t* sink) {
  ProfScope ps(K, "probe_touch");
  hipLaunchKernelGGL(k_probe_touch, dim3(256), dim3(256), 0, K.s, static_cast<const uint8_t*>(src), nbytes, stride, sink);
  return hipGetLastError();
}

// Flag round trips between two workgroups, a and b, through the device-coherent level, the
// hand-off the fused decode kernels use (agent-scope stores and polling loads). Thread 0 of a
// stores i to word 0 and polls word 32 (another 128-byte line) until it reads i; thread 0 of b
// polls word 0 for i and stores i to word 32; i = 1 .. n. Workgroups are dealt to the XCDs in
// turn (b mod 8), so b - a = 8 keeps both on one XCD and an odd difference puts them on two.
// Every poll gives up once the device clock has run limit ticks (100 MHz) past the start of the
// wait, so both threads end whatever happens. res: [0] clock ticks a spent on the n round trips,
// [1] round trips completed, [2] a's XCC_ID << 32 | HW_ID, [3] the same of b. The words are zero
// when the kernel starts (the host clears them).
__global__ __launch_bounds__(64) void k_probe_flags(uint32_t* w, int a, int b, int n, uint64_t limit,
                                                    unsigned long long* res) {
  if (threadIdx.x != 0 || ((int)blockIdx.x != a && (int)blockIdx.x != b)) return;
  const bool is_a = (int)blockIdx.x == a;
  uint32_t* mine = w + (is_a ? 0 : 32);
  const uint32_t* theirs = w + (is_a ? 32 : 0);
  const unsigned long long id = ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
                                (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  int done = 0;
  for (int i = 1; i <= n; ++i) {
    if (is_a) __hip_atomic_store(mine, (uint32_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long w0 = __builtin_amdgcn_s_memrealtime();
    bool seen = false;
    while (!(seen = __hip_atomic_load(theirs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)i) &&
           __builtin_amdgcn_s_memrealtime() - w0 < limit) {
    }
    if (!seen) break;
    if (!is_a) __hip_atomic_store(mine, (uint32_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    done = i;
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (is_a) {
    res[0] = t1 - t0;
    res[1] = (unsigned long long)done;
    res[2] = id;
  } else {
    res[3] = id;
  }
}

hipError_t launch_probe_flags(const Launch& K, uint32_t* words, int a, int b, int n, unsigned long long* res) {
  ProfScope ps(K, "probe_flags");
  const hipError_t e = hipMemsetAsync(words, 0, 64 * sizeof(uint32_t), K.s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_probe_flags, dim3((unsigned)(std::max(a, b) + 1)), dim3(64), 0, K.s, words, a, b, n,
                     (uint64_t)10000000 /* 100 ms */, res);
  return hipGetLastError();
}

hipError_t launch_probe_empty(const Launch& K, uint32_t n_wg) {
  ProfScope ps(K, "probe_empty");
  hipLaunchKernelGGL(k_probe_empty, dim3(n_wg), dim3(256), 0, K.s);
  return hipGetLastError();
}

}  // namespace mr
