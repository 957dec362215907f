// mr_valu.hip -- router, top-k and vector-ALU expert kernels for gfx950.
//
// These kernels are the straightforward decode path: one launch per step
// (router GEMV, top-k, gate+up+SwiGLU, down+combine), one wave per output
// row, activations staged in LDS. They are the correctness baseline the fused
// decode kernels (mr_fused.hip, mr_fused_q4k.hip) are checked and timed against,
// and they run every layout the ABI accepts (MXFP4 and Q4_K, any H, I multiple of
// the block).
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"

namespace mr {

// ---------------------------------------------------------------------------
// zero fill (graph-capture safe replacement for hipMemsetAsync)
__global__ void k_zero(uint32_t* __restrict__ p, uint64_t n_words) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n_words; i += stride) p[i] = 0u;
}

hipError_t launch_zero(const Launch& K, void* dst, uint64_t nbytes) {
  uint64_t words = nbytes / 4;
  if (words == 0) return hipSuccess;
  uint32_t blocks = (uint32_t)((words + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  ProfScope ps(K, "zero");
  hipLaunchKernelGGL(k_zero, dim3(blocks), dim3(256), 0, K.s, (uint32_t*)dst, words);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Router GEMV: logits[t][e] = x[t] . Wr[e] + b[e] + mask[e]  (layer.rs:806-837, 1016-1026)
// One wave per expert row; float4 loads; grid (ceil(E/4), T).
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ x,
                                                       const float* __restrict__ wr,
                                                       const float* __restrict__ br,
                                                       const float* __restrict__ mask,
                                                       float* __restrict__ logits, int H, int E) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const int t = blockIdx.y;
  if (e >= E) return;
  const float* xr = x + (size_t)t * H;
  const float* w = wr + (size_t)e * H;
  float acc = 0.f;
  for (int c = lane * 4; c < H; c += 256) {
    f32x4 a = *reinterpret_cast<const f32x4*>(xr + c);
    f32x4 b = *reinterpret_cast<const f32x4*>(w + c);
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    acc = __builtin_fmaf(a.w, b.w, acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if (br) acc = acc + br[e];
    if (mask) acc = acc + mask[e];
    logits[(size_t)t * E + e] = acc;
  }
}

// Router GEMM for many tokens on the fp32 MFMA (v_mfma_f32_16x16x4f32): a 1024-thread
// workgroup takes 16 tokens x 16 experts x one of nks ranges of H's 16-element blocks; its
// 16 waves take the range's blocks in turn (wave w: blocks w, w+16, ...), each issuing all of
// its loads before its first MFMA, and the 16 partial tiles are summed in LDS in wave order.
// A CU reaches only a fraction of HBM bandwidth with its own loads, so H is split over
// workgroups until the grid spans the CUs (k_router_topk_finish adds the nks partials in
// order: the same bits on every run). MFMA operands: lane (i, g) = lane % 16, lane / 16 holds
// x[t0+i][k..k+3] and Wr[e0+i][k..k+3] for k = 16b + 4g, and MFMA j of the block multiplies
// their element j, so the four MFMAs cover the block's 16 elements; D[4g + r][i] is token
// t0+4g+r, expert e0+i. Tokens past T and experts past E repeat the last row (not stored).
// part: [nks][T][E]. H % 4 == 0 and ceil(H/16) <= nks * 16 * kRouterBlocks.
constexpr int kRouterWaves = 16, kRouterBlocks = 6, kRouterMaxSplit = 4;
__global__ __launch_bounds__(1024) void k_router_logits_mfma(const float* __restrict__ x,
                                                             const float* __restrict__ wr,
                                                             float* __restrict__ part, int T, int H, int E,
                                                             int nks) {
  __shared__ f32x4 red[kRouterWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
  const int nb = (H + 15) >> 4, per = (nb + nks - 1) / nks;
  const int kb0 = (int)blockIdx.z * per, kb1 = min(nb, kb0 + per);
  const float* xr = x + (size_t)min(t0 + i, T - 1) * H + 4 * g;
  const float* wrow = wr + (size_t)min(e0 + i, E - 1) * H + 4 * g;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 a[kRouterBlocks], w[kRouterBlocks];
#pragma unroll
  for (int j = 0; j < kRouterBlocks; ++j) {
    const int b = kb0 + wave + kRouterWaves * j;
    const bool in = b < kb1 && 16 * b + 4 * g < H;
    a[j] = in ? *reinterpret_cast<const f32x4*>(xr + 16 * b) : z;
    w[j] = in ? *reinterpret_cast<const f32x4*>(wrow + 16 * b) : z;
  }
  f32x4 acc = z;
#pragma unroll
  for (int j = 0; j < kRouterBlocks; ++j) {
    if (kb0 + wave + kRouterWaves * j < kb1) {  // wave-uniform
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].x, w[j].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].y, w[j].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].z, w[j].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].w, w[j].w, acc, 0, 0, 0);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 s = red[0][lane];
#pragma unroll
    for (int q = 1; q < kRouterWaves; ++q) {
      const f32x4 p = red[q][lane];
      s = f32x4{s[0] + p[0], s[1] + p[1], s[2] + p[2], s[3] + p[3]};
    }
    const int e = e0 + i;
    float* out = part + (size_t)blockIdx.z * T * E;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * g + r;
      if (t < T && e < E) out[(size_t)t * E + e] = s[r];
    }
  }
}

hipError_t launch_router_logits(const Launch& K, const mr_layer& L, const float* x, uint32_t T,
                                float* logits) {
  ProfScope ps(K, "router_logits");
  dim3 grid((L.E + 3) / 4, T);
  hipLaunchKernelGGL(k_router_logits, grid, dim3(256), 0, K.s, x, L.d.router_w, L.d.router_b,
                     L.d.dummy_mask, logits, (int)L.H, (int)L.E);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Top-k (top_k_routing, layer.rs:2346-2403; softmax_topk_kernel,
// fused_ops.metal:131-316). One wave per token; each lane holds up to 8 of the
// E <= 512 values. Selection = first k of a stable descending sort: the
// largest value wins, ties go to the lower expert index.
// Top-k of the logits v[j] of experts lane + 64 j (live[j]: e < E): by logit, and in the
// standard mode, where two logits at the selection boundary could round to one probability,
// again by the probabilities as the reference computes them (prob_exact_needed, prob_keys);
// rows whose probabilities are NaN then take experts 0..k-1, as the reference's stable sort does.
__device__ void topk_vals(float (&v)[8], bool (&live)[8], int k, uint32_t flags, int32_t* out_idx,
                          float* out_w, float* sel_v /* LDS [16] */, int* sel_i /* LDS [16] */) {
  static_assert(kRouteVals == 8, "one key column per lane value");
  const int lane = threadIdx.x & 63;
  const bool softmax_after = (flags & MR_ROUTE_SOFTMAX_AFTER_TOPK) != 0u;
  int E = 0;  // live[j] is e < E
#pragma unroll
  for (int j = 0; j < 8; ++j) E += __popcll(__ballot(live[j]));
  // keys: + 0.f makes -0.0 and +0.0 share a key; a NaN takes key 1, below every number
  // (-inf is 0x007FFFFF), as in the fused routing
  uint32_t hk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) hk[j] = live[j] ? (v[j] == v[j] ? order_key(v[j] + 0.f) : 1u) : 0u;
  // k rounds of a wave argmax on 64-bit keys: the value's order key above the complemented
  // expert index, so the larger value wins and, between equal values, the lower index. DPP
  // steps inside 16-lane rows, then the four rows by readlane. Returns the k-th key.
  auto select = [&]() {
    bool lv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) lv[j] = live[j];
    uint32_t kth = 0u;
    for (int r = 0; r < k; ++r) {
      uint64_t best = 0ull;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t e = (uint32_t)(lane + 64 * j);
        const uint64_t key = ((uint64_t)hk[j] << 32) | (0xFFFFFFFFu - e);
        if (lv[j]) best = key > best ? key : best;
      }
      best = wave_max_u64(best);
      const int bi = (int)(0xFFFFFFFFu - (uint32_t)best);
      if ((bi & 63) == lane) lv[bi >> 6] = false;
      if (lane == 0) sel_i[r] = bi;
      kth = (uint32_t)(best >> 32);
    }
    __builtin_amdgcn_wave_barrier();
    return kth;
  };
  const uint32_t kth = select();
  if (!softmax_after && prob_exact_needed(hk, kth)) {
    prob_keys(v, E, hk);
    select();
  }
  // the selected logits
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    const float lr = entry_value(v, sel_i[r]);
    if (lane == 0) sel_v[r] = lr;
  }
  __builtin_amdgcn_wave_barrier();
  float mx_all = 0.f, sum_all = 1.f;
  if (!softmax_after) {  // standard mode: probabilities over all experts
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j]) m = fmaxf(m, v[j]);
    mx_all = wave_max(m);
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j]) sm += __expf(v[j] - mx_all);
    sum_all = wave_sum(sm);
  }
  if (lane == 0) {
    if (softmax_after) {
      float m = -INFINITY;
      for (int r = 0; r < k; ++r) m = fmaxf(m, sel_v[r]);
      float ex[16], sx = 0.f;
      for (int r = 0; r < k; ++r) {
        ex[r] = __expf(sel_v[r] - m);
        sx = sx + ex[r];
      }
      for (int r = 0; r < k; ++r) out_w[r] = ex[r] / sx;
    } else {
      float pr[16];
      for (int r = 0; r < k; ++r) pr[r] = __expf(sel_v[r] - mx_all) / sum_all;
      if (flags & MR_ROUTE_NORM_TOPK) {
        float sx = 0.f;
        for (int r = 0; r < k; ++r) sx = sx + pr[r];
        for (int r = 0; r < k; ++r) out_w[r] = pr[r] / sx;
      } else {
        for (int r = 0; r < k; ++r) out_w[r] = pr[r];
      }
    }
    for (int r = 0; r < k; ++r) out_idx[r] = sel_i[r];
  }
}

__device__ void topk_wave(const float* row, int E, int k, uint32_t flags, int32_t* out_idx,
                          float* out_w, float* sel_v /* LDS [16] */, int* sel_i /* LDS [16] */) {
  const int lane = threadIdx.x & 63;
  float v[8];
  bool live[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int e = lane + 64 * j;
    live[j] = e < E;
    v[j] = live[j] ? row[e] : 0.f;
  }
  topk_vals(v, live, k, flags, out_idx, out_w, sel_v, sel_i);
}

// Router logits from the H-split partials of k_router_logits_mfma (summed in split order,
// then + bias + mask, the order of k_router_logits), written to logits, then the top-k.
__global__ __launch_bounds__(64) void k_router_topk_finish(const float* __restrict__ part, int nks, int T,
                                                           const float* __restrict__ br,
                                                           const float* __restrict__ mask,
                                                           float* __restrict__ logits, int E, int k,
                                                           uint32_t flags, int32_t* __restrict__ idx,
                                                           float* __restrict__ w) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int t = blockIdx.x, lane = threadIdx.x & 63;
  float v[8];
  bool live[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    live[j] = e < E;
    float s = 0.f;
    if (live[j]) {
      s = part[(size_t)t * E + e];
      for (int q = 1; q < nks; ++q) s = s + part[((size_t)q * T + t) * E + e];
      if (br) s = s + br[e];
      if (mask) s = s + mask[e];
      logits[(size_t)t * E + e] = s;
    }
    v[j] = s;
  }
  topk_vals(v, live, k, flags, idx + (size_t)t * k, w + (size_t)t * k, sv, si);
}

hipError_t launch_router_topk(const Launch& K, const mr_layer& L, const float* x, uint32_t T, float* logits,
                              float* part, int32_t* idx, float* w) {
  const uint32_t nb = (L.H + 15) / 16, tiles = ((L.E + 15) / 16) * ((T + 15) / 16);
  uint32_t nks = std::max<uint32_t>((nb + 16 * kRouterBlocks - 1) / (16 * kRouterBlocks), (256 + tiles - 1) / tiles);
  nks = std::min<uint32_t>(nks, kRouterMaxSplit);
  if (T < 16 || L.H % 4 != 0 || nb > nks * 16u * kRouterBlocks) {
    hipError_t e = launch_router_logits(K, L, x, T, logits);
    return e == hipSuccess ? launch_topk(K, logits, T, L.E, L.d.top_k, L.d.route_flags, idx, w) : e;
  }
  {
    ProfScope ps(K, "router_logits");
    hipLaunchKernelGGL(k_router_logits_mfma, dim3((L.E + 15) / 16, (T + 15) / 16, nks), dim3(64 * kRouterWaves), 0,
                       K.s, x, L.d.router_w, part, (int)T, (int)L.H, (int)L.E, (int)nks);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  ProfScope ps(K, "topk");
  hipLaunchKernelGGL(k_router_topk_finish, dim3(T), dim3(64), 0, K.s, part, (int)nks, (int)T, L.d.router_b,
                     L.d.dummy_mask, logits, (int)L.E, (int)L.d.top_k, L.d.route_flags, idx, w);
  return hipGetLastError();
}

__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ logits, int E, int k,
                                             uint32_t flags, int32_t* __restrict__ idx,
                                             float* __restrict__ w) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int t = blockIdx.x;
  topk_wave(logits + (size_t)t * E, E, k, flags, idx + (size_t)t * k, w + (size_t)t * k, sv, si);
}

hipError_t launch_topk(const Launch& K, const float* logits, uint32_t T, uint32_t E, uint32_t k,
                       uint32_t flags, int32_t* idx, float* w) {
  ProfScope ps(K, "topk");
  hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, K.s, logits, (int)E, (int)k, flags, idx, w);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Row dot products of one quantized weight row with an LDS-resident vector.
// Each lane returns its partial sum; units of 32 elements are spread over lanes.

// MXFP4: unit = one 17-byte block; sum_b d_b * sum_j kvalue_j x_j.
__device__ __forceinline__ float row_dot_mxfp4(const uint8_t* __restrict__ row,
                                               const float* xs, int in_features, int lane) {
  const int nb = in_features >> 5;
  float acc = 0.f;
  for (int b = lane; b < nb; b += 64) {
    uint32_t sc, q[4];
    mx_load_block(row + (size_t)b * 17, sc, q);
    float kd = mx_block_kdot(q, xs + 32 * b);
    acc = __builtin_fmaf(kd, e8m0_half(sc), acc);
  }
  return acc;
}

// Q4_K: unit = one 32-element sub-block s of a 144-byte super-block:
// (d*sc) * sum q x - (dmin*m) * sum x  (dequant.rs:218-262 regrouped).
__device__ __forceinline__ float row_dot_q4k(const uint8_t* __restrict__ row, const float* xs,
                                             int in_features, int lane) {
  const int nu = in_features >> 5;  // 8 sub-blocks per 256
  float acc = 0.f;
  for (int u = lane; u < nu; u += 64) {
    const int b = u >> 3, s = u & 7;
    const uint8_t* blk = row + (size_t)b * 144;
    const uint32_t* bw = reinterpret_cast<const uint32_t*>(blk);
    uint32_t dd = bw[0];
    uint32_t scw[3] = {bw[1], bw[2], bw[3]};
    uint32_t sc, m;
    q4k_scale_min((uint32_t)s, scw, sc, m);
    float d = h2f(dd & 0xFFFFu), dmin = h2f(dd >> 16);
    const uint32_t* qw = bw + 4 + 8 * (s >> 1);
    const int shift = (s & 1) * 4;
    const float* xb = xs + 32 * u;
    float sq = 0.f, sx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t word = (qw[i] >> shift) & 0x0F0F0F0Fu;
      f32x4 xv = *reinterpret_cast<const f32x4*>(xb + 4 * i);
      sq = __builtin_fmaf((float)((word >> 0) & 0xFFu), xv.x, sq);
      sq = __builtin_fmaf((float)((word >> 8) & 0xFFu), xv.y, sq);
      sq = __builtin_fmaf((float)((word >> 16) & 0xFFu), xv.z, sq);
      sq = __builtin_fmaf((float)((word >> 24) & 0xFFu), xv.w, sq);
      sx += (xv.x + xv.y) + (xv.z + xv.w);
    }
    acc += (d * (float)sc) * sq - (dmin * (float)m) * sx;
  }
  return acc;
}

template <int TYPE>
__device__ __forceinline__ float row_dot(const uint8_t* row, const float* xs, int n, int lane) {
  if constexpr (TYPE == MR_GGML_MXFP4)
    return row_dot_mxfp4(row, xs, n, lane);
  else
    return row_dot_q4k(row, xs, n, lane);
}

__host__ __device__ constexpr uint64_t row_bytes_of(int type, uint64_t cols) {
  return type == MR_GGML_MXFP4 ? (cols / 32) * 17 : (cols / 256) * 144;
}

// ---------------------------------------------------------------------------
// Kernel (2): gate+up dequant-matvec + bias + SwiGLU for each (token, slot).
// grid (ceil(I / 16), slots, T), 256 threads: 4 waves x 4 rows each.
struct GateUpArgs {
  const uint8_t* gate;
  const uint8_t* up;
  const uint64_t* gate_off;  // [E] byte offsets
  const uint64_t* up_off;
  const float* gate_b;       // [E, I] or null
  const float* up_b;
  const float* x;            // [T, H]
  const int32_t* idx;        // [T, k] or null (shared expert: expert 0)
  float* act;                // [T, k, I]
  const float* sh_gate_inp;  // shared expert only: [H] or null
  float* sh_sig;             // shared expert only: [T] sigmoid(x . gate_inp)
  int H, I, E, k, act_kind;
  float alpha, limit;
};

template <int TYPE>
__global__ __launch_bounds__(256) void k_gateup_valu(GateUpArgs a) {
  extern __shared__ float xs[];  // [H]
  const int t = blockIdx.z, slot = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* xt = a.x + (size_t)t * a.H;
  for (int c = threadIdx.x * 4; c < a.H; c += 1024)
    *reinterpret_cast<f32x4*>(xs + c) = *reinterpret_cast<const f32x4*>(xt + c);
  __syncthreads();
  const int e = a.idx ? a.idx[(size_t)t * a.k + slot] : 0;
  if (e < 0 || e >= a.E) return;  // invalid routing entry contributes nothing
  if (a.sh_sig && blockIdx.x == 0 && wave == 0) {
    float z = 0.f;
    if (a.sh_gate_inp)
      for (int c = lane; c < a.H; c += 64) z = __builtin_fmaf(xs[c], a.sh_gate_inp[c], z);
    z = wave_sum(z);
    if (lane == 0) a.sh_sig[t] = a.sh_gate_inp ? sigmoidf_(z) : 1.0f;
  }
  const uint8_t* G = a.gate + a.gate_off[e];
  const uint8_t* U = a.up + a.up_off[e];
  const uint64_t rb = row_bytes_of(TYPE, (uint64_t)a.H);
  const int row0 = blockIdx.x * 16 + wave * 4;
  for (int i = 0; i < 4; ++i) {
    const int r = row0 + i;
    if (r >= a.I) break;
    float g = wave_sum(row_dot<TYPE>(G + (uint64_t)r * rb, xs, a.H, lane));
    float u = wave_sum(row_dot<TYPE>(U + (uint64_t)r * rb, xs, a.H, lane));
    if (lane == 0) {
      if (a.gate_b) g = g + a.gate_b[(size_t)e * a.I + r];
      if (a.up_b) u = u + a.up_b[(size_t)e * a.I + r];
      float h = a.act_kind == MR_ACT_SWIGLU_OAI ? swiglu_oai(g, u, a.alpha, a.limit) : silu_mul(g, u);
      a.act[((size_t)t * a.k + slot) * a.I + r] = h;
    }
  }
}

// Kernel (3): down dequant-matvec + bias + weighted combine over the k routed
// experts in ascending expert index (layer.rs:1092-1106, 1446-1448), then the
// shared expert scaled by its sigmoid gate (layer.rs:1935-1951).
// grid (ceil(H / 16), T), 256 threads; LDS holds the token's k activations.
struct DownArgs {
  const uint8_t* down;
  const uint64_t* down_off;
  const float* down_b;   // [E, H] or null
  const float* act;      // [T, k, I]
  const int32_t* idx;    // [T, k]
  const float* w;        // [T, k]
  float* y;              // [T, H]
  int H, I, E, k;
  // shared expert (optional)
  const uint8_t* sh_down;  // [H, Ish] (type sh_type)
  const float* act_sh;     // [T, Ish]
  const float* sh_sig;     // [T]
  int Ish;
};

template <int TYPE, int SH_TYPE>
__global__ __launch_bounds__(256) void k_down_valu(DownArgs a) {
  extern __shared__ float lds[];  // [k * I] + [Ish]
  __shared__ int order[16];
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* at = a.act + (size_t)t * a.k * a.I;
  const int n_act = a.k * a.I;
  for (int c = threadIdx.x * 4; c < n_act; c += 1024)
    *reinterpret_cast<f32x4*>(lds + c) = *reinterpret_cast<const f32x4*>(at + c);
  float* lds_sh = lds + n_act;
  if (a.sh_down)
    for (int c = threadIdx.x * 4; c < a.Ish; c += 1024)
      *reinterpret_cast<f32x4*>(lds_sh + c) =
          *reinterpret_cast<const f32x4*>(a.act_sh + (size_t)t * a.Ish + c);
  if (threadIdx.x == 0) {
    // slots sorted by expert index, ascending (insertion sort, k <= 16)
    const int32_t* it = a.idx + (size_t)t * a.k;
    for (int s = 0; s < a.k; ++s) {
      int j = s;
      while (j > 0 && it[order[j - 1]] > it[s]) {
        order[j] = order[j - 1];
        --j;
      }
      order[j] = s;
    }
  }
  __syncthreads();
  const uint64_t rb = row_bytes_of(TYPE, (uint64_t)a.I);
  const uint64_t rb_sh = row_bytes_of(SH_TYPE, (uint64_t)a.Ish);
  const int row0 = blockIdx.x * 16 + wave * 4;
  for (int i = 0; i < 4; ++i) {
    const int r = row0 + i;
    if (r >= a.H) break;
    float yv = 0.f;
    for (int j = 0; j < a.k; ++j) {
      const int slot = order[j];
      const int e = a.idx[(size_t)t * a.k + slot];
      if (e < 0 || e >= a.E) continue;
      const uint8_t* D = a.down + a.down_off[e] + (uint64_t)r * rb;
      float o = wave_sum(row_dot<TYPE>(D, lds + slot * a.I, a.I, lane));
      if (a.down_b) o = o + a.down_b[(size_t)e * a.H + r];
      yv = yv + o * a.w[(size_t)t * a.k + slot];
    }
    if (a.sh_down) {
      float s = wave_sum(row_dot<SH_TYPE>(a.sh_down + (uint64_t)r * rb_sh, lds_sh, a.Ish, lane));
      yv = yv + s * a.sh_sig[t];
    }
    if (lane == 0) a.y[(size_t)t * a.H + r] = yv;
  }
}

template <int TYPE>
static hipError_t gateup_dispatch(const Launch& K, const char* name, const GateUpArgs& a,
                                  uint32_t slots, uint32_t T) {
  dim3 grid((a.I + 15) / 16, slots, T);
  size_t lds = (size_t)a.H * sizeof(float);
  ProfScope ps(K, name);
  hipLaunchKernelGGL(k_gateup_valu<TYPE>, grid, dim3(256), lds, K.s, a);
  return hipGetLastError();
}

template <int TYPE, int SH>
static hipError_t down_dispatch2(const Launch& K, const DownArgs& a, uint32_t T) {
  dim3 grid((a.H + 15) / 16, T);
  size_t lds = ((size_t)a.k * a.I + (a.sh_down ? a.Ish : 0)) * sizeof(float);
  ProfScope ps(K, "down");
  hipLaunchKernelGGL((k_down_valu<TYPE, SH>), grid, dim3(256), lds, K.s, a);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t down_dispatch(const Launch& K, const DownArgs& a, int sh_type, uint32_t T) {
  if (sh_type == MR_GGML_MXFP4) return down_dispatch2<TYPE, MR_GGML_MXFP4>(K, a, T);
  return down_dispatch2<TYPE, MR_GGML_Q4_K>(K, a, T);
}

hipError_t launch_experts_valu(const Launch& s, const mr_layer& L, const float* x, uint32_t T,
                               const int32_t* idx, const float* w, float* act, float* act_sh,
                               float* y) {
  const mr_pack& G = *L.d.gate;
  const mr_pack& U = *L.d.up;
  const mr_pack& D = *L.d.down;
  const bool has_sh = L.d.sh_gate != nullptr;
  float* sh_sig = has_sh ? act_sh + (size_t)T * L.Ish : nullptr;
  hipError_t err;
  if (has_sh) {
    const mr_pack& SG = *L.d.sh_gate;
    GateUpArgs sa{SG.base, L.d.sh_up->base, SG.d_offsets, L.d.sh_up->d_offsets, nullptr, nullptr,
                  x, nullptr, act_sh, L.d.sh_gate_inp, sh_sig, (int)L.H, (int)L.Ish, 1, 1,
                  MR_ACT_SILU, 0.f, 0.f};
    err = SG.type == MR_GGML_MXFP4 ? gateup_dispatch<MR_GGML_MXFP4>(s, "shared_gateup", sa, 1, T)
                                   : gateup_dispatch<MR_GGML_Q4_K>(s, "shared_gateup", sa, 1, T);
    if (err != hipSuccess) return err;
  }
  GateUpArgs ga{G.base, U.base, G.d_offsets, U.d_offsets, L.d.gate_bias, L.d.up_bias, x, idx, act,
                nullptr, nullptr, (int)L.H, (int)L.I, (int)L.E, (int)L.d.top_k, (int)L.d.act,
                L.d.alpha, L.d.limit};
  err = L.type == MR_GGML_MXFP4 ? gateup_dispatch<MR_GGML_MXFP4>(s, "gateup", ga, L.d.top_k, T)
                                : gateup_dispatch<MR_GGML_Q4_K>(s, "gateup", ga, L.d.top_k, T);
  if (err != hipSuccess) return err;
  DownArgs da{D.base, D.d_offsets, L.d.down_bias, act, idx, w, y, (int)L.H, (int)L.I, (int)L.E,
              (int)L.d.top_k, has_sh ? L.d.sh_down->base : nullptr, act_sh, sh_sig, (int)L.Ish};
  const int sh_type = has_sh ? L.d.sh_down->type : MR_GGML_Q4_K;
  return L.type == MR_GGML_MXFP4 ? down_dispatch<MR_GGML_MXFP4>(s, da, sh_type, T)
                                 : down_dispatch<MR_GGML_Q4_K>(s, da, sh_type, T);
}

// ---------------------------------------------------------------------------
// Dequantization (dequantize_mxfp4 dequant.rs:605-628; dequantize_q4k 218-262),
// bit-exact: single multiplies, no contraction.
__global__ void k_dequant_mxfp4(const uint8_t* __restrict__ src, float* __restrict__ out,
                                uint64_t n_blocks) {
  uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  uint32_t sc, q[4];
  mx_load_block(src + b * 17, sc, q);
  const float d = e8m0_half(sc);
  float* y = out + b * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2 v0 = MR_KV2(q[i], 0), v1 = MR_KV2(q[i], 1), v2 = MR_KV2(q[i], 2),
                v3 = MR_KV2(q[i], 3);
    y[4 * i + 0] = v0.x * d, y[16 + 4 * i + 0] = v0.y * d;
    y[4 * i + 1] = v1.x * d, y[16 + 4 * i + 1] = v1.y * d;
    y[4 * i + 2] = v2.x * d, y[16 + 4 * i + 2] = v2.y * d;
    y[4 * i + 3] = v3.x * d, y[16 + 4 * i + 3] = v3.y * d;
  }
}

__global__ void k_dequant_q4k(const uint8_t* __restrict__ src, float* __restrict__ out,
                              uint64_t n_units) {
#pragma clang fp contract(off)
  uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= n_units) return;
  const uint64_t b = u >> 3;
  const uint32_t s = (uint32_t)(u & 7);
  const uint32_t* bw = reinterpret_cast<const uint32_t*>(src + b * 144);
  uint32_t dd = bw[0];
  uint32_t scw[3] = {bw[1], bw[2], bw[3]};
  uint32_t sc, m;
  q4k_scale_min(s, scw, sc, m);
  const float d1 = h2f(dd & 0xFFFFu) * (float)sc;
  const float m1 = h2f(dd >> 16) * (float)m;
  const uint32_t* qw = bw + 4 + 8 * (s >> 1);
  const int shift = (s & 1) * 4;
  float* y = out + u * 32;
  for (int i = 0; i < 8; ++i) {
    uint32_t word = (qw[i] >> shift) & 0x0F0F0F0Fu;
    for (int j = 0; j < 4; ++j) {
      float p = d1 * (float)((word >> (8 * j)) & 0xFFu);
      y[4 * i + j] = p - m1;
    }
  }
}

hipError_t launch_dequant(const Launch& K, const mr_pack& p, uint32_t expert, float* out) {
  ProfScope ps(K, "dequant");
  hipStream_t s = K.s;
  const uint8_t* src = p.base + p.h_offsets[expert];
  const uint64_t n_el = (uint64_t)p.out_features * p.in_features;
  if (p.type == MR_GGML_MXFP4) {
    uint64_t nb = n_el / 32;
    hipLaunchKernelGGL(k_dequant_mxfp4, dim3((uint32_t)((nb + 255) / 256)), dim3(256), 0, s, src,
                       out, nb);
  } else {
    uint64_t nu = n_el / 32;
    hipLaunchKernelGGL(k_dequant_q4k, dim3((uint32_t)((nu + 255) / 256)), dim3(256), 0, s, src,
                       out, nu);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic blocks (same arithmetic as moe_rocm/synth.py).
__global__ void k_synth_mxfp4(uint8_t* __restrict__ dst, uint64_t n_blocks, uint64_t first,
                              uint64_t seed) {
  uint64_t l = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (l >= n_blocks) return;
  const uint64_t b = first + l;
  uint64_t d0 = draw(seed, 3 * b), d1 = draw(seed, 3 * b + 1), d2 = draw(seed, 3 * b + 2);
  uint8_t* p = dst + l * 17;
  p[0] = (uint8_t)(119u + (uint32_t)(((d0 >> 32) * 9ull) >> 32));
  for (int i = 0; i < 8; ++i) p[1 + i] = (uint8_t)(d1 >> (8 * i));
  for (int i = 0; i < 8; ++i) p[9 + i] = (uint8_t)(d2 >> (8 * i));
}

__device__ __forceinline__ float irwin_hall12(uint64_t a, uint64_t b, uint64_t c) {
  uint32_t s = 0;
  for (int i = 0; i < 4; ++i) s += (uint32_t)((a >> (16 * i)) & 0xFFFFu);
  for (int i = 0; i < 4; ++i) s += (uint32_t)((b >> (16 * i)) & 0xFFFFu);
  for (int i = 0; i < 4; ++i) s += (uint32_t)((c >> (16 * i)) & 0xFFFFu);
  return ((float)s - 393216.0f) * (1.0f / 65536.0f);
}

__global__ void k_synth_q4k(uint8_t* __restrict__ dst, uint64_t n_blocks, uint64_t first,
                            uint64_t seed) {
#pragma clang fp contract(off)
  uint64_t l = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (l >= n_blocks) return;
  const uint64_t b = first + l;
  uint64_t d[24];
  for (int i = 0; i < 24; ++i) d[i] = draw(seed, 24 * b + i);
  float zd = irwin_hall12(d[0], d[1], d[2]);
  float zm = irwin_hall12(d[3], d[4], d[5]);
  uint32_t hd = f2h_rne(fabsf(zd) * 0.01f);
  uint32_t hm = f2h_rne(fabsf(zm) * 0.005f);
  uint8_t* p = dst + l * 144;
  p[0] = (uint8_t)hd, p[1] = (uint8_t)(hd >> 8), p[2] = (uint8_t)hm, p[3] = (uint8_t)(hm >> 8);
  for (int i = 0; i < 140; ++i) p[4 + i] = (uint8_t)(d[6 + i / 8] >> (8 * (i % 8)));
}

hipError_t launch_synth(const Launch& K, int type, void* dst, uint64_t n_blocks, uint64_t seed) {
  hipStream_t s = K.s;
  const uint64_t per = 65535ull * 256ull;
  for (uint64_t off = 0; off < n_blocks; off += per) {
    uint64_t n = n_blocks - off < per ? n_blocks - off : per;
    dim3 grid((uint32_t)((n + 255) / 256));
    if (type == MR_GGML_MXFP4)
      hipLaunchKernelGGL(k_synth_mxfp4, grid, dim3(256), 0, s, (uint8_t*)dst + off * 17, n, off,
                         seed);
    else
      hipLaunchKernelGGL(k_synth_q4k, grid, dim3(256), 0, s, (uint8_t*)dst + off * 144, n, off,
                         seed);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mr
