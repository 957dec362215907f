// mr_fused.hip -- single-launch MXFP4 MoE decode layer for gfx950 (CDNA4).
//
// One kernel per layer and token does the whole of gpu_routed_moe_forward_metal
// (metal/mod.rs:1512-1677): router GEMV + top-k, gate+up dequant-matvec with
// bias and SwiGLU, down dequant-matvec with bias and the weighted combine.
//
// Matvecs run on v_mfma_scale_f32_16x16x128_f8f6f4 with the weights fed
// straight from their native 17-byte GGUF blocks: the 16 code bytes of a block
// are the A operand of one lane (32 K values), its e8m0 byte is that lane's A
// scale (GGUF kvalue*2^(e-128) == OCP e2m1*2^(e-127)). The activation vector is
// the B operand, split into kTerms e4m3 terms (B columns 0..kTerms-1, each with
// its own e8m0 scale per 32-element block); the column sum of D is the matvec.
// K inside a block is ordered so that MFMA k=2j <-> GGUF element j and
// k=2j+1 <-> element j+16 (byte j holds both), so no weight is repacked.
//
// Work is split into three groups of workgroups in one grid, producers first:
//   [0, R)        router: 4 experts per WG (one wave each) + the x split for
//                 a share of the 32-element blocks; each wave publishes its
//                 logit as a 64-bit (epoch+1, bits) word.
//   [R, R+NG)     gate/up: 32 rows of one routed slot, both projections;
//                 4 waves = 2 row tiles x 2 K halves. Epilogue: bias, SwiGLU,
//                 * routing weight, split into the down projection's B image.
//   [R+NG, grid)  down: 16 output rows; wave w takes slots w, w+4, ... Its down
//                 weights are loaded into registers before the gate/up results
//                 exist, so their HBM traffic overlaps the gate/up phase.
// Cross-workgroup data moves through agent-coherent (sc1) loads and stores,
// ordered by s_waitcnt; every wait is bounded (kSpinLimit) and a timeout sets
// an error word the host reads at mr_sync, so no launch can hang.
#include "mr_device.h"
#include "mr_internal.h"

#include <algorithm>

namespace mr {

constexpr int kTerms = 4;        // e4m3 terms of an activation split (B columns used)
constexpr int kGuSteps = 12;     // K steps (4 blocks each) per gate/up wave: H <= 3072
constexpr int kDnSteps = 23;     // K steps per down wave: I <= 2944
constexpr int kImgBytes = kTerms * 32;  // B image bytes per 32-element block
constexpr int kRouterVec = 12;  // float4 per lane of a router row: H <= 3072
constexpr int kSplitRounds = 12; // split blocks per half-wave of a router WG
constexpr int kImgRegs = 6;      // x image u64 words per thread: H <= 3072

// sync words (uint32 indices into Scratch::sync); tags start at byte 512
enum : int { SW_EPOCH = 0, SW_GU_DONE = 32, SW_WG_DONE = 64, SW_ERR = 96, SW_TAG0 = 128 };

struct FusedArgs {
  const uint8_t* gate;
  const uint8_t* up;
  const uint8_t* down;
  const uint64_t* gate_off;
  const uint64_t* up_off;
  const uint64_t* down_off;
  const float* gate_b;
  const float* up_b;
  const float* down_b;
  const float* router_w;
  const float* router_b;
  const float* mask;
  const float* x;
  float* y;
  uint32_t* sync;
  uint8_t* ximg;    // [nbH][kImgBytes] x split image
  uint32_t* xsc;    // [nbH] 4 e8m0 bytes (one per term)
  uint8_t* dimg;    // [k][nbI][kImgBytes] down B image
  uint32_t* dsc;    // [k][nbI]
  int H, I, E, k;
  uint32_t flags;
  int act;
  float alpha, limit;
  int R, NG, ND;
  uint32_t spin_limit;
  uint32_t lds_img_bytes;  // dynamic LDS: image bytes, then 4-byte scales
};

// ---- agent-coherent accesses (global_load/store ... sc1) ----------------------
__device__ __forceinline__ uint32_t ld_sc1(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_sc1(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_sc1(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// All vector memory operations of this wave issued so far have completed.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- DPP reductions ------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
#define DPP_XOR1 0xB1      // quad_perm [1,0,3,2]
#define DPP_XOR2 0x4E      // quad_perm [2,3,0,1]
#define DPP_HMIRROR 0x141  // row_half_mirror
#define DPP_MIRROR 0x140   // row_mirror

// max over each aligned group of 32 lanes, result in every lane of the group
__device__ __forceinline__ float max32(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HMIRROR>(v));
  v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
  return fmaxf(v, __shfl_xor(v, 16, 64));
}
// sum over each quad (lanes 4m..4m+3), result in every lane of the quad
__device__ __forceinline__ float sum4(float v) {
  v += dpp_f<DPP_XOR1>(v);
  return v + dpp_f<DPP_XOR2>(v);
}

// ---- e4m3 activation split ---------------------------------------------------------
// OCP e4m3 (bias 7) code of v, |v| < 256, round to nearest even; dec = its value.
__device__ __forceinline__ uint32_t e4m3_rne(float v, float& dec) {
  const float a = fabsf(v);
  uint32_t code;
  if (a < 0.015625f) {  // subnormal range: multiples of 2^-9
    const float q = rintf(a * 512.0f);
    code = (uint32_t)q;
    dec = q * (1.0f / 512.0f);
  } else {
    const uint32_t b = __float_as_uint(a);
    const uint32_t r = (b + 0x7FFFFu + ((b >> 20) & 1u)) & ~0xFFFFFu;
    dec = __uint_as_float(r);
    code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
  }
  if (v < 0.0f) {
    dec = -dec;
    code |= 0x80u;
  }
  return code;
}

// Split one 32-element block held one element per lane (32-lane group, lane p
// holds MFMA position p) into kTerms e4m3 terms. Term t uses the scale
// 2^(floor(log2(max|r_t|)) - 7), so max|r_t|/scale is in [128, 256) and each
// term adds 4 bits; the residual after the terms is below 2^-16 of the block max.
// Returns the 4 codes packed (term t in byte t) and the 4 scale bytes likewise.
__device__ __forceinline__ void split32(float v, uint32_t& codes, uint32_t& scales) {
  float r = v;
  codes = 0u, scales = 0u;
#pragma unroll
  for (int t = 0; t < kTerms; ++t) {
    const float m = max32(fabsf(r));
    const int e = (int)((__float_as_uint(m) >> 23) & 0xFFu) - 127;  // m == 0 -> e = -127
    const int sb = e + 120;  // e8m0 byte of 2^(e-7)
    uint32_t code = 0u;
    float dec = 0.0f;
    if (sb > 0 && m > 0.0f) {
      code = e4m3_rne(r * __uint_as_float((uint32_t)(254 - sb) << 23), dec);  // r * 2^-(e-7)
      dec = dec * __uint_as_float((uint32_t)sb << 23);                        // * 2^(e-7)
    }
    r -= dec;
    codes |= code << (8 * t);
    scales |= (uint32_t)(sb > 0 && m > 0.0f ? sb : 0) << (8 * t);
  }
}

// Gather byte t of `codes` from the 4 lanes of each quad into one dword (in the
// quad's first lane): bytes of positions 4m..4m+3 of term t.
__device__ __forceinline__ uint32_t quad_pack(uint32_t codes, int t) {
  uint32_t b = (codes >> (8 * t)) & 0xFFu;
  const int lane = threadIdx.x & 63;
  uint32_t b1 = __shfl(b, lane + 1, 64), b2 = __shfl(b, lane + 2, 64), b3 = __shfl(b, lane + 3, 64);
  return b | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Split the 32-element block at lanes [32h, 32h+32) of the wave and store its
// image with sc1 dword stores: img[t*32 + p] = code of position p, term t.
__device__ __forceinline__ void split_store(float v, uint8_t* img, uint32_t* sc, bool active) {
  uint32_t codes, scales;
  split32(v, codes, scales);
  const int p = threadIdx.x & 31;
#pragma unroll
  for (int t = 0; t < kTerms; ++t) {
    const uint32_t dw = quad_pack(codes, t);
    if (active && (p & 3) == 0) st_sc1(reinterpret_cast<uint32_t*>(img + t * 32 + p), dw);
  }
  if (active && p == 0) st_sc1(sc, scales);
}

// ---- operands ------------------------------------------------------------------
// B operand of lane (col i, group g) for K step st from a B image in LDS:
// data bytes 0..15 = K [16g, 16g+16) = block 4st+g/2, half g&1; bytes 16..31 =
// K [64+16g, ...) = block 4st+2+g/2; scale = block 4st+g (MFMA scale indexing).
__device__ __forceinline__ void load_b(const uint8_t* img, const uint32_t* sc, int st, int nb,
                                       int i, int g, i32x8& B, int& sb) {
  B = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
  sb = 127;
  if (i < kTerms) {
    const int b0 = 4 * st + (g >> 1), b1 = b0 + 2, off = i * 32 + 16 * (g & 1);
    if (b0 < nb) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(img + (size_t)b0 * kImgBytes + off);
      B[0] = v[0], B[1] = v[1], B[2] = v[2], B[3] = v[3];
    }
    if (b1 < nb) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(img + (size_t)b1 * kImgBytes + off);
      B[4] = v[0], B[5] = v[1], B[6] = v[2], B[7] = v[3];
    }
    const int bs = 4 * st + g;
    if (bs < nb) sb = (int)((sc[bs] >> (8 * i)) & 0xFFu);
  }
}

__device__ __forceinline__ f32x4 mfma_fp4(const uint32_t a[4], uint32_t sa, const i32x8& B, int sb,
                                          f32x4 acc) {
  const i32x8 A = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 4, 0, 0, (int)sa, 0, sb);
}

// ---- routing ---------------------------------------------------------------------
// Wave 0 of a consumer workgroup: wait until every expert's logit of this
// launch is published, then select the top-k (same rule as k_topk: largest
// first, ties to the lower index) and write slot -> (expert, weight) to LDS.
__device__ bool route_wave(const FusedArgs& a, uint32_t epoch, int* sel_i, float* sel_w) {
  const int lane = threadIdx.x & 63;
  const unsigned long long* tags = reinterpret_cast<const unsigned long long*>(a.sync + SW_TAG0);
  const uint32_t want = epoch + 1u;
  float v[8];
  bool live[8];
  uint32_t it = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      live[j] = e < a.E;
      v[j] = 0.f;
      if (live[j]) {
        const unsigned long long t = ld_sc1(tags + e);
        ok = ok && (uint32_t)(t >> 32) == want;
        v[j] = __uint_as_float((uint32_t)t);
      }
    }
    if (__all(ok)) break;
    if (++it > a.spin_limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  const bool softmax_after = (a.flags & MR_ROUTE_SOFTMAX_AFTER_TOPK) != 0u;
  if (!softmax_after) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j]) m = fmaxf(m, v[j]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j]) v[j] = __expf(v[j] - m), s += v[j];
    s = wave_sum(s);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j]) v[j] = v[j] / s;
  }
  float selv = 0.f;
  for (int r = 0; r < a.k; ++r) {
    float bv = 0.f;
    int bi = -1;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j] && (bi < 0 || v[j] > bv)) bv = v[j], bi = lane + 64 * j;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) bv = ov, bi = oi;
    }
    if (bi >= 0 && (bi & 63) == lane) live[bi >> 6] = false;
    if (lane == r) selv = bv;
    if (lane == 0) sel_i[r] = bi;
  }
  // weights: lanes 0..k-1 hold the selected values, in selection order
  const bool in = lane < a.k;
  if (softmax_after) {
    float m = wave_max(in ? selv : -INFINITY);
    float ex = in ? __expf(selv - m) : 0.f;
    float s = wave_sum(ex);
    if (in) sel_w[lane] = ex / s;
  } else if (a.flags & MR_ROUTE_NORM_TOPK) {
    float s = wave_sum(in ? selv : 0.f);
    if (in) sel_w[lane] = selv / s;
  } else if (in) {
    sel_w[lane] = selv;
  }
  return true;
}

__device__ __forceinline__ void fail(const FusedArgs& a) { st_sc1(a.sync + SW_ERR, 1u); }

// A operands of one 16-row tile of a down matrix, all K steps.
__device__ __forceinline__ void load_down_rows(const uint8_t* D, int S, int nbI, int g,
                                               uint32_t (&ad)[kDnSteps][4], uint32_t (&sd)[kDnSteps]) {
#pragma unroll
  for (int j = 0; j < kDnSteps; ++j) {
    const int c = 4 * j + g;
    if (j < S && c < nbI) {
      mx_load_block(D + (size_t)c * 17, sd[j], ad[j]);
    } else {
      sd[j] = 127u;
      ad[j][0] = ad[j][1] = ad[j][2] = ad[j][3] = 0u;
    }
  }
}

// ---- the kernel ------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_fused_mxfp4(FusedArgs a) {
  extern __shared__ __align__(16) uint8_t lds_dyn[];  // x image (gate/up) or down images + scales
  uint8_t* lds_img = lds_dyn;
  uint32_t* lds_sc = reinterpret_cast<uint32_t*>(lds_dyn + a.lds_img_bytes);
  __shared__ float lds_part[2 * 2 * 2 * 16];
  __shared__ float lds_act[32];
  __shared__ int sel_i[16];
  __shared__ float sel_w[16];
  __shared__ int ok_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int bid = blockIdx.x;
  const uint32_t epoch = ld_sc1(a.sync + SW_EPOCH);
  const int nbH = a.H >> 5, nbI = a.I >> 5;

  if (bid < a.R) {
    // ------------------------------------------------------------- router
    // Issue every load first: this wave's router row and x for the dot, and
    // the x elements of this workgroup's share of the split blocks.
    const int e = bid * 4 + wave;
    const bool has_e = e < a.E;
    const float* wrow = a.router_w + (size_t)(has_e ? e : 0) * a.H;
    f32x4 xr[kRouterVec], wr[kRouterVec];
#pragma unroll
    for (int j = 0; j < kRouterVec; ++j) {
      const int c = (lane + 64 * j) * 4;
      if (has_e && c < a.H) {
        xr[j] = *reinterpret_cast<const f32x4*>(a.x + c);
        wr[j] = *reinterpret_cast<const f32x4*>(wrow + c);
      } else {
        xr[j] = f32x4{0.f, 0.f, 0.f, 0.f}, wr[j] = xr[j];
      }
    }
    const int bpw = (nbH + a.R - 1) / a.R;
    const int half = lane >> 5, p = lane & 31;
    const int elem = (p >> 1) + 16 * (p & 1);  // MFMA position p <-> GGUF element
    float xs[kSplitRounds];
#pragma unroll
    for (int j = 0; j < kSplitRounds; ++j) {
      const int jb = (wave * 2 + half) + 8 * j, b = bid * bpw + jb;
      xs[j] = (jb < bpw && b < nbH) ? a.x[b * 32 + elem] : 0.f;
    }
    // x split of the share; stored before this workgroup publishes any logit,
    // so a consumer that sees all logits also sees the whole x image
#pragma unroll
    for (int j = 0; j < kSplitRounds; ++j) {
      const int jb0 = wave * 2 + 8 * j;  // first half-wave's block of this round
      if (jb0 < bpw) {
        const int jb = jb0 + half, b = bid * bpw + jb;
        const bool act = jb < bpw && b < nbH;
        split_store(xs[j], a.ximg + (size_t)(act ? b : 0) * kImgBytes, a.xsc + (act ? b : 0), act);
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kRouterVec; ++j) {
      acc = __builtin_fmaf(xr[j].x, wr[j].x, acc);
      acc = __builtin_fmaf(xr[j].y, wr[j].y, acc);
      acc = __builtin_fmaf(xr[j].z, wr[j].z, acc);
      acc = __builtin_fmaf(xr[j].w, wr[j].w, acc);
    }
    acc = wave_sum(acc);
    vm_drain();       // this wave's split stores are complete ...
    __syncthreads();  // ... and so are those of the other waves
    if (has_e && lane == 0) {
      if (a.router_b) acc = acc + a.router_b[e];
      if (a.mask) acc = acc + a.mask[e];
      st_sc1(reinterpret_cast<unsigned long long*>(a.sync + SW_TAG0) + e,
             ((unsigned long long)(epoch + 1u) << 32) | __float_as_uint(acc));
    }
  } else if (bid < a.R + a.NG) {
    // ------------------------------------------------------------- gate/up
    const int gid = bid - a.R;
    const int nrp = a.I >> 5;
    const int slot = gid / nrp, pair = gid % nrp;
    if (tid == 0) ok_flag = 1;
    if (wave == 0 && !route_wave(a, epoch, sel_i, sel_w)) {
      if (lane == 0) ok_flag = 0, fail(a);
    }
    __syncthreads();
    if (ok_flag) {
      const int e = sel_i[slot];
      const float wsl = sel_w[slot];
      // x split image (complete once every logit is published): issue its
      // loads first, then the weight loads, then move the image to LDS
      const int n8 = nbH * kImgBytes / 8;
      const unsigned long long* xsrc = reinterpret_cast<const unsigned long long*>(a.ximg);
      unsigned long long ximg[kImgRegs];
      uint32_t xscr = 0u;
#pragma unroll
      for (int j = 0; j < kImgRegs; ++j) {
        const int idx = tid + 256 * j;
        ximg[j] = idx < n8 ? ld_sc1(xsrc + idx) : 0ull;
      }
      if (tid < nbH) xscr = ld_sc1(a.xsc + tid);
      const int tile = wave & 1, kh = wave >> 1;
      const int S = (nbH + 3) >> 2, S0 = (S + 1) >> 1;
      const int st0 = kh * S0, nst = min(S0, S - st0);
      const int row = pair * 32 + tile * 16 + i;
      const uint64_t rb = (uint64_t)nbH * 17;
      const uint8_t* G = a.gate + a.gate_off[e] + (uint64_t)row * rb;
      const uint8_t* U = a.up + a.up_off[e] + (uint64_t)row * rb;
      uint32_t ag[kGuSteps][4], au[kGuSteps][4], sg[kGuSteps], su[kGuSteps];
#pragma unroll
      for (int j = 0; j < kGuSteps; ++j) {
        const int c = 4 * (st0 + j) + g;
        if (j < nst && c < nbH) {
          mx_load_block(G + (size_t)c * 17, sg[j], ag[j]);
          mx_load_block(U + (size_t)c * 17, su[j], au[j]);
        } else {
          sg[j] = su[j] = 127u;
          ag[j][0] = ag[j][1] = ag[j][2] = ag[j][3] = 0u;
          au[j][0] = au[j][1] = au[j][2] = au[j][3] = 0u;
        }
      }
      {
        unsigned long long* dst = reinterpret_cast<unsigned long long*>(lds_img);
#pragma unroll
        for (int j = 0; j < kImgRegs; ++j) {
          const int idx = tid + 256 * j;
          if (idx < n8) dst[idx] = ximg[j];
        }
        if (tid < nbH) lds_sc[tid] = xscr;
      }
      __syncthreads();  // x image in LDS
      f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kGuSteps; ++j) {
        if (j < nst) {
          i32x8 B;
          int sb;
          load_b(lds_img, lds_sc, st0 + j, nbH, i, g, B, sb);
          dg = mfma_fp4(ag[j], sg[j], B, sb, dg);
          du = mfma_fp4(au[j], su[j], B, sb, du);
        }
      }
      // column sum over the kTerms columns (= quad 0 of each 16-lane row)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gs = sum4(dg[r]), us = sum4(du[r]);
        if (i == 0) {
          lds_part[((kh * 2 + tile) * 2 + 0) * 16 + 4 * g + r] = gs;
          lds_part[((kh * 2 + tile) * 2 + 1) * 16 + 4 * g + r] = us;
        }
      }
      __syncthreads();
      if (wave == 0) {
        // lanes 0..31: rows pair*32 + lane; bias, SwiGLU, routing weight
        if (lane < 32) {
          const int t2 = lane >> 4, r16 = lane & 15;
          float gv = lds_part[((0 * 2 + t2) * 2 + 0) * 16 + r16] + lds_part[((1 * 2 + t2) * 2 + 0) * 16 + r16];
          float uv = lds_part[((0 * 2 + t2) * 2 + 1) * 16 + r16] + lds_part[((1 * 2 + t2) * 2 + 1) * 16 + r16];
          const int rr = pair * 32 + lane;
          if (a.gate_b) gv = gv + a.gate_b[(size_t)e * a.I + rr];
          if (a.up_b) uv = uv + a.up_b[(size_t)e * a.I + rr];
          const float h = a.act == MR_ACT_SWIGLU_OAI ? swiglu_oai(gv, uv, a.alpha, a.limit) : silu_mul(gv, uv);
          lds_act[lane] = h * wsl;
        }
        __builtin_amdgcn_wave_barrier();
        const int p = lane & 31;
        const float v = lds_act[(p >> 1) + 16 * (p & 1)];
        const size_t blk = (size_t)slot * nbI + pair;
        split_store(v, a.dimg + blk * kImgBytes, a.dsc + blk, lane < 32);
        vm_drain();
        if (lane == 0) add_sc1(a.sync + SW_GU_DONE, 1u);
      }
    }
  } else {
    // ------------------------------------------------------------- down
    const int q = bid - a.R - a.NG;
    if (tid == 0) ok_flag = 1;
    if (wave == 0 && !route_wave(a, epoch, sel_i, sel_w)) {
      if (lane == 0) ok_flag = 0, fail(a);
    }
    __syncthreads();
    if (ok_flag) {
      const int S = (nbI + 3) >> 2;
      const int row = q * 16 + i;
      const uint64_t rb = (uint64_t)nbI * 17;
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
      // prefetch this wave's first slot's down weights (independent of gate/up)
      uint32_t ad[kDnSteps][4], sd[kDnSteps];
      int slot = wave;
      if (slot < a.k) load_down_rows(a.down + a.down_off[sel_i[slot]] + (uint64_t)row * rb, S, nbI, g, ad, sd);
      // wait for every gate/up workgroup of this launch
      if (tid == 0) {
        uint32_t it = 0;
        while (ld_sc1(a.sync + SW_GU_DONE) < (uint32_t)a.NG) {
          if (++it > a.spin_limit) {
            ok_flag = 0, fail(a);
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      }
      __syncthreads();
      if (ok_flag) {
        // all k down B images -> LDS
        const int n8 = a.k * nbI * kImgBytes / 8;
        const unsigned long long* src = reinterpret_cast<const unsigned long long*>(a.dimg);
        unsigned long long* dst = reinterpret_cast<unsigned long long*>(lds_img);
        for (int j = tid; j < n8; j += 256) dst[j] = ld_sc1(src + j);
        for (int j = tid; j < a.k * nbI; j += 256) lds_sc[j] = ld_sc1(a.dsc + j);
        __syncthreads();
        for (; slot < a.k; slot += 4) {
          if (slot != wave) load_down_rows(a.down + a.down_off[sel_i[slot]] + (uint64_t)row * rb, S, nbI, g, ad, sd);
          const uint8_t* img = lds_img + (size_t)slot * nbI * kImgBytes;
          const uint32_t* sc = lds_sc + slot * nbI;
#pragma unroll
          for (int j = 0; j < kDnSteps; ++j) {
            if (j < S) {
              i32x8 B;
              int sb;
              load_b(img, sc, j, nbI, i, g, B, sb);
              d = mfma_fp4(ad[j], sd[j], B, sb, d);
            }
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float s = sum4(d[r]);
          if (i == 0) lds_part[wave * 16 + 4 * g + r] = s;
        }
        __syncthreads();
        if (tid < 16) {
          const int rr = q * 16 + tid;
          float yv = ((lds_part[tid] + lds_part[16 + tid]) + lds_part[32 + tid]) + lds_part[48 + tid];
          if (a.down_b)
            for (int s = 0; s < a.k; ++s)
              yv = yv + sel_w[s] * a.down_b[(size_t)sel_i[s] * a.H + rr];
          if (rr < a.H) a.y[rr] = yv;
        }
      }
    }
  }
  // ----------------------------------------------------------------- exit
  __syncthreads();
  if (tid == 0) {
    vm_drain();
    const uint32_t total = (uint32_t)(a.R + a.NG + a.ND);
    if (add_sc1(a.sync + SW_WG_DONE, 1u) == total - 1u) {
      st_sc1(a.sync + SW_GU_DONE, 0u);
      st_sc1(a.sync + SW_WG_DONE, 0u);
      st_sc1(a.sync + SW_EPOCH, epoch + 1u);
    }
  }
}

// Shapes the fused kernel runs; others take the VALU path.
bool fused_supported(const mr_layer& L) {
  if (L.type != MR_GGML_MXFP4 || L.d.sh_gate) return false;
  const int nbH = L.H / 32, nbI = L.I / 32;
  if ((nbH + 3) / 4 > 2 * kGuSteps) return false;
  if ((nbI + 3) / 4 > kDnSteps) return false;
  if ((size_t)L.d.top_k * nbI * (kImgBytes + 4) > 64 * 1024) return false;
  if ((size_t)nbH * kImgBytes / 8 > (size_t)256 * kImgRegs) return false;
  if (L.I % 32 != 0 || L.H % 16 != 0) return false;
  return true;
}

uint64_t fused_scratch_bytes(uint64_t H, uint64_t I, uint64_t k) {
  return (H / 32) * (kImgBytes + 4) + k * (I / 32) * (kImgBytes + 4) + 1024;
}

hipError_t launch_fused(const Launch& K, const mr_layer& L, const float* x, float* y,
                        uint32_t* sync, uint8_t* img_base, uint32_t spin_limit) {
  FusedArgs a{};
  a.gate = L.d.gate->base, a.up = L.d.up->base, a.down = L.d.down->base;
  a.gate_off = L.d.gate->d_offsets, a.up_off = L.d.up->d_offsets, a.down_off = L.d.down->d_offsets;
  a.gate_b = L.d.gate_bias, a.up_b = L.d.up_bias, a.down_b = L.d.down_bias;
  a.router_w = L.d.router_w, a.router_b = L.d.router_b, a.mask = L.d.dummy_mask;
  a.x = x, a.y = y, a.sync = sync;
  const uint64_t nbH = L.H / 32, nbI = L.I / 32;
  uint8_t* p = img_base;
  a.ximg = p, p += nbH * kImgBytes;
  a.xsc = reinterpret_cast<uint32_t*>(p), p += ((nbH * 4 + 255) / 256) * 256;
  a.dimg = p, p += (uint64_t)L.d.top_k * nbI * kImgBytes;
  a.dsc = reinterpret_cast<uint32_t*>(p);
  a.H = (int)L.H, a.I = (int)L.I, a.E = (int)L.E, a.k = (int)L.d.top_k;
  a.flags = L.d.route_flags, a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  a.R = (int)((L.E + 3) / 4);
  a.NG = (int)(L.d.top_k * (L.I / 32));
  a.ND = (int)((L.H + 15) / 16);
  a.spin_limit = spin_limit;
  const uint64_t img = std::max<uint64_t>(nbH, (uint64_t)L.d.top_k * nbI) * kImgBytes;
  const uint64_t nsc = std::max<uint64_t>(nbH, (uint64_t)L.d.top_k * nbI);
  a.lds_img_bytes = (uint32_t)img;
  const size_t lds = img + nsc * 4;
  ProfScope ps(K, "fused_layer");
  hipLaunchKernelGGL(k_fused_mxfp4, dim3(a.R + a.NG + a.ND), dim3(256), lds, K.s, a);
  return hipGetLastError();
}

}  // namespace mr
