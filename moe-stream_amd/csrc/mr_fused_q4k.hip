// mr_fused_q4k.hip -- single-launch Q4_K MoE decode layer for gfx950 (CDNA4).
//
// The Q4_K counterpart of k_fused_mxfp4: one kernel per layer and token does
// the router GEMV (+ the shared-expert gate), top-k routing, gate+up
// dequant-matvec with SwiGLU/SiLU, down dequant-matvec with the weighted
// combine in ascending expert order, and the sigmoid-gated shared expert
// (layer.rs:1012-1027, 1818-1953, 2346-2403; per-expert QMatMul path
// layer.rs:2099-2147).
//
// Dot products on the int8 MFMA (v_mfma_i32_16x16x64_i8). The activation (x for gate/up;
// for down, h = the activation times the routing weight) is split per 16-element group G
// into two int8 terms, v = s0*t0 + (s0/256)*t1 with s0 = max|v|/127, so
// |v - s0*t0 - s0*t1/256| <= s0/256 (about 3e-5 of the group max).
//
// A work unit is 16 rows x one 256-element super-block. A super-block row is 144 bytes: a
// header chunk (d, dmin, 12 scale bytes) and 8 quant chunks; the low nibbles of quant chunk
// p are elements 16hf..16hf+15 of sub-block 2jj, its high nibbles the same elements of
// sub-block 2jj+1 (jj = (p-1)/2, hf = (p-1)%2; dequantize_q4k, dequant.rs:218-262). Lane
// (i, g) = (lane & 15, lane >> 4) loads row i's header and its quant chunks 1+g and 5+g;
// a chunk is the B operand (16 int8 of weight row i) of two MFMAs after one AND (low
// nibbles) or a shift and an AND (high nibbles). The A operand of MFMA (L, hi) carries in
// row m = 2*Gl + t term t of group 8L + Gl of the super-block, but only in lane group g
// whose chunk holds that group (Gl = 4(g>>1) + 2hi + (g&1)); the other lanes read a zero
// block. The int32 result D_L is then, per (group, term) row and weight row, the exact sum
// of q * t over the group. Lane (i, g) of D_L holds rows 4g..4g+3: both groups and both
// terms of sub-block 4L+g of weight row i, so its epilogue needs one (d*sc, dmin*m) pair:
//   sum_e w_e x_e = (d*sc) * sum_G s0_G/256 * (256*A0_G + A1_G) - (dmin*m) * sum_G X_G,
// with (d*sc, dmin*m) rounded as dequantize_q4k rounds them and X_G the group's f32 sum;
// |256*A0 + A1| < 2^24, so its conversion to float is exact.
//
// Roles (grid order; all workgroups resident, see fused_q4k_supported):
//   [0, R)       router: one logit per wave (E experts, then x . w_gi of the
//                shared expert when there is one).
//   [R, R+ND)    down: 16 output rows; wave w takes slots w, w+4, ... (routed slots, then
//                the shared expert). Its first units are loaded before the gate/up results
//                exist.
//   [R+ND, grid) gate/up: 16 rows of one slot; waves = (gate, up) x 2 halves of the
//                super-blocks. Epilogue: bias, activation, x routing weight (sigmoid
//                gate for the shared expert), int8 split of the 16 results (one group)
//                into the down input image.
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace mr {

constexpr int kQ4RouterVec = 8;   // float4s per lane per router pass (two passes: H <= 4096)
constexpr int kQ4RingG = 4;       // gate/up units loaded ahead (two rounds: H/512 <= 8)
constexpr int kQ4RingD = 6;       // down units loaded ahead (two rounds: ceil(ktot/4) * I/256 <= 12)
constexpr int kQ4MaxH = 4096, kQ4MaxI = 2048, kQ4MaxKI = 12288, kQ4MaxSlots = 17;
constexpr int kQ4MaxUnitsD = 2 * kQ4RingD;          // down units of one wave
#ifndef MR_Q4_PRESPLIT
#define MR_Q4_PRESPLIT 6  // all: C3 15.62 -> 15.31 us, C4 16.73 -> 16.38 us (2 and 4 gain less)
#endif
constexpr int kQ4PreSplit = MR_Q4_PRESPLIT;         // down units whose B operands are split before the wait
static_assert(kQ4PreSplit >= 0 && kQ4PreSplit <= kQ4RingD, "at most every ring unit");

// LDS carve-up (bytes): activation image [groups][2 terms][16 int8] (gate/up: x, H/16 groups;
// down: h of every slot, ktot * I/16 groups), group scales [groups] (s0/256, sum), a zero
// block. 1 KiB after the image and after the scales takes the direct-load overrun.
constexpr int kQImg = 0;
constexpr int kQSc = kQImg + kQ4MaxKI * 2 + 1024;
constexpr int kQZero = kQSc + kQ4MaxKI / 16 * 8 + 1024;
constexpr int kQ4Smem = kQZero + 16;
static_assert(kQ4MaxH <= kQ4MaxKI && 4 * 1024 <= kQSc, "the x image and the router prefetch fit");
static_assert(kQ4MaxKI / 16 <= 0xFFFF && kQ4MaxSlots <= 32, "a down unit's group and slot fit its table word");

struct Q4Args {
  ExpertLoc gate, up, down;
  const uint8_t* sh_gate;  // shared expert matrices (one expert) or null
  const uint8_t* sh_up;
  const uint8_t* sh_down;
  const float* gate_b;
  const float* up_b;
  const float* down_b;
  const float* router_w;
  const float* router_b;
  const float* mask;
  const float* sh_gate_inp;
  const float* x;
  float* y;
  float* logits_out;  // router logits [E] of this launch (the layer's logits output) or null
  uint32_t* fs;     // this layer's sync block
  uint32_t* err;    // context error word
  uint32_t* himg;   // [ktot][I/16][8 words] int8 terms of the down input
  float* hsc;       // [ktot][I/16][2] (s0/256, group sum)
  int H, I, E, k, ktot, has_sh;
  uint32_t flags;
  int act;
  float alpha, limit;
  int R, ND, NG;
  int gt;  // row tiles per gate/up workgroup
  WaitBound wb;  // time limit of the cross-workgroup waits
  PrefetchRows pf;  // the next layer's router rows (router workgroups read them)
  NormResid nr;     // fused RMSNorm of x and residual added to y (off: nr.w == nullptr)
  unsigned long long* trace;
  int nsh;  // slots of the shared expert: Ish / I (slot k + j: its rows and columns j*I .. j*I + I - 1)
};

// ---- int8 two-term split ------------------------------------------------------------------
// s0 = m/127 (m = max|v| of the group); t0 = rn(v/s0), t1 = rn((v - s0*t0) * 256/s0), both
// clamped to +-127 (|v - s0*t0| <= s0/2 can round t1 to 128; the clamp costs at most s0/256).
__device__ __forceinline__ void split_i8(float v, float m, int& t0, int& t1, float& s0) {
  if (!(m > 0.f)) {
    t0 = t1 = 0, s0 = 0.f;
    return;
  }
  s0 = m / 127.f;
  t0 = (int)fminf(fmaxf(rintf(v / s0), -127.f), 127.f);
  const float r = fmaf(-(float)t0, s0, v);
  t1 = (int)fminf(fmaxf(rintf(r / s0 * 256.f), -127.f), 127.f);
}

// ---- work units: 16 rows x one super-block ----------------------------------------------
// Per-lane constants. Lane (i, g): B operand = weight row i, chunks 1+g / 5+g; A operand row
// m = i (group Gl = i >> 1, term i & 1), live in MFMA (., hi) when Gl = 4(g>>1) + 2hi + (g&1).
struct UnitLane {
  uint32_t o_hd, o_w0, o_w1;  // byte offsets of the lane's header and quant chunks in a unit
  uint32_t nz[2];             // 1: the lane's A operand is live in MFMA (., hi)
  uint32_t ab[2];             // live: 16 * i (the unit's image offset is added); else the zero block
  uint32_t sc_off;            // 16 * g: the lane's two group scales within a super-block half
  uint32_t sh8;               // 8 * g: the lane's byte in a header scale word
};
__device__ __forceinline__ UnitLane unit_lane(uint32_t rb) {
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  UnitLane u;
  u.o_hd = (uint32_t)i * rb;
  u.o_w0 = u.o_hd + 16u * (uint32_t)(1 + g);
  u.o_w1 = u.o_hd + 16u * (uint32_t)(5 + g);
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const bool live = (i >> 1) == 4 * (g >> 1) + 2 * hi + (g & 1);
    u.nz[hi] = live ? 1u : 0u;
    u.ab[hi] = live ? 16u * (uint32_t)i : (uint32_t)kQZero;
  }
  u.sc_off = 16u * (uint32_t)g;
  u.sh8 = 8u * (uint32_t)g;
  return u;
}

// d: extra byte offset of the lane's row (rows of another stride than the UnitLane's)
__device__ __forceinline__ void unit_load(const uint8_t* p, const UnitLane& ul, uint4& hd, uint4& w0, uint4& w1,
                                          uint32_t d = 0u) {
  hd = *reinterpret_cast<const uint4*>(p + (ul.o_hd + d));
  w0 = *reinterpret_cast<const uint4*>(p + (ul.o_w0 + d));
  w1 = *reinterpret_cast<const uint4*>(p + (ul.o_w1 + d));
}
// No extra row offset: the units of a ring share the UnitLane's row stride.
struct NoRowDelta {
  __device__ uint32_t operator()(int) const { return 0u; }
};

// The LDS operands of one unit against the activation groups gb .. gb+15 (image and scales in
// LDS at smem): the A operands of its four MFMAs and the lane's two group-scale pairs.
struct UnitOps {
  i32x4 av[2][2];
  float4 sc[2];
};
__device__ __forceinline__ UnitOps unit_ops(const UnitLane& ul, uint32_t gb, const uint8_t* smem) {
  const uint32_t uofs = (uint32_t)kQImg + gb * 32u;
  UnitOps o;
#pragma unroll
  for (int L = 0; L < 2; ++L)
#pragma unroll
    for (int hi = 0; hi < 2; ++hi)
      o.av[L][hi] = *reinterpret_cast<const i32x4*>(smem + __umul24(ul.nz[hi], uofs + 256u * (uint32_t)L) + ul.ab[hi]);
#pragma unroll
  for (int L = 0; L < 2; ++L)
    o.sc[L] = *reinterpret_cast<const float4*>(smem + kQSc + gb * 8u + 64u * (uint32_t)L + ul.sc_off);
  return o;
}

// The weight side of one unit: the B operands of its four MFMAs (nibbles as int8) and the
// lane's (d*sc, dmin*m) of sub-blocks g (L = 0) and 4 + g (L = 1).
struct UnitPrep {
  i32x4 b[2][2];
  float dsc[2], dm[2];
};
// The lane's (d*sc, dmin*m) of sub-blocks g (L = 0) and 4 + g (L = 1) from the unit's header.
struct UnitScales {
  float dsc[2], dm[2];
};
__device__ __forceinline__ UnitScales unit_scales(const uint4& hd, const UnitLane& ul) {
  // get_scale_min_k4 (dequant.rs:199-209): j < 4 takes the low 6 bits of bytes j, j+4; j >= 4
  // the nibbles of byte j+4 and the top 2 bits of bytes j-4, j
  const float d = __half2float(__ushort_as_half((unsigned short)(hd.x & 0xFFFFu)));
  const float dmin = __half2float(__ushort_as_half((unsigned short)(hd.x >> 16)));
  const uint32_t s = ul.sh8;
  const uint32_t sc0 = __builtin_amdgcn_ubfe(hd.y, s, 6u), m0 = __builtin_amdgcn_ubfe(hd.z, s, 6u);
  const uint32_t sc1 = __builtin_amdgcn_ubfe(hd.w, s, 4u) | (__builtin_amdgcn_ubfe(hd.y, s + 6u, 2u) << 4);
  const uint32_t m1 = __builtin_amdgcn_ubfe(hd.w, s + 4u, 4u) | (__builtin_amdgcn_ubfe(hd.z, s + 6u, 2u) << 4);
  UnitScales u;
  u.dsc[0] = __fmul_rn(d, (float)sc0), u.dsc[1] = __fmul_rn(d, (float)sc1);
  u.dm[0] = __fmul_rn(dmin, (float)m0), u.dm[1] = __fmul_rn(dmin, (float)m1);
  return u;
}
__device__ __forceinline__ UnitPrep unit_prep(const UnitScales& u, const uint4& w0, const uint4& w1) {
  UnitPrep p;
#pragma unroll
  for (int L = 0; L < 2; ++L) {
    const uint4 w = L ? w1 : w0;
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const uint32_t s = hi ? 4u : 0u;
      p.b[L][hi] = i32x4{(int)((w.x >> s) & 0x0F0F0F0Fu), (int)((w.y >> s) & 0x0F0F0F0Fu),
                         (int)((w.z >> s) & 0x0F0F0F0Fu), (int)((w.w >> s) & 0x0F0F0F0Fu)};
    }
    p.dsc[L] = u.dsc[L], p.dm[L] = u.dm[L];
  }
  return p;
}
__device__ __forceinline__ UnitPrep unit_prep(const uint4& hd, const uint4& w0, const uint4& w1, const UnitLane& ul) {
  return unit_prep(unit_scales(hd, ul), w0, w1);
}

// One unit: this lane's share of row i's dot product (lanes i, i+16, i+32, i+48 hold the four
// shares).
__device__ __forceinline__ float unit_dot(const UnitPrep& p, const UnitOps& o) {
  float r = 0.f;
#pragma unroll
  for (int L = 0; L < 2; ++L) {
    i32x4 D = {0, 0, 0, 0};
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) D = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.av[L][hi], p.b[L][hi], D, 0, 0, 0);
    const float v = fmaf(o.sc[L].z, (float)(D[2] * 256 + D[3]), o.sc[L].x * (float)(D[0] * 256 + D[1]));
    r = fmaf(p.dsc[L], v, r);
    r = fmaf(-p.dm[L], o.sc[L].y + o.sc[L].w, r);
  }
  return r;
}
__device__ __forceinline__ float unit_dot(const uint4& hd, const uint4& w0, const uint4& w1, const UnitLane& ul,
                                          const UnitOps& o) {
  return unit_dot(unit_prep(hd, w0, w1, ul), o);
}
__device__ __forceinline__ float unit_dot(const uint4& hd, const uint4& w0, const uint4& w1, const UnitLane& ul,
                                          uint32_t gb, const uint8_t* smem) {
  return unit_dot(unit_prep(hd, w0, w1, ul), unit_ops(ul, gb, smem));
}

// The four shares of a row summed: every lane holds its row i's total.
__device__ __forceinline__ float row_total(float v) {
  return add_xor32(add_xor16(v));
}

// A wave's units 0..nu-1 (nu >= 1): RING of them are loaded by units_issue (all RING loads are
// issued, units past nu repeat the last one, so the waits before each unit's use are exact);
// units_process runs them in order. STREAM (a separate kernel instantiation, for shapes with
// more units than RING): once unit u is done, unit u + RING (or again the last unit) is loaded
// into its registers, every load again unconditional. base(u): the unit's 144-byte
// super-block in row 0.
template <int RING>
struct UnitRegs {
  uint4 hd[RING], w0[RING], w1[RING];
};
template <int RING, class BaseFn, class DFn = NoRowDelta>
__device__ __forceinline__ void units_issue(UnitRegs<RING>& R, int nu, BaseFn base, const UnitLane& ul,
                                            DFn dfn = DFn{}) {
#pragma unroll
  for (int r = 0; r < RING; ++r) {
    const int u = min(r, nu - 1);
    unit_load(base(u), ul, R.hd[r], R.w0[r], R.w1[r], dfn(u));
  }
}
template <bool STREAM, int RING, class BaseFn, class Proc, class DFn = NoRowDelta>
__device__ __forceinline__ void units_process(UnitRegs<RING>& R, int nu, BaseFn base, const UnitLane& ul, Proc proc,
                                              DFn dfn = DFn{}) {
  if (!STREAM) {
#pragma unroll
    for (int r = 0; r < RING; ++r)
      if (r < nu) proc(r, R.hd[r], R.w0[r], R.w1[r]);
  } else {
    for (int u0 = 0; u0 < nu; u0 += RING) {
#pragma unroll
      for (int r = 0; r < RING; ++r) {
        if (u0 + r < nu) proc(u0 + r, R.hd[r], R.w0[r], R.w1[r]);
        // the refill stays after unit r: the loads are invariant, and the scheduler would
        // otherwise issue every refill first, with all their registers live at once
        __builtin_amdgcn_sched_barrier(0);
        const int un = min(u0 + r + RING, nu - 1);
        unit_load(base(un), ul, R.hd[r], R.w0[r], R.w1[r], dfn(un));
      }
    }
  }
}

__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// One 16-element group of the x image: terms at xq + 32 G, (s0/256, sum) at xs[G].
__device__ __forceinline__ void x_group(const float (&v)[16], uint8_t* xq, float2* xs, int G) {
  float m = 0.f, sum = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) m = fmaxf(m, fabsf(v[q])), sum = sum + v[q];
  uint32_t p0[4] = {0u, 0u, 0u, 0u}, p1[4] = {0u, 0u, 0u, 0u};
  float s0 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    int t0, t1;
    split_i8(v[q], m, t0, t1, s0);
    p0[q >> 2] |= ((uint32_t)t0 & 0xFFu) << (8 * (q & 3));
    p1[q >> 2] |= ((uint32_t)t1 & 0xFFu) << (8 * (q & 3));
  }
  *reinterpret_cast<uint4*>(xq + G * 32) = uint4{p0[0], p0[1], p0[2], p0[3]};
  *reinterpret_cast<uint4*>(xq + G * 32 + 16) = uint4{p1[0], p1[1], p1[2], p1[3]};
  xs[G] = float2{s0 * (1.f / 256.f), sum};
}

// NORM: the input is rms_norm(x) and the residual x is added to y (mr_moe_forward_residual);
// a separate instantiation, so the plain decode path compiles without that code.
// DN > 0: I = 256 * DN and every wave's units fit its registers (straight-line unit code, no
// per-unit branches, so the compiler overlaps one unit's LDS reads and MFMAs with another's
// epilogue); DN == 0: any supported shape, table-driven units streamed through the registers.
template <bool NORM, int DN>
__global__ __launch_bounds__(256, 3) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_fused_q4k(Q4Args a) {
  constexpr bool STREAM = DN == 0;
  __shared__ __align__(16) uint8_t smem[kQ4Smem];
  __shared__ int sel_i[16];
  __shared__ float sel_w[kQ4MaxSlots];  // [k ..]: weight of the shared expert (each of its slots)
  __shared__ int sel_o[16];
  __shared__ uint32_t sel_k[16];
  __shared__ uint32_t route_tmp[128];  // routing: compacted candidates
  __shared__ int ok_flag;
  __shared__ float gu_part[2][2][16];  // [gate, up][super-block half][row]
  __shared__ __align__(16) int8_t hb[32];
  __shared__ float dn_part[kQ4MaxSlots][16];
  __shared__ const uint8_t* dn_tab[4][kQ4MaxUnitsD];  // down: unit table of each wave
  __shared__ uint32_t dn_grp[4][kQ4MaxUnitsD];
  __shared__ float dn_spare[4][64];  // down: stores of repeated slots and of lanes 16-63

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: wave-level branches stay scalar
  // role index = dispatch slot: the role permutation of the MXFP4 kernel (role_index) measured
  // 4-5% slower on these grids, whose CUs with two gate/up units already hold nothing else
  const int bid = blockIdx.x;
  const int nsbH = a.H >> 8, nsbI = a.I >> 8, nGI = a.I >> 4;
  TRACE(0);
  const uint32_t seq = ld_sc1(wg_seq_word(a.fs));
  const RouteCfg rc{a.fs, (uint32_t)(a.E + a.has_sh), a.E, a.k, a.flags, a.wb, a.trace};

  if (bid < a.R) {
    // ------------------------------------------------------------- router
    __builtin_amdgcn_s_setprio(2);  // the logits gate every other role: router loads issue first
    const int e = bid * 4 + wave;
    if (e < a.E + a.has_sh) {
      const float* w = e < a.E ? a.router_w + (size_t)e * a.H : a.sh_gate_inp;
      // bias and mask are loaded with the rows, not after the reduction (an HBM round trip)
      const float rbias = (e < a.E && a.router_b) ? a.router_b[e] : 0.f;
      const float rmask = (e < a.E && a.mask) ? a.mask[e] : 0.f;
      float inv = 1.f;
      if (NORM && w) {  // x = rms_norm(h)
        f32x4 hv[2 * kQ4RouterVec];
        load_lanes4(a.x, a.H, hv);
        inv = rms_inv(hv, a.H, a.nr.eps);
      }
      float acc = 0.f;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (p * kQ4RouterVec * 256 >= a.H) break;
        f32x4 xv[kQ4RouterVec], wv[kQ4RouterVec];
#pragma unroll
        for (int j = 0; j < kQ4RouterVec; ++j) {
          const int c = (lane + 64 * (p * kQ4RouterVec + j)) * 4;
          const bool in = c < a.H && w != nullptr;
          xv[j] = in ? *reinterpret_cast<const f32x4*>(a.x + c) : f32x4{0.f, 0.f, 0.f, 0.f};
          wv[j] = in ? *reinterpret_cast<const f32x4*>(w + c) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (NORM && w) {
#pragma unroll
          for (int j = 0; j < kQ4RouterVec; ++j) {
            const int c = (lane + 64 * (p * kQ4RouterVec + j)) * 4;
            const f32x4 nv = c < a.H ? *reinterpret_cast<const f32x4*>(a.nr.w + c) : f32x4{0.f, 0.f, 0.f, 0.f};
            xv[j] = f32x4{norm1(xv[j].x, inv, nv.x), norm1(xv[j].y, inv, nv.y), norm1(xv[j].z, inv, nv.z),
                          norm1(xv[j].w, inv, nv.w)};
          }
        }
#pragma unroll
        for (int j = 0; j < kQ4RouterVec; ++j) {
          acc = __builtin_fmaf(xv[j].x, wv[j].x, acc);
          acc = __builtin_fmaf(xv[j].y, wv[j].y, acc);
          acc = __builtin_fmaf(xv[j].z, wv[j].z, acc);
          acc = __builtin_fmaf(xv[j].w, wv[j].w, acc);
        }
      }
      acc = wave_sum_fast(acc);  // the same bits in every lane (butterfly of commutative adds)
      if (e < a.E) {
        if (a.router_b) acc = acc + rbias;
        if (a.mask) acc = acc + rmask;
      }
      put_logit(a.fs, (uint32_t)(a.E + a.has_sh), e, seq, acc);
      if (a.logits_out && e < a.E && lane == 0) a.logits_out[e] = acc;
    }
    TRACE(1);
    prefetch_rows(a.pf, bid, a.R, smem);
  } else if (bid >= a.R + a.ND) {
    // ------------------------------------------------------------- gate/up
    const int gid = bid - a.R - a.ND;
    // the gate/up loads issue ahead of the down workgroups' loads on the same CU
    __builtin_amdgcn_s_setprio(1);
    uint8_t* xq = smem + kQImg;
    float2* xs = reinterpret_cast<float2*>(smem + kQSc);
    if (tid == 0) *reinterpret_cast<uint4*>(smem + kQZero) = uint4{0u, 0u, 0u, 0u};
    // x = rms_norm(h) when fused: each wave derives inv the way the router waves do
    float inv = 1.f;
    if (NORM) {
      f32x4 hv[2 * kQ4RouterVec];
      load_lanes4(a.x, a.H, hv);
      inv = rms_inv(hv, a.H, a.nr.eps);
    }
    // The routing wave differs between the (up to four) workgroups that share a CU (dispatch
    // slots b and b + 256 share one), so their polls and selections run on different SIMDs.
    const int rw = (int)(blockIdx.x >> 8) & 3;
    // x image first, one 16-element group per thread, then the poll: a poll issued before the
    // router has published its logits returned only well after they were published (traced: issued
    // at 1.2 us, complete at 4.4 us, published by 2.7 us), while one issued after the x image
    // returns within a few hundred ns (C3 +2.7%, C4 +3.5% over polling from the start)
    for (int G = tid; G < (a.H >> 4); G += 256) {
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(a.x + G * 16 + 4 * q);
        v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
      }
      if (NORM) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 nw = *reinterpret_cast<const f32x4*>(a.nr.w + G * 16 + 4 * q);
          v[4 * q] = norm1(v[4 * q], inv, nw.x), v[4 * q + 1] = norm1(v[4 * q + 1], inv, nw.y);
          v[4 * q + 2] = norm1(v[4 * q + 2], inv, nw.z), v[4 * q + 3] = norm1(v[4 * q + 3], inv, nw.w);
        }
      }
      x_group(v, xq, xs, G);
    }
    TRACE(1);
    __syncthreads();  // the x image is complete before the routing wave polls
    RouteState rs;  // the routing wave: the selection, finished (weights, order) once its loads are issued
    if (wave == rw) {  // ok_flag written by this wave alone: it is 0 exactly when the selection failed
      const bool routed = route_select(rc, seq, sel_i, sel_k, route_tmp, rs);
      if (lane == 0) ok_flag = routed ? 1 : 0;
      if (!routed && lane == 0) fail(a.err);
    }
    __syncthreads();  // selection and the x image ready
    TRACE(2);
    if (ok_flag) {
      // the workgroup's gt row tiles of one slot, one after another (gt > 1 only in the streaming
      // instantiation, for grids that would not fit the CUs with one tile per workgroup)
      const int gt = STREAM ? a.gt : 1, nub = nGI / gt;
      const int slot = gid / nub, ub = gid - slot * nub;
      for (int t = 0; t < gt; ++t) {
      const int urow = ub * gt + t;
      const bool sh = slot >= a.k;
      const int mat = wave >> 1, kh = wave & 1;
      const int e = sh ? 0 : sel_i[slot];
      const uint32_t rb = (uint32_t)nsbH * 144u;
      // shared slot k + j: rows j*I .. j*I + I - 1 of the shared gate and up matrices (j > 0
      // only in the streaming instantiation)
      const uint8_t* W = sh ? (mat ? a.sh_up : a.sh_gate) + (STREAM ? (size_t)(slot - a.k) * a.I * rb : 0)
                            : expert_at(mat ? a.up : a.gate, e);
      const int nlo = (nsbH + 1) >> 1;  // super-blocks of half 0 (half 1 takes the rest)
      const int c0 = kh ? nlo : 0, nu = kh ? nsbH - nlo : nlo;
      const uint8_t* Wr = uniform_ptr(W + (size_t)(urow * 16) * rb + (size_t)c0 * 144);
      // loads used only by the epilogue issue first: the waits for the units never wait for them
      float gbias = 0.f, ubias = 0.f;
      // every lane, no condition (a load under a lane condition is waited for at once): the
      // shared gate logit, or the first logit when there is no shared expert (unused then)
      const float zsh = get_logit(a.fs, (uint32_t)(a.E + a.has_sh), a.has_sh ? a.E : 0);
      if (wave == 0 && lane < 16 && !sh) {  // the epilogue's biases
        const size_t bi = (size_t)e * a.I + urow * 16 + lane;
        if (a.gate_b) gbias = a.gate_b[bi];
        if (a.up_b) ubias = a.up_b[bi];
      }
      const UnitLane ul = unit_lane(rb);
      auto base = [&](int u) { return Wr + (size_t)u * 144; };
      float acc = 0.f;
      UnitRegs<kQ4RingG> R;
      if constexpr (!STREAM) {
        // every unit slot is loaded and run; those past nu (a duplicate of unit nu - 1, or for
        // nu == 0 of the row block's first super-block) add nothing
        const uint8_t* Wl = nu > 0 ? Wr : uniform_ptr(W + (size_t)(urow * 16) * rb);
        units_issue(R, max(nu, 1), [&](int u) { return Wl + (size_t)u * 144; }, ul);
        if (wave == rw && t == 0) route_finish(rc, rs, sel_w, sel_o);  // routing weights while the rows load
        // the LDS operands of unit r + 1 are read before unit r's MFMAs
        UnitOps op = unit_ops(ul, (uint32_t)min(c0, nsbH - 1) * 16u, smem);
#pragma unroll
        for (int r = 0; r < kQ4RingG; ++r) {
          const UnitOps cur = op;
          if (r + 1 < kQ4RingG) op = unit_ops(ul, (uint32_t)min(c0 + r + 1, nsbH - 1) * 16u, smem);
          const float v = unit_dot(R.hd[r], R.w0[r], R.w1[r], ul, cur);
          acc += r < nu ? v : 0.f;
        }
      } else {
        if (nu > 0) units_issue(R, nu, base, ul);
        if (wave == rw && t == 0) route_finish(rc, rs, sel_w, sel_o);
        if (nu > 0)
          units_process<STREAM>(R, nu, base, ul, [&](int u, const uint4& hd, const uint4& w0, const uint4& w1) {
            acc += unit_dot(hd, w0, w1, ul, (uint32_t)(c0 + u) * 16u, smem);
          });
      }
      XTRACE(wave);  // per wave: dot products done
      acc = row_total(acc);
      if (wave == 0 && (STREAM ? lane < a.nsh : a.has_sh && lane == 0))
        sel_w[a.k + (STREAM ? lane : 0)] = a.sh_gate_inp ? sigmoidf_(zsh) : 1.f;
      if (lane < 16) gu_part[mat][kh][lane] = acc;
      TRACE(3);
      __syncthreads();
      if (wave == 0 && lane < 16) {
        float g = gu_part[0][0][lane] + gu_part[0][1][lane], u = gu_part[1][0][lane] + gu_part[1][1][lane];
        if (!sh && a.gate_b) g = g + gbias;
        if (!sh && a.up_b) u = u + ubias;
        const float hact = (!sh && a.act == MR_ACT_SWIGLU_OAI) ? swiglu_oai(g, u, a.alpha, a.limit) : silu_mul(g, u);
        const float h = hact * sel_w[slot];
        float m = max8(fabsf(h));
        m = fmaxf(m, dpp_f<kDppMirror>(m));
        float sum = sum8(h);
        sum = sum + dpp_f<kDppMirror>(sum);
        int t0, t1;
        float s0;
        split_i8(h, m, t0, t1, s0);
        hb[lane] = (int8_t)t0, hb[16 + lane] = (int8_t)t1;
        lds_drain();
        __builtin_amdgcn_wave_barrier();
        const size_t blk = (size_t)slot * nGI + urow;
        if (lane < 8) st_sc1(a.himg + blk * 8 + lane, reinterpret_cast<const uint32_t*>(hb)[lane]);
        if (lane == 0) st_sc1(reinterpret_cast<uint32_t*>(a.hsc) + blk * 2, __float_as_uint(s0 * (1.f / 256.f)));
        if (lane == 1) st_sc1(reinterpret_cast<uint32_t*>(a.hsc) + blk * 2 + 1, __float_as_uint(sum));
        vm_drain();  // image stores complete before the count that announces them
      }
      if (t + 1 < gt) __syncthreads();  // gu_part and hb are free for the next tile
      }
      TRACE(4);
    }
    // counted even when routing failed, so later launches stay in step
    if (tid == 0) count<128>(a.fs + FS_GU, gid);
  } else {
    // ------------------------------------------------------------- down
    const int q = bid - a.R;
    if (tid == 0) ok_flag = 1, *reinterpret_cast<uint4*>(smem + kQZero) = uint4{0u, 0u, 0u, 0u};
    RouteState rs;  // wave 0: the selection, finished (weights, order) once the loads are issued
    // the routing wave runs at the gate/up waves' priority while it selects (its weight
    // loads, issued after, stay below the gate/up streams)
    if (wave == 0) __builtin_amdgcn_s_setprio(1);
    if (wave == 0 && !route_select<MR_ROUTE_SLEEP_DOWN>(rc, seq, sel_i, sel_k, route_tmp, rs)) {
      if (lane == 0) ok_flag = 0, fail(a.err);
    }
    if (wave == 0) __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    TRACE(1);
    if (ok_flag) {
      const uint32_t rb = (uint32_t)nsbI * 144u;
      // The shared expert's down rows are nsh times longer (sh_rb bytes apart); its slots take
      // one column range each (the streaming instantiation alone runs nsh > 1): row i of a unit
      // of a shared slot sits i * (sh_rb - rb) bytes further than the UnitLane's i * rb.
      const uint32_t sh_rb = rb * (uint32_t)max(a.nsh, 1);
      const uint32_t dsh = (uint32_t)(lane & 15) * (sh_rb - rb);
      const int ush0 = max(0, (a.k - wave + 3) >> 2) * nsbI;  // the wave's first unit of a shared slot
      [[maybe_unused]] auto row_delta = [&](int u) { return u >= ush0 ? dsh : 0u; };
      const int nsw = (a.ktot - wave + 3) >> 2;  // slots of this wave: wave, wave + 4, ...
      const int nu = nsw * nsbI;                 // units: slot-major, super-blocks within
      const UnitLane ul = unit_lane(rb);
      // fixed shape: slot j of the wave holds units j*DN .. j*DN+DN-1; slots past nsw repeat the
      // last slot (loaded and run, never stored)
      constexpr int NSL = DN > 0 ? kQ4RingD / DN : 1;
      int sj[NSL];
      const uint8_t* pj[NSL];
      UnitRegs<kQ4RingD> R;
      if constexpr (!STREAM) {
#pragma unroll
        for (int j = 0; j < NSL; ++j) {
          sj[j] = min(wave + 4 * j, a.ktot - 1);
          const uint8_t* D = sj[j] >= a.k ? a.sh_down : expert_at(a.down, sel_i[min(sj[j], a.k - 1)]);
          pj[j] = uniform_ptr(D + (size_t)(q * 16) * rb);
        }
#pragma unroll
        for (int r = 0; r < kQ4RingD; ++r) unit_load(pj[r / DN] + (size_t)(r % DN) * 144, ul, R.hd[r], R.w0[r], R.w1[r]);
      } else {
        // unit table of this wave (lane u < nu): the unit's super-block in row 0 of row block
        // q of its slot's down matrix; its first activation group, its slot, and whether it
        // ends the slot (bits 0-15, 16-20, 31)
        if (nu > 0) {
          const int u = min(lane, nu - 1), j = u / nsbI, c = u - j * nsbI, s = wave + 4 * j;
          // shared slot k + j': columns j'*I .. of the shared down rows, which are nsh times longer
          const uint8_t* D = s >= a.k ? a.sh_down + (size_t)(s - a.k) * rb + (size_t)(q * 16) * sh_rb
                                      : expert_at(a.down, sel_i[min(s, a.k - 1)]) + (size_t)(q * 16) * rb;
          if (lane < kQ4MaxUnitsD) {
            dn_tab[wave][lane] = D + (size_t)c * 144;
            dn_grp[wave][lane] = (uint32_t)(s * nGI + c * 16) | ((uint32_t)s << 16) | (c == nsbI - 1 ? 0x80000000u : 0u);
          }
          lds_drain();
          __builtin_amdgcn_wave_barrier();
          units_issue(R, nu, [&](int u) { return uniform_ptr(dn_tab[wave][u]); }, ul, row_delta);
        }
      }
      if (wave == 0) route_finish(rc, rs, sel_w, sel_o);  // wave 0 alone uses weights and order
      const float yres = (tid < 16 && NORM) ? a.nr.resid[q * 16 + tid] : 0.f;
      float ybias = 0.f;  // this row's routed bias terms (layer.rs:1417-1444)
      if (tid < 16 && a.down_b)
        for (int s2 = 0; s2 < a.k; ++s2) ybias = ybias + sel_w[s2] * a.down_b[(size_t)sel_i[s2] * a.H + q * 16 + tid];
      // every unit's sub-block scales are decoded while the gate/up results are awaited (the
      // weights land long before the count completes; the scales take the header's registers)
      // The first kQ4PreSplit units (all of them by default) also get their nibbles split into
      // the int8 B operands here, so after the wait only the LDS operands, the MFMAs and the
      // epilogue remain per unit.
      [[maybe_unused]] UnitScales US[STREAM ? 1 : kQ4RingD];
      [[maybe_unused]] UnitPrep PS[STREAM ? 1 : kQ4PreSplit];
      if constexpr (!STREAM) {
#pragma unroll
        for (int r = 0; r < kQ4RingD; ++r) {
          US[r] = unit_scales(R.hd[r], ul);
          // materialised here: the compiler would otherwise sink the decode to its use
          asm volatile("" : "+v"(US[r].dsc[0]), "+v"(US[r].dsc[1]), "+v"(US[r].dm[0]), "+v"(US[r].dm[1]));
          if (r < kQ4PreSplit) {
            PS[r] = unit_prep(US[r], R.w0[r], R.w1[r]);
            asm volatile("" : "+v"(PS[r].b[0][0]), "+v"(PS[r].b[0][1]), "+v"(PS[r].b[1][0]), "+v"(PS[r].b[1][1]));
          }
        }
      }
      TRACE(2);
      if (wave == 0 && !wait_count<MR_GU_WAIT_SLEEP, 128, 4>(a.fs + FS_GU, (seq + 1u) * (uint32_t)a.NG, a.wb,
                                                         (uint32_t)a.NG / 4) && lane == 0)
        ok_flag = 0, fail(a.err);
      __syncthreads();
      TRACE(3);
      if (ok_flag) {
        // down input image of every slot -> LDS (agent-coherent direct-to-LDS loads)
        {
          const int nq = a.ktot * nGI * 2;  // 16-byte pieces of the terms
          const uint8_t* src = reinterpret_cast<const uint8_t*>(a.himg);
          for (int b = wave; b * 64 < nq; b += 4) {
            const int idx = min(b * 64 + lane, nq - 1);
            __builtin_amdgcn_global_load_lds(src + (size_t)idx * 16, smem + kQImg + b * 1024, 16, 0, 16 /* sc1 */);
          }
          const int npc = (a.ktot * nGI + 1) / 2;  // 16-byte pieces of the (s0/256, sum) pairs
          const uint8_t* ssrc = reinterpret_cast<const uint8_t*>(a.hsc);
          for (int b = wave; b * 64 < npc; b += 4) {
            const int idx = min(b * 64 + lane, npc - 1);
            __builtin_amdgcn_global_load_lds(ssrc + (size_t)idx * 16, smem + kQSc + b * 1024, 16, 0, 16 /* sc1 */);
          }
          vm_drain();
        }
        __syncthreads();
        TRACE(4);
        float acc = 0.f;
        if constexpr (!STREAM) {
          // the LDS operands of unit r + 1 are read before unit r's MFMAs
          UnitOps op = unit_ops(ul, (uint32_t)(sj[0] * nGI), smem);
#pragma unroll
          for (int r = 0; r < kQ4RingD; ++r) {
            const int j = r / DN, c = r % DN;
            const UnitOps cur = op;
            if (r + 1 < kQ4RingD)
              op = unit_ops(ul, (uint32_t)(sj[(r + 1) / DN] * nGI + ((r + 1) % DN) * 16), smem);
            acc += unit_dot(r < kQ4PreSplit ? PS[r < kQ4PreSplit ? r : 0] : unit_prep(US[r], R.w0[r], R.w1[r]), cur);
            if (c == DN - 1) {  // the slot's last super-block: lanes 0-15 store its rows (repeated
                                // slots and the other lanes store to this wave's spare row)
              acc = row_total(acc);
              const bool st = lane < 16 && j < nsw;
              float* dst = st ? &dn_part[sj[j]][lane] : &dn_spare[wave][lane];
              *dst = acc;
              acc = 0.f;
            }
          }
        } else if (nu > 0) {
          units_process<STREAM>(R, nu, [&](int u) { return uniform_ptr(dn_tab[wave][u]); }, ul,
                                [&](int u, const uint4& hd, const uint4& w0, const uint4& w1) {
                                  const uint32_t gw = __builtin_amdgcn_readfirstlane(dn_grp[wave][u]);
                                  acc += unit_dot(hd, w0, w1, ul, gw & 0xFFFFu, smem);
                                  if (gw >> 31) {  // the slot's last super-block
                                    acc = row_total(acc);
                                    if (lane < 16) dn_part[(gw >> 16) & 31u][lane] = acc;
                                    acc = 0.f;
                                  }
                                }, row_delta);
        }
        XTRACE(wave);  // per wave: dot products done
        __syncthreads();
        if (tid < 16) {
          const int rr = q * 16 + tid;
          float yv = 0.f;  // routed slots in ascending expert order (layer.rs:1092-1106)
          for (int p = 0; p < a.k; ++p) yv = yv + dn_part[sel_o[p]][tid];
          yv = yv + ybias;
          if (a.has_sh) {  // shared expert after the routed sum, its slots in column order
            float ysh = dn_part[a.k][tid];
            if constexpr (STREAM)
              for (int s2 = 1; s2 < a.nsh; ++s2) ysh = ysh + dn_part[a.k + s2][tid];
            yv = yv + ysh;
          }
          if (NORM) yv = yres + yv;  // hidden = residual + moe_out (layer.rs:473)
          a.y[rr] = yv;
        }
        XTRACE(4 + wave);  // per wave: combine done
      }
    }
  }
  // ----------------------------------------------------------------- exit
  __syncthreads();
  TRACE(5);
#ifdef MR_FUSED_TRACE
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * 32 + 7] = __smid();
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * 32 + 6] = (unsigned long long)bid + 1;  // role index
  if (a.trace && (threadIdx.x & 63) == 0)  // HW_ID: wave, SIMD, CU, SE of each wave
    a.trace[blockIdx.x * 32 + 26 + (threadIdx.x >> 6)] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
#endif
  if (tid == 0) st_sc1(wg_seq_word(a.fs), seq + 1u);
}

namespace {
struct Q4Grid {
  uint64_t R, ND, NG, gt;
  uint64_t total() const { return R + ND + NG; }
};
// Roles of a launch: gt row tiles per gate/up workgroup, the fewest (1, 2 or 4) that keep the
// grid within 3 workgroups per CU.
// Slots of the shared expert: Ish / I column ranges of I (0 without one).
uint64_t q4_nsh(const mr_layer& L) { return L.d.sh_gate ? L.Ish / L.I : 0u; }
Q4Grid q4_grid(const mr_layer& L, int n_cu) {
  const uint64_t has_sh = L.d.sh_gate ? 1u : 0u, ktot = L.d.top_k + q4_nsh(L), nGI = L.I / 16;
  const uint64_t R = (L.E + has_sh + 3) / 4, ND = L.H / 16;
  const uint64_t cap = std::min<uint64_t>(3ull * (uint64_t)n_cu, (uint64_t)kMaxGrid);
  uint64_t gt = 1;
  while (R + ND + ktot * nGI / gt > cap && gt < 4 && nGI % (2 * gt) == 0) gt *= 2;
  return Q4Grid{R, ND, ktot * nGI / gt, gt};
}
// Units of the busiest gate/up and down waves.
uint64_t q4_units_gu(const mr_layer& L) { return (L.H / 256 + 1) / 2; }
uint64_t q4_units_dn(const mr_layer& L) {
  const uint64_t ktot = L.d.top_k + q4_nsh(L);
  return (ktot + 3) / 4 * (L.I / 256);
}
// The instantiation for a shape: DN = I/256 when every wave's units fit its registers
// (I <= 768, H <= 2048, the down waves' slots within kQ4RingD / DN, one row tile per gate/up
// workgroup, a shared expert no wider than the routed ones), else 0 (streaming).
int q4_dn(const mr_layer& L, int n_cu) {
  const uint64_t dn = L.I / 256, ktot = L.d.top_k + q4_nsh(L);
  if (dn >= 1 && dn <= 3 && q4_nsh(L) <= 1 && q4_units_gu(L) <= (uint64_t)kQ4RingG && (ktot + 3) / 4 <= (uint64_t)(kQ4RingD / dn) &&
      q4_grid(L, n_cu).gt == 1)
    return (int)dn;
  return 0;
}
template <bool NORM>
const void* q4_kernel(int dn) {
  switch (dn) {
    case 1: return reinterpret_cast<const void*>(k_fused_q4k<NORM, 1>);
    case 2: return reinterpret_cast<const void*>(k_fused_q4k<NORM, 2>);
    case 3: return reinterpret_cast<const void*>(k_fused_q4k<NORM, 3>);
    default: return reinterpret_cast<const void*>(k_fused_q4k<NORM, 0>);
  }
}
}  // namespace

// Shapes the fused Q4_K kernel runs; others take the VALU path.
bool fused_q4k_supported(const mr_layer& L, int n_cu) {
  if (L.type != MR_GGML_Q4_K || L.H % 256 != 0 || L.I % 256 != 0 || L.H == 0 || L.I == 0) return false;
  if (L.H > (uint32_t)kQ4MaxH || L.I > (uint32_t)kQ4MaxI) return false;
  const uint32_t has_sh = L.d.sh_gate ? 1u : 0u;
  if (has_sh && (L.d.sh_gate->type != MR_GGML_Q4_K || L.d.sh_up->type != MR_GGML_Q4_K ||
                 L.d.sh_down->type != MR_GGML_Q4_K || L.Ish % L.I != 0))
    return false;  // a shared expert as nsh = Ish / I slots of the routed width
  const uint64_t ktot = L.d.top_k + q4_nsh(L);
  if (L.d.top_k > 16 || ktot > (uint64_t)kQ4MaxSlots || L.E > 512 || L.E + has_sh > (uint32_t)kMaxLogits) return false;
  if (ktot * L.I > (uint64_t)kQ4MaxKI) return false;  // the down input image of every slot in LDS
  if (q4_units_dn(L) > (uint64_t)kQ4MaxUnitsD) return false;  // the down waves' unit tables
  // every workgroup resident at once (3 per CU are assumed; fused_q4k_resident checks)
  const uint64_t grid = q4_grid(L, n_cu).total();
  return grid <= 3ull * n_cu && grid <= (uint64_t)kMaxGrid;
}

// Every workgroup of a launch must be resident at once (workgroups wait on each other):
// the occupancy the runtime reports for the instantiations this layer launches (registers and
// LDS), on an otherwise idle device, times the CU count must cover the grid.
bool fused_q4k_resident(const mr_layer& L, int n_cu) {
  const int64_t grid = (int64_t)q4_grid(L, n_cu).total();
  const int dn = q4_dn(L, n_cu);
  int b0 = 0, b1 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b0, q4_kernel<false>(dn), 256, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&b1, q4_kernel<true>(dn), 256, 0) != hipSuccess)
    return false;
  if ((int64_t)std::min(b0, b1) * n_cu < grid) return false;
  // as for the MXFP4 kernel: LDS rounded up to 2 KB per workgroup must fit the CU as well
  int dev = 0, cu_lds = 0;
  hipFuncAttributes fa{}, fb{};
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cu_lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
      hipFuncGetAttributes(&fa, q4_kernel<false>(dn)) != hipSuccess || hipFuncGetAttributes(&fb, q4_kernel<true>(dn)) != hipSuccess)
    return false;
  const int64_t wg_lds = (int64_t)((std::max(fa.sharedSizeBytes, fb.sharedSizeBytes) + 2047) & ~(size_t)2047);
  return wg_lds * ((grid + n_cu - 1) / n_cu) <= (int64_t)cu_lds;
}

hipError_t launch_fused_q4k(const Launch& K, const mr_layer& L, const float* x, float* y, uint32_t* err,
                            uint8_t* img_base, const NormResid& nr) {
  Q4Args a{};
#ifdef MR_FUSED_TRACE
  a.trace = g_fused_trace;
#endif
  a.gate = expert_loc(L.d.gate), a.up = expert_loc(L.d.up), a.down = expert_loc(L.d.down);
  a.has_sh = L.d.sh_gate ? 1 : 0;
  if (a.has_sh) {
    a.sh_gate = L.d.sh_gate->base + L.d.sh_gate->h_offsets[0];
    a.sh_up = L.d.sh_up->base + L.d.sh_up->h_offsets[0];
    a.sh_down = L.d.sh_down->base + L.d.sh_down->h_offsets[0];
  }
  a.gate_b = L.d.gate_bias, a.up_b = L.d.up_bias, a.down_b = L.d.down_bias;
  a.router_w = L.d.router_w, a.router_b = L.d.router_b, a.mask = L.d.dummy_mask;
  a.sh_gate_inp = L.d.sh_gate_inp;
  a.x = x, a.y = y, a.fs = L.fused_sync, a.err = err;
  a.logits_out = L.logits_out;
  a.nsh = (int)q4_nsh(L);
  a.H = (int)L.H, a.I = (int)L.I, a.E = (int)L.E, a.k = (int)L.d.top_k, a.ktot = a.k + a.nsh;
  const uint64_t nGI = L.I / 16;
  a.himg = reinterpret_cast<uint32_t*>(img_base);
  a.hsc = reinterpret_cast<float*>(img_base + (uint64_t)a.ktot * nGI * 32);
  a.flags = L.d.route_flags, a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  const int n_cu = L.ctx->n_cu;
  const Q4Grid g = q4_grid(L, n_cu);
  a.R = (int)g.R, a.ND = (int)g.ND, a.NG = (int)g.NG, a.gt = (int)g.gt;
  a.wb = wait_bound(*L.ctx);
  a.pf = prefetch_plan(L.next);
  a.nr = nr;
  ProfScope ps(K, "fused_layer");
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel(nr.w ? q4_kernel<true>(q4_dn(L, n_cu)) : q4_kernel<false>(q4_dn(L, n_cu)),
                                       dim3((unsigned)g.total()), dim3(256), args, 0, K.s);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace mr
