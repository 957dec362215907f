// mr_fused_q4k.hip -- single-launch Q4_K MoE decode layer for gfx950 (CDNA4).
//
// The Q4_K counterpart of k_fused_mxfp4: one kernel per layer and token does
// the router GEMV (+ the shared-expert gate), top-k routing, gate+up
// dequant-matvec with SwiGLU/SiLU, down dequant-matvec with the weighted
// combine in ascending expert order, and the sigmoid-gated shared expert
// (layer.rs:1012-1027, 1818-1953, 2346-2403; per-expert QMatMul path
// layer.rs:2099-2147).
//
// Weight streaming. A wave owns a region of 8 consecutive rows of one expert
// matrix; the rows are contiguous in the GGUF layout, so lane l simply loads
// 16-byte chunks l, l+64, ... of the region (fully coalesced 1 KiB per wave
// load). A 144-byte super-block is 9 chunks: chunk 0 is the header (d, dmin,
// 12 scale bytes), chunks 1..8 are the 128 quant bytes. Header chunks are
// staged in LDS and decoded once per super-block into (d*sc_j, dmin*m_j);
// quant chunk p (qs bytes 16(p-1)..16p) holds 16 low nibbles = elements
// 64jj+16hf+t of sub-block 2jj and 16 high nibbles = elements 64jj+32+16hf+t of
// sub-block 2jj+1 (jj = (p-1)/2, hf = (p-1)%2; dequantize_q4k, dequant.rs:218-262).
//
// Dot products. The activation vector is split per 16-element group into two
// int8 terms: v = s0*t0 + s1*t1 with s0 = max|v|/127, s1 = s0/254, so
// |v - s0*t0 - s1*t1| <= s0/508 (about 1.6e-5 of the group max). The nibbles
// (0..15) are already int8 operands after one AND, so a chunk's 32 products
// are 8 v_dot4_i32_i8 per term, exact in int32. Per sub-block half:
//   sum_j w_j x_j = (d*sc) * (s0*A0 + s1*A1) - (dmin*m) * sum_j x_j
// with A0/A1 the integer dot products and sum_j x_j the group sum, the same
// weights w_j = (d*sc)*q_j - dmin*m the reference dequantizes.
//
// Roles (grid order; all workgroups resident, see fused_q4k_supported):
//   [0, R)       router: one logit per wave (E experts, then x . w_gi of the
//                shared expert when there is one).
//   [R, R+ND)    down: 8 output rows; wave w takes slots w, w+4, w+8 (routed
//                slots, then the shared expert). Down weights are prefetched into
//                registers before the gate/up results exist.
//   [R+ND, grid) gate/up: 16 rows of one slot; waves = (gate, up) x 2 halves of
//                8 rows. Epilogue: bias, activation, x routing weight (sigmoid
//                gate for the shared expert), int8 split of the 16 results into
//                the down input image.
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"

#include <algorithm>

namespace mr {

constexpr int kQ4RouterVec = 12;  // float4 pairs per lane of a router row: H <= 3072
constexpr int kQ4GuIt = 9;        // chunks per lane of a gate/up region (8 rows x H/256 sb): H <= 2048
constexpr int kQ4DnIt = 4;        // chunks per lane per slot of a down region (8 rows x I/256 sb): I <= 768
constexpr int kQ4DnSlots = 3;     // slots per down wave: k + shared <= 12
constexpr int kQ4MaxH = 2048, kQ4MaxI = 768, kQ4MaxSlots = 4 * kQ4DnSlots;
constexpr float kInv254 = 1.0f / 254.0f;

// LDS carve-up (bytes), gate/up workgroups
constexpr int kGuXq = 0;                                 // [H/16][2 x 16 int8] x terms
constexpr int kGuXs = kGuXq + kQ4MaxH * 2;               // [H/16] float2 (s0, group sum)
constexpr int kGuHdec = kGuXs + kQ4MaxH / 16 * 8;        // [4 waves][64 sb][16 floats] decoded headers
constexpr int kGuVbuf = kGuHdec + 4 * 64 * 64;           // [4][576] chunk partials
constexpr int kGuEnd = kGuVbuf + 4 * 576 * 4;
// down workgroups. A wave takes ns = ceil(ktot/4) slots; per-wave header and
// partial arrays hold ns regions of 8 rows x I/256 super-blocks: ns*I/256 <= kDnSbW/8.
constexpr int kDnSbW = 48;                                  // super-blocks per wave (all its regions)
constexpr int kDnHq = 0;                                    // [slots][I/16][32] h terms
constexpr int kDnHqBytes = kQ4MaxSlots * 512 * 2;           // ktot * I * 2 <= 12 * 512 * 2
constexpr int kDnHs = kDnHq + kDnHqBytes + 1024;            // [slots][I/16] float2 (+ 1 KiB load overrun)
constexpr int kDnHdec = kDnHs + kDnHqBytes / 4 + 1024;      // [4 waves][kDnSbW][16 floats]
constexpr int kDnVbuf = kDnHdec + 4 * kDnSbW * 64;          // [4][kDnSbW * 9] partials; raw headers alias it
constexpr int kDnEnd = kDnVbuf + 4 * kDnSbW * 9 * 4;
constexpr int kQ4Smem = kGuEnd > kDnEnd ? kGuEnd : kDnEnd;
static_assert(kDnSbW * 9 * 4 >= kDnSbW * 16, "raw headers fit in the partials slice");
static_assert(kQ4MaxH / 256 <= 8 && kQ4GuIt == 9 && kQ4MaxI / 256 <= 3 && kQ4DnIt == 4,
              "a wave's loads cover its 8-row region (chunk map: 9 loads for 8 super-blocks per row, "
              "4 for up to 3)");
static_assert(72 * (kQ4MaxH / 256) <= 576, "per-wave LDS slices hold a gate/up region");

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
  uint32_t* fs;     // this layer's sync block
  uint32_t* err;    // context error word
  uint32_t* himg;   // [ktot][I/16][8 words] int8 terms of the down input
  float* hsc;       // [ktot][I/16][2] (s0, group sum)
  int H, I, E, k, ktot, has_sh;
  uint32_t flags;
  int act;
  float alpha, limit;
  int R, ND, NG;
  uint32_t spin_limit;
  PrefetchRows pf;  // the next layer's router rows (router workgroups read them)
  NormResid nr;     // fused RMSNorm of x and residual added to y (off: nr.w == nullptr)
  unsigned long long* trace;
};

// ---- int8 two-term split ------------------------------------------------------------------
// s0 = m/127 (m = max|v| of the group), s1 = s0/254; t0 = rn(v/s0), t1 = rn((v - s0*t0)/s1).
__device__ __forceinline__ void split_i8(float v, float m, int& t0, int& t1, float& s0) {
  if (!(m > 0.f)) {
    t0 = t1 = 0, s0 = 0.f;
    return;
  }
  s0 = m / 127.f;
  const float s1 = s0 * kInv254;
  t0 = (int)fminf(fmaxf(rintf(v / s0), -127.f), 127.f);
  const float r = fmaf(-(float)t0, s0, v);
  t1 = (int)fminf(fmaxf(rintf(r / s1), -127.f), 127.f);
}

// ---- regions: 8 rows of a Q4_K matrix each -------------------------------------------------
// A region's chunk c = row * P + pos (P = 9 * nsb chunks per row, nsb <= 8) is held by one
// (load j, lane) pair:
//   nsb == 8:  loads j < 8 hold row j at pos = lane; load 8 holds row lane/8 at pos 64 + lane%8;
//   nsb < 8:   rp = 64 / P rows per load; lane = h * P + pos holds row j * rp + h (lanes with
//              h >= rp, and rows past 7, hold no chunk).
// Each load is 1 KiB of consecutive bytes (nsb == 8, last load: 8 runs of 128 B), and a lane's
// position is the same in every load but nsb == 8's last, so the activation operands of that
// position are read from LDS once per region instead of once per chunk.
struct QMap {
  int rp, h, pos;  // rows per load, this lane's row within a load, its position
  int trow, tpos;  // nsb == 8: row and position of the last load
  bool wide;       // nsb == 8
};
__device__ __forceinline__ QMap q_map(int nsb) {
  const int lane = threadIdx.x & 63;
  QMap m;
  m.wide = nsb == 8;
  if (m.wide) {
    m.rp = 1, m.h = 0, m.pos = lane, m.trow = lane >> 3, m.tpos = 64 + (lane & 7);
  } else {
    const int P = 9 * nsb;
    m.rp = 64 / P, m.h = lane / P, m.pos = lane - m.h * P, m.trow = 8, m.tpos = m.pos;
  }
  return m;
}
// Row held by load j (8: none) and the position of that load.
__device__ __forceinline__ int q_row(const QMap& m, int j) {
  if (m.wide) return j < 8 ? j : m.trow;
  return m.h < m.rp ? min(j * m.rp + m.h, 8) : 8;
}
__device__ __forceinline__ int q_pos(const QMap& m, int j) { return j == 8 ? m.tpos : m.pos; }

// A super-block header (d, dmin, 12 scale bytes) decoded into (d*sc_j, dmin*m_j) for its
// 8 sub-blocks: 16 floats at out.
__device__ __forceinline__ void header_decode(const uint4& h, float* out16) {
  const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
  const uint32_t s3[3] = {h.y, h.z, h.w};
  float4* out = reinterpret_cast<float4*>(out16);
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    uint32_t sc0, m0, sc1, m1;
    q4k_scale_min((uint32_t)j, s3, sc0, m0);
    q4k_scale_min((uint32_t)j + 1u, s3, sc1, m1);
    out[j / 2] = float4{__fmul_rn(d, (float)sc0), __fmul_rn(dmin, (float)m0),
                        __fmul_rn(d, (float)sc1), __fmul_rn(dmin, (float)m1)};
  }
}

// Phase 1 (needs only the weights): stage each super-block's header chunk in
// LDS (hraw), then decode it into (d*sc_j, dmin*m_j) for its 8 sub-blocks (hdec,
// 16 floats per super-block, regions one after another).
template <int IT, int NS>
__device__ __forceinline__ void region_headers(const uint4 (&ch)[NS][IT], const QMap& m, int nsb, int ns,
                                               uint4* hraw, float* hdec) {
  const int lane = threadIdx.x & 63;
  const int nsbr = 8 * nsb;
  const int col = m.pos / 9;
  const bool hpos = m.pos - 9 * col == 0;  // header chunks sit at positions 9 * col (never in the last
                                           // load of nsb == 8: positions 64..71)
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    if (r < ns) {
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        const int row = q_row(m, j);
        if (j < 8 && hpos && row < 8) hraw[r * nsbr + row * nsb + col] = ch[r][j];
      }
    }
  }
  lds_drain();
  __builtin_amdgcn_wave_barrier();
  for (int b = lane; b < ns * nsbr; b += 64) header_decode(hraw[b], hdec + b * 16);
  lds_drain();
  __builtin_amdgcn_wave_barrier();
}

// Header of a region's super-block lane (row lane / nsb, column lane % nsb), for lanes
// below 8 * nsb, as one load issued ahead of the region's chunks: it lands first, so the
// headers decode while the chunks stream in.
__device__ __forceinline__ uint4 region_header_load(const uint8_t* base, int nsb) {
  const int lane = threadIdx.x & 63;
  const int b = min(lane, 8 * nsb - 1), row = b / nsb;
  return *reinterpret_cast<const uint4*>(base + (size_t)row * nsb * 144 + (size_t)(b - row * nsb) * 144);
}

// Activation operands of chunk position pos (quant chunk p = pos % 9 of super-block
// column pos / 9): the int8 terms of its two 16-element groups (low nibbles: group G,
// high nibbles: G + 2) and their (s0, group sum). Header positions (p == 0) read
// position 1's operands; their products are discarded.
struct XOps {
  uint32_t l0[4], l1[4], h0[4], h1[4];
  float2 gl, gh;
  int hoff;  // float offset of the position's (d*sc, dmin*m) pairs within a super-block's 16
  int col;
  bool hdr;
};
__device__ __forceinline__ void x_ops(const uint8_t* xq, const float2* xs, int pos, XOps& o) {
  const int col = pos / 9, p = pos - 9 * col;
  o.hdr = p == 0;
  const int pp = o.hdr ? 0 : p - 1, jj = pp >> 1, hf = pp & 1;
  const int G = col * 16 + jj * 4 + hf;
  const uint4 l0 = *reinterpret_cast<const uint4*>(xq + G * 32);
  const uint4 l1 = *reinterpret_cast<const uint4*>(xq + G * 32 + 16);
  const uint4 h0 = *reinterpret_cast<const uint4*>(xq + (G + 2) * 32);
  const uint4 h1 = *reinterpret_cast<const uint4*>(xq + (G + 2) * 32 + 16);
  o.l0[0] = l0.x, o.l0[1] = l0.y, o.l0[2] = l0.z, o.l0[3] = l0.w;
  o.l1[0] = l1.x, o.l1[1] = l1.y, o.l1[2] = l1.z, o.l1[3] = l1.w;
  o.h0[0] = h0.x, o.h0[1] = h0.y, o.h0[2] = h0.z, o.h0[3] = h0.w;
  o.h1[0] = h1.x, o.h1[1] = h1.y, o.h1[2] = h1.z, o.h1[3] = h1.w;
  o.gl = xs[G], o.gh = xs[G + 2];
  o.hoff = 4 * jj, o.col = col;
}

// One quant chunk (16 low nibbles of sub-block 2jj, 16 high nibbles of sub-block 2jj+1)
// against its activation operands: per half, (d*sc) * (s0*A0 + s1*A1) - (dmin*m) * sum.
__device__ __forceinline__ float chunk_dot(const uint4& wc, const XOps& o, const float4& dm) {
  const uint32_t w[4] = {wc.x, wc.y, wc.z, wc.w};
  int a0 = 0, a1 = 0, b0 = 0, b1 = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int lo = (int)(w[d] & 0x0F0F0F0Fu), hi = (int)((w[d] >> 4) & 0x0F0F0F0Fu);
    a0 = __builtin_amdgcn_sdot4(lo, (int)o.l0[d], a0, false);
    a1 = __builtin_amdgcn_sdot4(lo, (int)o.l1[d], a1, false);
    b0 = __builtin_amdgcn_sdot4(hi, (int)o.h0[d], b0, false);
    b1 = __builtin_amdgcn_sdot4(hi, (int)o.h1[d], b1, false);
  }
  const float xlo = o.gl.x * (float)a0 + (o.gl.x * kInv254) * (float)a1;
  const float xhi = o.gh.x * (float)b0 + (o.gh.x * kInv254) * (float)b1;
  return ((dm.x * xlo - dm.y * o.gl.y) + dm.z * xhi) - dm.w * o.gh.y;
}

// Phase 2: quant-chunk dot products against the activation images (xq[r]: [G][32 B]
// int8 terms, xs[r]: [G] (s0, group sum)) into vbuf (chunk order), then each row's sum;
// out[r] is left in lanes 8*row (row = 0..7). vbuf may alias hraw (headers are decoded).
// Header chunks and lanes without a chunk write 0 (the latter to chunk 0, a header).
template <int IT, int NS>
__device__ __forceinline__ void region_dots(const uint4 (&ch)[NS][IT], const QMap& m, int nsb, int ns,
                                            const uint8_t* const (&xq)[NS], const float2* const (&xs)[NS],
                                            const float* hdec, float* vbuf, float (&out)[NS]) {
  const int lane = threadIdx.x & 63;
  const int P = 9 * nsb, nch = 8 * P, nsbr = 8 * nsb;
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    if (r < ns) {
      XOps xm, xt;
      x_ops(xq[r], xs[r], m.pos, xm);
      if (IT > 8) x_ops(xq[r], xs[r], m.tpos, xt);
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        const XOps& o = j < 8 ? xm : xt;
        const int row = q_row(m, j);
        const bool ok = row < 8 && !o.hdr;
        const int sb = min(row, 7) * nsb + o.col;
        const float4 dm = *reinterpret_cast<const float4*>(hdec + (r * nsbr + sb) * 16 + o.hoff);
        const float v = chunk_dot(ch[r][j], o, dm);
        vbuf[r * nch + (row < 8 ? row * P + q_pos(m, j) : 0)] = ok ? v : 0.f;
      }
    }
  }
  lds_drain();
  __builtin_amdgcn_wave_barrier();
  // row sums: 8 lanes per row, each over every 8th chunk of the row (at most IT: P <= 8 * IT),
  // then DPP; the reads are issued together
  const int row = lane >> 3, j8 = lane & 7;
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    float sm = 0.f;
    if (r < ns) {
      float e[IT];
#pragma unroll
      for (int t = 0; t < IT; ++t) e[t] = j8 + 8 * t < P ? vbuf[r * nch + row * P + j8 + 8 * t] : 0.f;
#pragma unroll
      for (int t = 0; t < IT; ++t) sm += e[t];
    }
    out[r] = sum8(sm);
  }
}

// Loads of one region (8 rows x nsb super-blocks at `base`); a lane without a chunk in a
// load reads chunk 0 (ignored).
template <int IT>
__device__ __forceinline__ void region_load(const uint8_t* base, const QMap& m, int nsb, uint4 (&ch)[IT]) {
  const int P = 9 * nsb;
#pragma unroll
  for (int j = 0; j < IT; ++j) {
    const int row = q_row(m, j);
    const int c = row < 8 ? row * P + q_pos(m, j) : 0;
    ch[j] = *reinterpret_cast<const uint4*>(base + (size_t)c * 16);
  }
}

// NORM: the input is rms_norm(x) and the residual x is added to y (mr_moe_forward_residual);
// a separate instantiation, so the plain decode path compiles without that code.
template <bool NORM>
__global__ __launch_bounds__(256, 3) void k_fused_q4k(Q4Args a) {
  __shared__ __align__(16) uint8_t smem[kQ4Smem];
  __shared__ int sel_i[16];
  __shared__ float sel_w[17];  // [k]: weight of the shared expert
  __shared__ int sel_o[16];
  __shared__ uint32_t sel_k[16];
  __shared__ uint32_t route_tmp[128];  // routing: compacted candidates
  __shared__ int ok_flag;
  __shared__ float gu_part[2][16];
  __shared__ __align__(16) int8_t hb[32];
  __shared__ float dn_part[kQ4MaxSlots][8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: wave-level branches stay scalar
  const int bid = blockIdx.x;
  const int nsbH = a.H >> 8, nsbI = a.I >> 8, nGI = a.I >> 4;
  TRACE(0);
  const uint32_t seq = ld_sc1(wg_seq_word(a.fs));
  const RouteCfg rc{a.fs, (uint32_t)(a.E + a.has_sh), a.E, a.k, a.flags, a.spin_limit, a.trace};

  if (bid < a.R) {
    // ------------------------------------------------------------- router
    __builtin_amdgcn_s_setprio(2);  // the logits gate every other role: router loads issue first
    const int e = bid * 4 + wave;
    if (e < a.E + a.has_sh) {
      const float* w = e < a.E ? a.router_w + (size_t)e * a.H : a.sh_gate_inp;
      // bias and mask are loaded with the rows, not after the reduction (an HBM round trip)
      const float rbias = (e < a.E && a.router_b) ? a.router_b[e] : 0.f;
      const float rmask = (e < a.E && a.mask) ? a.mask[e] : 0.f;
      f32x4 xv[kQ4RouterVec], wv[kQ4RouterVec];
#pragma unroll
      for (int j = 0; j < kQ4RouterVec; ++j) {
        const int c = (lane + 64 * j) * 4;
        const bool in = c < a.H && w != nullptr;
        xv[j] = in ? *reinterpret_cast<const f32x4*>(a.x + c) : f32x4{0.f, 0.f, 0.f, 0.f};
        wv[j] = in ? *reinterpret_cast<const f32x4*>(w + c) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if (NORM && w) {  // x = rms_norm(h)
        f32x4 nv[kQ4RouterVec];
        load_lanes4(a.nr.w, a.H, nv);
        const float inv = rms_inv(xv, a.H, a.nr.eps);
#pragma unroll
        for (int j = 0; j < kQ4RouterVec; ++j)
          xv[j] = f32x4{norm1(xv[j].x, inv, nv[j].x), norm1(xv[j].y, inv, nv[j].y),
                        norm1(xv[j].z, inv, nv[j].z), norm1(xv[j].w, inv, nv[j].w)};
      }
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kQ4RouterVec; ++j) {
        acc = __builtin_fmaf(xv[j].x, wv[j].x, acc);
        acc = __builtin_fmaf(xv[j].y, wv[j].y, acc);
        acc = __builtin_fmaf(xv[j].z, wv[j].z, acc);
        acc = __builtin_fmaf(xv[j].w, wv[j].w, acc);
      }
      acc = wave_sum(acc);  // the same bits in every lane (butterfly of commutative adds)
      if (e < a.E) {
        if (a.router_b) acc = acc + rbias;
        if (a.mask) acc = acc + rmask;
      }
      put_logit(a.fs, (uint32_t)(a.E + a.has_sh), e, seq, acc);
    }
    TRACE(1);
    prefetch_rows(a.pf, bid, a.R, smem);
  } else if (bid >= a.R + a.ND) {
    // ------------------------------------------------------------- gate/up
    const int gid = bid - a.R - a.ND;
    // the gate/up loads issue ahead of the down workgroups' prefetch on the same CU
    __builtin_amdgcn_s_setprio(1);
    uint8_t* xq = smem + kGuXq;
    float2* xs = reinterpret_cast<float2*>(smem + kGuXs);
    // x = rms_norm(h) when fused: each wave derives inv the way the router waves do
    float inv = 1.f;
    if (NORM) {
      f32x4 hv[kQ4RouterVec];
      load_lanes4(a.x, a.H, hv);
      inv = rms_inv(hv, a.H, a.nr.eps);
    }
    // x image: one 16-element group per thread
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
      xs[G] = float2{s0, sum};
    }
    TRACE(1);
    if (tid == 0) ok_flag = 1;
    RouteState rs;  // wave 0: the selection, finished (weights, order) once its loads are issued
    if (wave == 0 && !route_select(rc, seq, sel_i, sel_k, route_tmp, rs)) {
      if (lane == 0) ok_flag = 0, fail(a.err);
    }
    __syncthreads();  // selection and the x image ready
    TRACE(2);
    if (ok_flag) {
      const int slot = gid / nGI, urow = gid - slot * nGI;
      const bool sh = slot >= a.k;
      const int mat = wave >> 1, half = wave & 1;
      const int e = sh ? 0 : sel_i[slot];
      const uint8_t* W = sh ? (mat ? a.sh_up : a.sh_gate) : expert_at(mat ? a.up : a.gate, e);
      const size_t rb = (size_t)nsbH * 144;
      const QMap qm = q_map(nsbH);
      const uint8_t* Wr = W + (size_t)(urow * 16 + half * 8) * rb;
      // loads used only by the epilogue issue first: a wait for the region's header (the next
      // load) or for its chunks then never waits for them
      float zsh = 0.f, gbias = 0.f, ubias = 0.f;
      if (wave == 0 && a.has_sh && lane == 0) zsh = get_logit(a.fs, (uint32_t)(a.E + a.has_sh), a.E);
      if (wave == 0 && lane < 16 && !sh) {  // the epilogue's biases
        const size_t bi = (size_t)e * a.I + urow * 16 + lane;
        if (a.gate_b) gbias = a.gate_b[bi];
        if (a.up_b) ubias = a.up_b[bi];
      }
      const uint4 hdr = region_header_load(Wr, nsbH);
      uint4 ch[1][kQ4GuIt];
      region_load<kQ4GuIt>(Wr, qm, nsbH, ch[0]);
      if (wave == 0) route_finish(rc, rs, sel_w, sel_o);  // routing weights while the rows load
      float* hdec = reinterpret_cast<float*>(smem + kGuHdec) + wave * 64 * 16;
      if (lane < 8 * nsbH) header_decode(hdr, hdec + lane * 16);
      lds_drain();
      __builtin_amdgcn_wave_barrier();
      XTRACE(wave);  // per wave: weights landed, headers decoded
      const uint8_t* const xqs[1] = {xq};
      const float2* const xss[1] = {xs};
      float r[1];
      region_dots<kQ4GuIt, 1>(ch, qm, nsbH, 1, xqs, xss, hdec, reinterpret_cast<float*>(smem + kGuVbuf) + wave * 576, r);
      XTRACE(4 + wave);  // per wave: dot products done
      if (wave == 0 && a.has_sh && lane == 0) sel_w[a.k] = a.sh_gate_inp ? sigmoidf_(zsh) : 1.f;
      if ((lane & 7) == 0) gu_part[mat][half * 8 + (lane >> 3)] = r[0];
      TRACE(3);
      __syncthreads();
      if (wave == 0 && lane < 16) {
        const int rr = urow * 16 + lane;
        float g = gu_part[0][lane], u = gu_part[1][lane];
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
        if (lane == 0) st_sc1(reinterpret_cast<uint32_t*>(a.hsc) + blk * 2, __float_as_uint(s0));
        if (lane == 1) st_sc1(reinterpret_cast<uint32_t*>(a.hsc) + blk * 2 + 1, __float_as_uint(sum));
        vm_drain();  // image stores complete before the count that announces them
      }
      TRACE(4);
    }
    // counted even when routing failed, so later launches stay in step
    if (tid == 0) count<128>(a.fs + FS_GU, gid);
  } else {
    // ------------------------------------------------------------- down
    const int q = bid - a.R;
    if (tid == 0) ok_flag = 1;
    RouteState rs;  // wave 0: the selection, finished (weights, order) once the prefetch is issued
    // the routing wave runs at the gate/up waves' priority while it selects (its weight
    // prefetch, issued after, stays below the gate/up streams)
    if (wave == 0) __builtin_amdgcn_s_setprio(1);
    if (wave == 0 && !route_select<MR_ROUTE_SLEEP_DOWN>(rc, seq, sel_i, sel_k, route_tmp, rs)) {
      if (lane == 0) ok_flag = 0, fail(a.err);
    }
    if (wave == 0) __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    TRACE(1);
    if (ok_flag) {
      const size_t rb = (size_t)nsbI * 144;
      const QMap qm = q_map(nsbI);
      uint4 ch[kQ4DnSlots][kQ4DnIt];
#pragma unroll
      for (int j = 0; j < kQ4DnSlots; ++j) {
        const int s = wave + 4 * j;
        const int sc = s < a.ktot ? s : 0;
        const uint8_t* D = sc >= a.k ? a.sh_down : expert_at(a.down, sel_i[sc]);
        if (s < a.ktot) region_load<kQ4DnIt>(D + (size_t)(q * 8) * rb, qm, nsbI, ch[j]);
      }
      if (wave == 0) route_finish(rc, rs, sel_w, sel_o);  // wave 0 alone uses weights and order
      const float yres = (tid < 8 && NORM && q * 8 + tid < a.H) ? a.nr.resid[q * 8 + tid] : 0.f;
      float ybias = 0.f;  // this row's routed bias terms (layer.rs:1417-1444)
      if (tid < 8 && a.down_b)
        for (int s2 = 0; s2 < a.k; ++s2) ybias = ybias + sel_w[s2] * a.down_b[(size_t)sel_i[s2] * a.H + q * 8 + tid];
      // headers of this wave's slots: independent of the gate/up results
      const int nsw = (a.ktot - wave + 3) >> 2;  // slots of this wave: wave, wave + 4, ...
      float* hdec = reinterpret_cast<float*>(smem + kDnHdec) + wave * kDnSbW * 16;
      float* vbuf = reinterpret_cast<float*>(smem + kDnVbuf) + wave * kDnSbW * 9;
      region_headers<kQ4DnIt, kQ4DnSlots>(ch, qm, nsbI, nsw, reinterpret_cast<uint4*>(vbuf), hdec);
      TRACE(2);
      if (wave == 0 && !wait_count<MR_GU_WAIT_SLEEP, 128, 4>(a.fs + FS_GU, (seq + 1u) * (uint32_t)a.NG, a.spin_limit,
                                                         (uint32_t)a.NG / 4) && lane == 0)
        ok_flag = 0, fail(a.err);
      __syncthreads();
      TRACE(3);
      if (ok_flag) {
        // down input image of every slot -> LDS (agent-coherent direct-to-LDS loads)
        uint8_t* hq = smem + kDnHq;
        float2* hs = reinterpret_cast<float2*>(smem + kDnHs);
        {
          const int nq = a.ktot * nGI * 2;  // 16-byte pieces of the terms
          const uint8_t* src = reinterpret_cast<const uint8_t*>(a.himg);
          for (int b = wave; b * 64 < nq; b += 4) {
            const int idx = min(b * 64 + lane, nq - 1);
            __builtin_amdgcn_global_load_lds(src + (size_t)idx * 16, hq + b * 1024, 16, 0, 16 /* sc1 */);
          }
          const int npc = (a.ktot * nGI + 1) / 2;  // 16-byte pieces of the (s0, sum) pairs
          const uint8_t* ssrc = reinterpret_cast<const uint8_t*>(a.hsc);
          for (int b = wave; b * 64 < npc; b += 4) {
            const int idx = min(b * 64 + lane, npc - 1);
            __builtin_amdgcn_global_load_lds(ssrc + (size_t)idx * 16, reinterpret_cast<uint8_t*>(hs) + b * 1024, 16, 0,
                                             16 /* sc1 */);
          }
          vm_drain();
        }
        __syncthreads();
        TRACE(4);
        const uint8_t* xqs[kQ4DnSlots];
        const float2* xss[kQ4DnSlots];
#pragma unroll
        for (int j = 0; j < kQ4DnSlots; ++j) {
          const int sj = min(wave + 4 * j, a.ktot - 1);
          xqs[j] = hq + (size_t)sj * nGI * 32, xss[j] = hs + (size_t)sj * nGI;
        }
        float r[kQ4DnSlots];
        region_dots<kQ4DnIt, kQ4DnSlots>(ch, qm, nsbI, nsw, xqs, xss, hdec, vbuf, r);
        XTRACE(wave);  // per wave: dot products and row sums done
#pragma unroll
        for (int j = 0; j < kQ4DnSlots; ++j)
          if (j < nsw && (lane & 7) == 0) dn_part[wave + 4 * j][lane >> 3] = r[j];
        __syncthreads();
        if (tid < 8) {
          const int rr = q * 8 + tid;
          float yv = 0.f;  // routed slots in ascending expert order (layer.rs:1092-1106)
          for (int p = 0; p < a.k; ++p) yv = yv + dn_part[sel_o[p]][tid];
          yv = yv + ybias;
          if (a.has_sh) yv = yv + dn_part[a.k][tid];  // shared expert after the routed sum
          if (NORM) yv = yres + yv;  // hidden = residual + moe_out (layer.rs:473)
          if (rr < a.H) a.y[rr] = yv;
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
  if (a.trace && (threadIdx.x & 63) == 0)  // HW_ID: wave, SIMD, CU, SE of each wave
    a.trace[blockIdx.x * 32 + 26 + (threadIdx.x >> 6)] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
#endif
  if (tid == 0) st_sc1(wg_seq_word(a.fs), seq + 1u);
}

// Shapes the fused Q4_K kernel runs; others take the VALU path.
bool fused_q4k_supported(const mr_layer& L, int n_cu) {
  if (L.type != MR_GGML_Q4_K || L.H % 256 != 0 || L.I % 256 != 0) return false;
  if (L.H > (uint32_t)kQ4MaxH || L.I > (uint32_t)kQ4MaxI || L.H > 4u * kQ4RouterVec * 64) return false;
  const uint32_t has_sh = L.d.sh_gate ? 1u : 0u;
  if (has_sh && (L.d.sh_gate->type != MR_GGML_Q4_K || L.d.sh_up->type != MR_GGML_Q4_K ||
                 L.d.sh_down->type != MR_GGML_Q4_K || L.Ish != L.I))
    return false;
  const uint64_t ktot = L.d.top_k + has_sh;
  if (ktot > (uint64_t)kQ4MaxSlots || L.E > 512 || L.E + has_sh > (uint32_t)kMaxLogits) return false;
  // per-wave LDS slices (down): ceil(ktot/4) regions of 8 rows x I/256 super-blocks; h image
  if ((ktot + 3) / 4 * 8 * (L.I / 256) > (uint64_t)kDnSbW || ktot * L.I * 2 > (uint64_t)kDnHqBytes) return false;
  const uint64_t R = (L.E + has_sh + 3) / 4, ND = L.H / 8, NG = ktot * (L.I / 16);
  // every workgroup resident at once (106 VGPRs and 36 KB LDS allow 4 per CU; 3 are assumed)
  if (R + ND + NG > 3ull * n_cu || R + ND + NG > (uint64_t)kMaxGrid) return false;
  return true;
}

// Every workgroup of a launch must be resident at once (workgroups wait on each other):
// the occupancy the runtime reports for this kernel's registers and LDS, on an otherwise
// idle device, times the CU count must cover the grid (both instantiations).
bool fused_q4k_resident(const mr_layer& L, int n_cu) {
  const uint64_t has_sh = L.d.sh_gate ? 1u : 0u, ktot = L.d.top_k + has_sh;
  const int64_t grid = (int64_t)((L.E + has_sh + 3) / 4 + L.H / 8 + ktot * (L.I / 16));
  int b0 = 0, b1 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b0, k_fused_q4k<false>, 256, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&b1, k_fused_q4k<true>, 256, 0) != hipSuccess)
    return false;
  return (int64_t)std::min(b0, b1) * n_cu >= grid;
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
  a.H = (int)L.H, a.I = (int)L.I, a.E = (int)L.E, a.k = (int)L.d.top_k, a.ktot = a.k + a.has_sh;
  const uint64_t nGI = L.I / 16;
  a.himg = reinterpret_cast<uint32_t*>(img_base);
  a.hsc = reinterpret_cast<float*>(img_base + (uint64_t)a.ktot * nGI * 32);
  a.flags = L.d.route_flags, a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  a.R = (a.E + a.has_sh + 3) / 4;
  a.ND = (int)(L.H / 8);
  a.NG = (int)((uint64_t)a.ktot * nGI);
  a.spin_limit = L.ctx->spin_limit;
  a.pf = prefetch_plan(L.next);
  a.nr = nr;
  ProfScope ps(K, "fused_layer");
  if (nr.w)
    hipLaunchKernelGGL(k_fused_q4k<true>, dim3(a.R + a.ND + a.NG), dim3(256), 0, K.s, a);
  else
    hipLaunchKernelGGL(k_fused_q4k<false>, dim3(a.R + a.ND + a.NG), dim3(256), 0, K.s, a);
  return hipGetLastError();
}

}  // namespace mr
