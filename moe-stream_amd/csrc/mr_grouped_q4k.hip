// mr_grouped_q4k.hip -- multi-token (prefill / batched) Q4_K MoE experts as grouped GEMMs on
// the gfx950 int8 MFMA (v_mfma_i32_16x16x32_i8).
//
// The reference runs each expert once over all of its tokens (index_select, gate/up/act/down,
// index_add: layer.rs:2148-2183; on the GPU one projection per expert, metal/mod.rs:911-962).
// Here, after the grouping of mr_grouped.hip (k_group: (token, slot) pairs by expert):
//   k_split_q4k        activation rows -> two int8 terms per element and a scale per 256-element
//                      super-block: v = s*(t0 + t1/128), s = max|v|/127 (|error| <= s/256), plus
//                      the f32 sum of every 32-element sub-block.
//   k_grouped_q4k<1>   gate and up for one (expert, 32-row tile, 32-pair tile); epilogue bias +
//                      activation x routing weight -> h [pair][I] (f32).
//   k_split_q4k        h rows -> terms.
//   k_grouped_q4k<0>   down for one (expert, 64-row tile, 32-pair tile) -> o [pair][H].
//   k_combine          (mr_grouped.hip) the pairs of a token in ascending expert order, then the
//                      shared expert scaled by its sigmoid gate (layer.rs:1092-1106, 1935-1951).
// A work item reads its expert's weight rows once for its 32 pairs, so an expert's weights are
// read ceil(n_e / 32) times per call (from HBM once, the repeats from the XCD's L2), against once
// per (token, slot) on the per-token path.
//
// Arithmetic per sub-block j of a Q4_K super-block (dequant.rs:218-262 regrouped):
//   sum_k w_k x_k = d*sc_j * sum_k q_k x_k - (dmin*m_j) * sum_k x_k,
// with sum_k q_k x_k = s * (A0 + A1/128), A_t = sum_k q_k t_k exact in int32 (one MFMA per term:
// A = 16 rows x 32 nibbles as int8, B = 32 elements x 16 pairs). The sc_j weighting is summed
// over the super-block in int32 (|sum| < 8 * 63 * 32*15*127 < 2^31), then scaled by d*s in f32.
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"

#include <algorithm>

namespace mr {

typedef int i32x4v __attribute__((ext_vector_type(4)));

constexpr int kQPairs = 32;    // pairs per work item (2 MFMA column groups of 16)
constexpr int kQXcds = 8;      // workgroups are dispatched round robin over the 8 XCDs

// ---- activation rows -> terms ---------------------------------------------------------------
// One wave per (row, 256-element super-block): lane l holds elements 4l .. 4l+3.
__global__ __launch_bounds__(256) void k_split_q4k(const float* __restrict__ src, int n_rows, int D,
                                                   int8_t* __restrict__ t0, int8_t* __restrict__ t1,
                                                   float* __restrict__ s_out, float* __restrict__ x_sum) {
  const int lane = threadIdx.x & 63;
  const int nsb = D >> 8;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)n_rows * nsb) return;  // uniform per wave
  const int64_t r = item / nsb;
  const int sb = (int)(item - r * nsb);
  const size_t off = (size_t)r * D + (size_t)sb * 256 + 4 * lane;
  const f32x4 v = *reinterpret_cast<const f32x4*>(src + off);
  float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  mx = wave_max(mx);
  // sub-block sums: lanes 8j .. 8j+7 hold sub-block j (elements in order within a lane, then
  // a butterfly over the 8 lanes)
  float ps = (v.x + v.y) + (v.z + v.w);
  ps += __shfl_xor(ps, 1, 64);
  ps += __shfl_xor(ps, 2, 64);
  ps += __shfl_xor(ps, 4, 64);
  const float s = mx / 127.f;
  const float inv = mx > 0.f ? 127.f / mx : 0.f;
  const float inv1 = mx > 0.f ? 128.f * inv : 0.f;
  uint32_t w0 = 0, w1 = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float x = v[c];
    const float a = fminf(fmaxf(rintf(x * inv), -127.f), 127.f);
    const float res = __builtin_fmaf(-a, s, x);  // x - s*t0, one rounding
    const float b = fminf(fmaxf(rintf(res * inv1), -127.f), 127.f);
    w0 |= ((uint32_t)(int)a & 0xFFu) << (8 * c);
    w1 |= ((uint32_t)(int)b & 0xFFu) << (8 * c);
  }
  *reinterpret_cast<uint32_t*>(t0 + off) = w0;
  *reinterpret_cast<uint32_t*>(t1 + off) = w1;
  if (lane == 0) s_out[(size_t)r * nsb + sb] = s;
  if ((lane & 7) == 0) x_sum[(size_t)r * (D >> 5) + sb * 8 + (lane >> 3)] = ps;
}

// ---- shared-expert gate: sigmoid(x . gate_inp) per token (layer.rs:1935-1951) -------------------
// The order of the per-token path (k_gateup_valu): lane-strided fma, then a wave sum.
__global__ __launch_bounds__(64) void k_sh_gate(const float* __restrict__ x, int H, const float* __restrict__ gi,
                                                float* __restrict__ sig) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float z = 0.f;
  if (gi)
#pragma unroll 8
    for (int c = lane; c < H; c += 64) z = __builtin_fmaf(x[(size_t)t * H + c], gi[c], z);  // loads issued ahead
  z = wave_sum(z);
  if (lane == 0) sig[t] = gi ? sigmoidf_(z) : 1.0f;
}

// ---- grouped GEMM ---------------------------------------------------------------------------
struct GQ4Args {
  ExpertLoc w0;              // gate (GATEUP) or down
  ExpertLoc w1;              // up (GATEUP)
  const float* b0;           // gate bias [E][M] or null (GATEUP)
  const float* b1;           // up bias
  const int8_t* t0;          // B terms [rows][K]
  const int8_t* t1;
  const float* bs;           // [rows][K/256] term scale
  const float* bx;           // [rows][K/32] sub-block sums
  const int32_t* pair_tok;   // B row of pair p, or null (row = p)
  const float* pair_w;       // GATEUP: routing weight of pair p, or null (1)
  const int32_t* exp_off;    // [E+1] pair offsets (null: one expert of single_p pairs)
  const int32_t* tile_off;   // [E+1] 32-pair tile offsets
  int single_p;
  float* out;                // GATEUP: h [P][M]; down: o [P][M]
  int M, K, E, act;
  float alpha, limit;
};

// Work item: (expert e, row tile, 32-pair tile); 4 waves of 16 rows each (gate/up: waves 0-1 gate,
// 2-3 up, the same 32 rows; down: 64 rows). Per 256-element super-block of K:
//   A: the wave's 16 rows x 144 bytes as 16-byte pieces (3 loads per lane, each covering about
//      seven rows' whole super-blocks), one super-block ahead in registers, then written to the
//      wave's LDS slice; lanes g = 0 decode their row's 16-byte header from it (d, dmin*m_j, sc_j)
//      and lane (i, g) reads the 8 bytes of row i that hold elements [8g, 8g+8) of a sub-block
//      pair (low nibbles: even sub-blocks, high: odd).
//   B: the pairs' two term rows (32 x 2 x 256 bytes), scales and sub-block sums, staged in LDS by
//      all 256 threads (one super-block ahead in registers, double-buffered LDS) in MFMA operand
//      order: the 8 bytes that lane l takes for (term, pair group, sub-block j) sit in slot
//      l ^ 2j of a 512-byte block, so every LDS read of a wave is 64 consecutive 8-byte slots
//      and the staging writes of one pair's 16 chunks spread over 8 bank pairs.
//   min term: sum_j (dmin*m_j)[row] * X_j[pair] is a [16 x 8] x [8 x 16] f32 product per pair
//      group, two v_mfma_f32_16x16x4_f32 per super-block instead of 8 FMAs per lane and sub-block.
// D layout of the MFMAs: lane (i, g) holds rows 4g .. 4g+3 of the wave's tile, pair column i.
template <bool GATEUP>
__global__ __launch_bounds__(256, 3) void k_grouped_q4k(GQ4Args a) {
  __shared__ __align__(16) uint8_t bst[2][2 * 2 * 8 * 512];  // [buf][term][pair group][sub-block][64 slots x 8 B]
  __shared__ float bsx[2][2 * 2 * 64];                       // [buf][pair group][j / 4][lane]: sub-block sums
  __shared__ float bss[2][kQPairs];                          // term scales
  __shared__ __align__(16) int hsc[4][8][16];                // [wave][sub-block][row] sc_j
  __shared__ float hm[4][2 * 64];                            // [wave][j / 4][lane]: dmin*m_j of row lane & 15
  __shared__ __align__(16) float hd[4][16];                  // d
  __shared__ __align__(16) uint8_t ast[4][16 * 144];         // [wave][row][super-block bytes]
  __shared__ float pw[kQPairs];                                    // routing weights (GATEUP)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  constexpr int kRows = GATEUP ? 32 : 64;  // output rows of one matrix per work item
  const int n_rt = (a.M + kRows - 1) / kRows;
  const int n_tiles = a.exp_off ? a.tile_off[a.E] : (a.single_p + kQPairs - 1) / kQPairs;
  const int n_work = n_rt * n_tiles;
  const int per_xcd = (n_work + kQXcds - 1) / kQXcds;
  const int loc = blockIdx.x / kQXcds;
  const int w = (blockIdx.x % kQXcds) * per_xcd + loc;
  if (loc >= per_xcd || w >= n_work) return;  // uniform
  int e = 0, tl = 0, rt = 0, p0 = 0, np = 0;
  if (a.exp_off) {
    int lo = 0, hi = a.E;  // expert: n_rt * tile_off[e] <= w < n_rt * tile_off[e+1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (n_rt * a.tile_off[mid] <= w) lo = mid; else hi = mid;
    }
    e = lo;
    const int nt_e = a.tile_off[e + 1] - a.tile_off[e];
    const int wl = w - n_rt * a.tile_off[e];
    rt = wl / nt_e, tl = wl - rt * nt_e;
    p0 = a.exp_off[e] + tl * kQPairs;
    np = min(kQPairs, a.exp_off[e + 1] - p0);
  } else {
    rt = w / n_tiles, tl = w - rt * n_tiles;
    p0 = tl * kQPairs;
    np = min(kQPairs, a.single_p - p0);
  }
  const int nsb = a.K >> 8;
  const uint64_t rb = (uint64_t)nsb * 144;
  const int m = GATEUP ? (wave >> 1) : 0;
  const int wrow0 = rt * kRows + (GATEUP ? (wave & 1) : wave) * 16;
  const bool tile_in = wrow0 < a.M;  // uniform
  const uint8_t* W = expert_at(m ? a.w1 : a.w0, e);
  // A pieces of this lane: slot it*64 + lane < 144 = (row slot / 9, 16-byte piece slot % 9)
  const uint8_t* asrc[3];
  int adst[3];
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int sl = min(it * 64 + lane, 143);
    asrc[it] = W + (uint64_t)min(wrow0 + sl / 9, a.M - 1) * rb + (sl % 9) * 16;
    adst[it] = (sl / 9) * 144 + (sl % 9) * 16;
  }
  if (GATEUP && tid < kQPairs) pw[tid] = a.pair_w ? a.pair_w[p0 + min(tid, np - 1)] : 1.f;

  // B pieces of this thread: piece j*256 + tid = (term, pair, 16-byte chunk); the chunk holds
  // elements [8 g0, 8 g0 + 16) of sub-block ch / 2, g0 = 2 (ch & 1): two operand slots
  const int8_t* bsrc[4];
  int bdst0[4], bdst1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pc = j * 256 + tid;
    const int term = pc >> 9, pr = (pc >> 4) & 31, ch = pc & 15;
    const int p = p0 + min(pr, np - 1);
    const int row = a.pair_tok ? a.pair_tok[p] : p;
    bsrc[j] = (term ? a.t1 : a.t0) + (size_t)row * a.K + ch * 16;
    const int sbj = ch >> 1, g0 = 2 * (ch & 1), ii = pr & 15;
    const int blk = ((term * 2 + (pr >> 4)) * 8 + sbj) * 512;
    bdst0[j] = blk + ((16 * g0 + ii) ^ (2 * sbj)) * 8;
    bdst1[j] = blk + ((16 * (g0 + 1) + ii) ^ (2 * sbj)) * 8;
  }
  // this thread's sub-block sum (pair tid / 8, sub-block tid % 8) in B operand order
  const int xdst = (((tid >> 3) >> 4) * 2 + ((tid & 7) >> 2)) * 64 + 16 * (tid & 3) + ((tid >> 3) & 15);
  const int xrow = [&] {  // pair of this thread's sub-block sum (tid = pair * 8 + sub-block)
    const int p = p0 + min(tid >> 3, np - 1);
    return a.pair_tok ? a.pair_tok[p] : p;
  }();
  const int srow = [&] {
    const int p = p0 + min(tid & 31, np - 1);
    return a.pair_tok ? a.pair_tok[p] : p;
  }();
  struct BRegs {
    i32x4 v[4];
    float x, s;
  };
  auto load_b = [&](int sbk, BRegs& br) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      br.v[j] = *(const __attribute__((address_space(1))) i32x4*)(bsrc[j] + (size_t)sbk * 256);
    br.x = a.bx[(size_t)xrow * (a.K >> 5) + sbk * 8 + (tid & 7)];
    br.s = a.bs[(size_t)srow * nsb + sbk];
  };
  auto store_b = [&](const BRegs& br, int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<uint64_t*>(&bst[buf][0] + bdst0[j]) =
          ((uint64_t)(uint32_t)br.v[j][1] << 32) | (uint32_t)br.v[j][0];
      *reinterpret_cast<uint64_t*>(&bst[buf][0] + bdst1[j]) =
          ((uint64_t)(uint32_t)br.v[j][3] << 32) | (uint32_t)br.v[j][2];
    }
    bsx[buf][xdst] = br.x;
    if (tid < kQPairs) bss[buf][tid] = br.s;
  };
  struct ARegs {
    i32x4 v[3];
  };
  auto load_a = [&](int sbk, ARegs& ar) {
#pragma unroll
    for (int it = 0; it < 3; ++it)
      if (it < 2 || lane < 16)
        ar.v[it] = *(const __attribute__((address_space(1))) i32x4*)(asrc[it] + (size_t)sbk * 144);
  };
  auto store_a = [&](const ARegs& ar) {  // the wave's slice: its reads of the last super-block are done
#pragma unroll
    for (int it = 0; it < 3; ++it)
      if (it < 2 || lane < 16) *reinterpret_cast<i32x4*>(&ast[wave][adst[it]]) = ar.v[it];
  };
  // header of row i (lanes g == 0, from the wave's slice) -> LDS: d, dmin*m_j (the reference's f32
  // products), sc_j
  auto decode_hdr = [&]() {
    if (g == 0) {
      const i32x4 hdr = *reinterpret_cast<const i32x4*>(&ast[wave][i * 144]);
      const uint32_t dd = (uint32_t)hdr[0];
      const uint32_t s3[3] = {(uint32_t)hdr[1], (uint32_t)hdr[2], (uint32_t)hdr[3]};
      const float d = h2f(dd & 0xFFFFu), dmin = h2f(dd >> 16);
      hd[wave][i] = d;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t sc, mm;
        q4k_scale_min((uint32_t)j, s3, sc, mm);
        hsc[wave][j][i] = (int)sc;
        hm[wave][(j >> 2) * 64 + 16 * (j & 3) + i] = dmin * (float)mm;
      }
    }
  };

  f32x4 acc[2];
  acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  BRegs bR;
  ARegs aR;
  load_b(0, bR);
  load_a(0, aR);
  for (int sbk = 0; sbk < nsb; ++sbk) {
    const int buf = sbk & 1;
    store_b(bR, buf);  // buffer buf was last read in super-block sbk-2, before the last barrier
    store_a(aR);
    decode_hdr();      // this wave's header slots were last read before the last barrier
    __syncthreads();   // the stages of super-block sbk and the headers are in LDS
    if (sbk + 1 < nsb) {
      load_b(sbk + 1, bR);
      load_a(sbk + 1, aR);
    }
    if (tile_in) {
      const uint8_t* bb = &bst[buf][0];
      int I0[2][4], I1[2][4];
#pragma unroll
      for (int pg = 0; pg < 2; ++pg)
#pragma unroll
        for (int r = 0; r < 4; ++r) I0[pg][r] = I1[pg][r] = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // A: elements [8g, 8g+8) of sub-block j of row i as int8 (low nibbles: even j)
        const uint64_t qb = *reinterpret_cast<const uint64_t*>(&ast[wave][i * 144 + 16 + 32 * (j >> 1) + 8 * g]);
        const uint32_t lo = (uint32_t)qb, hi = (uint32_t)(qb >> 32);
        const uint32_t sh = (j & 1) * 4;
        const long av = (long)(((uint64_t)((hi >> sh) & 0x0F0F0F0Fu) << 32) | ((lo >> sh) & 0x0F0F0F0Fu));
        const i32x4v scv = *reinterpret_cast<const i32x4v*>(&hsc[wave][j][4 * g]);
        const int slot = (lane ^ (2 * j)) * 8;
#pragma unroll
        for (int pg = 0; pg < 2; ++pg) {
          const long bv0 = *reinterpret_cast<const long*>(bb + ((0 * 2 + pg) * 8 + j) * 512 + slot);
          const long bv1 = *reinterpret_cast<const long*>(bb + ((1 * 2 + pg) * 8 + j) * 512 + slot);
          const i32x4v z = {0, 0, 0, 0};
          const i32x4v d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv0, z, 0, 0, 0);
          const i32x4v d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv1, z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            I0[pg][r] += __mul24(scv[r], d0[r]);
            I1[pg][r] += __mul24(scv[r], d1[r]);
          }
        }
      }
      // min term: [16 rows x 8 sub-blocks] x [8 sub-blocks x 16 pairs] per pair group
      f32x4 Mn[2];
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) {
        Mn[pg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 2; ++c)
          Mn[pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(hm[wave][c * 64 + lane], bsx[buf][(pg * 2 + c) * 64 + lane],
                                                        Mn[pg], 0, 0, 0);
      }
      const f32x4 dv = *reinterpret_cast<const f32x4*>(&hd[wave][4 * g]);
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) {
        const float s = bss[buf][pg * 16 + i];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = __builtin_fmaf((float)I1[pg][r], 0.0078125f, (float)I0[pg][r]);  // A0 + A1/128
          acc[pg][r] = __builtin_fmaf(dv[r] * s, v, acc[pg][r]) - Mn[pg][r];
        }
      }
    }
  }
  if (GATEUP) {
    __syncthreads();  // every wave is done with the stages: reuse them for the gate/up tiles
    float* ep = reinterpret_cast<float*>(&bst[0][0]);  // [mat][32 rows][32 pairs]
#pragma unroll
    for (int pg = 0; pg < 2; ++pg)
#pragma unroll
      for (int r = 0; r < 4; ++r) ep[(m * 32 + (wave & 1) * 16 + 4 * g + r) * kQPairs + pg * 16 + i] = acc[pg][r];
    __syncthreads();
    const int r0 = rt * kRows;
    for (int q = tid; q < 32 * kQPairs; q += 256) {
      const int pl = q >> 5, rr = q & 31;  // consecutive threads: consecutive rows of one pair
      const int row = r0 + rr;
      if (pl >= np || row >= a.M) continue;
      float gv = ep[rr * kQPairs + pl], uv = ep[(32 + rr) * kQPairs + pl];
      if (a.b0) gv = gv + a.b0[(size_t)e * a.M + row];
      if (a.b1) uv = uv + a.b1[(size_t)e * a.M + row];
      const float h = a.act == MR_ACT_SWIGLU_OAI ? swiglu_oai(gv, uv, a.alpha, a.limit) : silu_mul(gv, uv);
      a.out[(size_t)(p0 + pl) * a.M + row] = h * pw[pl];
    }
  } else if (tile_in) {
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      const int pl = pg * 16 + i;
      if (pl < np && wrow0 + 4 * g < a.M)
        *reinterpret_cast<f32x4*>(a.out + (size_t)(p0 + pl) * a.M + wrow0 + 4 * g) = acc[pg];
    }
  }
}

// ---- host side -------------------------------------------------------------------------------
namespace {
constexpr uint64_t kQAlign = 256;
uint64_t qup(uint64_t v) { return (v + kQAlign - 1) / kQAlign * kQAlign; }
struct TermsPlan {
  uint64_t t0, t1, s, x, total;
};
TermsPlan terms_plan(uint64_t rows, uint64_t D, uint64_t o) {
  TermsPlan p{};
  p.t0 = o, o += qup(rows * D);
  p.t1 = o, o += qup(rows * D);
  p.s = o, o += qup(rows * (D / 256) * 4);
  p.x = o, o += qup(rows * (D / 32) * 4);
  p.total = o;
  return p;
}
struct Q4Plan {
  uint64_t pair_tok, pair_w, pair_of, exp_off, tile_off;
  TermsPlan xt, ht, hst;
  uint64_t h, o, hsh, osh, sig, total;
};
Q4Plan q4_plan(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish) {
  Q4Plan p{};
  const uint64_t P = T * k;
  uint64_t o = 0;
  p.pair_tok = o, o += qup(P * 4);
  p.pair_w = o, o += qup(P * 4);
  p.pair_of = o, o += qup(P * 4);
  p.exp_off = o, o += qup((E + 1) * 4);
  p.tile_off = o, o += qup((E + 1) * 4);
  p.xt = terms_plan(T, H, o), o = p.xt.total;
  p.h = o, o += qup(P * I * 4);
  p.ht = terms_plan(P, I, o), o = p.ht.total;
  p.o = o, o += qup(P * H * 4);
  if (Ish) {
    p.hsh = o, o += qup(T * Ish * 4);
    p.hst = terms_plan(T, Ish, o), o = p.hst.total;
    p.osh = o, o += qup(T * H * 4);
    p.sig = o, o += qup(T * 4);
  }
  p.total = o;
  return p;
}
struct Terms {
  int8_t* t0;
  int8_t* t1;
  float* s;
  float* x;
};
Terms terms_at(char* b, const TermsPlan& p) {
  return Terms{reinterpret_cast<int8_t*>(b + p.t0), reinterpret_cast<int8_t*>(b + p.t1),
               reinterpret_cast<float*>(b + p.s), reinterpret_cast<float*>(b + p.x)};
}
hipError_t split(const Launch& K, const float* src, uint64_t rows, uint32_t D, const Terms& t) {
  const uint64_t items = rows * (D / 256);
  ProfScope ps(K, "split_q4k");
  hipLaunchKernelGGL(k_split_q4k, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, K.s, src, (int)rows, (int)D, t.t0,
                     t.t1, t.s, t.x);
  return hipGetLastError();
}
}  // namespace

uint64_t grouped_q4k_scratch_bytes(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish) {
  return q4_plan(T, k, E, I, H, Ish).total;
}

hipError_t launch_sh_gate(const Launch& K, const float* x, uint32_t T, int H, const float* gate_inp, float* sig) {
  ProfScope ps(K, "shared_gate");
  hipLaunchKernelGGL(k_sh_gate, dim3(T), dim3(64), 0, K.s, x, H, gate_inp, sig);
  return hipGetLastError();
}

// Q4_K routed experts (and a Q4_K shared expert) with K dimensions in whole super-blocks.
bool grouped_q4k_supported(const mr_layer& L) {
  if (L.type != MR_GGML_Q4_K || L.d.top_k > 16 || L.E > 1024) return false;
  if (L.H % 256 != 0 || L.I % 256 != 0 || L.H % 4 != 0) return false;
  if (L.d.sh_gate && (L.d.sh_gate->type != MR_GGML_Q4_K || L.d.sh_down->type != MR_GGML_Q4_K || L.Ish % 256 != 0))
    return false;
  return true;
}

hipError_t launch_grouped_q4k(const Launch& K, const mr_layer& L, const float* x, uint32_t T, const int32_t* idx,
                              const float* w, float* y, void* scratch) {
  const int k = (int)L.d.top_k, E = (int)L.E, H = (int)L.H, I = (int)L.I, Ish = L.d.sh_gate ? (int)L.Ish : 0;
  const int P = (int)T * k;
  const Q4Plan p = q4_plan(T, k, E, I, H, Ish);
  char* b = static_cast<char*>(scratch);
  int32_t* pair_tok = reinterpret_cast<int32_t*>(b + p.pair_tok);
  float* pair_w = reinterpret_cast<float*>(b + p.pair_w);
  int32_t* pair_of = reinterpret_cast<int32_t*>(b + p.pair_of);
  int32_t* exp_off = reinterpret_cast<int32_t*>(b + p.exp_off);
  int32_t* tile_off = reinterpret_cast<int32_t*>(b + p.tile_off);
  const Terms xt = terms_at(b, p.xt), ht = terms_at(b, p.ht);
  float* h = reinterpret_cast<float*>(b + p.h);
  float* o = reinterpret_cast<float*>(b + p.o);
  hipError_t e;
  if ((e = launch_group(K, idx, w, P, k, E, pair_tok, pair_w, pair_of, exp_off, tile_off)) != hipSuccess) return e;
  if ((e = split(K, x, T, (uint32_t)H, xt)) != hipSuccess) return e;
  const int max_tiles = (P + kQPairs - 1) / kQPairs + E;
  GQ4Args a{};
  a.w0 = expert_loc(L.d.gate), a.w1 = expert_loc(L.d.up), a.b0 = L.d.gate_bias, a.b1 = L.d.up_bias;
  a.t0 = xt.t0, a.t1 = xt.t1, a.bs = xt.s, a.bx = xt.x;
  a.pair_tok = pair_tok, a.pair_w = pair_w, a.exp_off = exp_off, a.tile_off = tile_off;
  a.out = h, a.M = I, a.K = H, a.E = E, a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  {
    ProfScope ps(K, "grouped_q4k_gateup");
    hipLaunchKernelGGL(k_grouped_q4k<true>, dim3(grouped_grid((uint64_t)((I + 31) / 32) * max_tiles)), dim3(256), 0, K.s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = split(K, h, (uint64_t)P, (uint32_t)I, ht)) != hipSuccess) return e;
  GQ4Args d{};
  d.w0 = expert_loc(L.d.down);
  d.t0 = ht.t0, d.t1 = ht.t1, d.bs = ht.s, d.bx = ht.x;
  d.exp_off = exp_off, d.tile_off = tile_off, d.out = o, d.M = H, d.K = I, d.E = E;
  {
    ProfScope ps(K, "grouped_q4k_down");
    hipLaunchKernelGGL(k_grouped_q4k<false>, dim3(grouped_grid((uint64_t)((H + 63) / 64) * max_tiles)), dim3(256), 0, K.s, d);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  float* osh = nullptr;
  float* sig = nullptr;
  if (Ish) {  // the shared expert: one expert over all T tokens, weight 1, then its sigmoid gate
    float* hsh = reinterpret_cast<float*>(b + p.hsh);
    const Terms hst = terms_at(b, p.hst);
    osh = reinterpret_cast<float*>(b + p.osh);
    sig = reinterpret_cast<float*>(b + p.sig);
    const int tiles = ((int)T + kQPairs - 1) / kQPairs;
    GQ4Args s{};
    s.w0 = expert_loc(L.d.sh_gate), s.w1 = expert_loc(L.d.sh_up);
    s.t0 = xt.t0, s.t1 = xt.t1, s.bs = xt.s, s.bx = xt.x;
    s.single_p = (int)T, s.out = hsh, s.M = Ish, s.K = H, s.E = 1, s.act = MR_ACT_SILU;
    {
      ProfScope ps(K, "grouped_q4k_shared_gateup");
      hipLaunchKernelGGL(k_grouped_q4k<true>, dim3(grouped_grid((uint64_t)((Ish + 31) / 32) * tiles)), dim3(256), 0, K.s, s);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if ((e = split(K, hsh, T, (uint32_t)Ish, hst)) != hipSuccess) return e;
    GQ4Args sd{};
    sd.w0 = expert_loc(L.d.sh_down);
    sd.t0 = hst.t0, sd.t1 = hst.t1, sd.bs = hst.s, sd.bx = hst.x;
    sd.single_p = (int)T, sd.out = osh, sd.M = H, sd.K = Ish, sd.E = 1;
    {
      ProfScope ps(K, "grouped_q4k_shared_down");
      hipLaunchKernelGGL(k_grouped_q4k<false>, dim3(grouped_grid((uint64_t)((H + 63) / 64) * tiles)), dim3(256), 0, K.s, sd);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if ((e = launch_sh_gate(K, x, T, H, L.d.sh_gate_inp, sig)) != hipSuccess) return e;
  }
  return launch_combine(K, o, pair_of, idx, w, L.d.down_bias, T, k, H, osh, sig, y);
}

}  // namespace mr
