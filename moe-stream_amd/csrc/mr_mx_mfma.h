// mr_mx_mfma.h -- MXFP4 weights x e4m3-split activations on the gfx950 scaled
// MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), shared by the fused decode kernel
// (mr_fused.hip) and the grouped multi-token kernels (mr_grouped.hip).
//
// A operand: 16 weight rows in native GGUF MXFP4 blocks (17 bytes: e8m0 scale
// byte + 16 code bytes); the block's scale byte is the lane's hardware A scale
// (GGUF kvalue*2^(e-128) == OCP e2m1*2^(e-127)), so no weight is dequantized.
// B operand: an activation vector split into kTerms e4m3 terms, one B column per
// term, each term with its own e8m0 scale per 32-element block; summing the
// kTerms columns of D gives the f32 dot product to ~2^-16 of each block's max.
//
// Operand layout (lane = 16*g + i):
//   A (fp4): row i, K [32g, 32g+32), nibble n (byte n/2, low nibble first) = K 32g+n;
//   B (fp8): column i, bytes 0..15 = K [16g, 16g+16), bytes 16..31 = K [64+16g, +16);
//            scale_b of lane (i, g) applies to K block g = K [32g, 32g+32);
//   D:       D[4g + r][i] in element r.
// Within a block, MFMA k=2j <-> GGUF element j and k=2j+1 <-> element j+16 (byte j
// holds both), so weight bytes are consumed exactly as stored.
//
// Activation image layout ("B image"): per 32-element block, kImgBytes bytes =
// kTerms x 32 codes in MFMA K order, plus one u32 of kTerms e8m0 scale bytes.
#pragma once

#include "mr_device.h"
#include "mr_fused_common.h"

namespace mr {

constexpr int kTerms = 4;               // e4m3 terms of an activation split (B columns used)
constexpr int kImgBytes = kTerms * 32;  // B image bytes per 32-element block

// ---- e4m3 activation split -----------------------------------------------------------
// One 32-element block is held by 8 lanes; lane m holds MFMA positions
// 4m..4m+3 = GGUF elements 2m, 2m+16, 2m+1, 2m+17 of the block.
// Term t: scale 2^(floor(log2 max|r_t|) - 7) so max|r_t|/scale is in [128, 256);
// codes by v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest even); the residual
// after kTerms terms is below 2^-16 of the block max. codes[t] is the code
// dword of term t; the kTerms scale bytes are packed into `scales`. NT < kTerms
// computes only the first NT terms (codes[t >= NT] and their scale bytes are 0).
template <int NT = kTerms>
__device__ __forceinline__ void split_block8(float v0, float v1, float v2, float v3,
                                             uint32_t codes[kTerms], uint32_t& scales) {
  static_assert(NT >= 1 && NT <= kTerms, "1..kTerms terms");
  float r0 = v0, r1 = v1, r2 = v2, r3 = v3;
  scales = 0u;
#pragma unroll
  for (int t = NT; t < kTerms; ++t) codes[t] = 0u;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float m = max8(fmaxf(fmaxf(fabsf(r0), fabsf(r1)), fmaxf(fabsf(r2), fabsf(r3))));
    const int ex = (int)((__float_as_uint(m) >> 23) & 0xFFu);  // biased exponent; 0: zero/denormal
    const int sb = ex - 7;                                     // e8m0 byte of 2^(e-7)
    uint32_t c = 0u;
    if (sb > 0) {
      const float inv = __uint_as_float((uint32_t)(254 - sb) << 23);  // 2^-(e-7)
      const float sc = __uint_as_float((uint32_t)sb << 23);           // 2^(e-7)
      c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r0 * inv, r1 * inv, 0, false);
      c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r2 * inv, r3 * inv, (int)c, true);
      const f32x2 d01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, false);
      const f32x2 d23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, true);
      r0 -= d01.x * sc, r1 -= d01.y * sc, r2 -= d23.x * sc, r3 -= d23.y * sc;
      scales |= (uint32_t)sb << (8 * t);
    }
    codes[t] = c;
  }
}

// The same split with the block's 32 elements in 4 lanes (this lane and the lanes xor 16 and
// xor 32), each holding split lanes 2n and 2n+1: a0..a3 the elements of lane 2n, b0..b3 those
// of lane 2n+1 (in the order of split_block8). ca/cb get the code dwords of both; the codes
// and scales are the same bits as split_block8's for the same block.
template <int NT = kTerms>
__device__ __forceinline__ void split_block_x2(float a0, float a1, float a2, float a3, float b0, float b1, float b2,
                                               float b3, uint32_t ca[kTerms], uint32_t cb[kTerms], uint32_t& scales) {
  static_assert(NT >= 1 && NT <= kTerms, "1..kTerms terms");
  scales = 0u;
#pragma unroll
  for (int t = NT; t < kTerms; ++t) ca[t] = cb[t] = 0u;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float m = fmaxf(fmaxf(fmaxf(fabsf(a0), fabsf(a1)), fmaxf(fabsf(a2), fabsf(a3))),
                    fmaxf(fmaxf(fabsf(b0), fabsf(b1)), fmaxf(fabsf(b2), fabsf(b3))));
    m = max_xor32(max_xor16(m));
    const int ex = (int)((__float_as_uint(m) >> 23) & 0xFFu);  // biased exponent; 0: zero/denormal
    const int sb = ex - 7;                                     // e8m0 byte of 2^(e-7)
    uint32_t c = 0u, d = 0u;
    if (sb > 0) {
      const float inv = __uint_as_float((uint32_t)(254 - sb) << 23);  // 2^-(e-7)
      const float sc = __uint_as_float((uint32_t)sb << 23);           // 2^(e-7)
      c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a0 * inv, a1 * inv, 0, false);
      c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a2 * inv, a3 * inv, (int)c, true);
      d = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(b0 * inv, b1 * inv, 0, false);
      d = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(b2 * inv, b3 * inv, (int)d, true);
      if (t + 1 < NT) {  // the residual feeds the next term
        const f32x2 c01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, false), c23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, true);
        const f32x2 d01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false), d23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
        a0 -= c01.x * sc, a1 -= c01.y * sc, a2 -= c23.x * sc, a3 -= c23.y * sc;
        b0 -= d01.x * sc, b1 -= d01.y * sc, b2 -= d23.x * sc, b3 -= d23.y * sc;
      }
      scales |= (uint32_t)sb << (8 * t);
    }
    ca[t] = c, cb[t] = d;
  }
}

// ---- operands ----------------------------------------------------------------------------
// B operand of lane (col i, group g) for K step st from a B image in LDS.
// Columns i >= kTerms and blocks past nb read `zero` (32 zero bytes in LDS),
// so the loads need no per-lane branches.
__device__ __forceinline__ void load_b(const uint8_t* img, const uint32_t* sc, const uint8_t* zero,
                                       int st, int nb, int i, int g, i32x8& B, int& sb) {
  const bool col = i < kTerms;
  const int b0 = 4 * st + (g >> 1), b1 = b0 + 2, off = i * 32 + 16 * (g & 1);
  const uint8_t* p0 = (col && b0 < nb) ? img + (size_t)b0 * kImgBytes + off : zero;
  const uint8_t* p1 = (col && b1 < nb) ? img + (size_t)b1 * kImgBytes + off : zero;
  const i32x4 v0 = *reinterpret_cast<const i32x4*>(p0);
  const i32x4 v1 = *reinterpret_cast<const i32x4*>(p1);
  B = i32x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  const int bs = min(4 * st + g, nb - 1);
  // Columns past kTerms multiply a zero B operand, so any finite scale serves them: every
  // lane takes a byte of the block's scale word (bytes are <= 247, never the NaN code 0xFF),
  // with no branch around the LDS load. A byte load: the value needs no ALU step, which the
  // scheduler would otherwise hoist above the previous MFMA together with a wait for it.
  sb = (int)reinterpret_cast<const uint8_t*>(sc)[bs * 4 + (i & 3)];
}

// Raw 20-byte window (5 aligned dwords) holding one 17-byte block.
struct RawBlk {
  uint32_t d[5];
};
// Global (not flat) loads: a flat load also counts on the LDS counter, so a later wait for
// its data would also wait for every LDS read issued meanwhile.
__device__ __forceinline__ void raw_load(const uint8_t* p, RawBlk& r) {
  const __attribute__((address_space(1))) uint32_t* w =
      (const __attribute__((address_space(1))) uint32_t*)(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)3);
  r.d[0] = w[0], r.d[1] = w[1], r.d[2] = w[2], r.d[3] = w[3], r.d[4] = w[4];
}
__device__ __forceinline__ void raw_zero(RawBlk& r) { r.d[0] = r.d[1] = r.d[2] = r.d[3] = r.d[4] = 0u; }

// A operand of one lane from a raw block window (sh = block address & 3; the 16 code
// bytes start at byte sh+1): the 4 code dwords and the e8m0 scale byte. An invalid
// block (past the row end) becomes all-zero codes, so it adds exactly 0 whatever B holds
// (as long as B is finite).
struct AOp {
  uint32_t q[4];
};
__device__ __forceinline__ AOp prep_a(const RawBlk& r, uint32_t sh, bool valid, int& sa) {
  const uint32_t t = sh + 1u;
  AOp a;
  if (t == 4u) {
    a.q[0] = r.d[1], a.q[1] = r.d[2], a.q[2] = r.d[3], a.q[3] = r.d[4];
  } else {
    a.q[0] = __builtin_amdgcn_alignbyte(r.d[1], r.d[0], t);
    a.q[1] = __builtin_amdgcn_alignbyte(r.d[2], r.d[1], t);
    a.q[2] = __builtin_amdgcn_alignbyte(r.d[3], r.d[2], t);
    a.q[3] = __builtin_amdgcn_alignbyte(r.d[4], r.d[3], t);
  }
  sa = valid ? (int)((r.d[0] >> (8u * sh)) & 0xFFu) : 127;
  if (!valid) a.q[0] = a.q[1] = a.q[2] = a.q[3] = 0u;
  return a;
}
__device__ __forceinline__ f32x4 mfma_op(const AOp& a, int sa, const i32x8& B, int sb, f32x4 acc) {
  const i32x8 A = {(int)a.q[0], (int)a.q[1], (int)a.q[2], (int)a.q[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 4, 0, 0, sa, 0, sb);
}

// One MFMA on a raw block window; sh = block address & 3. The 16 code bytes
// start at byte sh+1 of the window.
__device__ __forceinline__ f32x4 mfma_raw(const RawBlk& r, uint32_t sh, bool valid, const i32x8& B,
                                          int sb, f32x4 acc) {
  // selects, not a branch: a divergent branch per step splits the chain into basic blocks,
  // across which the compiler reorders the MFMAs away from their operands
  const uint32_t t = sh + 1u;
  const bool hi = t == 4u;
  const uint32_t q0 = hi ? r.d[1] : __builtin_amdgcn_alignbyte(r.d[1], r.d[0], t);
  const uint32_t q1 = hi ? r.d[2] : __builtin_amdgcn_alignbyte(r.d[2], r.d[1], t);
  const uint32_t q2 = hi ? r.d[3] : __builtin_amdgcn_alignbyte(r.d[3], r.d[2], t);
  const uint32_t q3 = hi ? r.d[4] : __builtin_amdgcn_alignbyte(r.d[4], r.d[3], t);
  const int sa = valid ? (int)((r.d[0] >> (8u * sh)) & 0xFFu) : 127;
  const i32x8 A = {(int)q0, (int)q1, (int)q2, (int)q3, 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 4, 0, 0, sa, 0, sb);
}

// mfma_raw without a branch: each code dword is the 64-bit dword pair shifted right by
// sh+1 bytes (a shift of 4 bytes selects the upper dword). For chains whose windows are read
// just before use, where a divergent branch around the shifts would cost more than the shifts.
__device__ __forceinline__ f32x4 mfma_raw_nb(const RawBlk& r, uint32_t sh, bool valid, const i32x8& B,
                                             int sb, f32x4 acc) {
  const uint32_t t8 = 8u * (sh + 1u);
  const uint32_t q0 = (uint32_t)((((uint64_t)r.d[1] << 32) | r.d[0]) >> t8);
  const uint32_t q1 = (uint32_t)((((uint64_t)r.d[2] << 32) | r.d[1]) >> t8);
  const uint32_t q2 = (uint32_t)((((uint64_t)r.d[3] << 32) | r.d[2]) >> t8);
  const uint32_t q3 = (uint32_t)((((uint64_t)r.d[4] << 32) | r.d[3]) >> t8);
  const int sa = valid ? (int)((r.d[0] >> (8u * sh)) & 0xFFu) : 127;
  const i32x8 A = {(int)q0, (int)q1, (int)q2, (int)q3, 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 4, 0, 0, sa, 0, sb);
}

// B operand for a prepared-A chain: column i reads term i%4 (columns 4..15 repeat
// the terms; only columns 0..3 are summed afterwards, and the data is finite), block
// indices clamp to the last block (the A operand of an invalid block is zero).
// base = image + (i%4)*32 + 16*(g&1) of this lane.
__device__ __forceinline__ void load_b_fast(const uint8_t* base, const uint32_t* sc, int st, int nb, int i,
                                            int g, i32x8& B, int& sb) {
  const int b0 = min(4 * st + (g >> 1), nb - 1), b1 = min(4 * st + 2 + (g >> 1), nb - 1);
  const i32x4 v0 = *reinterpret_cast<const i32x4*>(base + b0 * kImgBytes);
  const i32x4 v1 = *reinterpret_cast<const i32x4*>(base + b1 * kImgBytes);
  B = i32x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  sb = (int)reinterpret_cast<const uint8_t*>(sc)[min(4 * st + g, nb - 1) * 4 + (i & 3)];
}
}  // namespace mr
