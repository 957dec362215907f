// mr_device.h -- gfx950 device helpers shared by the MoE kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mr {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bits_f32(uint32_t b) { return __uint_as_float(b); }

// e8m0 byte -> 2^(e-128), the half scale of dequant.rs:589-597 (denormal for e < 2).
__device__ __forceinline__ float e8m0_half(uint32_t e) {
  return e < 2u ? bits_f32(0x00200000u << e) : bits_f32((e - 1u) << 23);
}

// IEEE binary16 bits -> float, exact (half::f16::to_f32, dequant.rs:37-41).
__device__ __forceinline__ float h2f(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (ex == 0) {
    float v = (float)man * 5.9604644775390625e-08f;  // man * 2^-24, exact
    return bits_f32(__float_as_uint(v) | sign);
  }
  if (ex == 31) return bits_f32(sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u));
  return bits_f32(sign | ((ex + 112u) << 23) | (man << 13));
}

// float -> IEEE binary16 bits, round to nearest even, integer-only (matches
// numpy's float32 -> float16 conversion; used by the synthetic generator).
__device__ __forceinline__ uint32_t f2h_rne(float f) {
  uint32_t x = __float_as_uint(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u);
  if (ax >= 0x477FF000u) return sign | 0x7C00u;  // rounds to >= 65520 -> inf
  if (ax < 0x38800000u) {                        // below 2^-14: f16 subnormal or zero
    if (ax < 0x33000000u) return sign;           // < 2^-25 rounds to zero
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;  // value = m * 2^(e-150); f16 sub unit 2^-24 -> shift = 126 - e
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return sign | q;
  }
  uint32_t e = (ax >> 23) - 112u;
  uint32_t m = ax & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  return sign | q;
}

// Load one 17-byte MXFP4 block at any byte alignment with five aligned dword
// loads and byte funnel shifts. Each dword read contains at least one byte of
// the block, so no access leaves the block's own 4-byte-aligned words.
__device__ __forceinline__ void mx_load_block(const uint8_t* p, uint32_t& scale, uint32_t q[4]) {
  uintptr_t a = reinterpret_cast<uintptr_t>(p);
  uint32_t sh = (uint32_t)(a & 3u);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(a - sh);
  uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[4];
  scale = (d0 >> (8u * sh)) & 0xFFu;
  uint32_t t = sh + 1u;  // first code byte offset within d0..d4 (1..4)
  if (t == 4u) {
    q[0] = d1, q[1] = d2, q[2] = d3, q[3] = d4;
  } else {
    q[0] = __builtin_amdgcn_alignbyte(d1, d0, t);
    q[1] = __builtin_amdgcn_alignbyte(d2, d1, t);
    q[2] = __builtin_amdgcn_alignbyte(d3, d2, t);
    q[3] = __builtin_amdgcn_alignbyte(d4, d3, t);
  }
}

// Two MXFP4 codes of byte `sel` of a code dword -> (low nibble, high nibble) as
// doubled e2m1 values {0,1,2,3,4,6,8,12,-0,...} (MXFP4_VALUES, dequant.rs:580).
#define MR_KV2(word, sel) __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((word), 2.0f, (sel))

// Sum over one block of kvalue_j * x_j for the 32 elements of the block (GGUF
// order: byte j low nibble -> element j, high nibble -> element j+16). The
// caller multiplies by the block's half scale.
__device__ __forceinline__ float mx_block_kdot(const uint32_t q[4], const float* xb) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x4 xl = *reinterpret_cast<const f32x4*>(xb + 4 * i);
    const f32x4 xh = *reinterpret_cast<const f32x4*>(xb + 16 + 4 * i);
    f32x2 v0 = MR_KV2(q[i], 0);
    f32x2 v1 = MR_KV2(q[i], 1);
    f32x2 v2 = MR_KV2(q[i], 2);
    f32x2 v3 = MR_KV2(q[i], 3);
    s0 = __builtin_fmaf(v0.x, xl.x, s0);
    s1 = __builtin_fmaf(v0.y, xh.x, s1);
    s0 = __builtin_fmaf(v1.x, xl.y, s0);
    s1 = __builtin_fmaf(v1.y, xh.y, s1);
    s0 = __builtin_fmaf(v2.x, xl.z, s0);
    s1 = __builtin_fmaf(v2.y, xh.z, s1);
    s0 = __builtin_fmaf(v3.x, xl.w, s0);
    s1 = __builtin_fmaf(v3.y, xh.w, s1);
  }
  return s0 + s1;
}

// Q4_K get_scale_min_k4 (dequant.rs:199-209) on the 12 scale bytes held in
// three little-endian dwords.
__device__ __forceinline__ void q4k_scale_min(uint32_t j, const uint32_t s[3], uint32_t& sc,
                                              uint32_t& m) {
  auto byte = [&](uint32_t i) -> uint32_t { return (s[i >> 2] >> (8u * (i & 3u))) & 0xFFu; };
  if (j < 4u) {
    sc = byte(j) & 63u;
    m = byte(j + 4u) & 63u;
  } else {
    sc = (byte(j + 4u) & 0x0Fu) | ((byte(j - 4u) >> 6) << 4);
    m = (byte(j + 4u) >> 4) | ((byte(j) >> 6) << 4);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Butterfly steps across lanes l and l ^ 32 (l ^ 16) with gfx950's lane-swap instructions
// instead of an LDS permute: v_permlane32_swap (v_permlane16_swap) with one register as both
// operands leaves {v[l], v[l ^ 32]} ({v[l], v[l ^ 16]}) in the two results of lane l, so their
// sum (maximum) is the step's value, the same bits in both lanes of a pair since the operation
// is commutative. All 64 lanes active.
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// v + v[l ^ 8] and v + v[l ^ 4] by DPP inside each row of 16 lanes: row_ror:8 reads lane
// l ^ 8; lanes 0-3 and 8-11 (banks 0, 2) read four lanes up with row_ror:12, lanes 4-7 and
// 12-15 (banks 1, 3) four down with row_ror:4.
__device__ __forceinline__ float add_xor8(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
}
__device__ __forceinline__ float add_xor4(float v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xA, false);
  return v + __int_as_float(__builtin_amdgcn_update_dpp(lo, __float_as_int(v), 0x12C, 0xF, 0x5, false));
}
// wave_sum's butterfly (the pairs l, l ^ o for o = 32 .. 1, so the same bits in every lane and
// the same bits as wave_sum) without LDS permutes; all 64 lanes active.
__device__ __forceinline__ float wave_sum_fast(float v) {
  v = add_xor32(v);
  v = add_xor16(v);
  v = add_xor8(v);
  v = add_xor4(v);
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // l ^ 2
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // l ^ 1
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// OAI SwiGLU (activation.rs:25-38): min(g,L)*sigmoid(alpha*min(g,L))*(clamp(u,-L,L)+1).
__device__ __forceinline__ float swiglu_oai(float g, float u, float alpha, float limit) {
  float gc = fminf(g, limit);
  float uc = fminf(fmaxf(u, -limit), limit);
  float sig = 1.0f / (__expf(-(gc * alpha)) + 1.0f);
  return (gc * sig) * (uc + 1.0f);
}

// SiLU-gated (activation.rs:13-15): g / (1 + exp(-g)) * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + __expf(-g))) * u;
}

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (__expf(-z) + 1.0f); }

// Counter-based SplitMix64 (moe_rocm/synth.py).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t draw(uint64_t seed, uint64_t i) {
  return mix64(seed + (i + 1ull) * 0x9E3779B97F4A7C15ull);
}

}  // namespace mr
