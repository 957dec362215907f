// mr_fused_common.h -- pieces shared by the single-launch decode kernels
// (mr_fused.hip: MXFP4 on MFMA; mr_fused_q4k.hip: Q4_K on integer dot products).
//
// A fused decode launch splits its grid into roles (router, gate/up, down) that
// hand results to each other through HBM inside the one launch. Hand-offs use:
//  * agent-coherent accesses (global_load/store ... sc1: they bypass the
//    non-coherent per-CU caches and meet in L2), ordered by s_waitcnt;
//  * monotonic counters in a per-layer sync block: launch n of a layer waits
//    until a counter reaches (n+1) * producers, so nothing is reset between
//    launches. Producers increment one of kCopies copies (spread over separate
//    cache lines) without waiting for a return value; waiters sum the copies.
//    Each workgroup keeps its own launch number n (no exit atomic);
//  * bounded waits: a wait that runs past its time limit (device clock) sets the
//    context error word (read and cleared by mr_sync) and the launch still exits normally.
#pragma once

#include "../../include/moe_rocm.h"
#include "mr_device.h"
#include "mr_internal.h"

namespace mr {

constexpr int kCopies = 128;    // room for this many copies of each producer counter, one 128-byte line apart
constexpr int kCopyStride = 32;  // words
constexpr int kMaxLogits = 1024;
constexpr int kMaxGrid = 1024;
#ifndef MR_LOGIT_COPIES
#define MR_LOGIT_COPIES 32
#endif
constexpr int kLogitCopies = MR_LOGIT_COPIES;  // copies of the published logits (consumers spread their polls)
static_assert(kLogitCopies >= 1 && kLogitCopies <= 64, "one copy per lane of the publishing wave");
enum : int {
  FS_GU = 0,                                   // [kCopies] counter: gate/up units finished
  FS_WGSEQ = FS_GU + kCopies * kCopyStride,    // [grid] launches completed, one word per workgroup
  FS_DN = FS_WGSEQ + kMaxGrid,                 // [row groups] down slot groups finished (MXFP4, > 4 slots)
  FS_LOGITS = FS_DN + kMaxGrid                 // [kLogitCopies][n_logits] (logit bits, launch flag)
                                               // word pairs: E experts, then extras
};
// The block's size for n_logits published logits (logit_copy's stride times the copies).
inline uint64_t layer_sync_words(uint32_t n_logits) {
  return (uint64_t)FS_LOGITS + (uint64_t)kLogitCopies * ((2u * n_logits + 31u) & ~31u);
}

// Launch sequence number of this layer's kernel. Every launch of a layer runs
// the same grid, so each workgroup keeps its own count (read at entry, stored
// +1 at exit): all workgroups of a launch read the same value, with no atomic.
__device__ __forceinline__ uint32_t* wg_seq_word(uint32_t* fs) { return fs + FS_WGSEQ + blockIdx.x; }

// Role order of a fused launch: [routers R | down ND | gate/up NG | split down halves]. The
// dispatcher hands workgroup b to CU b mod nc in round b / nc (one per CU per round, in index
// order), so with the identity order the CUs that run two gate/up units can also get a down
// group, and those gate/up units finish last. role_index maps the dispatch slot pb to a role
// index so that they get nothing else: round 0 holds the routers and down groups on CUs
// [0, nc - n2) and gate/up units on the other n2 = NG - nc CUs, round 1 a gate/up unit on every
// CU, round 2 the remaining down groups (and split halves) on CUs [0, grid - 2 nc). Valid when
// 2 nc <= grid <= 3 nc and nc <= NG <= 2 nc, with every router in round 0 (role_perm_nc); nc = 0
// is the identity.
__device__ __forceinline__ int role_index(int pb, int nc, int R, int ND, int NG) {
  if (!nc) return pb;
  const int r = pb / nc, c = pb - r * nc, n2 = NG - nc;
  if (r == 1) return R + ND + n2 + c;
  if (r == 0 && c >= nc - n2) return R + ND + (c - (nc - n2));
  const int x = r == 0 ? c : (nc - n2) + c;  // the x-th router / down group / split half
  return x < R + ND ? x : NG + x;
}
inline int role_perm_nc(int grid, int R, int NG, int n_cu) {
  return (2 * n_cu <= grid && grid <= 3 * n_cu && n_cu <= NG && NG <= 2 * n_cu && R <= 2 * n_cu - NG) ? n_cu : 0;
}

__device__ __forceinline__ const uint8_t* expert_at(const ExpertLoc& l, int e) {
  return l.base + (l.tab ? l.tab[e] : (uint64_t)e * l.stride);
}

#ifdef MR_FUSED_TRACE
#define TRACE(slot)                                                                       \
  do {                                                                                    \
    if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * 32 + (slot)] = wall_clock64(); \
  } while (0)
#define XTRACE(slot)                                                                              \
  do {                                                                                            \
    if (a.trace && (threadIdx.x & 63) == 0) a.trace[blockIdx.x * 32 + 16 + (slot)] = wall_clock64(); \
  } while (0)
#define RTRACE(slot)                                                                             \
  do {                                                                                           \
    if (rc.trace && threadIdx.x == 0) rc.trace[blockIdx.x * 32 + 8 + (slot)] = wall_clock64(); \
  } while (0)
#else
#define TRACE(slot) \
  do {              \
  } while (0)
#define RTRACE(slot) \
  do {               \
  } while (0)
#define XTRACE(slot) \
  do {               \
  } while (0)
#endif

// ---- DPP ---------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppHMirror = 0x141;  // row_half_mirror: lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;   // row_mirror: lane i <-> 15-i within 16

// max over each aligned group of 8 lanes, in every lane of the group
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  return fmaxf(v, dpp_f<kDppHMirror>(v));
}
// sum over each quad, in every lane of the quad
__device__ __forceinline__ float sum4(float v) {
  v += dpp_f<kDppXor1>(v);
  return v + dpp_f<kDppXor2>(v);
}
// sum over each aligned group of 8 lanes, in every lane of the group
__device__ __forceinline__ float sum8(float v) {
  v = sum4(v);
  return v + dpp_f<kDppHMirror>(v);
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int L>
__device__ __forceinline__ uint32_t lane_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, L);
}
template <int L>
__device__ __forceinline__ float lane_f(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), L));
}
// Whole-wave reductions (all 64 lanes active), result uniform: DPP inside each
// row of 16 lanes, then the four row results through readlane.
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
  v += dpp_u<kDppXor1>(v);
  v += dpp_u<kDppXor2>(v);
  v += dpp_u<kDppHMirror>(v);
  v += dpp_u<kDppMirror>(v);
  return (lane_u<0>(v) + lane_u<16>(v)) + (lane_u<32>(v) + lane_u<48>(v));
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
  v = max(v, dpp_u<kDppXor1>(v));
  v = max(v, dpp_u<kDppXor2>(v));
  v = max(v, dpp_u<kDppHMirror>(v));
  v = max(v, dpp_u<kDppMirror>(v));
  return max(max(lane_u<0>(v), lane_u<16>(v)), max(lane_u<32>(v), lane_u<48>(v)));
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  auto mx = [](uint64_t a, uint32_t hi, uint32_t lo) {
    const uint64_t b = ((uint64_t)hi << 32) | lo;
    return a > b ? a : b;
  };
  v = mx(v, dpp_u<kDppXor1>((uint32_t)(v >> 32)), dpp_u<kDppXor1>((uint32_t)v));
  v = mx(v, dpp_u<kDppXor2>((uint32_t)(v >> 32)), dpp_u<kDppXor2>((uint32_t)v));
  v = mx(v, dpp_u<kDppHMirror>((uint32_t)(v >> 32)), dpp_u<kDppHMirror>((uint32_t)v));
  v = mx(v, dpp_u<kDppMirror>((uint32_t)(v >> 32)), dpp_u<kDppMirror>((uint32_t)v));
  uint64_t r = 0ull;
  r = mx(r, lane_u<0>((uint32_t)(v >> 32)), lane_u<0>((uint32_t)v));
  r = mx(r, lane_u<16>((uint32_t)(v >> 32)), lane_u<16>((uint32_t)v));
  r = mx(r, lane_u<32>((uint32_t)(v >> 32)), lane_u<32>((uint32_t)v));
  return mx(r, lane_u<48>((uint32_t)(v >> 32)), lane_u<48>((uint32_t)v));
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
  v = min(v, dpp_u<kDppXor1>(v));
  v = min(v, dpp_u<kDppXor2>(v));
  v = min(v, dpp_u<kDppHMirror>(v));
  v = min(v, dpp_u<kDppMirror>(v));
  return min(min(lane_u<0>(v), lane_u<16>(v)), min(lane_u<32>(v), lane_u<48>(v)));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(lane_f<0>(v), lane_f<16>(v)), fmaxf(lane_f<32>(v), lane_f<48>(v)));
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return (lane_f<0>(v) + lane_f<16>(v)) + (lane_f<32>(v) + lane_f<48>(v));
}

// ---- agent-coherent accesses (global_load/store ... sc1) ---------------------------
__device__ __forceinline__ uint32_t ld_sc1(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_sc1(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld64_sc1(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Published logits: kLogitCopies copies of n_logits 64-bit words (logit bits, seq + 1),
// each copy starting on a 128-byte line. A reader that sees the flag half sees the value
// half (aligned 8-byte stores are single-copy atomic), so no counter or store drain is
// needed; the flag of the previous launch is seq, never seq + 1, and the block starts
// zeroed (flag 0). Consumer workgroups poll copy (blockIdx % kLogitCopies), which
// spreads their polls over many lines instead of one.
__device__ __forceinline__ uint64_t* logit_copy(const uint32_t* fs, uint32_t n_logits, int copy) {
  const uint32_t stride = (2u * n_logits + 31u) & ~31u;  // words
  return reinterpret_cast<uint64_t*>(const_cast<uint32_t*>(fs) + FS_LOGITS + (size_t)copy * stride);
}
// Lane c < kLogitCopies of a wave stores copy c of logit e (v is wave-uniform).
__device__ __forceinline__ void put_logit(uint32_t* fs, uint32_t n_logits, int e, uint32_t seq, float v) {
  const int lane = threadIdx.x & 63;
  if (lane < kLogitCopies) {
    const uint64_t w = ((uint64_t)(seq + 1u) << 32) | (uint64_t)__float_as_uint(v);
    __hip_atomic_store(logit_copy(fs, n_logits, lane) + e, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
// Logit e of the current launch; valid once route_wave has returned true in this wave.
__device__ __forceinline__ float get_logit(const uint32_t* fs, uint32_t n_logits, int e) {
  const uint64_t* p = logit_copy(fs, n_logits, (int)(blockIdx.x % kLogitCopies)) + e;
  return __uint_as_float(ld_sc1(reinterpret_cast<const uint32_t*>(p)));
}
// All vector memory operations this wave has issued have completed.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// All LDS operations this wave has issued have completed.
__device__ __forceinline__ void lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Time limit of a cross-workgroup wait, on the device's constant-rate clock (wall_clock64,
// s_memrealtime). `free` polls come without a clock read (every wait of a normal launch ends
// well within them); from then on every poll reads the clock and compares the reading of the
// poll before with the clock at poll `free`, so no poll waits for its own clock read. A wait
// therefore gives up at most `free` polls plus `ticks` after it began.
// (WaitBound, the launch argument: mr_internal.h.)
struct WaitTimer {
  uint64_t t0 = 0, t1 = 0;
  // at poll `it` of a wait: whether the limit has passed
  __device__ __forceinline__ bool out(uint32_t it, const WaitBound& b) {
    if (it < b.free) return false;
    if (it == b.free) {
      t0 = t1 = (uint64_t)wall_clock64();
      return false;
    }
    const bool o = t1 - t0 > (uint64_t)b.ticks;
    t1 = (uint64_t)wall_clock64();
    return o;
  }
};

// Count n finished producer items on copy (id % NC) (no return value is waited for).
// NC copies in use (64 or 128: fewer lines to poll against fewer producers per line).
template <int NC>
__device__ __forceinline__ void count(uint32_t* copies, int id, uint32_t n = 1u) {
  static_assert(NC == 64 || NC == 128, "one or two copies per lane of the waiting wave");
  (void)__hip_atomic_fetch_add(copies + kCopyStride * (id % NC), n, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}
// Bounded wait (one full wave) until the counter copies sum to at least `target`
// (wrap-around safe); false if its time limit ran out. SLEEP: s_sleep units (64 clocks)
// between polls (longer for waits that overlap weight streaming).
#ifndef MR_GU_WAIT_SLEEP
#define MR_GU_WAIT_SLEEP 32  // the down workgroups' wait for the gate/up count
#endif
// Once at most `near` items are missing, polls come every SLEEP_NEAR units instead: the
// last producers are seen sooner without polling fast through the whole wait.
template <int SLEEP, int NC, int SLEEP_NEAR = SLEEP>
__device__ __forceinline__ bool wait_count(const uint32_t* copies, uint32_t target, const WaitBound& wb,
                                           uint32_t near = 0u) {
  const int lane = threadIdx.x & 63;
  WaitTimer tm;
  for (uint32_t it = 0;; ++it) {
    uint32_t c = ld_sc1(copies + kCopyStride * lane);
    if (NC > 64) c += ld_sc1(copies + kCopyStride * (lane + 64));
    const uint32_t sum = wave_sum_u(c);
    const int32_t missing = (int32_t)(target - sum);
    if (missing <= 0) return true;
    if (tm.out(it, wb)) return false;
    if ((uint32_t)missing <= near)
      __builtin_amdgcn_s_sleep(SLEEP_NEAR);
    else
      __builtin_amdgcn_s_sleep(SLEEP);
  }
}


// ---- fused RMSNorm and residual (norm.rs:16-37; layer.rs:462-473) ---------------------------
// mr_moe_forward_residual: the layer's input is rms_norm(h) = (h * inv) * w with
// inv = 1 / sqrt(mean(h^2) + eps), and its output is h + moe(rms_norm(h)). w == nullptr: the
// input is used as given and nothing is added.
// (NormResid, the launch argument, is declared with the launchers.)
// inv of the RMSNorm from a wave's lane-strided float4s of h (lane l holds elements
// 4*(l + 64*j) .. +3, zero past H): squares rounded, then summed in a fixed order per lane
// and a butterfly across lanes, so every wave that calls this gets the same bits.
// (No contraction: squares and sums are rounded separately; sqrtf and the division are
// the correctly rounded HIP forms.)
template <int NV>
__device__ __forceinline__ float rms_inv(const f32x4 (&xv)[NV], int H, float eps) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    s = s + xv[j].x * xv[j].x;
    s = s + xv[j].y * xv[j].y;
    s = s + xv[j].z * xv[j].z;
    s = s + xv[j].w * xv[j].w;
  }
  s = wave_sum(s);  // the same bits in every lane
  return 1.f / sqrtf(s / (float)H + eps);
}
// An in-bounds float4 load whatever the index (the index clamped to the last float4), zero
// selected afterwards for indices past n (a multiple of 4). A load under a per-lane condition
// is compiled into a branch of its own, and the wait at the branch's end can make a run of
// such loads one memory round trip each; these issue together. Where loads are off the
// critical path the conditional form can be the faster one (it adds fewer requests while the
// critical ones are in flight): the choice is measured per use.
__device__ __forceinline__ f32x4 ld4_or0(const float* v, int c, int n) {
  const f32x4 t = *reinterpret_cast<const f32x4*>(v + min(c, n - 4));
  return c < n ? t : f32x4{0.f, 0.f, 0.f, 0.f};
}
// A wave's lane-strided float4s of v (zero past H).
template <int NV>
__device__ __forceinline__ void load_lanes4(const float* v, int H, f32x4 (&out)[NV]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    out[j] = c < H ? *reinterpret_cast<const f32x4*>(v + c) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
}
// The same, every load unconditional (ld4_or0).
template <int NV>
__device__ __forceinline__ void load_lanes4_all(const float* v, int H, f32x4 (&out)[NV]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NV; ++j) out[j] = ld4_or0(v, (lane + 64 * j) * 4, H);
}
__device__ __forceinline__ float norm1(float x, float inv, float w) { return (x * inv) * w; }

// ---- next-layer router prefetch -----------------------------------------------------------
// Router rows of the layer that runs next (rows 0..E-1 of its router weights, then its
// shared-expert gate row if it has one). Its router workgroup b reads rows 4b..4b+3; router
// workgroup b of this launch reads the rows of next workgroups b, b + R, ... into LDS and
// drops them, after publishing its own logits, so they are in the caches when the next
// launch starts (workgroup b runs on XCD b mod 8 in both launches).
struct PrefetchRows {
  const float* w;   // [E, H] f32, or nullptr: no prefetch
  const float* sh;  // row E (shared-expert gate) or nullptr
  int rows, E, H;
  int rpw;          // rows per router workgroup of the next layer's MXFP4 kernel, 0: four, one per wave
};
// The next layer's router workgroup nb computes rows nb * rpw .. nb * rpw + rpw - 1: with four
// rows per workgroup (rpw = 0; the Q4_K kernel) one per wave, whole rows; otherwise (the MXFP4
// kernel: rpw rows, quarter w of every row's columns in wave w) wave w reads quarter w of each.
__device__ __forceinline__ void prefetch_rows(const PrefetchRows& p, int bid, int R, uint8_t* lds) {
  if (!p.w) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rpw = p.rpw ? p.rpw : 4;
  const int nj = (p.H + 255) / 256;                   // 64 lanes x 16 bytes per load
  const int jq = p.rpw ? (nj + 3) / 4 : nj;           // loads per row and wave
  const int j0 = p.rpw ? wave * jq : 0, j1 = min(nj, j0 + jq);
  for (int nb = bid; nb * rpw < p.rows; nb += R) {
    for (int r = p.rpw ? 0 : wave; r < rpw; r += p.rpw ? 1 : 4) {
      const int e = nb * rpw + r;
      if (e < p.rows) {
        const float* src = e < p.E ? p.w + (size_t)e * p.H : p.sh;
        for (int j = j0; j < j1; ++j) {
          const int c = min(j * 256 + lane * 4, p.H - 4);
          __builtin_amdgcn_global_load_lds(src + c, lds + wave * 1024, 16, 0, 0);
        }
      }
    }
  }
  vm_drain();  // the loads complete before this workgroup's LDS is released
}
// The next layer's norm weights (mr_layer_set_norm), which every router and gate/up workgroup
// of that layer reads: each of the first eight router workgroups (one per XCD, workgroups being
// dealt to the XCDs in turn) reads all H of them, its four waves a quarter each.
__device__ __forceinline__ void prefetch_norm(const float* nw, int H, int bid, uint8_t* lds) {
  if (!nw || bid >= 8) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int j = wave; j * 256 < H; j += 4) {
    const int c = min(j * 256 + lane * 4, H - 4);
    __builtin_amdgcn_global_load_lds(nw + c, lds + wave * 1024, 16, 0, 0);
  }
  vm_drain();
}
// Host side: the plan for the hint set with mr_layer_set_next (no prefetch without one).
inline PrefetchRows prefetch_plan(const mr_layer* n) {
  PrefetchRows p{nullptr, nullptr, 0, 0, 0, 0};
  if (!n || !n->d.router_w || n->H < 4) return p;
  p.w = n->d.router_w;
  p.sh = n->d.sh_gate ? n->d.sh_gate_inp : nullptr;
  p.E = (int)n->E;
  p.rows = (int)n->E + (p.sh ? 1 : 0);
  p.H = (int)n->H;
  return p;
}

// ---- routing ----------------------------------------------------------------------------
struct RouteCfg {
  const uint32_t* fs;  // layer sync block
  uint32_t n_logits;   // logits published per launch (E, plus extras)
  int E, k;
  uint32_t flags;      // MR_ROUTE_*
  WaitBound wb;
  unsigned long long* trace;  // MR_FUSED_TRACE builds only
};

// Order-preserving key of a float: larger float <=> larger unsigned key.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

constexpr int kRouteVals = 8;  // experts per lane in routing: E <= 512
// s_sleep units (64 clocks) between polls of the published logits: every workgroup polls,
// so the poll rate is weighed against the traffic it adds to the lines being waited on.
#ifndef MR_ROUTE_SLEEP
#define MR_ROUTE_SLEEP 2
#endif
#ifndef MR_ROUTE_SLEEP_DOWN
#define MR_ROUTE_SLEEP_DOWN 100  // down workgroups: their weights are needed only after gate/up
#endif

// ---- Qwen-mode ranking: probabilities, ties to the lower index --------------------------
// The standard mode ranks p_i = expf(l_i - max) / sum in f32 (sum in expert order; layer.rs:
// 2371-2394) with a stable sort whose comparator calls unordered pairs equal. exp and the
// division are monotonic, so ranking by logit selects the same set unless
//  - the k-th selected logit lk and the largest logit below it lb are so close that their
//    probabilities can round to one value: the f32 difference l - max is exact to 2^-24
//    |l - max|, expf and the division round once each, so lk - lb > 2^-20 (1 + max - lb) keeps
//    p(lk) > p(lb) while p(lk) is a normal number, which max - lk <= 80 ensures (expf(-80) / 512
//    > 2^-126); below that, probabilities lose precision or flush to 0 and tie;
//  - a probability is NaN: a NaN logit, a +inf maximum (inf - inf) or a row of -inf make the
//    sum, hence every probability, NaN; every comparison is then "equal" and the stable sort
//    keeps expert order: experts 0..k-1 with NaN weights.
// prob_exact_needed tells those rows apart; they are ranked again on the probabilities.
// key: this lane's key columns (valid logits have keys >= 2, NaN 1, absent 0), T the k-th
// largest key. The common answer costs a wave max and one compare pass.
// NJ: the key columns that can be live (E <= 64 NJ).
template <int NJ = kRouteVals>
__device__ __forceinline__ bool prob_exact_needed(const uint32_t (&key)[kRouteVals], uint32_t T) {
  uint32_t mk = 0u;
#pragma unroll
  for (int j = 0; j < NJ; ++j) mk = max(mk, key[j]);
  const float lk = key_value(T), m = key_value(wave_max_u(mk)), d = m - lk;
  // lb >= lk - tau with tau = 2^-20 (1 + m - lb) <= 2^-20 (1 + m - lk) (1 + 2^-19): any key in
  // [key(lk - tau), T) is a near tie
  const uint32_t lo = order_key(lk - 0x1p-20f * (1.f + d) * (1.f + 0x1p-19f));
  // Branch-free (bitwise, not short-circuit: the compiler would turn every || into a branch
  // on the exec mask): NaN or infinite ends, or p(lk) below the normal range; then per key a
  // near tie or a NaN (which makes every probability NaN; absent keys, 0, lie below lo).
  uint32_t hit = !(d <= 80.f) ? 1u : 0u;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    hit |= ((key[j] >= lo ? 1u : 0u) & (key[j] < T ? 1u : 0u)) | (key[j] == 1u ? 1u : 0u);
  return __ballot(hit != 0u) != 0ull;
}
// Order keys of the probabilities as the reference computes them: expf of the f32 difference
// (correctly rounded: computed in double), the sum in expert order (each term read from its
// lane in turn, so every lane adds the same sequence), IEEE division. NaN probabilities get key
// 1 (equal to each other), absent experts (past E) key 0. Returns whether they are NaN. Registers only, and rolled where it can be: the path is rare, and it must not
// weigh on the caller's registers or LDS.
__device__ __forceinline__ bool prob_keys(const float (&v)[kRouteVals], int E, uint32_t (&key)[kRouteVals]) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j)
    if (lane + 64 * j < E) m = fmaxf(m, v[j]);
  m = wave_max_f(m);
  float p[kRouteVals], s = 0.f;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    p[j] = lane + 64 * j < E ? (float)exp((double)(v[j] - m)) : 0.f;
    const int n = min(64, E - 64 * j);  // experts of column j
#pragma unroll 1
    for (int l = 0; l < n; ++l) s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j]), l));
  }
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    const float q = p[j] / s;
    key[j] = lane + 64 * j < E ? (q == q ? order_key(q + 0.f) : 1u) : 0u;
  }
  return !(s == s);  // the sum (the same in every lane) is NaN exactly when every probability is
}
// The value of lane-held entry e (lane e & 63, column e >> 6), in every lane.
__device__ __forceinline__ float entry_value(const float (&v)[kRouteVals], int e) {
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    const float t = __shfl(v[j], e & 63);
    if ((e >> 6) == j) r = t;
  }
  return r;
}

// Lanes below this one in a 64-bit wave mask.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// The k-th largest key of the wave's NJ key columns: the largest T with at least k
// keys >= T, fixed one bit at a time from the top (per bit, one ballot per column; the
// compares issue before the first scalar count reads a mask). A lone wave issues about
// one instruction per four cycles, so fewer instructions per bit beat fewer steps. Once
// exactly k keys are >= the prefix, the k-th largest is the least of them: one wave
// minimum ends the search (for spread-out logits, after about half of the 32 bits).
template <int NJ>
__device__ __forceinline__ uint32_t kth_key(const uint32_t (&key)[kRouteVals], int k) {
  uint32_t T = 0u;
  bool exact = false;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t t = T | (1u << b);
    uint64_t m[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) m[j] = __ballot(key[j] >= t);
    int c = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) c += __popcll(m[j]);
    __builtin_amdgcn_sched_group_barrier(0x2, NJ, 0);
    __builtin_amdgcn_sched_group_barrier(0x4, 2 * NJ + 3, 0);
    if (c >= k) {
      T = t;
      if (c == k) {  // wave-uniform
        exact = true;
        break;
      }
    }
  }
  if (exact) {
    uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NJ; ++j) mn = key[j] >= T ? min(mn, key[j]) : mn;
    T = wave_min_u(mn);
  }
  return T;
}

// The selected set: keys above T, then of the keys equal to T the lowest expert indices.
// Expert indices idx[j] ascend with j, then with the lane (e = lane + 64*j, or a list
// compacted in that order). Slot = rank of the expert index among the selected, so slots
// run in ascending expert order. sel_i/sel_k[slot] get the expert and its key. Returns T,
// the k-th largest key.
template <int NJ>
__device__ __forceinline__ uint32_t topk_slots(const uint32_t (&key)[kRouteVals], const int (&idx)[kRouteVals], int k,
                                               int* sel_i, uint32_t* sel_k) {
  const uint32_t T = kth_key<NJ>(key, k);
  int above = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) above += __popcll(__ballot(key[j] > T));
  const int need = k - above;  // ties at T to take (>= 1)
  int ties = 0, before = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint64_t eq = __ballot(key[j] == T);
    const bool s = key[j] > T || (key[j] == T && ties + lanes_below(eq) < need);
    ties += __popcll(eq);
    const uint64_t sm = __ballot(s);
    if (s) {
      const int slot = before + lanes_below(sm);
      sel_i[slot] = idx[j], sel_k[slot] = key[j];
    }
    before += __popcll(sm);
  }
  return T;
}

// Many columns (E > 128): the k-th largest lane maximum H bounds the threshold from
// below (k lanes hold a key >= H), so only keys >= H can be selected. When those fit one
// column they are compacted in ascending expert order through LDS (tmp: 128 of its words) and
// selected there; otherwise all columns are searched.
__device__ __forceinline__ uint32_t topk_slots_wide(const uint32_t (&key)[kRouteVals], int k, int* sel_i,
                                                    uint32_t* sel_k, uint32_t* tmp) {
  const int lane = threadIdx.x & 63;
  uint32_t hm[kRouteVals], hk = 0u;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) hk = max(hk, key[j]);
  hm[0] = hk;
  const uint32_t H = kth_key<1>(hm, k);
  int before = 0;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    const bool s = key[j] >= H;
    const uint64_t sm = __ballot(s);
    const int slot = before + lanes_below(sm);
    if (s && slot < 64) tmp[slot] = key[j], tmp[64 + slot] = (uint32_t)(lane + 64 * j);
    before += __popcll(sm);
  }
  int idx[kRouteVals];
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) idx[j] = lane + 64 * j;
  if (before > 64) return topk_slots<kRouteVals>(key, idx, k, sel_i, sel_k);
  lds_drain();
  __builtin_amdgcn_wave_barrier();
  uint32_t ck[kRouteVals];
  ck[0] = lane < before ? tmp[lane] : 0u;
  idx[0] = lane < before ? (int)tmp[64 + lane] : 0;
  return topk_slots<1>(ck, idx, k, sel_i, sel_k);
}

// Wave 0 of a consumer workgroup (all 64 lanes): wait until every logit of this
// launch is published, then select the top-k (tmp: kRouteVals * 64 words of LDS scratch) (largest first, ties to the lower
// index; top_k_routing layer.rs:2346-2403). Expert e = lane + 64*j is value j of
// a lane. Slots are numbered in ascending expert index, the combine order of
// layer.rs:1092-1106; slot r's expert goes to sel_i[r] (LDS) and, for route_finish,
// stays in the state (lane r = slot r).
struct RouteState {
  float v[kRouteVals];  // this lane's logits
  uint32_t my_key;
  int my_e;
  float xv;  // the extra entry E + lane (lane < n_logits - E) as polled, else 0
};
// The selection by key (topk_slots for one or two key columns, else topk_slots_wide) into
// sel_i/sel_k; returns the k-th largest key. CHECK: need = prob_exact_needed on the live
// columns, computed while the slot stores drain.
template <bool CHECK>
__device__ __forceinline__ uint32_t select_keys(const uint32_t (&key)[kRouteVals], int nj, int k, int* sel_i,
                                                uint32_t* sel_k, uint32_t* tmp, bool& need) {
  const int lane = threadIdx.x & 63;
  int idx[kRouteVals];
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) idx[j] = lane + 64 * j;
  uint32_t T;
  need = false;
  if (nj <= 1) {
    T = topk_slots<1>(key, idx, k, sel_i, sel_k);
    if (CHECK) need = prob_exact_needed<1>(key, T);
  } else if (nj <= 2) {
    T = topk_slots<2>(key, idx, k, sel_i, sel_k);
    if (CHECK) need = prob_exact_needed<2>(key, T);
  } else {
    T = topk_slots_wide(key, k, sel_i, sel_k, tmp);
    if (CHECK) need = prob_exact_needed(key, T);
  }
  lds_drain();
  __builtin_amdgcn_wave_barrier();
  return T;
}

// The selection redone on probability keys (pkey: order keys of p, absent 0): k rounds of a wave
// argmax on (key, complemented index), then the k experts put in ascending expert order into
// sel_i/sel_k (sel_k: their logit keys, which route_finish weighs by; the NaN key 1 when the
// probabilities are NaN (pnan), so the weights come out NaN as the reference's do). Small and
// slow: such rows are rare, and this code must not weigh on the routing's registers.
__device__ __forceinline__ void prob_select(const uint32_t (&pkey)[kRouteVals], const float (&v)[kRouteVals], int E,
                                            int k, bool pnan, int* sel_i, uint32_t* sel_k) {
  const int lane = threadIdx.x & 63;
  bool live[kRouteVals];
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) live[j] = lane + 64 * j < E;
  int mine = 0;  // lane r: the r-th ranked expert
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0ull;
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j) {
      const uint64_t key = ((uint64_t)pkey[j] << 32) | (0xFFFFFFFFu - (uint32_t)(lane + 64 * j));
      if (live[j]) best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    const int bi = (int)(0xFFFFFFFFu - (uint32_t)best);
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j)
      if (bi == lane + 64 * j) live[j] = false;
    if (lane == r) mine = bi;
  }
  // slot = rank of the expert index among the selected
  int slot = 0;
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    const int o = __shfl(mine, r);
    slot += (lane < k && o < mine) ? 1 : 0;
  }
  const float ls = entry_value(v, mine);
  if (lane < k) sel_i[slot] = mine, sel_k[slot] = (ls == ls && !pnan) ? order_key(ls + 0.f) : 1u;
  lds_drain();
  __builtin_amdgcn_wave_barrier();
}

// One poll of the published logits: columns 0..NJ-1 (expert lane + 64 j) and the lane's extra
// entry, every load issued before the first is used. The loads are unconditional, with
// addresses clamped to a valid entry (absent experts re-read expert E - 1, lanes without an
// extra entry re-read entry 0): a load under a per-lane condition sits in its own branch, and
// the wait for it at the join would make the loads one round trip each. True when every
// entry carries this launch's flag; v gets the logits (-inf past E).
template <int NJ, bool XTRA>
__device__ __forceinline__ bool poll_logits(const uint64_t* lw, int E, int ex, uint32_t flag, float (&v)[kRouteVals],
                                            float& xv) {
  const int lane = threadIdx.x & 63;
  uint64_t w[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) w[j] = ld64_sc1(lw + min(lane + 64 * j, E - 1));
  const uint64_t wx = ld64_sc1(lw + (ex >= 0 ? ex : 0));
  uint32_t bad = (ex >= 0 && (uint32_t)(wx >> 32) != flag) ? 1u : 0u;
  if (XTRA) xv = ex >= 0 ? __uint_as_float((uint32_t)wx) : 0.f;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    const bool in = j < NJ && lane + 64 * j < E;
    v[j] = in ? __uint_as_float((uint32_t)w[j < NJ ? j : 0]) : -INFINITY;
    bad |= (in && (uint32_t)(w[j < NJ ? j : 0] >> 32) != flag) ? 1u : 0u;
  }
  return __ballot(bad != 0u) == 0ull;
}

// QWEN: compile in the near-tie check (layers whose flags lack MR_ROUTE_SOFTMAX_AFTER_TOPK rank
// probabilities); a kernel instantiated without it ranks by logit alone.
// XTRA: keep the polled extra entries (RouteState::xv).
template <int SLEEP = MR_ROUTE_SLEEP, bool QWEN = true, bool XTRA = false>
__device__ inline bool route_select(const RouteCfg& rc, uint32_t seq, int* sel_i, uint32_t* sel_k, uint32_t* tmp,
                                   RouteState& st) {
  const int lane = threadIdx.x & 63;
  RTRACE(0);
  const int nj = (rc.E + 63) >> 6;  // values per lane (wave-uniform)
  // Poll the flagged logit words until every entry (experts and extras) carries this
  // launch's flag; the values come with the flags, in the same loads. One poll at a time:
  // a poll is a round trip to the device-coherent level (about a microsecond), yet more
  // polls in flight (2-4, spaced over that round trip) delay the logits' own stores and
  // lose 3-35% (the publish lines are shared by every consumer workgroup).
  const uint64_t* lw = logit_copy(rc.fs, rc.n_logits, (int)(blockIdx.x % kLogitCopies));
  const uint32_t flag = seq + 1u;
  const int ex = lane < (int)rc.n_logits - rc.E ? rc.E + lane : -1;  // an extra entry of this lane
  float v[kRouteVals], xv = 0.f;
  WaitTimer tm;
  for (uint32_t it = 0;; ++it) {
    // nj is wave-uniform: one straight-line poll per column count (6 and 7 read 8 columns)
    const bool ok = nj <= 1   ? poll_logits<1, XTRA>(lw, rc.E, ex, flag, v, xv)
                    : nj <= 2 ? poll_logits<2, XTRA>(lw, rc.E, ex, flag, v, xv)
                    : nj <= 4 ? poll_logits<4, XTRA>(lw, rc.E, ex, flag, v, xv)
                              : poll_logits<8, XTRA>(lw, rc.E, ex, flag, v, xv);
    if (ok) {
#ifdef MR_FUSED_TRACE
      if (rc.trace && threadIdx.x == 0) rc.trace[blockIdx.x * 32 + 10] = it;  // polls before the logits were seen
#endif
      break;
    }
    if (tm.out(it, rc.wb)) return false;
    __builtin_amdgcn_s_sleep(SLEEP);
  }
  RTRACE(1);
  // Ranking: largest logit first, then in Qwen mode, where two logits at the selection
  // boundary could round to one probability, or that hold NaN probabilities, again on the
  // probabilities (prob_exact_needed).
  // Keys: + 0.f makes -0.0 and +0.0 share a key; a NaN takes key 1, below every number
  // (-inf is 0x007FFFFF) and above the absent entries past E (key 0), the order of k_topk.
  uint32_t key[kRouteVals];
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j)
    key[j] = (lane + 64 * j < rc.E) ? (v[j] == v[j] ? order_key(v[j] + 0.f) : 1u) : 0u;
  RTRACE(3);
  bool need;
  (void)select_keys<QWEN>(key, nj, rc.k, sel_i, sel_k, tmp, need);
  if (QWEN && need && !(rc.flags & MR_ROUTE_SOFTMAX_AFTER_TOPK)) {
    const bool pnan = prob_keys(v, rc.E, key);
    prob_select(key, v, rc.E, rc.k, pnan, sel_i, sel_k);
  }
  RTRACE(5);
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) st.v[j] = v[j];
  st.xv = xv;
  st.my_key = lane < rc.k ? sel_k[lane] : 0u;
  st.my_e = lane < rc.k ? sel_i[lane] : 0;
  RTRACE(7);
  return true;
}


// Weights and combine order of the selection (the top-k weights of top_k_routing,
// layer.rs:2346-2403; ascending expert order, layer.rs:1092-1106): sel_w[r] for slot r, and
// ord[p] = the slot holding the p-th smallest expert index (slot p: slots ascend with the
// expert index). Not needed to start streaming weights, so callers run it after their
// first loads are issued.
__device__ inline void route_finish(const RouteCfg& rc, const RouteState& st, float* sel_w, int* ord) {
  const int lane = threadIdx.x & 63;
  const float* v = st.v;
  const bool sel_softmax = (rc.flags & (MR_ROUTE_SOFTMAX_AFTER_TOPK | MR_ROUTE_NORM_TOPK)) != 0u;
  float m_all = 0.f, s_all = 1.f;  // plain softmax: the all-expert normaliser
  if (!sel_softmax) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j) m = fmaxf(m, v[j]);
    m_all = wave_max_f(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j)
      if (lane + 64 * j < rc.E) s += __expf(v[j] - m_all);
    s_all = wave_sum_f(s);
  }
  const bool in = lane < rc.k;
  const float l = in ? key_value(st.my_key) : 0.f;
  float w;
  if (sel_softmax) {
    const float m = wave_max_f(in ? l : -INFINITY);  // the largest selected logit
    const float ex = in ? __expf(l - m) : 0.f;
    w = ex / wave_sum_f(ex);
  } else {
    w = __expf(l - m_all) / s_all;
  }
  if (in) sel_w[lane] = w, ord[lane] = lane;
  lds_drain();
}

__device__ __forceinline__ void fail(uint32_t* err) { st_sc1(err, 1u); }

}  // namespace mr
