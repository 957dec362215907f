// mr_internal.h -- host-side objects behind the C ABI of include/moe_rocm.h,
// shared by the API layer (mr_api.cpp) and the kernel launchers (*.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/moe_rocm.h"

namespace mr {

constexpr uint32_t kMaxTopK = 16;        // softmax_topk_kernel limit (fused_ops.metal:150)
constexpr uint32_t kMaxExperts = 512;    // same limit (fused_ops.metal:158)
constexpr uint32_t kMaxHidden = 16384;   // LDS-staged activation limit of the VALU kernels
// Size of the static scratch array of mr_moe_forward_batched_noalloc (one per GPU).
constexpr uint64_t kStaticScratchBytes = MR_STATIC_SCRATCH_BYTES;

// Per-context scratch: routing outputs, intermediate activations, sync words.
// Sized by mr_reserve (or lazily on first use outside graph capture).
struct Scratch {
  void* base = nullptr;
  uint64_t bytes = 0;
  // carve-outs (device pointers into base)
  int32_t* idx = nullptr;      // [T, k]
  float* w = nullptr;          // [T, k]
  float* logits = nullptr;     // [T, E]
  float* rpart = nullptr;      // [4, T, E] router partial sums
  float* act = nullptr;        // [T, k, I] or grouped [T*k, I]
  float* act_sh = nullptr;     // [T, Ish] shared expert activation
  void* mfma_b = nullptr;      // MFMA B-operand images (x split / act split)
  uint32_t* sync = nullptr;    // sync words for the fused decode kernel
  int32_t* groups = nullptr;   // batched path: per-expert token lists
  void* grouped = nullptr;     // grouped MFMA path: activation images and per-pair outputs
  float* xn = nullptr;         // [T, H] normalised input (mr_moe_forward_residual, multi-kernel path)
  float* ytmp = nullptr;       // [T, H] MoE output before the residual add
  uint64_t cap_tokens = 0, cap_k = 0, cap_e = 0, cap_i = 0, cap_h = 0, cap_ish = 0;
};

// Optional per-kernel timing: an event pair around every kernel launch on the
// context stream (enabled by MR_OPT_PROFILE, never during graph capture).
struct Prof {
  bool on = false;
  struct Rec {
    int name;
    hipEvent_t a, b;
  };
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  std::vector<Rec> recs;
  std::vector<std::string> names;
  hipEvent_t next_event();
  int name_id(const char* n);
};

// What a launcher needs: the stream and, when profiling, the recorder.
struct Launch {
  hipStream_t s;
  Prof* prof;  // nullptr when not profiling
};

// RAII bracket around one kernel launch.
struct ProfScope {
  Launch L;
  const char* name;
  hipEvent_t a = nullptr;
  ProfScope(const Launch& l, const char* n) : L(l), name(n) {
    if (L.prof) {
      a = L.prof->next_event();
      (void)hipEventRecord(a, L.s);
    }
  }
  ~ProfScope() {
    if (L.prof && a) {
      hipEvent_t b = L.prof->next_event();
      (void)hipEventRecord(b, L.s);
      L.prof->recs.push_back({L.prof->name_id(name), a, b});
    }
  }
};

}  // namespace mr

struct mr_ctx {
  int device = MR_DEVICE_NONE;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  int n_cu = 0;
  int decode_kernel = MR_DECODE_AUTO;
  uint32_t wait_limit_us = 50000;  // time limit of the fused kernels' cross-workgroup waits
  int wall_khz = 100000;           // rate of the device's constant clock (wall_clock64)
  bool fused_used = false;
  std::string err;
  mr::Scratch scratch;
  // Scratch allocations superseded by a larger one while a graph captured since their
  // allocation may still address them: these stay allocated (and their fused-kernel error
  // words are still checked by mr_sync) until mr_ctx_destroy. A superseded allocation that
  // no capture has seen is freed at once.
  std::vector<void*> retired;
  std::vector<uint32_t*> retired_err;
  bool captured_since_alloc = false;  // mr_graph_begin ran since the scratch was allocated
  bool pending_wait_err = false;      // a freed scratch's error word was set, not yet reported
  // This device's static scratch array (mr_moe_forward_batched_noalloc), resolved at
  // mr_ctx_create; nullptr with static_err set when the lookup failed.
  void* static_scratch = nullptr;
  hipError_t static_err = hipSuccess;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  bool capturing = false;
  mr::Prof prof;
  mr::Launch launch() { return mr::Launch{stream, (prof.on && !capturing) ? &prof : nullptr}; }
};

struct mr_pack {
  mr_ctx* ctx = nullptr;
  int type = 0;
  uint32_t n_experts = 0, out_features = 0, in_features = 0;
  const uint8_t* base = nullptr;   // device bytes
  uint64_t nbytes = 0;
  bool owned = false;
  uint64_t matrix_bytes = 0;       // bytes of one expert matrix
  std::vector<uint64_t> h_offsets; // per-expert byte offsets from base
  uint64_t* d_offsets = nullptr;   // same on the device (nullptr for host-only ctx)
  bool uniform = false;            // h_offsets[e] == uni_off0 + e * uni_stride for every e
  uint64_t uni_off0 = 0, uni_stride = 0;
};

namespace mr {
// Where the fused kernels find expert e: base + e * stride when the pack's experts sit
// one stride apart (no table read between the routing and the weight loads), else
// base + tab[e].
struct ExpertLoc {
  const uint8_t* base;
  const uint64_t* tab;  // nullptr: uniform stride
  uint64_t stride;
};
inline ExpertLoc expert_loc(const mr_pack* p) {
  if (p->uniform) return ExpertLoc{p->base + p->uni_off0, nullptr, p->uni_stride};
  return ExpertLoc{p->base, p->d_offsets, 0};
}
}  // namespace mr

struct mr_layer {
  mr_ctx* ctx = nullptr;
  mr_layer_desc d{};
  uint32_t H = 0, I = 0, E = 0, Ish = 0;
  int type = 0;
  uint32_t* fused_sync = nullptr;  // device sync block of the fused decode kernel
  const mr_layer* next = nullptr;  // layer run after this one (router prefetch hint) or NULL
  const float* norm_w = nullptr;   // norm weights of this layer's residual forwards (prefetch hint) or NULL
  float* logits_out = nullptr;     // router logits [T, E] of every forward call, or NULL
  uint32_t logits_cap = 0;         // tokens logits_out holds
  std::vector<mr_pack*> own_packs;  // device objects the layer owns (mr_gguf_layer_create)
  std::vector<void*> own_dev;
};

struct mr_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace mr {

// Launchers implemented in the .hip files. Each returns a hipError_t from the launch.
hipError_t launch_zero(const Launch& L, void* dst, uint64_t nbytes);
hipError_t launch_router_logits(const Launch& K, const mr_layer& L, const float* x, uint32_t T,
                                float* logits);
// Router logits (written to logits) and top-k for T tokens; part: [4][T][E] floats of scratch.
hipError_t launch_router_topk(const Launch& K, const mr_layer& L, const float* x, uint32_t T, float* logits,
                              float* part, int32_t* idx, float* w);
hipError_t launch_topk(const Launch& K, const float* logits, uint32_t T, uint32_t E, uint32_t k,
                       uint32_t flags, int32_t* idx, float* w);
hipError_t launch_experts_valu(const Launch& K, const mr_layer& L, const float* x, uint32_t T,
                               const int32_t* idx, const float* w, float* act, float* act_sh,
                               float* y);
hipError_t launch_dequant(const Launch& K, const mr_pack& p, uint32_t expert, float* out);
hipError_t launch_rms_norm(const Launch& K, const float* h, const float* w, float eps, uint32_t T, uint32_t H,
                           float* out);
hipError_t launch_residual_add(const Launch& K, const float* h, const float* m, uint64_t n, float* out);
hipError_t launch_synth(const Launch& K, int type, void* dst, uint64_t n_blocks, uint64_t seed);
// Measurement probes (mr_probe.hip).
hipError_t launch_probe_read(const Launch& K, const void* src, uint64_t nbytes, uint32_t n_wg, uint32_t depth,
                             uint32_t* sink);
hipError_t launch_probe_tiles(const Launch& K, const void* src, uint32_t rb, uint32_t n_tiles, uint32_t n_wg,
                              uint32_t depth, uint32_t* sink);
hipError_t launch_probe_touch(const Launch& K, const void* src, uint64_t nbytes, uint32_t stride, uint32_t* sink);
hipError_t launch_probe_empty(const Launch& K, uint32_t n_wg);
hipError_t launch_probe_flags(const Launch& K, uint32_t* words, int a, int b, int n, unsigned long long* res);
// With `device` current: this device's address of the static scratch array (looked up once
// per device).
hipError_t static_scratch_init(int device, void** out);

// Records an error on the context (or the calling thread when ctx is NULL); returns code.
int set_error(mr_ctx* ctx, int code, const char* msg);
// Hands packs and device buffers to a layer, which frees them in mr_layer_destroy.
void layer_adopt(mr_layer* L, mr_pack* const* packs, size_t n_packs, void* const* dev, size_t n_dev);

// Fused RMSNorm of the layer input and residual added to its output
// (mr_moe_forward_residual; norm.rs:16-37, layer.rs:462-473). w == nullptr: off.
struct NormResid {
  const float* w = nullptr;      // [H] norm weight
  float eps = 0.f;
  const float* resid = nullptr;  // [H] residual h (the un-normalised input)
};

// Time limit of a fused kernel's cross-workgroup waits (mr_fused_common.h): the context's limit in
// ticks of the device clock; limits below 100 us (a limit forced by a test) consult the clock from
// the first poll, longer ones after 64 polls.
struct WaitBound {
  uint32_t free;   // polls before the clock is consulted
  uint32_t ticks;  // time limit in clock ticks
};
inline WaitBound wait_bound(const mr_ctx& c) {
  const uint64_t t = (uint64_t)c.wait_limit_us * (uint64_t)c.wall_khz / 1000u;
  return WaitBound{c.wait_limit_us < 100u ? 0u : 64u, (uint32_t)std::min<uint64_t>(t, 0xFFFFFFFFull)};
}

// Fused single-launch MXFP4 decode layer (mr_fused.hip).
constexpr int kSyncErrWord = 96;  // uint32 index of the fused kernel's error word
bool fused_supported(const mr_layer& L, int n_cu);
bool fused_resident(const mr_layer& L, int n_cu);      // the whole grid fits the CUs at once
hipError_t launch_fused(const Launch& K, const mr_layer& L, const float* x, float* y,
                        uint32_t* err, uint8_t* img_base, WaitBound wb, int n_cu,
                        const NormResid& nr = NormResid{});
uint64_t fused_layer_sync_bytes(const mr_layer& L);  // sync block of one layer (its logit count)

// Scratch of the grouped multi-token MXFP4 path (device pointers; P = T * top_k pairs).
struct GroupedScratch {
  int32_t* pair_tok;  // [P] token of sorted pair p
  float* pair_w;      // [P] its routing weight
  int32_t* pair_of;   // [P] sorted index of (token, slot)
  int32_t* exp_off;   // [E+1] pair offset of each expert
  int32_t* tile_off;  // [E+1] 16-pair tile offset of each expert
  uint8_t* img_x;     // [T][H/32][128] x images
  uint32_t* sc_x;     // [T][H/32]
  uint8_t* img_h;     // [P][I/32][128] h images
  uint32_t* sc_h;     // [P][I/32]
  float* obuf;        // [P][H] down results
  uint8_t* img_hsh;   // [T][Ish/32][128] shared-expert h images
  uint32_t* sc_hsh;   // [T][Ish/32]
  float* osh;         // [T][H] shared-expert down results
  float* sig;         // [T] its sigmoid gate
};
GroupedScratch grouped_scratch(const Scratch& s, uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H,
                               uint64_t Ish);
uint64_t grouped_scratch_bytes(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish);
// sigmoid(x_t . gate_inp) per token t, or 1 without gate_inp (mr_grouped_q4k.hip)
hipError_t launch_sh_gate(const Launch& K, const float* x, uint32_t T, int H, const float* gate_inp, float* sig);
bool grouped_supported(const mr_layer& L);
hipError_t launch_grouped(const Launch& K, const mr_layer& L, const float* x, uint32_t T, const int32_t* idx,
                          const float* w, float* y, const GroupedScratch& gs);
// Pair grouping, grid size and the ascending-expert combine shared by the grouped paths
// (mr_grouped.hip).
unsigned grouped_grid(uint64_t items);
hipError_t launch_group(const Launch& K, const int32_t* idx, const float* w, int P, int k, int E, int32_t* pair_tok,
                        float* pair_w, int32_t* pair_of, int32_t* exp_off, int32_t* tile_off);
hipError_t launch_combine(const Launch& K, const float* o, const int32_t* pair_of, const int32_t* idx, const float* w,
                          const float* down_b, uint32_t T, int k, int H, const float* o_sh, const float* sh_sig,
                          float* y);
// Grouped multi-token Q4_K path on the int8 MFMA (mr_grouped_q4k.hip); scratch: one block of
// grouped_q4k_scratch_bytes.
bool grouped_q4k_supported(const mr_layer& L);
uint64_t grouped_q4k_scratch_bytes(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish);
hipError_t launch_grouped_q4k(const Launch& K, const mr_layer& L, const float* x, uint32_t T, const int32_t* idx,
                              const float* w, float* y, void* scratch);
bool fused_q4k_supported(const mr_layer& L, int n_cu);
bool fused_q4k_resident(const mr_layer& L, int n_cu);
hipError_t launch_fused_q4k(const Launch& K, const mr_layer& L, const float* x, float* y, uint32_t* err,
                            uint8_t* img_base, const NormResid& nr = NormResid{});
#ifdef MR_FUSED_TRACE
extern unsigned long long* g_fused_trace;
#endif

}  // namespace mr
