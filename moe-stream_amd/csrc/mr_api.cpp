// mr_api.cpp -- C ABI of include/moe_rocm.h: contexts, device memory, expert
// packs, layers, argument validation and dispatch to the gfx950 kernels.
//
// Every entry point validates its arguments before touching the device, so a
// host-only context (MR_DEVICE_NONE) exercises every error path without a GPU.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <new>

#include "mr_internal.h"

namespace {

thread_local std::string g_err;  // errors of calls that have no context

int set_err(mr_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (c)
    c->err = buf;
  else
    g_err = buf;
  return code;
}

int hip_fail(mr_ctx* c, hipError_t e, const char* what) {
  int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? MR_E_NOMEM : MR_E_LAUNCH;
  return set_err(c, code, "%s: %s", what, hipGetErrorString(e));
}

bool has_dev(const mr_ctx* c) { return c && c->device >= 0; }

// Make the context's device current for this host thread.
int bind(mr_ctx* c) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return set_err(c, MR_E_LAUNCH, "hipGetDevice failed");
  if (cur != c->device) {
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
  }
  return MR_OK;
}

uint64_t block_elems(int type) { return type == MR_GGML_MXFP4 ? 32u : 256u; }

bool valid_type(int type) { return type == MR_GGML_MXFP4 || type == MR_GGML_Q4_K; }

constexpr uint64_t kAlign = 256;
uint64_t align_up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int pack_common(mr_ctx* c, int type, const void* bytes, uint64_t nbytes, uint32_t E, uint32_t out,
                uint32_t in, const uint64_t* host_offsets, mr_pack** res) {
  if (!res) return set_err(c, MR_E_INVAL, "out pointer is NULL");
  *res = nullptr;
  if (!valid_type(type)) return set_err(c, MR_E_UNSUPPORTED, "ggml type %d is not MXFP4 (39) or Q4_K (12)", type);
  if (!bytes) return set_err(c, MR_E_INVAL, "weight bytes are NULL");
  if (E == 0 || out == 0 || in == 0) return set_err(c, MR_E_INVAL, "empty expert shape E=%u out=%u in=%u", E, out, in);
  if (in % block_elems(type) != 0)
    return set_err(c, MR_E_INVAL, "in_features %u is not a multiple of the %llu-element block", in,
                   (unsigned long long)block_elems(type));
  const uint64_t mb = mr_matrix_bytes(type, out, in);
  std::vector<uint64_t> off(E);
  for (uint32_t e = 0; e < E; ++e) {
    off[e] = host_offsets ? host_offsets[e] : (uint64_t)e * mb;
    if (off[e] > nbytes || nbytes - off[e] < mb)
      return set_err(c, MR_E_INVAL, "expert %u slice [%llu, +%llu) exceeds %llu bytes", e,
                     (unsigned long long)off[e], (unsigned long long)mb, (unsigned long long)nbytes);
    if (type == MR_GGML_Q4_K && (off[e] % 4 != 0))
      return set_err(c, MR_E_INVAL, "Q4_K expert %u offset %llu is not 4-byte aligned", e,
                     (unsigned long long)off[e]);
  }
  mr_pack* p = new (std::nothrow) mr_pack;
  if (!p) return set_err(c, MR_E_NOMEM, "host allocation failed");
  p->ctx = c;
  p->type = type;
  p->n_experts = E;
  p->out_features = out;
  p->in_features = in;
  p->nbytes = nbytes;
  p->matrix_bytes = mb;
  p->h_offsets = std::move(off);
  p->uniform = true;
  p->uni_off0 = p->h_offsets[0];
  p->uni_stride = E > 1 ? p->h_offsets[1] - p->h_offsets[0] : 0;
  for (uint32_t e = 1; e < E && p->uniform; ++e)
    p->uniform = p->h_offsets[e] >= p->uni_off0 && p->h_offsets[e] - p->uni_off0 == (uint64_t)e * p->uni_stride;
  *res = p;
  return MR_OK;
}

int upload_offsets(mr_ctx* c, mr_pack* p) {
  if (!has_dev(c)) return MR_OK;
  hipError_t e = hipMalloc(&p->d_offsets, sizeof(uint64_t) * p->n_experts);
  if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(offsets)");
  e = hipMemcpy(p->d_offsets, p->h_offsets.data(), sizeof(uint64_t) * p->n_experts,
                hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(c, e, "hipMemcpy(offsets)");
  return MR_OK;
}

// Scratch layout for T tokens of a layer shape.
struct ScratchPlan {
  uint64_t idx, w, logits, rpart, act, act_sh, mfma_b, sync, groups, grouped, xn, ytmp, total;
};

ScratchPlan plan_scratch(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish) {
  ScratchPlan p{};
  uint64_t o = 0;
  p.idx = o, o += align_up(T * k * 4);
  p.w = o, o += align_up(T * k * 4);
  p.logits = o, o += align_up(T * E * 4);
  p.rpart = o, o += align_up(4 * T * E * 4);
  p.act = o, o += align_up(T * k * I * 4);
  p.act_sh = o, o += align_up(T * (Ish + 1) * 4);
  // MFMA B-operand images: x split (H/32 blocks) and act split (k*I/32 blocks, then Ish/32 of
  // the shared expert), 16 columns x 33 bytes per block, rounded generously; then the fused
  // MXFP4 kernel's per-slot down rows (top_k + shared slots of H floats).
  p.mfma_b = o, o += align_up(((H / 32) + ((k * I + Ish) / 32) + 64) * 16 * 40 + (k + 1) * H * 4 + 256);
  p.sync = o, o += align_up(4096);
  p.groups = o, o += align_up((T * k + E + 64) * 8);
  p.grouped = o, o += align_up(std::max(mr::grouped_scratch_bytes(T, k, E, I, H, Ish),
                                        mr::grouped_q4k_scratch_bytes(T, k, E, I, H, Ish)));
  p.xn = o, o += align_up(T * H * 4);
  p.ytmp = o, o += align_up(T * H * 4);
  p.total = o;
  return p;
}

// Scratch of one batched call (mr_moe_forward_batched_noalloc): routing outputs, logits and
// router partials, then either the grouped MFMA path's pair lists and images, or the VALU
// path's activations [T, k, I] and shared activations [T, Ish + 1].
struct BatchedPlan {
  uint64_t idx, w, logits, rpart, work, work_sh, total;
};

// Which multi-token path a layer takes (mr_moe_forward_batched and its static-scratch variant).
enum class Batched { valu, grouped_mx, grouped_q4k };
Batched batched_kind(const mr_ctx* c, const mr_layer& L) {
  if (c->decode_kernel == MR_DECODE_VALU) return Batched::valu;
  if (mr::grouped_supported(L)) return Batched::grouped_mx;
  if (mr::grouped_q4k_supported(L)) return Batched::grouped_q4k;
  return Batched::valu;
}

BatchedPlan plan_batched(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish, Batched kind) {
  BatchedPlan p{};
  uint64_t o = 0;
  p.idx = o, o += align_up(T * k * 4);
  p.w = o, o += align_up(T * k * 4);
  p.logits = o, o += align_up(T * E * 4);
  p.rpart = o, o += align_up(4 * T * E * 4);
  p.work = o;
  if (kind == Batched::grouped_mx) {
    o += align_up(mr::grouped_scratch_bytes(T, k, E, I, H, Ish));
    p.work_sh = o;
  } else if (kind == Batched::grouped_q4k) {
    o += align_up(mr::grouped_q4k_scratch_bytes(T, k, E, I, H, Ish));
    p.work_sh = o;
  } else {
    o += align_up(T * k * I * 4);
    p.work_sh = o, o += align_up(T * (Ish + 1) * 4);
  }
  p.total = o;
  return p;
}

// Scratch grows to cover the largest shape and token count seen. A call that needs more
// tokens than the scratch holds grows it to at least twice its token capacity (mr_reserve
// asks for exactly max_tokens), so a token count that creeps up costs O(log T) allocations.
// The superseded allocation is freed once the stream has drained, unless a graph was
// captured since it was allocated: such a graph may still address it, so it is kept (with
// its fused-kernel error word still checked by mr_sync) until mr_ctx_destroy.
int ensure_scratch(mr_ctx* c, const mr_layer* L, uint64_t T, bool exact = false) {
  mr::Scratch& s = c->scratch;
  uint64_t k = L->d.top_k, E = L->E, I = L->I, H = L->H, Ish = L->Ish;
  if (s.base && T <= s.cap_tokens && k <= s.cap_k && E <= s.cap_e && I <= s.cap_i && H <= s.cap_h &&
      Ish <= s.cap_ish)
    return MR_OK;
  if (c->capturing)
    return set_err(c, MR_E_INVAL, "scratch too small during graph capture; call mr_reserve first");
  const uint64_t grown = T > s.cap_tokens && !exact ? std::max<uint64_t>(T, 2 * s.cap_tokens) : T;
  uint64_t nT = std::max<uint64_t>(grown, s.cap_tokens), nk = std::max<uint64_t>(k, s.cap_k);
  uint64_t nE = std::max<uint64_t>(E, s.cap_e), nI = std::max<uint64_t>(I, s.cap_i);
  uint64_t nH = std::max<uint64_t>(H, s.cap_h), nS = std::max<uint64_t>(Ish, s.cap_ish);
  ScratchPlan p = plan_scratch(nT, nk, nE, nI, nH, nS);
  hipError_t e;
  if (s.base) {
    if (c->captured_since_alloc) {
      c->retired.push_back(s.base);
      c->retired_err.push_back(s.sync + mr::kSyncErrWord);
    } else {
      // no graph addresses it: drain the stream, keep an unreported wait failure, free it
      e = hipStreamSynchronize(c->stream);
      if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
      if (c->fused_used && s.sync) {
        uint32_t word = 0;
        e = hipMemcpy(&word, s.sync + mr::kSyncErrWord, 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(c, e, "read fused error word");
        if (word) c->pending_wait_err = true;
      }
      e = hipFree(s.base);
      if (e != hipSuccess) return hip_fail(c, e, "hipFree(scratch)");
    }
    s = mr::Scratch{};
  }
  void* base = nullptr;
  e = hipMalloc(&base, p.total);
  if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(scratch)");
  c->captured_since_alloc = false;
  // sync words and counters must start at zero; later calls keep them balanced
  e = mr::launch_zero(mr::Launch{c->stream, nullptr}, base, p.total);
  if (e != hipSuccess) return hip_fail(c, e, "zero scratch");
  char* b = static_cast<char*>(base);
  s.base = base;
  s.bytes = p.total;
  s.idx = reinterpret_cast<int32_t*>(b + p.idx);
  s.w = reinterpret_cast<float*>(b + p.w);
  s.logits = reinterpret_cast<float*>(b + p.logits);
  s.rpart = reinterpret_cast<float*>(b + p.rpart);
  s.act = reinterpret_cast<float*>(b + p.act);
  s.act_sh = reinterpret_cast<float*>(b + p.act_sh);
  s.mfma_b = b + p.mfma_b;
  s.sync = reinterpret_cast<uint32_t*>(b + p.sync);
  s.groups = reinterpret_cast<int32_t*>(b + p.groups);
  s.grouped = b + p.grouped;
  s.xn = reinterpret_cast<float*>(b + p.xn);
  s.ytmp = reinterpret_cast<float*>(b + p.ytmp);
  s.cap_tokens = nT, s.cap_k = nk, s.cap_e = nE, s.cap_i = nI, s.cap_h = nH, s.cap_ish = nS;
  return MR_OK;
}

bool misaligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; }

// Kernels read f32 activations and router rows as 16-byte vectors and index/weight
// arrays as 4-byte words.
int check_io_align(mr_ctx* c, const float* x, const float* y, const void* idx, const float* w, const float* logits) {
  if (misaligned(x, 16) || misaligned(y, 16))
    return set_err(c, MR_E_INVAL, "x and y must be 16-byte aligned");
  if (misaligned(idx, 4) || misaligned(w, 4) || misaligned(logits, 4))
    return set_err(c, MR_E_INVAL, "idx, w and logits must be 4-byte aligned");
  return MR_OK;
}

int check_layer(mr_ctx* c, const mr_layer* L) {
  if (!L) return set_err(c, MR_E_INVAL, "layer is NULL");
  if (L->ctx != c) return set_err(c, MR_E_INVAL, "layer belongs to another context");
  return MR_OK;
}

// The array a T-token forward call of L writes its router logits to: the layer's logits output
// (mr_layer_set_logits_out) when set, else `own` (scratch). Calls of more tokens than the
// output holds are refused before anything is launched.
int logits_dst(mr_ctx* c, const mr_layer* L, uint32_t T, float* own, float** out) {
  if (!L->logits_out) {
    *out = own;
    return MR_OK;
  }
  if (T > L->logits_cap)
    return set_err(c, MR_E_INVAL, "n_tokens %u exceeds the %u tokens of the layer's logits output", T, L->logits_cap);
  *out = L->logits_out;
  return MR_OK;
}

}  // namespace

namespace mr {

hipEvent_t Prof::next_event() {
  if (used == pool.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    pool.push_back(e);
  }
  return pool[used++];
}

int Prof::name_id(const char* n) {
  for (size_t i = 0; i < names.size(); ++i)
    if (names[i] == n) return (int)i;
  names.emplace_back(n);
  return (int)names.size() - 1;
}

}  // namespace mr

extern "C" {

const char* mr_status_string(int status) {
  switch (status) {
    case MR_OK: return "ok";
    case MR_E_INVAL: return "invalid argument";
    case MR_E_NOMEM: return "out of device memory";
    case MR_E_NODEV: return "no HIP device";
    case MR_E_LAUNCH: return "HIP launch or runtime failure";
    case MR_E_UNSUPPORTED: return "unsupported";
    default: return "unknown status";
  }
}

const char* mr_last_error(const mr_ctx* ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

int mr_ctx_create(int device, mr_ctx** out) {
  if (!out) return set_err(nullptr, MR_E_INVAL, "out pointer is NULL");
  *out = nullptr;
  if (device < MR_DEVICE_NONE) return set_err(nullptr, MR_E_INVAL, "device %d is invalid", device);
  mr_ctx* c = new (std::nothrow) mr_ctx;
  if (!c) return set_err(nullptr, MR_E_NOMEM, "host allocation failed");
  if (device == MR_DEVICE_NONE) {
    *out = c;
    return MR_OK;
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    delete c;
    return set_err(nullptr, MR_E_NODEV, "no HIP device visible");
  }
  if (device >= n) {
    delete c;
    return set_err(nullptr, MR_E_INVAL, "device %d out of range (have %d)", device, n);
  }
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&c->ev0);
  if (e == hipSuccess) e = hipEventCreate(&c->ev1);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, device);
  if (e == hipSuccess && hipDeviceGetAttribute(&c->wall_khz, hipDeviceAttributeWallClockRate, device) != hipSuccess)
    c->wall_khz = 100000;  // the documented 100 MHz when the runtime does not report it
  if (e != hipSuccess) {
    int rc = hip_fail(nullptr, e, "context setup");
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return rc;
  }
  c->device = device;
  c->own_stream = true;
  // the device's static scratch (mr_moe_forward_batched_noalloc), resolved once per device
  // with the device current; a failure is reported by that entry point only
  c->static_err = mr::static_scratch_init(device, &c->static_scratch);
  *out = c;
  return MR_OK;
}

void mr_ctx_destroy(mr_ctx* c) {
  if (!c) return;
  if (has_dev(c)) {
    (void)bind(c);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->scratch.base) (void)hipFree(c->scratch.base);
    for (void* r : c->retired) (void)hipFree(r);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    for (hipEvent_t ev : c->prof.pool) (void)hipEventDestroy(ev);
    if (c->own_stream && c->stream) (void)hipStreamDestroy(c->stream);
  }
  delete c;
}

int mr_ctx_device(const mr_ctx* c) { return c ? c->device : MR_DEVICE_NONE; }

int mr_ctx_set_stream(mr_ctx* c, void* hip_stream) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context has no stream");
  if (c->capturing) return set_err(c, MR_E_INVAL, "cannot change stream during capture");
  if (c->own_stream && c->stream) {
    (void)hipStreamSynchronize(c->stream);
    (void)hipStreamDestroy(c->stream);
  }
  c->stream = static_cast<hipStream_t>(hip_stream);
  c->own_stream = false;
  return MR_OK;
}

void* mr_ctx_stream(const mr_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int mr_ctx_set_option(mr_ctx* c, int option, int value) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (option == MR_OPT_DECODE_KERNEL) {
    if (value < MR_DECODE_AUTO || value > MR_DECODE_FUSED)
      return set_err(c, MR_E_INVAL, "decode kernel %d unknown", value);
    c->decode_kernel = value;
    return MR_OK;
  }
  if (option == MR_OPT_WAIT_LIMIT_US) {
    if (value < 0) return set_err(c, MR_E_INVAL, "wait limit %d us is negative", value);
    c->wait_limit_us = value == 0 ? 50000u : (uint32_t)value;
    return MR_OK;
  }
  if (option == MR_OPT_PROFILE) {
    if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
    c->prof.on = value != 0;
    return MR_OK;
  }
  return set_err(c, MR_E_INVAL, "option %d unknown", option);
}

int mr_sync(mr_ctx* c) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
  if (c->fused_used && c->scratch.sync) {
    // the current scratch's error word and those of superseded scratch (graphs captured
    // before the scratch grew still write there)
    bool ran_out = c->pending_wait_err;
    c->pending_wait_err = false;
    const size_t n_words = 1 + c->retired_err.size();
    for (size_t i = 0; i < n_words; ++i) {
      uint32_t* dev = i == 0 ? c->scratch.sync + mr::kSyncErrWord : c->retired_err[i - 1];
      uint32_t word = 0;
      e = hipMemcpy(&word, dev, 4, hipMemcpyDeviceToHost);
      if (e != hipSuccess) return hip_fail(c, e, "read fused error word");
      if (word) {
        const uint32_t zero = 0;
        e = hipMemcpy(dev, &zero, 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(c, e, "reset fused error word");
        ran_out = true;
      }
    }
    if (ran_out)
      return set_err(c, MR_E_LAUNCH, "fused decode kernel: a cross-workgroup wait ran out (results of that launch are invalid)");
  }
  return MR_OK;
}

int mr_dev_alloc(mr_ctx* c, uint64_t nbytes, void** out) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!out) return set_err(c, MR_E_INVAL, "out pointer is NULL");
  *out = nullptr;
  if (nbytes == 0) return set_err(c, MR_E_INVAL, "zero-byte allocation");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if (c->capturing) return set_err(c, MR_E_INVAL, "allocation during graph capture");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipMalloc(out, nbytes);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "hipMalloc");
}

int mr_dev_free(mr_ctx* c, void* p) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!p) return MR_OK;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  (void)hipStreamSynchronize(c->stream);
  hipError_t e = hipFree(p);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "hipFree");
}

int mr_upload(mr_ctx* c, void* dst, const void* src, uint64_t n) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if ((!dst || !src) && n) return set_err(c, MR_E_INVAL, "NULL buffer");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if (n == 0) return MR_OK;
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "upload");
}

int mr_download(mr_ctx* c, void* dst, const void* src, uint64_t n) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if ((!dst || !src) && n) return set_err(c, MR_E_INVAL, "NULL buffer");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if (n == 0) return MR_OK;
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "download");
}

int mr_dev_zero(mr_ctx* c, void* dst, uint64_t n) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!dst && n) return set_err(c, MR_E_INVAL, "NULL buffer");
  if (n % 4) return set_err(c, MR_E_INVAL, "zero fill size %llu is not a multiple of 4", (unsigned long long)n);
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = mr::launch_zero(c->launch(), dst, n);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "zero fill");
}

uint64_t mr_matrix_bytes(int type, uint64_t rows, uint64_t cols) {
  if (type == MR_GGML_MXFP4) return rows * (cols / 32) * 17;
  if (type == MR_GGML_Q4_K) return rows * (cols / 256) * 144;
  return 0;
}

int mr_pack_upload(mr_ctx* c, int type, const void* host_bytes, uint64_t nbytes, uint32_t E,
                   uint32_t out, uint32_t in, const uint64_t* host_offsets, mr_pack** res) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = pack_common(c, type, host_bytes, nbytes, E, out, in, host_offsets, res);
  if (rc) return rc;
  mr_pack* p = *res;
  if (!has_dev(c)) {
    // host-only: keep the layout, no device copy (used by validation tests)
    p->base = static_cast<const uint8_t*>(host_bytes);
    return MR_OK;
  }
  if ((rc = bind(c))) {
    delete p, *res = nullptr;
    return rc;
  }
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, nbytes + 64);
  if (e != hipSuccess) {
    delete p, *res = nullptr;
    return hip_fail(c, e, "hipMalloc(pack)");
  }
  e = hipMemcpy(d, host_bytes, nbytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    delete p, *res = nullptr;
    return hip_fail(c, e, "hipMemcpy(pack)");
  }
  p->base = static_cast<const uint8_t*>(d);
  p->owned = true;
  if ((rc = upload_offsets(c, p))) {
    mr_pack_destroy(p), *res = nullptr;
    return rc;
  }
  return MR_OK;
}

int mr_pack_wrap(mr_ctx* c, int type, const void* dev_bytes, uint64_t nbytes, uint32_t E,
                 uint32_t out, uint32_t in, const uint64_t* host_offsets, mr_pack** res) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = pack_common(c, type, dev_bytes, nbytes, E, out, in, host_offsets, res);
  if (rc) return rc;
  mr_pack* p = *res;
  if (type == MR_GGML_Q4_K && (reinterpret_cast<uintptr_t>(dev_bytes) % 4 != 0)) {
    delete p, *res = nullptr;
    return set_err(c, MR_E_INVAL, "Q4_K device bytes must be 4-byte aligned");
  }
  p->base = static_cast<const uint8_t*>(dev_bytes);
  if (has_dev(c)) {
    if ((rc = bind(c)) || (rc = upload_offsets(c, p))) {
      mr_pack_destroy(p), *res = nullptr;
      return rc;
    }
  }
  return MR_OK;
}

void mr_pack_destroy(mr_pack* p) {
  if (!p) return;
  if (has_dev(p->ctx)) {
    (void)bind(p->ctx);
    (void)hipStreamSynchronize(p->ctx->stream);
    if (p->owned && p->base) (void)hipFree(const_cast<uint8_t*>(p->base));
    if (p->d_offsets) (void)hipFree(p->d_offsets);
  }
  delete p;
}

int mr_dequant(mr_ctx* c, const mr_pack* p, uint32_t expert, float* out) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!p || !out) return set_err(c, MR_E_INVAL, "NULL pack or output");
  if (p->ctx != c) return set_err(c, MR_E_INVAL, "pack belongs to another context");
  if (expert >= p->n_experts) return set_err(c, MR_E_INVAL, "expert %u out of range (E=%u)", expert, p->n_experts);
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = mr::launch_dequant(c->launch(), *p, expert, out);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "dequant launch");
}

int mr_layer_create(mr_ctx* c, const mr_layer_desc* d, mr_layer** res) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!d || !res) return set_err(c, MR_E_INVAL, "NULL descriptor or out pointer");
  *res = nullptr;
  if (!d->gate || !d->up || !d->down) return set_err(c, MR_E_INVAL, "gate, up and down packs are required");
  if (d->gate->ctx != c || d->up->ctx != c || d->down->ctx != c)
    return set_err(c, MR_E_INVAL, "packs belong to another context");
  const int type = d->gate->type;
  if (d->up->type != type || d->down->type != type)
    return set_err(c, MR_E_INVAL, "gate/up/down packs have different block types");
  const uint32_t E = d->gate->n_experts, I = d->gate->out_features, H = d->gate->in_features;
  if (d->up->n_experts != E || d->down->n_experts != E)
    return set_err(c, MR_E_INVAL, "expert counts differ (%u/%u/%u)", E, d->up->n_experts, d->down->n_experts);
  if (d->up->out_features != I || d->up->in_features != H)
    return set_err(c, MR_E_INVAL, "up pack is [%u,%u], expected [%u,%u]", d->up->out_features, d->up->in_features, I, H);
  if (d->down->out_features != H || d->down->in_features != I)
    return set_err(c, MR_E_INVAL, "down pack is [%u,%u], expected [%u,%u]", d->down->out_features, d->down->in_features, H, I);
  if (!d->router_w) return set_err(c, MR_E_INVAL, "router weights are required");
  for (const float* f : {d->router_w, d->router_b, d->dummy_mask, d->gate_bias, d->up_bias, d->down_bias,
                         d->sh_gate_inp})
    if (misaligned(f, 16))
      return set_err(c, MR_E_INVAL, "router, bias, mask and shared-gate arrays must be 16-byte aligned");
  if (E > mr::kMaxExperts) return set_err(c, MR_E_UNSUPPORTED, "n_experts %u > %u", E, mr::kMaxExperts);
  if (d->top_k == 0 || d->top_k > mr::kMaxTopK || d->top_k > E)
    return set_err(c, MR_E_INVAL, "top_k %u must be in 1..min(16, E=%u)", d->top_k, E);
  if (d->act != MR_ACT_SILU && d->act != MR_ACT_SWIGLU_OAI) return set_err(c, MR_E_INVAL, "activation %u unknown", d->act);
  if (d->route_flags & ~(MR_ROUTE_SOFTMAX_AFTER_TOPK | MR_ROUTE_NORM_TOPK))
    return set_err(c, MR_E_INVAL, "unknown routing flags 0x%x", d->route_flags);
  if (H > mr::kMaxHidden) return set_err(c, MR_E_UNSUPPORTED, "hidden %u > %u", H, mr::kMaxHidden);
  uint32_t Ish = 0;
  const bool any_sh = d->sh_gate || d->sh_up || d->sh_down;
  if (any_sh) {
    if (!d->sh_gate || !d->sh_up || !d->sh_down)
      return set_err(c, MR_E_INVAL, "shared expert needs gate, up and down packs");
    if (d->sh_gate->ctx != c || d->sh_up->ctx != c || d->sh_down->ctx != c)
      return set_err(c, MR_E_INVAL, "shared packs belong to another context");
    if (d->sh_gate->type != d->sh_up->type)
      return set_err(c, MR_E_INVAL, "shared gate/up packs have different block types");
    Ish = d->sh_gate->out_features;
    if (d->sh_gate->n_experts != 1 || d->sh_up->n_experts != 1 || d->sh_down->n_experts != 1)
      return set_err(c, MR_E_INVAL, "shared expert packs must hold exactly one expert");
    if (d->sh_gate->in_features != H || d->sh_up->out_features != Ish || d->sh_up->in_features != H ||
        d->sh_down->out_features != H || d->sh_down->in_features != Ish)
      return set_err(c, MR_E_INVAL, "shared expert shapes do not match hidden %u / inter %u", H, Ish);
  }
  if ((uint64_t)d->top_k * I + Ish > mr::kMaxHidden)
    return set_err(c, MR_E_UNSUPPORTED, "top_k*inter + shared inter = %llu exceeds %u",
                   (unsigned long long)d->top_k * I + Ish, mr::kMaxHidden);
  mr_layer* L = new (std::nothrow) mr_layer;
  if (!L) return set_err(c, MR_E_NOMEM, "host allocation failed");
  L->ctx = c;
  L->d = *d;
  L->H = H, L->I = I, L->E = E, L->Ish = Ish, L->type = type;
  if (has_dev(c) && ((mr::fused_supported(*L, c->n_cu) && mr::fused_resident(*L, c->n_cu)) ||
                     (mr::fused_q4k_supported(*L, c->n_cu) && mr::fused_q4k_resident(*L, c->n_cu)))) {
    // sync block of the fused decode kernel: counters start at zero
    int rc = bind(c);
    void* fs = nullptr;
    hipError_t e = rc ? hipSuccess : hipMalloc(&fs, mr::fused_layer_sync_bytes(*L));
    if (!rc && e == hipSuccess) e = hipMemset(fs, 0, mr::fused_layer_sync_bytes(*L));
    if (rc || e != hipSuccess) {
      if (fs) (void)hipFree(fs);
      delete L;
      return rc ? rc : hip_fail(c, e, "hipMalloc(fused sync)");
    }
    L->fused_sync = static_cast<uint32_t*>(fs);
  }
  *res = L;
  return MR_OK;
}

int mr_layer_set_logits_out(mr_layer* L, float* logits, uint32_t max_tokens) {
  if (!L) return set_err(nullptr, MR_E_INVAL, "mr_layer_set_logits_out: layer is NULL");
  if (logits && max_tokens == 0) return set_err(L->ctx, MR_E_INVAL, "mr_layer_set_logits_out: max_tokens is 0");
  if (misaligned(logits, 4)) return set_err(L->ctx, MR_E_INVAL, "mr_layer_set_logits_out: logits must be 4-byte aligned");
  L->logits_out = logits;
  L->logits_cap = logits ? max_tokens : 0;
  return MR_OK;
}

int mr_layer_set_norm(mr_layer* L, const float* norm_w) {
  if (!L) return set_err(nullptr, MR_E_INVAL, "mr_layer_set_norm: layer is NULL");
  if (misaligned(norm_w, 16)) return set_err(L->ctx, MR_E_INVAL, "mr_layer_set_norm: norm_w must be 16-byte aligned");
  L->norm_w = norm_w;
  return MR_OK;
}

int mr_layer_set_next(mr_layer* L, const mr_layer* next) {
  if (!L) return set_err(nullptr, MR_E_INVAL, "mr_layer_set_next: layer is NULL");
  if (next && next->ctx != L->ctx) return set_err(L->ctx, MR_E_INVAL, "mr_layer_set_next: layers of different contexts");
  L->next = next;
  return MR_OK;
}

void mr_layer_destroy(mr_layer* L) {
  if (!L) return;
  if (L->fused_sync && has_dev(L->ctx)) {
    (void)bind(L->ctx);
    (void)hipStreamSynchronize(L->ctx->stream);
    (void)hipFree(L->fused_sync);
  }
  for (mr_pack* p : L->own_packs) mr_pack_destroy(p);
  for (void* d : L->own_dev) (void)mr_dev_free(L->ctx, d);
  delete L;
}


int mr_reserve(mr_ctx* c, const mr_layer* L, uint32_t max_tokens) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (max_tokens == 0) return set_err(c, MR_E_INVAL, "max_tokens is 0");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c))) return rc;
  return ensure_scratch(c, L, max_tokens, true);
}

int mr_router_topk(mr_ctx* c, const mr_layer* L, const float* x, uint32_t T, int32_t* idx,
                   float* w, float* logits) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!x || !idx || !w) return set_err(c, MR_E_INVAL, "NULL x, idx or w");
  if ((rc = check_io_align(c, x, nullptr, idx, w, logits))) return rc;
  if (T == 0) return MR_OK;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c)) || (rc = ensure_scratch(c, L, T))) return rc;
  float* lg = logits ? logits : c->scratch.logits;
  hipError_t e = mr::launch_router_topk(c->launch(), *L, x, T, lg, c->scratch.rpart, idx, w);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "router launch");
}

int mr_topk(mr_ctx* c, const float* logits, uint32_t T, uint32_t E, uint32_t k, uint32_t flags,
            int32_t* idx, float* w) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!logits || !idx || !w) return set_err(c, MR_E_INVAL, "NULL logits, idx or w");
  if (E == 0 || E > mr::kMaxExperts) return set_err(c, MR_E_INVAL, "n_experts %u must be in 1..%u", E, mr::kMaxExperts);
  if (k == 0 || k > mr::kMaxTopK || k > E) return set_err(c, MR_E_INVAL, "top_k %u must be in 1..min(16, %u)", k, E);
  if (flags & ~(MR_ROUTE_SOFTMAX_AFTER_TOPK | MR_ROUTE_NORM_TOPK)) return set_err(c, MR_E_INVAL, "unknown routing flags 0x%x", flags);
  int rc = check_io_align(c, nullptr, nullptr, idx, w, logits);
  if (rc) return rc;
  if (T == 0) return MR_OK;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c))) return rc;
  hipError_t e = mr::launch_topk(c->launch(), logits, T, E, k, flags, idx, w);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "topk launch");
}

int mr_moe_experts(mr_ctx* c, const mr_layer* L, const float* x, uint32_t T, const int32_t* idx,
                   const float* w, float* y) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!x || !idx || !w || !y) return set_err(c, MR_E_INVAL, "NULL x, idx, w or y");
  if ((rc = check_io_align(c, x, y, idx, w, nullptr))) return rc;
  if (T == 0) return MR_OK;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c)) || (rc = ensure_scratch(c, L, T))) return rc;
  hipError_t e = mr::launch_experts_valu(c->launch(), *L, x, T, idx, w, c->scratch.act,
                                         c->scratch.act_sh, y);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "expert launch");
}

// One decode token through the layer. nr.w != nullptr: the input is rms_norm(x) and the
// output is x + moe(rms_norm(x)) (mr_moe_forward_residual); y may then alias x.
static int forward_one(mr_ctx* c, const mr_layer* L, const float* x, float* y, const mr::NormResid& nr) {
  int rc;
  if ((rc = bind(c)) || (rc = ensure_scratch(c, L, 1))) return rc;
  mr::Scratch& s = c->scratch;
  hipError_t e;
  if (c->decode_kernel != MR_DECODE_VALU && L->fused_sync) {
    uint32_t* err = s.sync + mr::kSyncErrWord;
    uint8_t* img = static_cast<uint8_t*>(s.mfma_b);
    if (mr::fused_supported(*L, c->n_cu)) {
      c->fused_used = true;
      e = mr::launch_fused(c->launch(), *L, x, y, err, img, mr::wait_bound(*c), c->n_cu, nr);
      return e == hipSuccess ? MR_OK : hip_fail(c, e, "fused moe forward launch");
    }
    if (mr::fused_q4k_supported(*L, c->n_cu)) {
      c->fused_used = true;
      e = mr::launch_fused_q4k(c->launch(), *L, x, y, err, img, nr);
      return e == hipSuccess ? MR_OK : hip_fail(c, e, "fused moe forward launch");
    }
  }
  if (c->decode_kernel == MR_DECODE_FUSED)
    return set_err(c, MR_E_UNSUPPORTED, "the fused decode kernels do not cover this layer shape");
  const float* xin = x;
  float* yout = y;
  e = hipSuccess;
  if (nr.w) {
    e = mr::launch_rms_norm(c->launch(), x, nr.w, nr.eps, 1, L->H, s.xn);
    xin = s.xn, yout = s.ytmp;
  }
  float* lg = L->logits_out ? L->logits_out : s.logits;
  if (e == hipSuccess) e = mr::launch_router_logits(c->launch(), *L, xin, 1, lg);
  if (e == hipSuccess) e = mr::launch_topk(c->launch(), lg, 1, L->E, L->d.top_k, L->d.route_flags, s.idx, s.w);
  if (e == hipSuccess) e = mr::launch_experts_valu(c->launch(), *L, xin, 1, s.idx, s.w, s.act, s.act_sh, yout);
  if (e == hipSuccess && nr.w) e = mr::launch_residual_add(c->launch(), x, s.ytmp, L->H, y);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "moe forward launch");
}

int mr_moe_forward(mr_ctx* c, const mr_layer* L, const float* x, float* y) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!x || !y) return set_err(c, MR_E_INVAL, "NULL x or y");
  if ((rc = check_io_align(c, x, y, nullptr, nullptr, nullptr))) return rc;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  return forward_one(c, L, x, y, mr::NormResid{});
}

int mr_moe_forward_residual(mr_ctx* c, const mr_layer* L, const float* h, const float* norm_w, float eps,
                            float* h_out) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!h || !norm_w || !h_out) return set_err(c, MR_E_INVAL, "NULL h, norm_w or h_out");
  if (!(eps >= 0.f) || eps > 1.f) return set_err(c, MR_E_INVAL, "eps %g is not in [0, 1]", (double)eps);
  if ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(h_out)) & 15u)
    return set_err(c, MR_E_INVAL, "h, norm_w and h_out must be 16-byte aligned");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  mr::NormResid nr;
  nr.w = norm_w, nr.eps = eps, nr.resid = h;
  return forward_one(c, L, h, h_out, nr);
}

// Routing and experts for T tokens (scratch already sized for T): the grouped GEMM path of the
// layer's type, else the per-token VALU kernels.
static hipError_t batched_core(mr_ctx* c, const mr_layer* L, const float* x, uint32_t T, float* y) {
  mr::Scratch& s = c->scratch;
  float* lg = L->logits_out ? L->logits_out : s.logits;  // T <= logits_cap checked by the caller
  hipError_t e = mr::launch_router_topk(c->launch(), *L, x, T, lg, s.rpart, s.idx, s.w);
  if (e == hipSuccess) {
    const Batched kind = batched_kind(c, *L);
    if (kind == Batched::grouped_mx)
      e = mr::launch_grouped(c->launch(), *L, x, T, s.idx, s.w, y,
                             mr::grouped_scratch(s, s.cap_tokens, s.cap_k, s.cap_e, s.cap_i, s.cap_h, s.cap_ish));
    else if (kind == Batched::grouped_q4k)
      e = mr::launch_grouped_q4k(c->launch(), *L, x, T, s.idx, s.w, y, s.grouped);
    else
      e = mr::launch_experts_valu(c->launch(), *L, x, T, s.idx, s.w, s.act, s.act_sh, y);
  }
  return e;
}

int mr_moe_forward_batched(mr_ctx* c, const mr_layer* L, const float* x, uint32_t T, float* y) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!x || !y) return set_err(c, MR_E_INVAL, "NULL x or y");
  if ((rc = check_io_align(c, x, y, nullptr, nullptr, nullptr))) return rc;
  if (T == 0) return MR_OK;
  float* lg;
  if ((rc = logits_dst(c, L, T, nullptr, &lg))) return rc;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c)) || (rc = ensure_scratch(c, L, T))) return rc;
  const hipError_t e = batched_core(c, L, x, T, y);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "batched moe launch");
}

int mr_moe_forward_batched_residual(mr_ctx* c, const mr_layer* L, const float* h, uint32_t T, const float* norm_w,
                                    float eps, float* h_out) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!h || !norm_w || !h_out) return set_err(c, MR_E_INVAL, "NULL h, norm_w or h_out");
  if (!(eps >= 0.f) || eps > 1.f) return set_err(c, MR_E_INVAL, "eps %g is not in [0, 1]", (double)eps);
  if ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(h_out)) & 15u)
    return set_err(c, MR_E_INVAL, "h, norm_w and h_out must be 16-byte aligned");
  if (T == 0) return MR_OK;
  float* lg;
  if ((rc = logits_dst(c, L, T, nullptr, &lg))) return rc;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if ((rc = bind(c)) || (rc = ensure_scratch(c, L, T))) return rc;
  mr::Scratch& s = c->scratch;
  hipError_t e = mr::launch_rms_norm(c->launch(), h, norm_w, eps, T, L->H, s.xn);
  if (e == hipSuccess) e = batched_core(c, L, s.xn, T, s.ytmp);
  if (e == hipSuccess) e = mr::launch_residual_add(c->launch(), h, s.ytmp, (uint64_t)T * L->H, h_out);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "batched moe residual launch");
}

int mr_moe_forward_batched_noalloc(mr_ctx* c, const mr_layer* L, const float* x, uint32_t T, float* y) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  int rc = check_layer(c, L);
  if (rc) return rc;
  if (!x || !y) return set_err(c, MR_E_INVAL, "NULL x or y");
  if ((rc = check_io_align(c, x, y, nullptr, nullptr, nullptr))) return rc;
  if (T == 0) return MR_OK;
  const Batched kind = batched_kind(c, *L);
  float* lg_out;
  if ((rc = logits_dst(c, L, T, nullptr, &lg_out))) return rc;
  const BatchedPlan p = plan_batched(T, L->d.top_k, L->E, L->I, L->H, L->Ish, kind);
  if (p.total > mr::kStaticScratchBytes)
    return set_err(c, MR_E_INVAL,
                   "n_tokens %u needs %llu bytes of scratch at this layer shape; the static scratch holds %llu "
                   "bytes (use mr_moe_forward_batched, or fewer tokens per call)",
                   T, (unsigned long long)p.total, (unsigned long long)mr::kStaticScratchBytes);
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if (!c->static_scratch) return hip_fail(c, c->static_err, "static scratch lookup (hipGetSymbolAddress)");
  if ((rc = bind(c))) return rc;
  char* b = static_cast<char*>(c->static_scratch);
  int32_t* idx = reinterpret_cast<int32_t*>(b + p.idx);
  float* w = reinterpret_cast<float*>(b + p.w);
  float* logits = lg_out ? lg_out : reinterpret_cast<float*>(b + p.logits);
  float* rpart = reinterpret_cast<float*>(b + p.rpart);
  // no profiling events here: recording them could create events (an allocation)
  const mr::Launch K{c->stream, nullptr};
  hipError_t e = mr::launch_router_topk(K, *L, x, T, logits, rpart, idx, w);
  if (e == hipSuccess) {
    if (kind == Batched::grouped_mx) {
      mr::Scratch view{};
      view.grouped = b + p.work;
      e = mr::launch_grouped(K, *L, x, T, idx, w, y,
                             mr::grouped_scratch(view, T, L->d.top_k, L->E, L->I, L->H, L->Ish));
    } else if (kind == Batched::grouped_q4k) {
      e = mr::launch_grouped_q4k(K, *L, x, T, idx, w, y, b + p.work);
    } else {
      e = mr::launch_experts_valu(K, *L, x, T, idx, w, reinterpret_cast<float*>(b + p.work),
                                  reinterpret_cast<float*>(b + p.work_sh), y);
    }
  }
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "batched moe launch (static scratch)");
}

int mr_probe_read(mr_ctx* c, const void* src, uint64_t nbytes, uint32_t n_wg, uint32_t depth, uint32_t* sink) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!src || !sink || n_wg == 0 || nbytes % 16 != 0) return set_err(c, MR_E_INVAL, "probe_read: bad arguments");
  if (depth != 4 && depth != 8 && depth != 16) return set_err(c, MR_E_INVAL, "probe_read: depth must be 4, 8 or 16");
  if (misaligned(src, 16)) return set_err(c, MR_E_INVAL, "probe_read: src must be 16-byte aligned");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  const hipError_t e = mr::launch_probe_read(c->launch(), src, nbytes, n_wg, depth, sink);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "probe_read launch");
}

int mr_probe_tiles(mr_ctx* c, const void* src, uint32_t row_bytes, uint32_t n_tiles, uint32_t n_wg, uint32_t depth,
                   uint32_t* sink) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!src || !sink || n_wg == 0 || row_bytes < 16 || n_tiles == 0) return set_err(c, MR_E_INVAL, "probe_tiles: bad arguments");
  if (depth != 2 && depth != 4 && depth != 8 && depth != 0x106 && depth != 0x10C && depth != 0x117)
    return set_err(c, MR_E_INVAL, "probe_tiles: depth must be 2, 4, 8 or 0x100 + 6, 12, 23");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  const hipError_t e = mr::launch_probe_tiles(c->launch(), src, row_bytes, n_tiles, n_wg, depth, sink);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "probe_tiles launch");
}

int mr_probe_touch(mr_ctx* c, const void* src, uint64_t nbytes, uint32_t stride, uint32_t* sink) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!src || !sink || nbytes < 4 || stride < 4 || stride % 4 != 0 || misaligned(src, 4))
    return set_err(c, MR_E_INVAL, "probe_touch: bad arguments");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  const hipError_t e = mr::launch_probe_touch(c->launch(), src, nbytes - 3, stride, sink);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "probe_touch launch");
}

int mr_probe_flags(mr_ctx* c, uint32_t* words, uint32_t wg_a, uint32_t wg_b, uint32_t n_round_trips,
                   unsigned long long* result) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!words || !result) return set_err(c, MR_E_INVAL, "probe_flags: NULL words or result");
  if (wg_a == wg_b || wg_a > 1023 || wg_b > 1023 || n_round_trips == 0 || n_round_trips > 100000)
    return set_err(c, MR_E_INVAL, "probe_flags: workgroups %u, %u and %u round trips out of range", wg_a, wg_b,
                   n_round_trips);
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  const hipError_t e = mr::launch_probe_flags(c->launch(), words, (int)wg_a, (int)wg_b, (int)n_round_trips, result);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "probe_flags launch");
}

int mr_probe_empty(mr_ctx* c, uint32_t n_wg) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (n_wg == 0) return set_err(c, MR_E_INVAL, "probe_empty: n_workgroups is 0");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  const hipError_t e = mr::launch_probe_empty(c->launch(), n_wg);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "probe_empty launch");
}

int mr_graph_begin(mr_ctx* c) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  if (c->capturing) return set_err(c, MR_E_INVAL, "capture already in progress");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamBeginCapture");
  c->capturing = true;
  c->captured_since_alloc = true;
  return MR_OK;
}

int mr_graph_end(mr_ctx* c, mr_graph** out) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!out) return set_err(c, MR_E_INVAL, "out pointer is NULL");
  *out = nullptr;
  if (!c->capturing) return set_err(c, MR_E_INVAL, "no capture in progress");
  c->capturing = false;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamEndCapture");
  mr_graph* G = new (std::nothrow) mr_graph;
  if (!G) {
    (void)hipGraphDestroy(g);
    return set_err(c, MR_E_NOMEM, "host allocation failed");
  }
  G->graph = g;
  e = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    mr_graph_destroy(G);
    return hip_fail(c, e, "hipGraphInstantiate");
  }
  *out = G;
  return MR_OK;
}

int mr_graph_launch(mr_ctx* c, const mr_graph* G) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!G || !G->exec) return set_err(c, MR_E_INVAL, "graph is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipGraphLaunch(G->exec, c->stream);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "hipGraphLaunch");
}

void mr_graph_destroy(mr_graph* G) {
  if (!G) return;
  if (G->exec) (void)hipGraphExecDestroy(G->exec);
  if (G->graph) (void)hipGraphDestroy(G->graph);
  delete G;
}

int mr_timer_start(mr_ctx* c) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipEventRecord(c->ev0, c->stream);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "hipEventRecord");
}

int mr_timer_stop(mr_ctx* c, float* ms) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!ms) return set_err(c, MR_E_INVAL, "out pointer is NULL");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipEventRecord(c->ev1, c->stream);
  if (e == hipSuccess) e = hipEventSynchronize(c->ev1);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, c->ev0, c->ev1);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "timer");
}

int mr_profile_read(mr_ctx* c, const char* kernel, uint64_t* count, double* total_ms) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!kernel || !count || !total_ms) return set_err(c, MR_E_INVAL, "NULL argument");
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
  uint64_t n = 0;
  double tot = 0.0;
  for (const auto& r : c->prof.recs) {
    if (c->prof.names[r.name] != kernel) continue;
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventElapsedTime");
    ++n, tot += ms;
  }
  *count = n, *total_ms = tot;
  return MR_OK;
}

int mr_profile_reset(mr_ctx* c) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (has_dev(c)) {
    int rc = bind(c);
    if (rc) return rc;
    (void)hipStreamSynchronize(c->stream);
  }
  c->prof.recs.clear();
  c->prof.used = 0;
  return MR_OK;
}

int mr_synth_blocks(mr_ctx* c, int type, void* dst, uint64_t n_blocks, uint64_t seed) {
  if (!c) return set_err(nullptr, MR_E_INVAL, "context is NULL");
  if (!valid_type(type)) return set_err(c, MR_E_UNSUPPORTED, "ggml type %d", type);
  if (!dst && n_blocks) return set_err(c, MR_E_INVAL, "NULL destination");
  if (n_blocks == 0) return MR_OK;
  if (!has_dev(c)) return set_err(c, MR_E_NODEV, "host-only context");
  int rc = bind(c);
  if (rc) return rc;
  hipError_t e = mr::launch_synth(c->launch(), type, dst, n_blocks, seed);
  return e == hipSuccess ? MR_OK : hip_fail(c, e, "synth launch");
}

}  // extern "C"

namespace mr {
int set_error(mr_ctx* ctx, int code, const char* msg) { return set_err(ctx, code, "%s", msg ? msg : ""); }
void layer_adopt(mr_layer* L, mr_pack* const* packs, size_t n_packs, void* const* dev, size_t n_dev) {
  L->own_packs.insert(L->own_packs.end(), packs, packs + n_packs);
  L->own_dev.insert(L->own_dev.end(), dev, dev + n_dev);
}
}  // namespace mr
