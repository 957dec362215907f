/*
 * moe_rocm.h -- C ABI of the MI355X (gfx950) MoE expert-FFN engine.
 *
 * Drop-in replacement for the expert-compute backend of moe-stream-core
 * (GOBA-AI-Labs/moe-stream), which today is the #[cfg(feature="metal")] module
 * crate::metal (moe-stream-core/src/lib.rs:7-8). Every entry point below names
 * the reference interface it replaces (path:line relative to
 * moe-stream-core/src/). Plain C: bindgen-clean, no C++ or HIP types.
 *
 * Conventions
 *  - Every function returns MR_OK (0) or a negative MR_E_* status. No
 *    exceptions or aborts cross the ABI. mr_last_error(ctx) describes the last
 *    failing call on that context (replaces candle_core::Error::Msg, e.g.
 *    metal/mod.rs:1308-1318).
 *  - Device pointers (`const float* x`, ...) are addresses in the context
 *    device's global memory, allocated with mr_dev_alloc or by any other HIP
 *    allocator on that device. Host pointers are marked `host_` and are only
 *    borrowed for the duration of the call.
 *  - All device work of a context is enqueued on that context's stream, in
 *    call order (the reference's single Metal command buffer,
 *    metal/mod.rs:6-14). Results are visible to the host after mr_sync or a
 *    download. Scratch buffers are owned by the context and reused by the
 *    next call (reference: BatchedMoeBuffers, metal/mod.rs:1222-1283), so
 *    calls on one context must not run concurrently from several host threads.
 *  - mr_moe_forward / mr_moe_forward_batched launch no allocation and no
 *    memset; with scratch reserved up front they may be captured into a HIP
 *    graph (mr_graph_* below).
 */
#ifndef MOE_ROCM_H
#define MOE_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define MR_OK 0
#define MR_E_INVAL (-1)       /* bad argument or shape */
#define MR_E_NOMEM (-2)       /* device allocation failed */
#define MR_E_NODEV (-3)       /* no HIP device, or a host-only context */
#define MR_E_LAUNCH (-4)      /* kernel launch or HIP runtime failure */
#define MR_E_UNSUPPORTED (-5) /* valid request outside what this build runs */

/* ---- GGML block types (reader.rs:34-128) --------------------------------- */
#define MR_GGML_Q4_K 12  /* 144-byte super-block of 256 elements */
#define MR_GGML_MXFP4 39 /* 17-byte block: e8m0 scale + 32 e2m1 codes */

/* ---- routing flags (top_k_routing, layer.rs:2346-2403) ------------------- */
/* GPT-OSS: top-k on raw logits, softmax over the k (softmax_weight=true). */
#define MR_ROUTE_SOFTMAX_AFTER_TOPK 1u
/* standard mode: renormalise the k probabilities (norm_topk_prob, config.rs:364). */
#define MR_ROUTE_NORM_TOPK 2u

/* ---- activations (ops/activation.rs:13-38) ----------------------------------- */
#define MR_ACT_SILU 0        /* silu(g) * u                                   */
#define MR_ACT_SWIGLU_OAI 1  /* min(g,L)*sigmoid(alpha*min(g,L))*(clamp(u,-L,L)+1) */

/* Device id for a host-only context: argument validation runs, device work
 * returns MR_E_NODEV. Lets every ABI/error test run without a GPU. */
#define MR_DEVICE_NONE (-1)

/* Kernel family used by the decode path (mr_ctx_set_option MR_OPT_DECODE_KERNEL). */
#define MR_OPT_DECODE_KERNEL 1
#define MR_DECODE_AUTO 0   /* fastest available */
#define MR_DECODE_VALU 1   /* vector-ALU dequant-matvec kernels, one launch per step */
#define MR_DECODE_FUSED 2  /* single fused launch per layer: router, top-k, experts, combine
                              (MXFP4 on the scaled MX-fp4 MFMA; Q4_K on the int8 MFMA) */
/* 1: record a HIP event pair around every kernel launch (read with mr_profile_read). */
#define MR_OPT_PROFILE 2
/* Time limit in microseconds of each cross-workgroup wait inside the fused decode
 * kernels (default 50000, i.e. 50 ms), measured on the device's constant-rate clock.
 * A wait that runs out ends the launch early and makes the next mr_sync return
 * MR_E_LAUNCH. A wait consults the clock from its 64th poll on (limits below 100 us:
 * from its first), so it gives up at most about 1 ms after the limit; a value of 0
 * restores the default. */
#define MR_OPT_WAIT_LIMIT_US 3

typedef struct mr_ctx mr_ctx;
typedef struct mr_pack mr_pack;
typedef struct mr_layer mr_layer;
typedef struct mr_graph mr_graph;
typedef struct mr_gguf mr_gguf;

/* ---- context, errors, streams -------------------------------------------- */
/* Replaces candle's Device::new_metal(0) handle (engine.rs:278-298). */
int mr_ctx_create(int device, mr_ctx** out);
void mr_ctx_destroy(mr_ctx* ctx);
const char* mr_last_error(const mr_ctx* ctx);
const char* mr_status_string(int status);
int mr_ctx_device(const mr_ctx* ctx);
/* Use a caller-owned hipStream_t (cast to void*) instead of the context's own. */
int mr_ctx_set_stream(mr_ctx* ctx, void* hip_stream);
void* mr_ctx_stream(const mr_ctx* ctx);
int mr_ctx_set_option(mr_ctx* ctx, int option, int value);
/* Wait for all work enqueued on the context stream (the reference syncs at
 * to_vec1 readbacks, layer.rs:938, engine.rs:2069). Also reports a fused decode
 * launch that ended early (MR_E_LAUNCH) since the previous mr_sync. */
int mr_sync(mr_ctx* ctx);

/* ---- device memory ------------------------------------------------------- */
int mr_dev_alloc(mr_ctx* ctx, uint64_t nbytes, void** out_dptr);
int mr_dev_free(mr_ctx* ctx, void* dptr);
/* Stream-ordered copies; both return after the copy has completed. */
int mr_upload(mr_ctx* ctx, void* dst, const void* host_src, uint64_t nbytes);
int mr_download(mr_ctx* ctx, void* host_dst, const void* src, uint64_t nbytes);
/* Enqueue a zero fill with a kernel (graph-capture safe, no memset node). */
int mr_dev_zero(mr_ctx* ctx, void* dst, uint64_t nbytes);

/* ---- expert weights in native GGUF layout --------------------------------- */
/* One projection (gate, up or down) of all experts of one layer: E matrices of
 * [out_features, in_features], expert e starting at host_offsets[e] bytes from
 * the buffer start (NULL = contiguous, e * bytes_per_expert, the layout of a
 * stacked ffn_*_exps tensor, reader.rs:394-444). The bytes stay in their
 * native block layout; nothing is repacked.
 * mr_pack_upload copies host bytes into a new device buffer the pack owns
 * (replaces upload_mxfp4_weights, metal/mod.rs:1823, and the packing loop of
 * preload_experts_gpu, engine.rs:1114-1148). */
int mr_pack_upload(mr_ctx* ctx, int ggml_type, const void* host_bytes, uint64_t nbytes,
                   uint32_t n_experts, uint32_t out_features, uint32_t in_features,
                   const uint64_t* host_offsets, mr_pack** out);
/* Same over device bytes the caller owns and keeps alive (zero copy; the
 * reference's Mxfp4Packed views, cache.rs:289-308). The kernels read whole
 * aligned 16-byte pieces, so the allocation must stay readable for 64 bytes past
 * the last expert's last block (mr_pack_upload allocates that slack itself). */
int mr_pack_wrap(mr_ctx* ctx, int ggml_type, const void* dev_bytes, uint64_t nbytes,
                 uint32_t n_experts, uint32_t out_features, uint32_t in_features,
                 const uint64_t* host_offsets, mr_pack** out);
void mr_pack_destroy(mr_pack* pack);
/* Bytes of one [rows, cols] matrix of a GGML block type (reader.rs:99-127). */
uint64_t mr_matrix_bytes(int ggml_type, uint64_t rows, uint64_t cols);
/* Dequantize expert `expert` of a pack to f32 [out_features, in_features]
 * (dequantize_mxfp4 dequant.rs:605, dequantize_q4k dequant.rs:218; the
 * arithmetic is bit-identical: no contraction). */
int mr_dequant(mr_ctx* ctx, const mr_pack* pack, uint32_t expert, float* out);

/* ---- one MoE layer ------------------------------------------------------- */
/* Bundles what run_moe reads for one layer (ResidentWeights fields,
 * cache.rs:319-398; GpuRoutingOffsets, metal/mod.rs:1440-1485;
 * ExpertBiasBuffers, metal/mod.rs:1202-1216). Device arrays are borrowed. */
typedef struct mr_layer_desc {
  const mr_pack* gate;        /* routed experts: [E, I, H] */
  const mr_pack* up;          /* [E, I, H] */
  const mr_pack* down;        /* [E, H, I] */
  const float* gate_bias;     /* [E, I] f32 or NULL (ffn_gate_exps.bias) */
  const float* up_bias;       /* [E, I] f32 or NULL */
  const float* down_bias;     /* [E, H] f32 or NULL */
  const float* router_w;      /* [E, H] f32 (ffn_gate_inp.weight) */
  const float* router_b;      /* [E] f32 or NULL (ffn_gate_inp.bias) */
  const float* dummy_mask;    /* [E] f32, 0 or -inf, or NULL (engine.rs:628-652) */
  /* optional always-on shared expert (layer.rs:1898-1953): NULL sh_gate disables */
  const mr_pack* sh_gate;     /* [1, Ish, H] */
  const mr_pack* sh_up;       /* [1, Ish, H] */
  const mr_pack* sh_down;     /* [1, H, Ish] */
  const float* sh_gate_inp;   /* [H] f32 or NULL (ffn_gate_inp_shexp.weight) */
  uint32_t top_k;             /* 1..16 */
  uint32_t route_flags;       /* MR_ROUTE_* */
  uint32_t act;               /* MR_ACT_* for the routed experts (shared expert: SiLU) */
  float alpha;                /* OAI SwiGLU alpha (1.702, layer.rs:873) */
  float limit;                /* OAI SwiGLU limit (7.0, layer.rs:874) */
} mr_layer_desc;

int mr_layer_create(mr_ctx* ctx, const mr_layer_desc* desc, mr_layer** out);
void mr_layer_destroy(mr_layer* layer);
/* Prefetch hint (no reference counterpart; the reference's decode loop runs the
 * layers in order, layer.rs:756-1980 per layer): `next` is the layer whose
 * mr_moe_forward follows this layer's. While this layer's fused decode kernel
 * streams expert weights, its router workgroups read the next layer's router
 * rows, so the next layer's router step finds them in the caches instead of
 * HBM. Results do not change. NULL clears the hint; `next` must belong to the
 * same context and stay alive (or be cleared here) while this layer is used. */
int mr_layer_set_next(mr_layer* layer, const mr_layer* next);
/* Prefetch hint for the fused residual decode (no reference counterpart): the
 * norm weights the caller passes to this layer's mr_moe_forward_residual
 * (the post-attention norm, layer.rs:462-463). The layer whose next layer
 * (mr_layer_set_next) this is reads them into the caches while it runs, as it
 * does the router rows. Results do not change. NULL clears it; norm_w must stay
 * valid while set (device f32 [H], 16-byte aligned). mr_gguf_layer_create sets
 * it to the norm weights the layer owns. */
int mr_layer_set_norm(mr_layer* layer, const float* norm_w);
/* Router logits out of the forward calls themselves: with an array set, every
 * mr_moe_forward(_residual) and mr_moe_forward_batched(_residual, _noalloc) of
 * this layer also writes its router logits (x . router row + bias + dummy mask,
 * the values top-k ranks) as f32 [n_tokens, E] to `logits` (device memory,
 * 4-byte aligned), in the same launches: the fused decode kernel's router
 * workgroups store them as they publish them, so no second router GEMV runs.
 * This is the readback the reference makes after the GPU MoE for router entropy
 * and routing statistics (layer.rs:879-905). Calls of more than max_tokens tokens
 * return MR_E_INVAL. NULL clears it. Graphs captured while it is set write to the
 * array they captured. Results of the calls do not change. */
int mr_layer_set_logits_out(mr_layer* layer, float* logits, uint32_t max_tokens);
/* Allocate context scratch for up to max_tokens tokens of this layer's shape
 * (BatchedMoeBuffers::new, metal/mod.rs:1240). Call before graph capture. A hot-path
 * call that needs more grows the scratch itself, to at least twice its token capacity;
 * the old allocation is freed, or, when a graph was captured since it was allocated,
 * kept until mr_ctx_destroy (the graph still addresses it). */
int mr_reserve(mr_ctx* ctx, const mr_layer* layer, uint32_t max_tokens);

/* ---- hot path -------------------------------------------------------------- */
/* Kernel (1): router GEMV + bias + dummy mask + softmax/top-k for n_tokens
 * tokens (layer.rs:806-837 + 1012-1027; softmax_topk_kernel,
 * fused_ops.metal:131-316). idx [T,k] i32, w [T,k] f32, logits [T,E] or NULL. */
int mr_router_topk(mr_ctx* ctx, const mr_layer* layer, const float* x, uint32_t n_tokens,
                   int32_t* idx, float* w, float* logits);
/* Top-k only, over given logits [T,E] (top_k_routing, layer.rs:2346-2403). */
int mr_topk(mr_ctx* ctx, const float* logits, uint32_t n_tokens, uint32_t n_experts,
            uint32_t top_k, uint32_t route_flags, int32_t* idx, float* w);
/* Kernels (2)+(3) with routing given: per token, gate+up dequant-matvec with
 * bias and SwiGLU, then down dequant-matvec with bias and the weighted combine
 * in ascending expert order, then the shared expert. y [T,H] is overwritten.
 * Replaces batched_moe_forward_metal (metal/mod.rs:1297-1435). */
int mr_moe_experts(mr_ctx* ctx, const mr_layer* layer, const float* x, uint32_t n_tokens,
                   const int32_t* idx, const float* w, float* y);
/* Whole layer for one decode token: router, top-k, experts, combine, shared
 * expert; no host synchronisation. Replaces gpu_routed_moe_forward_metal
 * (metal/mod.rs:1512-1677) and the CPU run_moe path (layer.rs:756-1980). */
int mr_moe_forward(mr_ctx* ctx, const mr_layer* layer, const float* x, float* y);
/* mr_moe_forward with the steps on either side of it fused in (layer.rs:462-473):
 * the input is rms_norm(h) = (h * inv) * norm_w, inv = 1 / sqrt(mean(h^2) + eps)
 * (ops/norm.rs:16-37, the post-attention norm), and h_out = h + moe(rms_norm(h))
 * (the residual add). h_out may equal h (in place). h, norm_w, h_out: [H] f32,
 * 16-byte aligned; 0 <= eps <= 1. */
int mr_moe_forward_residual(mr_ctx* ctx, const mr_layer* layer, const float* h, const float* norm_w,
                            float eps, float* h_out);
/* Whole layer for n_tokens tokens (prefill / batched): tokens are grouped by
 * expert and each expert's weights are read once for all its tokens.
 * Replaces the multi-token paths layer.rs:1449-1514 and 2148-2183. */
int mr_moe_forward_batched(mr_ctx* ctx, const mr_layer* layer, const float* x,
                           uint32_t n_tokens, float* y);
/* mr_moe_forward_batched with the post-attention RMSNorm and the residual add of every token
 * (layer.rs:462-473 over a [T, H] hidden state, the prefill form of mr_moe_forward_residual):
 * h_out[t] = h[t] + moe(rms_norm(h[t], norm_w, eps)). h_out may equal h. h, norm_w, h_out
 * 16-byte aligned; 0 <= eps <= 1. */
int mr_moe_forward_batched_residual(mr_ctx* ctx, const mr_layer* layer, const float* h, uint32_t n_tokens,
                                    const float* norm_w, float eps, float* h_out);
/* mr_moe_forward_batched without any allocation. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, serving
 * loops or harnesses that forbid hipMalloc). The same kernels and results, with their
 * scratch in a static device array of MR_STATIC_SCRATCH_BYTES that every GPU holds for
 * the life of the process (its address is looked up once per device by mr_ctx_create).
 * Calls whose scratch would not fit return MR_E_INVAL with the size in mr_last_error
 * (at the GPT-OSS shape, 64 MiB holds 631 tokens per call). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (several contexts or streams,
 * or several host threads) race and must be serialised by the caller. */
#define MR_STATIC_SCRATCH_BYTES (64ull << 20)
int mr_moe_forward_batched_noalloc(mr_ctx* ctx, const mr_layer* layer, const float* x,
                                   uint32_t n_tokens, float* y);

/* ---- GGUF files (gguf/reader.rs; preload of engine.rs:1079-1255) ----------------- */
/* Opens and memory-maps a GGUF v2/v3 file and parses its header, metadata and
 * tensor index (GgufReader::open, reader.rs:259-358: the same magic/version
 * checks, count limits, general.alignment (default 32) for the data start).
 * Errors: MR_E_INVAL for a malformed or truncated file (message in
 * mr_last_error(NULL)), MR_E_UNSUPPORTED for a tensor type outside
 * GgmlQuantType (reader.rs:39-86). Host only: no context needed. */
int mr_gguf_open(const char* path, mr_gguf** out);
void mr_gguf_close(mr_gguf* g);
uint64_t mr_gguf_n_tensors(const mr_gguf* g);
/* Name of tensor i (index order of the file), NULL past the end. */
const char* mr_gguf_tensor_name(const mr_gguf* g, uint64_t i);
/* One tensor's TensorInfo (reader.rs:131-154): ggml type, dims in GGUF order
 * (innermost first; pt_shape is the reverse), absolute data offset and raw byte
 * size (raw_size, reader.rs:114-127). dims has room for 4 entries. */
typedef struct mr_gguf_tensor {
  uint32_t ggml_type;
  uint32_t n_dims;
  uint64_t dims[4];
  uint64_t data_offset;
  uint64_t nbytes;
} mr_gguf_tensor;
int mr_gguf_tensor_info(const mr_gguf* g, const char* name, mr_gguf_tensor* out);
/* Read-only view of a tensor's bytes in the mapping (tensor_data, reader.rs:361-378;
 * bounds-checked against the file size). Valid until mr_gguf_close. */
int mr_gguf_tensor_data(const mr_gguf* g, const char* name, const void** data, uint64_t* nbytes);
/* Metadata lookups (get_metadata + MetadataValue::as_u32 / as_f32 / as_str,
 * reader.rs:170-218): MR_E_INVAL when the key is absent or of another type. */
int mr_gguf_meta_u32(const mr_gguf* g, const char* key, uint32_t* out);
int mr_gguf_meta_f32(const mr_gguf* g, const char* key, float* out);
/* The string's bytes (not NUL-terminated) and length; valid until mr_gguf_close. */
int mr_gguf_meta_str(const mr_gguf* g, const char* key, const char** str, uint64_t* len);
/* Element count and, if out != NULL, up to cap elements of an integer array
 * (as_u32_array, e.g. {arch}.experts_per_layer). */
int mr_gguf_meta_u32_array(const mr_gguf* g, const char* key, uint32_t* out, uint64_t cap, uint64_t* n);
/* Uploads a stacked expert tensor [E, out, in] (GGUF dims [in, out, E]) of
 * MXFP4 or Q4_K in its native bytes: expert e at e * bytes_per_expert
 * (expert_slice_data, reader.rs:394-444). */
int mr_gguf_upload_experts(mr_ctx* ctx, const mr_gguf* g, const char* name, mr_pack** out);
/* Options of mr_gguf_layer_create. */
typedef struct mr_gguf_layer_opts {
  uint32_t top_k;        /* 0: {arch}.expert_used_count */
  int32_t route_flags;   /* -1: from the architecture (gpt-oss: softmax after top-k; else renormalised
                            top-k, plain for general.name with Qwen1.5/Qwen2, config.rs:364) */
  int32_t act;           /* -1: MR_ACT_SWIGLU_OAI for gpt-oss, else MR_ACT_SILU */
  float alpha, limit;    /* OAI SwiGLU constants (layer.rs:873-874; 0: 1.702 and 7.0) */
} mr_gguf_layer_opts;
/* Builds MoE layer `layer` (tensors blk.<layer>.ffn_{gate,up,down}_exps.weight and
 * their .bias, ffn_gate_inp.weight/.bias, the shared expert ffn_{gate,up,down}_shexp
 * and ffn_gate_inp_shexp when present) on the device: experts uploaded natively,
 * f32/f16/bf16 vectors converted to f32 (load_weight). The layer owns what it
 * uploaded (freed by mr_layer_destroy). opts NULL: all defaults. The file can be
 * closed afterwards. Also returns the layer's post_attention_norm weight as
 * device f32 [H] in *norm_w (owned by the layer; NULL if the file has none) and
 * {arch}.attention.layer_norm_rms_epsilon in *eps (default 1e-6, config.rs:293),
 * for mr_moe_forward_residual; both outputs may be NULL. */
int mr_gguf_layer_create(mr_ctx* ctx, const mr_gguf* g, uint32_t layer, const mr_gguf_layer_opts* opts,
                         mr_layer** out, const float** norm_w, float* eps);

/* ---- graph capture of a sequence of calls (no reference counterpart: the
 * reference's Metal command buffer batching, metal/mod.rs:6-14) ----------- */
int mr_graph_begin(mr_ctx* ctx);
int mr_graph_end(mr_ctx* ctx, mr_graph** out);
int mr_graph_launch(mr_ctx* ctx, const mr_graph* graph);
void mr_graph_destroy(mr_graph* graph);

/* ---- timing on the context stream (bench support) ------------------------- */
/* Records an event pair around the work enqueued between the two calls and
 * returns the elapsed milliseconds after synchronising. */
int mr_timer_start(mr_ctx* ctx);
int mr_timer_stop(mr_ctx* ctx, float* out_ms);
/* With MR_OPT_PROFILE on: synchronise, then report how many launches of the
 * named kernel were recorded and their summed duration (ms). Kernel names:
 * "router_logits", "topk", "gateup", "down", "shared_gateup", "dequant",
 * "fused_layer", "grouped_gateup", "grouped_down", "group_tokens". */
int mr_profile_read(mr_ctx* ctx, const char* kernel, uint64_t* out_count, double* out_total_ms);
int mr_profile_reset(mr_ctx* ctx);

/* Bench and test support (synthetic weights, measurement probes) is declared in
 * moe_rocm_bench.h; it is not part of this interface. */

#ifdef __cplusplus
}
#endif
#endif /* MOE_ROCM_H */
