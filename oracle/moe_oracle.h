/*
 * moe_oracle.h -- CPU restatement of moe-stream's MoE expert-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product path (moe-stream_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * moe-stream-core/src/ of GOBA-AI-Labs/moe-stream). Built with
 * -O2 -ffp-contract=off and no fast-math, so each C float operation is one IEEE
 * rounding, matching Rust's no-contraction semantics.
 *
 * Parity pinning (what checks each function; see tests/test_oracle_*.py):
 *   or_fp16_to_f32        exhaustive over 65,536 patterns vs numpy.float16, KATs dequant.rs:808-816
 *   or_e8m0_to_f32_half   closed form 2^(e-128) for all 256 bytes (denormal branch included)
 *   or_dequant_mxfp4      closed form over 16 codes x 256 exponents; -0.0 for code 8
 *   or_mxfp4_matvec       one-hot inputs (exact column), f64 brute force on dequantized W
 *   or_get_scale_min_k4 / or_dequant_q4k
 *                         hand-built bit patterns per branch, KAT dequant.rs:818-837,
 *                         independent numpy restatement of ggml's Q4_K layout
 *   or_topk_routing       brute force vs numpy stable argsort; invariants (sum to 1,
 *                         ties -> lower index, -inf never chosen)
 *   or_swiglu_oai1 / or_silu_mul1 / or_sigmoid1
 *                         f64 closed forms incl. clamp branches; KATs activation.rs:67-81,
 *                         train.rs:1151-1184
 *   or_moe_forward        linearity in routing weights, single-expert identity,
 *                         zero-code -> bias-only, f64 numpy recomputation at tiny shapes
 *   or_rms_norm           KAT of norm.rs:44-56 (x = 1..4, w = 1); f64 recomputation; mean of squares
 *                         summed sequentially (candle's sum order is not reproducible here:
 *                         order parity unpinned, value pinned to f64 within tolerance)
 *   or_f32_matvec         restates candle's F32 gemm as a sequential fp32 sum; candle's
 *                         reduction order (gemm 0.17/0.18) is not reproducible here, so the
 *                         ORDER is parity unpinned (value pinned only to f64 within tolerance)
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_GGML_Q4_K 12
#define OR_GGML_MXFP4 39

float or_fp16_to_f32(uint16_t h);
float or_e8m0_to_f32_half(uint8_t e);
void or_dequant_mxfp4(const uint8_t* blocks, size_t n_elements, float* out);
void or_mxfp4_matvec(const uint8_t* w, const float* x, size_t out_features,
                     size_t in_features, float* y, int n_threads);
void or_mxfp4_matmul(const uint8_t* w, const float* x, size_t n_tokens,
                     size_t out_features, size_t in_features, float* y, int n_threads);
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);
void or_dequant_q4k(const uint8_t* blocks, size_t n_elements, float* out);
void or_f32_matvec(const float* w, const float* x, size_t out_features, size_t in_features,
                   float* y);
void or_topk_routing(const float* logits, size_t n_tokens, size_t n_experts, size_t k,
                     int normalize, int softmax_weight, uint32_t* idx, float* w);
float or_swiglu_oai1(float g, float u, float alpha, float limit);
float or_silu_mul1(float g, float u);
float or_sigmoid1(float x);
/* RMSNorm of n_rows rows of width: x / sqrt(mean(x^2) + eps) * weight (ops/norm.rs:32-36). */
void or_rms_norm(const float* x, const float* weight, size_t n_rows, size_t width, float eps, float* out);

/* Bytes of one [rows, cols] matrix in a GGML block type (reader.rs:99-127). */
uint64_t or_matrix_bytes(int ggml_type, uint64_t rows, uint64_t cols);

/* One MoE layer as the CPU path sees it. Stacked expert tensors are
 * [E][out][in] in native GGUF block layout, expert e at e*matrix_bytes
 * (reader.rs:394-444). Biases are [E][dim] f32 or NULL. */
typedef struct or_layer {
  int type;                 /* OR_GGML_MXFP4 or OR_GGML_Q4_K (routed experts) */
  uint32_t hidden, inter, n_experts, top_k;
  const uint8_t *gate, *up, *down;
  const float *gate_b, *up_b, *down_b;
  const float *router_w;    /* [E][H] */
  const float *router_b;    /* [E] or NULL */
  const float *dummy_mask;  /* [E] (0 or -inf) or NULL */
  int softmax_weight;       /* 1: GPT-OSS top-k on logits then softmax over the k */
  int norm_topk;            /* standard mode: renormalise the k probabilities */
  int act_oai;              /* 1: OAI SwiGLU (alpha, limit); 0: silu(g)*u */
  float alpha, limit;
  /* optional shared expert (Qwen3-Coder-Next): NULL sh_gate disables it */
  int sh_type;
  uint32_t sh_inter;
  const uint8_t *sh_gate, *sh_up, *sh_down;
  const float *sh_gate_inp; /* [H] or NULL */
} or_layer;

/* Full MoE layer for n_tokens tokens: router -> top-k -> experts in ascending
 * index order -> weighted combine -> shared expert. x [T][H] -> y [T][H].
 * idx/w/logits outputs are optional ([T][k], [T][k], [T][E]). */
int or_moe_forward(const or_layer* L, const float* x, size_t n_tokens, float* y,
                   uint32_t* idx_out, float* w_out, float* logits_out, int n_threads);

/* Expert part only, with routing given (idx/w [T][k]); accumulates into y
 * (caller zeroes it) and adds the shared expert when present. */
int or_moe_experts(const or_layer* L, const float* x, size_t n_tokens, const uint32_t* idx,
                   const float* w, float* y, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
