/*
 * moe_oracle.c -- CPU restatement of moe-stream's MoE expert-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product). Citations are
 * moe-stream-core/src/<file>:<line> of GOBA-AI-Labs/moe-stream. Build with
 * -O2 -ffp-contract=off (no fast-math): every expression below is a sequence
 * of single IEEE fp32 roundings in the order the Rust code performs them.
 */
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* IEEE binary16 -> binary32, exact. Restates half 2.7.1 f16::to_f32 used by
 * dequant.rs:37-41 (fp16_to_f32). NaNs come back quiet with their payload. */
float or_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (ex == 0) {
    /* zero or subnormal: man * 2^-24, exact in binary32 */
    float v = (float)man * 5.9604644775390625e-08f;
    uint32_t b;
    memcpy(&b, &v, 4);
    return bits_to_f32(b | sign);
  }
  if (ex == 31) {
    uint32_t b = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    return bits_to_f32(b);
  }
  return bits_to_f32(sign | ((ex + 112u) << 23) | (man << 13));
}

/* dequant.rs:589-597: 2^(e-128); bytes 0 and 1 take the denormal branch. */
float or_e8m0_to_f32_half(uint8_t e) {
  if (e < 2) return bits_to_f32(0x00200000u << e);
  return bits_to_f32(((uint32_t)e - 1u) << 23);
}

/* dequant.rs:580-583 (MXFP4_VALUES: doubled e2m1, code 8 is -0.0). */
static const float kMxfp4Values[16] = {0.0f,  1.0f,  2.0f,  3.0f,  4.0f,  6.0f,  8.0f,  12.0f,
                                       -0.0f, -1.0f, -2.0f, -3.0f, -4.0f, -6.0f, -8.0f, -12.0f};

/* dequant.rs:605-628: block b byte j: low nibble -> element 32b+j,
 * high nibble -> element 32b+j+16; y = lut * d. */
void or_dequant_mxfp4(const uint8_t* blocks, size_t n_elements, float* out) {
  size_t nb = n_elements / 32;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* x = blocks + b * 17;
    float d = or_e8m0_to_f32_half(x[0]);
    const uint8_t* qs = x + 1;
    float* y = out + b * 32;
    for (int j = 0; j < 16; ++j) {
      y[j] = kMxfp4Values[qs[j] & 0x0F] * d;
      y[j + 16] = kMxfp4Values[qs[j] >> 4] * d;
    }
  }
}

/* ---- dequant.rs:640-695 mxfp4_matvec_mul ------------------------------- */

typedef struct {
  const uint8_t* w;
  const float* x;
  float* y;
  size_t row0, row1, in_features;
} mxfp4_job;

static void mxfp4_rows(const mxfp4_job* jb) {
  size_t bpr = jb->in_features / 32;
  size_t row_bytes = bpr * 17;
  for (size_t i = jb->row0; i < jb->row1; ++i) {
    const uint8_t* row = jb->w + i * row_bytes;
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t* blk = row + b * 17;
      float d = or_e8m0_to_f32_half(blk[0]);
      const uint8_t* qs = blk + 1;
      const float* xin = jb->x + b * 32;
      for (int j = 0; j < 16; ++j) {
        float lo = kMxfp4Values[qs[j] & 0x0F];
        float hi = kMxfp4Values[qs[j] >> 4];
        /* acc += lo * d * input[j]; acc += hi * d * input[j+16]
         * Rust evaluates (lo*d)*x then acc + that, no contraction. */
        acc = acc + (lo * d) * xin[j];
        acc = acc + (hi * d) * xin[j + 16];
      }
    }
    jb->y[i] = acc;
  }
}

static void* mxfp4_rows_thread(void* p) {
  mxfp4_rows((const mxfp4_job*)p);
  return NULL;
}

/* Rows are split into ceil(out/threads) chunks, one scoped thread each,
 * threads spawned per call (dequant.rs:650-692). n_threads <= 1 runs inline;
 * the result is identical either way (each row is sequential). */
void or_mxfp4_matvec(const uint8_t* w, const float* x, size_t out_features,
                     size_t in_features, float* y, int n_threads) {
  size_t nt = n_threads < 1 ? 1 : (size_t)n_threads;
  if (nt > out_features) nt = out_features;
  if (nt <= 1) {
    mxfp4_job jb = {w, x, y, 0, out_features, in_features};
    mxfp4_rows(&jb);
    return;
  }
  size_t chunk = (out_features + nt - 1) / nt;
  pthread_t tid[256];
  mxfp4_job jobs[256];
  if (nt > 256) nt = 256, chunk = (out_features + 255) / 256;
  size_t launched = 0;
  for (size_t c = 0; c < nt; ++c) {
    size_t r0 = c * chunk, r1 = r0 + chunk;
    if (r0 >= out_features) break;
    if (r1 > out_features) r1 = out_features;
    jobs[c] = (mxfp4_job){w, x, y, r0, r1, in_features};
    if (pthread_create(&tid[c], NULL, mxfp4_rows_thread, &jobs[c]) != 0) {
      mxfp4_rows(&jobs[c]);
      tid[c] = 0;
    }
    launched = c + 1;
  }
  for (size_t c = 0; c < launched; ++c)
    if (tid[c]) pthread_join(tid[c], NULL);
}

/* dequant.rs:705-721: one matvec per token; weights re-read per token. */
void or_mxfp4_matmul(const uint8_t* w, const float* x, size_t n_tokens, size_t out_features,
                     size_t in_features, float* y, int n_threads) {
  for (size_t t = 0; t < n_tokens; ++t)
    or_mxfp4_matvec(w, x + t * in_features, out_features, in_features, y + t * out_features,
                    n_threads);
}

/* ---- Q4_K: dequant.rs:195-262 ------------------------------------------ */

/* dequant.rs:199-209 (ggml get_scale_min_k4). */
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* dequant.rs:218-262: per 144-byte block: d, dmin fp16 (LE), 12 scale bytes,
 * 128 qs bytes. Sub-blocks 2j/2j+1 take the low/high nibbles of qs[32j..].
 * y = (d*sc)*q - (dmin*m), each product rounded separately (no FMA). */
void or_dequant_q4k(const uint8_t* blocks, size_t n_elements, float* out) {
  size_t nb = n_elements / 256;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* x = blocks + b * 144;
    float* y = out + b * 256;
    float d = or_fp16_to_f32((uint16_t)(x[0] | (x[1] << 8)));
    float dmin = or_fp16_to_f32((uint16_t)(x[2] | (x[3] << 8)));
    const uint8_t* scales = x + 4;
    const uint8_t* qs = x + 16;
    int is = 0;
    size_t o = 0;
    for (int j = 0; j < 4; ++j) {
      uint8_t sc0, m0, sc1, m1;
      or_get_scale_min_k4(is, scales, &sc0, &m0);
      float d1 = d * (float)sc0;
      float m1f = dmin * (float)m0;
      or_get_scale_min_k4(is + 1, scales, &sc1, &m1);
      float d2 = d * (float)sc1;
      float m2f = dmin * (float)m1;
      for (int l = 0; l < 32; ++l) {
        float p = d1 * (float)(qs[j * 32 + l] & 0x0F);
        y[o++] = p - m1f;
      }
      for (int l = 0; l < 32; ++l) {
        float p = d2 * (float)(qs[j * 32 + l] >> 4);
        y[o++] = p - m2f;
      }
      is += 2;
    }
  }
}

/* candle F32 matmul (x [1,in] . W^T) as used at layer.rs:811/820/1825-1838/1921-1924.
 * Restated as a sequential fp32 sum in ascending column order; candle's gemm
 * reduction order is not reproducible here (parity of the ORDER unpinned). */
void or_f32_matvec(const float* w, const float* x, size_t out_features, size_t in_features,
                   float* y) {
  for (size_t r = 0; r < out_features; ++r) {
    const float* row = w + r * in_features;
    float acc = 0.0f;
    for (size_t c = 0; c < in_features; ++c) acc = acc + row[c] * x[c];
    y[r] = acc;
  }
}

/* or_f32_matvec with its rows split over threads (candle's F32 matmul runs on a thread
 * pool); each row is the same sequential sum, so the bits do not depend on the split. */
typedef struct {
  const float *w, *x;
  float* y;
  size_t r0, r1, in_features;
} f32_job;

static void* f32_rows_thread(void* p) {
  const f32_job* jb = (const f32_job*)p;
  or_f32_matvec(jb->w + jb->r0 * jb->in_features, jb->x, jb->r1 - jb->r0, jb->in_features, jb->y + jb->r0);
  return NULL;
}

static void f32_matvec_mt(const float* w, const float* x, size_t out_features, size_t in_features, float* y,
                          int n_threads) {
  size_t nt = n_threads < 1 ? 1 : (size_t)n_threads;
  if (nt > 256) nt = 256;
  if (nt > out_features) nt = out_features;
  if (nt <= 1) {
    or_f32_matvec(w, x, out_features, in_features, y);
    return;
  }
  size_t chunk = (out_features + nt - 1) / nt;
  pthread_t tid[256];
  f32_job jobs[256];
  size_t launched = 0;
  for (size_t c = 0; c < nt; ++c) {
    size_t r0 = c * chunk, r1 = r0 + chunk;
    if (r0 >= out_features) break;
    if (r1 > out_features) r1 = out_features;
    jobs[c] = (f32_job){w, x, y, r0, r1, in_features};
    if (pthread_create(&tid[c], NULL, f32_rows_thread, &jobs[c]) != 0) {
      f32_rows_thread(&jobs[c]);
      tid[c] = 0;
    }
    launched = c + 1;
  }
  for (size_t c = 0; c < launched; ++c)
    if (tid[c]) pthread_join(tid[c], NULL);
}

/* ---- routing: layer.rs:2346-2403 top_k_routing ---------------------------- */

/* a ranks above b in the descending order: the larger number; a NaN ranks below every
 * number. The reference's comparator (partial_cmp -> Equal) calls a NaN equal to everything:
 * where every value is NaN (standard mode: one NaN logit, a +inf maximum or a row of -inf makes
 * every probability NaN) its stable sort keeps index order, which this rule reproduces (no
 * value ranks above another, so the lowest remaining index is taken). A NaN among numbers
 * (softmax-after-top-k mode) makes that comparator inconsistent and the reference's order
 * depends on its sort algorithm; this build fixes NaN last for all paths. */
static int ranks_above(float a, float b) {
  if (isnan(a)) return 0;
  if (isnan(b)) return 1;
  return a > b;
}

/* First k entries of a stable descending sort (Rust sort_by with
 * b.partial_cmp(a), layer.rs:2358/2380): repeatedly take the largest
 * remaining value, ties resolved to the lower index. */
static void stable_desc_topk(const float* v, size_t n, size_t k, uint32_t* out_idx) {
  unsigned char taken[4096];
  unsigned char* tk = n <= sizeof(taken) ? taken : (unsigned char*)calloc(n, 1);
  memset(tk, 0, n);
  for (size_t r = 0; r < k && r < n; ++r) {
    size_t best = (size_t)-1;
    for (size_t i = 0; i < n; ++i) {
      if (tk[i]) continue;
      if (best == (size_t)-1 || ranks_above(v[i], v[best])) best = i;
    }
    tk[best] = 1;
    out_idx[r] = (uint32_t)best;
  }
  if (tk != taken) free(tk);
}

void or_topk_routing(const float* logits, size_t n_tokens, size_t n_experts, size_t k,
                     int normalize, int softmax_weight, uint32_t* idx, float* w) {
  float* tmp = (float*)malloc(sizeof(float) * (n_experts > k ? n_experts : k));
  for (size_t t = 0; t < n_tokens; ++t) {
    const float* row = logits + t * n_experts;
    uint32_t* ti = idx + t * k;
    float* tw = w + t * k;
    if (softmax_weight) {
      /* layer.rs:2355-2369: top-k by raw logit, softmax over the k. */
      stable_desc_topk(row, n_experts, k, ti);
      float mx = -INFINITY;
      for (size_t i = 0; i < k; ++i) mx = fmaxf(mx, row[ti[i]]);
      float sum = 0.0f;
      for (size_t i = 0; i < k; ++i) {
        tmp[i] = expf(row[ti[i]] - mx);
        sum = sum + tmp[i];
      }
      for (size_t i = 0; i < k; ++i) tw[i] = tmp[i] / sum;
    } else {
      /* layer.rs:2371-2394: softmax over all experts, top-k by probability,
       * optional renormalisation. */
      float mx = -INFINITY;
      for (size_t i = 0; i < n_experts; ++i) mx = fmaxf(mx, row[i]);
      float sum = 0.0f;
      for (size_t i = 0; i < n_experts; ++i) {
        tmp[i] = expf(row[i] - mx);
        sum = sum + tmp[i];
      }
      for (size_t i = 0; i < n_experts; ++i) tmp[i] = tmp[i] / sum;
      stable_desc_topk(tmp, n_experts, k, ti);
      if (normalize) {
        float ts = 0.0f;
        for (size_t i = 0; i < k; ++i) ts = ts + tmp[ti[i]];
        for (size_t i = 0; i < k; ++i) tw[i] = tmp[ti[i]] / ts;
      } else {
        for (size_t i = 0; i < k; ++i) tw[i] = tmp[ti[i]];
      }
    }
  }
  free(tmp);
}

/* ---- activations: ops/activation.rs ------------------------------------ */

/* activation.rs:25-38 swiglu_oai via candle ops: clamp = maximum(min).minimum(max);
 * `t * alpha` and `t + 1.0` are affine(mul, add) = v*mul + add. */
float or_swiglu_oai1(float g, float u, float alpha, float limit) {
  float gc = fminf(fmaxf(g, -INFINITY), limit);
  float uc = fminf(fmaxf(u, -limit), limit);
  float a = gc * alpha + 0.0f;
  float sig = 1.0f / (expf(-a) * 1.0f + 1.0f);
  float ga = gc * sig;
  float us = uc * 1.0f + 1.0f;
  return ga * us;
}

/* activation.rs:13-15: candle silu(v) = v / (1 + exp(-v)), then * up. */
float or_silu_mul1(float g, float u) {
  float s = g / (1.0f + expf(-g));
  return s * u;
}

/* activation.rs:41-45: recip(exp(-x) + 1). */
float or_sigmoid1(float x) { return 1.0f / (expf(-x) * 1.0f + 1.0f); }

/* ops/norm.rs:32-36 (CPU path): variance = mean(x^2) (sqr, then sum / n); inv_rms =
 * recip(sqrt(variance + eps)); out = (x * inv_rms) * weight. */
void or_rms_norm(const float* x, const float* weight, size_t n_rows, size_t width, float eps, float* out) {
  for (size_t r = 0; r < n_rows; ++r) {
    const float* xr = x + r * width;
    float s = 0.0f;
    for (size_t i = 0; i < width; ++i) {
      const float sq = xr[i] * xr[i];
      s = s + sq;
    }
    const float var = s / (float)width;
    const float inv = 1.0f / sqrtf(var + eps);
    for (size_t i = 0; i < width; ++i) out[r * width + i] = (xr[i] * inv) * weight[i];
  }
}

/* ---- layer: model/layer.rs run_moe ----------------------------------------- */

uint64_t or_matrix_bytes(int ggml_type, uint64_t rows, uint64_t cols) {
  if (ggml_type == OR_GGML_MXFP4) return rows * (cols / 32) * 17;
  if (ggml_type == OR_GGML_Q4_K) return rows * (cols / 256) * 144;
  return 0;
}

/* out = W . in for one expert matrix of the given type. MXFP4 uses the fused
 * matvec (QUANTIZED_MATMUL=1 path, layer.rs:1418-1440); Q4_K dequantizes to F32
 * and multiplies (default path, layer.rs:1750-1775 + 1818-1847). */
static void expert_matvec(int type, const uint8_t* wq, size_t rows, size_t cols, const float* in,
                          float* out, float* deq_scratch, int n_threads) {
  if (type == OR_GGML_MXFP4) {
    or_mxfp4_matvec(wq, in, rows, cols, out, n_threads);
  } else {
    or_dequant_q4k(wq, rows * cols, deq_scratch);  /* single-threaded, as dequant.rs:218 */
    f32_matvec_mt(deq_scratch, in, rows, cols, out, n_threads);
  }
}

/* One expert FFN for one token: layer.rs:1417-1444 (MXFP4) / 1818-1838 (F32). */
static void expert_ffn(const or_layer* L, uint32_t e, const float* x, float* o, float* g,
                       float* u, float* deq, int n_threads) {
  size_t H = L->hidden, I = L->inter;
  uint64_t gbytes = or_matrix_bytes(L->type, I, H);
  uint64_t dbytes = or_matrix_bytes(L->type, H, I);
  expert_matvec(L->type, L->gate + (uint64_t)e * gbytes, I, H, x, g, deq, n_threads);
  expert_matvec(L->type, L->up + (uint64_t)e * gbytes, I, H, x, u, deq, n_threads);
  if (L->gate_b)
    for (size_t i = 0; i < I; ++i) g[i] = g[i] + L->gate_b[(size_t)e * I + i];
  if (L->up_b)
    for (size_t i = 0; i < I; ++i) u[i] = u[i] + L->up_b[(size_t)e * I + i];
  for (size_t i = 0; i < I; ++i)
    g[i] = L->act_oai ? or_swiglu_oai1(g[i], u[i], L->alpha, L->limit) : or_silu_mul1(g[i], u[i]);
  expert_matvec(L->type, L->down + (uint64_t)e * dbytes, H, I, g, o, deq, n_threads);
  if (L->down_b)
    for (size_t j = 0; j < H; ++j) o[j] = o[j] + L->down_b[(size_t)e * H + j];
}

static int shared_expert(const or_layer* L, const float* x, float* y, int n_threads);

/* Expert assignment (layer.rs:1092-1106): experts visited in ascending index
 * order; each assigned token gets y[t] += out * w (layer.rs:1446-1448,
 * 1506-1513, 1845-1846). Duplicate picks of one expert for one token would sum
 * their weights (layer.rs:1415); top-k never returns duplicates. The shared
 * expert, when present, is added after the routed sum (layer.rs:1945-1951). */
int or_moe_experts(const or_layer* L, const float* x, size_t n_tokens, const uint32_t* idx,
                   const float* w, float* y, int n_threads) {
  size_t H = L->hidden, I = L->inter, k = L->top_k;
  size_t dq = (L->type == OR_GGML_Q4_K) ? I * H : 1;
  float* o = (float*)malloc(sizeof(float) * H);
  float* g = (float*)malloc(sizeof(float) * I);
  float* u = (float*)malloc(sizeof(float) * I);
  float* deq = (float*)malloc(sizeof(float) * dq);
  if (!o || !g || !u || !deq) {
    free(o), free(g), free(u), free(deq);
    return -1;
  }
  for (uint32_t e = 0; e < L->n_experts; ++e) {
    for (size_t t = 0; t < n_tokens; ++t) {
      float tw = 0.0f;
      int hit = 0;
      for (size_t s = 0; s < k; ++s)
        if (idx[t * k + s] == e) tw = hit ? tw + w[t * k + s] : w[t * k + s], hit = 1;
      if (!hit) continue;
      expert_ffn(L, e, x + t * H, o, g, u, deq, n_threads);
      float* yt = y + t * H;
      for (size_t j = 0; j < H; ++j) yt[j] = yt[j] + o[j] * tw;
    }
  }
  free(o), free(g), free(u), free(deq);
  int rc = 0;
  if (L->sh_gate)
    for (size_t t = 0; t < n_tokens && rc == 0; ++t) rc = shared_expert(L, x + t * H, y + t * H, n_threads);
  return rc;
}

/* Shared expert (layer.rs:1898-1953): dense SwiGLU on dequantized F32 weights,
 * scaled by sigmoid(sum(x * gate_inp)), added after the routed sum. */
static int shared_expert(const or_layer* L, const float* x, float* y, int n_threads) {
  size_t H = L->hidden, I = L->sh_inter;
  float* deq = (float*)malloc(sizeof(float) * H * I);
  float* g = (float*)malloc(sizeof(float) * I);
  float* u = (float*)malloc(sizeof(float) * I);
  float* s = (float*)malloc(sizeof(float) * H);
  if (!deq || !g || !u || !s) {
    free(deq), free(g), free(u), free(s);
    return -1;
  }
  expert_matvec(L->sh_type, L->sh_gate, I, H, x, g, deq, n_threads);
  expert_matvec(L->sh_type, L->sh_up, I, H, x, u, deq, n_threads);
  for (size_t i = 0; i < I; ++i) g[i] = or_silu_mul1(g[i], u[i]);
  expert_matvec(L->sh_type, L->sh_down, H, I, g, s, deq, n_threads);
  if (L->sh_gate_inp) {
    float z = 0.0f;
    for (size_t j = 0; j < H; ++j) z = z + x[j] * L->sh_gate_inp[j];
    float sg = or_sigmoid1(z);
    for (size_t j = 0; j < H; ++j) s[j] = s[j] * sg;
  }
  for (size_t j = 0; j < H; ++j) y[j] = y[j] + s[j];
  free(deq), free(g), free(u), free(s);
  return 0;
}

int or_moe_forward(const or_layer* L, const float* x, size_t n_tokens, float* y,
                   uint32_t* idx_out, float* w_out, float* logits_out, int n_threads) {
  size_t H = L->hidden, E = L->n_experts, k = L->top_k;
  float* logits = (float*)malloc(sizeof(float) * n_tokens * E);
  uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * n_tokens * k);
  float* w = (float*)malloc(sizeof(float) * n_tokens * k);
  if (!logits || !idx || !w) {
    free(logits), free(idx), free(w);
    return -1;
  }
  /* router GEMV + bias + dummy mask: layer.rs:806-837, 1016-1026 */
  for (size_t t = 0; t < n_tokens; ++t) {
    float* lt = logits + t * E;
    or_f32_matvec(L->router_w, x + t * H, E, H, lt);
    if (L->router_b)
      for (size_t e = 0; e < E; ++e) lt[e] = lt[e] + L->router_b[e];
    if (L->dummy_mask)
      for (size_t e = 0; e < E; ++e) lt[e] = lt[e] + L->dummy_mask[e];
  }
  or_topk_routing(logits, n_tokens, E, k, L->norm_topk, L->softmax_weight, idx, w);
  memset(y, 0, sizeof(float) * n_tokens * H);
  int rc = or_moe_experts(L, x, n_tokens, idx, w, y, n_threads);
  if (idx_out) memcpy(idx_out, idx, sizeof(uint32_t) * n_tokens * k);
  if (w_out) memcpy(w_out, w, sizeof(float) * n_tokens * k);
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * n_tokens * E);
  free(logits), free(idx), free(w);
  return rc;
}
