"""Independent numpy (f64) restatements used to pin the C oracle.

Written from the GGML block-format definitions and the reference's math
(moe-stream-core/src/gguf/dequant.rs, model/layer.rs, ops/activation.rs),
vectorised and in a different order from oracle/moe_oracle.c, so a transposed
operand, a wrong nibble order or a dropped term in either shows up as a
mismatch.
"""
from __future__ import annotations

import numpy as np

MAG = np.array([0, 1, 2, 3, 4, 6, 8, 12], dtype=np.float64)


def mxfp4_dequant(blocks: np.ndarray, n_el: int) -> np.ndarray:
    """dequant.rs:605-628 (vectorised): element 32b+j <- low nibble of byte j,
    32b+16+j <- high nibble; value = +-MAG[code&7] * 2^(e-128)."""
    b = blocks.reshape(-1, 17)[: n_el // 32]
    e = b[:, 0].astype(np.int64)
    scale = np.ldexp(1.0, e - 128)
    qs = b[:, 1:17]
    codes = np.concatenate([qs & 0x0F, qs >> 4], axis=1)  # [nb, 32] in element order
    mag = MAG[codes & 7]
    sign = np.where(codes >= 8, -1.0, 1.0)
    vals = sign * mag * scale[:, None]
    out = vals.astype(np.float32)
    # code 8 is -0.0 (sign bit set)
    out[(codes == 8)] = np.float32(-0.0)
    return out.reshape(-1)


def q4k_dequant(blocks: np.ndarray, n_el: int) -> np.ndarray:
    """ggml Q4_K layout restated with explicit 6-bit unpacking per sub-block;
    y = f32(f32(d*sc)*q) - f32(dmin*m) with fp32 rounding at each step."""
    b = blocks.reshape(-1, 144)[: n_el // 256]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(-1)
    s = b[:, 4:16].astype(np.uint32)
    sc = np.zeros((b.shape[0], 8), dtype=np.uint32)
    mn = np.zeros((b.shape[0], 8), dtype=np.uint32)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            mn[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:144].reshape(-1, 4, 32).astype(np.uint32)
    out = np.empty((b.shape[0], 8, 32), dtype=np.float32)
    for sub in range(8):
        q = (qs[:, sub // 2, :] >> (4 * (sub % 2))) & 0xF
        d1 = (d * sc[:, sub].astype(np.float32)).astype(np.float32)
        m1 = (dmin * mn[:, sub].astype(np.float32)).astype(np.float32)
        p = (d1[:, None] * q.astype(np.float32)).astype(np.float32)
        out[:, sub, :] = (p - m1[:, None]).astype(np.float32)
    return out.reshape(-1)


def dequant(ggml_type: int, blocks: np.ndarray, n_el: int) -> np.ndarray:
    return mxfp4_dequant(blocks, n_el) if ggml_type == 39 else q4k_dequant(blocks, n_el)


def sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def swiglu_oai(g, u, alpha=1.702, limit=7.0):
    gc = np.minimum(g, limit)
    uc = np.clip(u, -limit, limit)
    return gc * sigmoid(alpha * gc) * (uc + 1.0)


def silu_mul(g, u):
    return g * sigmoid(g) * u


def topk(logits: np.ndarray, k: int, normalize: bool, softmax_weight: bool):
    """top_k_routing (layer.rs:2346-2403) by a stable argsort, f64 weights."""
    T, E = logits.shape
    idx = np.zeros((T, k), dtype=np.int64)
    w = np.zeros((T, k), dtype=np.float64)
    for t in range(T):
        v = logits[t].astype(np.float64)
        if softmax_weight:
            order = np.argsort(-v, kind="stable")[:k]
            sel = v[order]
            ex = np.exp(sel - sel.max())
            w[t] = ex / ex.sum()
        else:
            p = np.exp(v - v.max())
            p /= p.sum()
            order = np.argsort(-p, kind="stable")[:k]
            w[t] = p[order] / p[order].sum() if normalize else p[order]
        idx[t] = order
    return idx, w


def expert_ffn(host: dict, e: int, x: np.ndarray) -> np.ndarray:
    """One expert in f64 on dequantized weights (layer.rs:1417-1444)."""
    spec = host["spec"]
    H, I, t = spec.hidden, spec.inter, spec.ggml_type
    from moe_rocm import synth as S

    gb = S.matrix_bytes(t, I, H)
    db = S.matrix_bytes(t, H, I)
    Wg = dequant(t, host["gate"][e * gb:(e + 1) * gb], I * H).reshape(I, H).astype(np.float64)
    Wu = dequant(t, host["up"][e * gb:(e + 1) * gb], I * H).reshape(I, H).astype(np.float64)
    Wd = dequant(t, host["down"][e * db:(e + 1) * db], H * I).reshape(H, I).astype(np.float64)
    g = Wg @ x
    u = Wu @ x
    if host["gate_b"] is not None:
        g = g + host["gate_b"].reshape(-1, I)[e]
        u = u + host["up_b"].reshape(-1, I)[e]
    h = swiglu_oai(g, u, spec.alpha, spec.limit) if spec.act == 1 else silu_mul(g, u)
    o = Wd @ h
    if host["down_b"] is not None:
        o = o + host["down_b"].reshape(-1, H)[e]
    return o


def shared_ffn(host: dict, x: np.ndarray) -> np.ndarray:
    spec = host["spec"]
    H, Is, t = spec.hidden, spec.sh_inter, spec.sh_type
    Wg = dequant(t, host["sh_gate"], Is * H).reshape(Is, H).astype(np.float64)
    Wu = dequant(t, host["sh_up"], Is * H).reshape(Is, H).astype(np.float64)
    Wd = dequant(t, host["sh_down"], H * Is).reshape(H, Is).astype(np.float64)
    s = Wd @ silu_mul(Wg @ x, Wu @ x)
    if host.get("sh_gate_inp") is not None:
        s = s * sigmoid(float(x @ host["sh_gate_inp"].astype(np.float64)))
    return s


def moe_forward(host: dict, x: np.ndarray, idx=None, w=None):
    """Whole layer in f64: router, top-k (or given routing), experts, shared."""
    spec = host["spec"]
    H, E = spec.hidden, spec.n_experts
    x = x.reshape(-1, H).astype(np.float64)
    Wr = host["router_w"].reshape(E, H).astype(np.float64)
    logits = x @ Wr.T
    if host["router_b"] is not None:
        logits = logits + host["router_b"]
    if idx is None:
        idx, w = topk(logits, spec.top_k, bool(spec.route_flags & 2), bool(spec.route_flags & 1))
    y = np.zeros_like(x)
    for t in range(x.shape[0]):
        for s in np.argsort(idx[t], kind="stable"):
            y[t] += w[t][s] * expert_ffn(host, int(idx[t][s]), x[t])
        if spec.sh_inter:
            y[t] += shared_ffn(host, x[t])
    return y, idx, w, logits
