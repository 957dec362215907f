"""Multi-token Q4_K layers on the grouped int8-MFMA path (mr_moe_forward_batched and
mr_moe_forward_batched_residual): every token against an oracle that follows the reference's
multi-token CPU path (layer.rs:1449-1514: each expert's matrices dequantized once by the oracle's
dequant_q4k, dequant.rs:218-262, then applied to all of the expert's tokens, here in float64; the
shared expert and its sigmoid gate after the routed sum, layer.rs:1898-1953), and against the
per-token VALU path. Bar: max relative error 1e-3 per token (2e-3 between the two GPU paths);
tokens whose k-th and (k+1)-th router logits lie within 1e-5 of the largest are tie-ambiguous
and skipped. Routing (indices exactly, weights to 1e-5) is compared with the oracle's
top_k_routing on the oracle's logits.
"""
from dataclasses import replace

import numpy as np
import pytest

import moe_rocm as M
import oracle
from moe_rocm import synth as S
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3

TINY_SH = W.LayerSpec(260, 0, W.GGML_Q4_K, 512, 256, 24, 5, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, False,
                      sh_inter=256)
TINY_PLAIN = W.LayerSpec(261, 0, W.GGML_Q4_K, 512, 256, 12, 3, 0, W.ACT_SILU, False, False)  # plain softmax
TINY_BIAS = W.LayerSpec(262, 0, W.GGML_Q4_K, 768, 512, 16, 4, W.ROUTE_SOFTMAX_AFTER_TOPK, W.ACT_SWIGLU_OAI,
                        True, True)  # expert biases and OAI SwiGLU on Q4_K weights


def rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.fixture(scope="module")
def built(gpu_ctx):
    cache = {}
    yield cache
    for dl, _ in cache.values():
        dl.close()


def get(gpu_ctx, built, spec):
    if spec not in built:
        dl = W.DeviceLayer(gpu_ctx, spec)
        host = dict(spec=spec)
        host.update(dl.download_quant())
        host.update(W.float_tensors(spec))
        built[spec] = (dl, host)
    return built[spec]


def _silu(g):
    with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: the limit 0 is right
        return g / (1.0 + np.exp(-g))


def _swiglu_oai(g, u, alpha, limit):
    g = np.minimum(g, limit)
    u = np.clip(u, -limit, limit)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-alpha * g)) * (u + 1.0)


def oracle_batched(host, x):
    """layer.rs:1449-1514 in float64 on the oracle's dequantized weights. Returns
    (y [T,H], idx, w, logits [T,E] f32 as the oracle computes them)."""
    spec = host["spec"]
    H, I, E, k, t = spec.hidden, spec.inter, spec.n_experts, spec.top_k, spec.ggml_type
    T = x.shape[0]
    rw = host["router_w"].reshape(E, H)
    logits = np.stack([oracle.f32_matvec(rw, x[i]) for i in range(T)]).astype(np.float32)
    if host["router_b"] is not None:
        logits = (logits + host["router_b"]).astype(np.float32)
    idx, w = oracle.topk_routing(logits, k, normalize=bool(spec.route_flags & 2),
                                 softmax_weight=bool(spec.route_flags & 1))
    y = np.zeros((T, H), dtype=np.float64)
    mb_gu, mb_d = S.matrix_bytes(t, I, H), S.matrix_bytes(t, H, I)
    xd = x.astype(np.float64)
    for e in np.unique(idx):
        rows, slots = np.nonzero(idx == e)
        order = np.argsort(rows, kind="stable")
        rows, slots = rows[order], slots[order]
        Wg = oracle.dequant(t, host["gate"][e * mb_gu:(e + 1) * mb_gu], I * H).reshape(I, H).astype(np.float64)
        Wu = oracle.dequant(t, host["up"][e * mb_gu:(e + 1) * mb_gu], I * H).reshape(I, H).astype(np.float64)
        Wd = oracle.dequant(t, host["down"][e * mb_d:(e + 1) * mb_d], H * I).reshape(H, I).astype(np.float64)
        g = xd[rows] @ Wg.T
        u = xd[rows] @ Wu.T
        if host["gate_b"] is not None:
            g += host["gate_b"].reshape(E, I)[e]
            u += host["up_b"].reshape(E, I)[e]
        h = _swiglu_oai(g, u, spec.alpha, spec.limit) if spec.act == W.ACT_SWIGLU_OAI else _silu(g) * u
        o = h @ Wd.T
        if host["down_b"] is not None:
            o += host["down_b"].reshape(E, H)[e]
        y[rows] += o * w[rows, slots][:, None].astype(np.float64)
    if spec.sh_inter:
        Is, st = spec.sh_inter, spec.sh_type
        Sg = oracle.dequant(st, host["sh_gate"], Is * H).reshape(Is, H).astype(np.float64)
        Su = oracle.dequant(st, host["sh_up"], Is * H).reshape(Is, H).astype(np.float64)
        Sd = oracle.dequant(st, host["sh_down"], H * Is).reshape(H, Is).astype(np.float64)
        so = (_silu(xd @ Sg.T) * (xd @ Su.T)) @ Sd.T
        gi = host["sh_gate_inp"]
        sig = 1.0 / (1.0 + np.exp(-(xd @ gi.astype(np.float64)))) if gi is not None else np.ones(T)
        y += sig[:, None] * so
    return y, idx, w, logits


def _ambiguous(lg, k):
    s = np.sort(lg)[::-1]
    return s[k - 1] - s[k] <= 1e-5 * np.abs(lg).max()


def _run(gpu_ctx, dl, x, kernel=M.DECODE_AUTO, residual=None):
    T, H = x.shape
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(T * H * 4)
    gpu_ctx.set_option(M.OPT_DECODE_KERNEL, kernel)
    try:
        if residual is None:
            dl.layer.forward_batched(dx, T, dy)
        else:
            nw, eps = residual
            dn = gpu_ctx.to_device(nw)
            dl.layer.forward_batched_residual(dx, T, dn, eps, dy)
            gpu_ctx.sync()
            dn.free()
        y = dy.download(np.float32).reshape(T, H)
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        dx.free(), dy.free()
    return y


def _check(gpu_ctx, dl, host, x, valu=True, min_checked=0.9):
    spec = dl.spec
    T = x.shape[0]
    gpu_ctx.profile_reset()
    gpu_ctx.set_option(M.OPT_PROFILE, 1)
    try:
        y = _run(gpu_ctx, dl, x)
        n_grouped = gpu_ctx.profile_read("grouped_q4k_gateup")[0]
    finally:
        gpu_ctx.set_option(M.OPT_PROFILE, 0)
    assert n_grouped == 1, "the grouped Q4_K kernels did not run"
    yv = _run(gpu_ctx, dl, x, M.DECODE_VALU) if valu else None
    ry, ridx, rw, rlg = oracle_batched(host, x)
    # routing on the GPU against the oracle's
    di, dw, dlg = (gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.top_k * 4),
                   gpu_ctx.alloc(T * spec.n_experts * 4))
    dx = gpu_ctx.to_device(x)
    dl.layer.router_topk(dx, T, di, dw, dlg)
    gi = di.download(np.int32).reshape(T, -1)
    gw = dw.download(np.float32).reshape(T, -1)
    for b in (di, dw, dlg, dx):
        b.free()
    checked = 0
    for t in range(T):
        if _ambiguous(rlg[t], spec.top_k):
            continue
        assert np.array_equal(np.sort(gi[t]), np.sort(ridx[t].astype(np.int32))), t
        assert np.allclose(np.sort(gw[t]), np.sort(rw[t]), rtol=1e-5, atol=1e-6), t
        assert rel_err(y[t], ry[t]) <= REL_TOL, (t, rel_err(y[t], ry[t]))
        if valu:
            assert rel_err(y[t], yv[t]) <= 2 * REL_TOL, (t, rel_err(y[t], yv[t]))
        checked += 1
    assert checked >= min_checked * T
    return y


def test_c3_shaped_512_tokens(gpu_ctx, built):
    """A Qwen3-30B-A3B-shaped layer (H 2048, I 768, 128 experts, top-8) with a 512-token batch:
    4,096 (token, slot) pairs, every expert holding tokens, most with a ragged last pair tile."""
    spec = W.qwen3_30b(3, 0)
    dl, host = get(gpu_ctx, built, spec)
    x = W.x_tokens(spec, 512, first_token=4000)
    _check(gpu_ctx, dl, host, x, valu=False)


def test_c4_shaped_with_shared_expert(gpu_ctx, built):
    """The Coder-Next-shaped layer 0 (410 experts, top-10, shared expert with its sigmoid gate)."""
    spec = W.coder_next(4, 0)
    dl, host = get(gpu_ctx, built, spec)
    x = W.x_tokens(spec, 96, first_token=5000)
    _check(gpu_ctx, dl, host, x)


@pytest.mark.parametrize("spec", [TINY_SH, TINY_PLAIN, TINY_BIAS], ids=["shared", "plain-softmax", "bias-oai"])
@pytest.mark.parametrize("T", [1, 7, 33, 97])
def test_tiny_shapes(gpu_ctx, built, spec, T):
    dl, host = get(gpu_ctx, built, spec)
    x = W.x_tokens(spec, T, first_token=60 + T)
    _check(gpu_ctx, dl, host, x, min_checked=0.8)


def test_batched_residual_matches_per_token_and_in_place(gpu_ctx, built):
    """mr_moe_forward_batched_residual: h + moe(rms_norm(h)) for every token; equal to the
    oracle's rms_norm then the batched MoE, and the same bits in place."""
    spec = TINY_SH
    dl, host = get(gpu_ctx, built, spec)
    T, H = 40, spec.hidden
    h = (W.x_tokens(spec, T, first_token=900) * np.float32(3.0)).astype(np.float32)
    nw = W.norm_weights(1, H)[0]
    eps = 1e-6
    got = _run(gpu_ctx, dl, h, residual=(nw, eps))
    xn = oracle.rms_norm(h, nw, eps)
    ry, _, _, rlg = oracle_batched(host, xn)
    checked = 0
    for t in range(T):
        if _ambiguous(rlg[t], spec.top_k):
            continue
        err = np.abs(got[t].astype(np.float64) - (h[t] + ry[t])).max() / np.abs(ry[t]).max()
        assert err <= REL_TOL, (t, err)
        checked += 1
    assert checked >= 0.8 * T
    dh, dn = gpu_ctx.to_device(h), gpu_ctx.to_device(nw)
    dl.layer.forward_batched_residual(dh, T, dn, eps, dh)
    assert np.array_equal(dh.download(np.float32).reshape(T, H), got)
    dh.free(), dn.free()


def test_batched_residual_mxfp4(gpu_ctx, built):
    """The same entry on an MXFP4 layer (grouped MX-fp4 GEMMs underneath)."""
    spec = W.LayerSpec(263, 0, W.GGML_MXFP4, 512, 384, 8, 2, W.ROUTE_SOFTMAX_AFTER_TOPK, W.ACT_SWIGLU_OAI,
                       True, True)
    dl, host = get(gpu_ctx, built, spec)
    T, H = 33, spec.hidden
    h = W.x_tokens(spec, T, first_token=70)
    nw = W.norm_weights(1, H)[0]
    got = _run(gpu_ctx, dl, h, residual=(nw, 1e-5))
    L = oracle.layer_from_host(host)
    for t in range(T):
        ref, _, _, lg = L.forward_residual(h[t], nw, 1e-5)
        if _ambiguous(lg[0], spec.top_k):
            continue
        err = np.abs(got[t].astype(np.float64) - ref[0]).max() / np.abs(ref[0].astype(np.float64) - h[t]).max()
        assert err <= REL_TOL, (t, err)


def test_grouped_q4k_noalloc_and_graph_match_batched(gpu_ctx, built):
    """The static-scratch entry and a captured graph (replayed with eager work between the
    replays) give the bits of mr_moe_forward_batched."""
    spec = TINY_SH
    dl, _ = get(gpu_ctx, built, spec)
    H = spec.hidden
    x = W.x_tokens(spec, 64, first_token=123)
    dx = gpu_ctx.to_device(x)
    ya, yb, yg = gpu_ctx.alloc(64 * H * 4), gpu_ctx.alloc(64 * H * 4), gpu_ctx.alloc(64 * H * 4)
    try:
        for T in (64, 9):
            dl.layer.forward_batched(dx, T, ya)
            dl.layer.forward_batched_noalloc(dx, T, yb)
            gpu_ctx.sync()
            assert np.array_equal(ya.download(np.float32, count=T * H), yb.download(np.float32, count=T * H)), T
        dl.layer.reserve(64)
        dl.layer.forward_batched(dx, 64, ya)
        gpu_ctx.graph_begin()
        dl.layer.forward_batched(dx, 64, yg)
        g = gpu_ctx.graph_end()
        try:
            for rep in range(3):
                g.launch()
                gpu_ctx.sync()
                assert np.array_equal(yg.download(np.float32), ya.download(np.float32)), rep
                dl.layer.forward_batched(dx, 17, yb)  # eager work between replays
                gpu_ctx.sync()
        finally:
            g.close()
    finally:
        for b in (dx, ya, yb, yg):
            b.free()
