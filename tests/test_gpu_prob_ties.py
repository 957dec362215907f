"""Qwen-mode routing (probabilities over all experts, then top-k) on every device path against
the oracle, on router logits where the logit order and the probability order select different
experts. top_k_routing (layer.rs:2371-2394) ranks p_i = expf(l_i - max) / sum in f32 with a
stable sort, so distinct logits whose probabilities round to one value tie, and the lower
expert index wins; ranking by logit would take the larger logit instead.

The logits are set through a zero router matrix and the router bias (x . 0 + b = b exactly):
 - at-max: experts 7 (the maximum 0.125), 9 (one ulp below) and 2 (two ulps below) all have
   expf(l - max) == 1.0f, so k = 2 selects {2, 7}, not {7, 9};
 - below-max: expert 0 at 1.0 and the same three: l - 1.0 rounds to one f32 value for all
   three, so k = 3 selects {0, 2, 7}, not {0, 7, 9};
 - close-distinct: 0.5 and 0.5 - 4 ulp under a maximum of 1.0: within the re-ranking margin
   but with distinct probabilities, so the logit order stands (k = 2: {0, 7});
 - underflow: one logit 0 and the others distinct in [-200, -150]: their probabilities flush
   to 0 and tie, so k = 3 selects {7, 0, 1};
 - nan-logit / inf-logit: a NaN logit, or a +inf one (inf - inf), makes the sum and so every
   probability NaN; the sort then keeps expert order: experts 0..k-1 with NaN weights, and the
   layer's output is NaN.
The expected selections are the oracle's (C, glibc expf); each tie pattern is checked to
differ from the logit-ranked one, so the test tells the two rules apart."""
import numpy as np
import pytest

import moe_rocm as M
import oracle
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
PATTERNS = {"at-max": 2, "below-max": 3, "close-distinct": 2, "underflow": 3, "nan-logit": 2, "inf-logit": 2}


def logits_for(E, pattern, seed=11):
    b = (np.random.default_rng(seed).random(E) * 0.05).astype(np.float32)
    base = np.float32(0.125)
    u = np.spacing(base)
    if pattern in ("at-max", "below-max"):
        b[7], b[9], b[2] = base, base - u, base - 2 * u
        if pattern == "below-max":
            b[0] = 1.0
    elif pattern == "close-distinct":
        h = np.float32(0.5)
        b[0], b[7], b[9] = 1.0, h, h - 4 * np.spacing(h)
    elif pattern == "underflow":
        b = np.random.default_rng(seed).uniform(-200, -150, E).astype(np.float32)
        b[7] = 0.0
    else:
        b[5] = np.nan if pattern == "nan-logit" else np.inf
    return b.astype(np.float32)


def assert_close(got, ref, what):
    """NaN exactly where the reference is NaN, within REL_TOL elsewhere."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (what, int(np.isnan(got).sum()), int(np.isnan(ref).sum()))
    fin = ~np.isnan(ref)
    if fin.any():
        assert rel_err(got[fin], ref[fin]) <= REL_TOL, what


def by_logit(b, k):
    return set(np.argsort(-b.astype(np.float64), kind="stable")[:k].tolist())


def rel_err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


SPECS = {
    "q4k-E32": lambda k: W.LayerSpec(230, 0, W.GGML_Q4_K, 256, 256, 32, k, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, True),
    "q4k-E300": lambda k: W.LayerSpec(231, 0, W.GGML_Q4_K, 256, 256, 300, k, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                      True),
    "mxfp4-E32-plain": lambda k: W.LayerSpec(232, 0, W.GGML_MXFP4, 256, 128, 32, k, 0, W.ACT_SWIGLU_OAI, True, True),
}


@pytest.mark.parametrize("pattern", list(PATTERNS))
@pytest.mark.parametrize("name", list(SPECS))
def test_probability_ties_take_the_lower_index(gpu_ctx, name, pattern):
    k = PATTERNS[pattern]
    spec = SPECS[name](k)
    E = spec.n_experts
    host = dict(spec=spec)
    host.update(W.quant_tensors(spec))
    host.update(W.float_tensors(spec))
    host["router_w"] = np.zeros_like(host["router_w"])
    b = logits_for(E, pattern)
    host["router_b"] = b
    normalize = bool(spec.route_flags & W.ROUTE_NORM_TOPK)
    ridx, rw = oracle.topk_routing(b[None, :], k, normalize, False)
    want = set(ridx[0].tolist())
    if pattern != "close-distinct":
        assert want != by_logit(b, k), "the pattern must separate the two rankings"
    else:
        assert want == by_logit(b, k)
    if pattern in ("nan-logit", "inf-logit"):
        assert want == set(range(k)) and np.isnan(rw).all()
    _check_every_path(gpu_ctx, spec, host, k, want, ridx, rw)


# The softmax-after-top-k (GPT-OSS) mode ranks raw logits with the same comparator. Where that
# order is fixed whatever the sort algorithm: a row of NaN (every comparison "equal": experts
# 0..k-1) and a +inf logit (ranked first; its weight exp(inf - inf) makes every weight NaN).
OAI_PATTERNS = {"all-nan": 3, "inf-logit": 3}


@pytest.mark.parametrize("pattern", list(OAI_PATTERNS))
def test_softmax_after_topk_nan_and_inf_rows(gpu_ctx, pattern):
    k = OAI_PATTERNS[pattern]
    spec = W.LayerSpec(233, 0, W.GGML_MXFP4, 256, 128, 32, k, W.ROUTE_SOFTMAX_AFTER_TOPK, W.ACT_SWIGLU_OAI,
                       True, True)
    host = dict(spec=spec)
    host.update(W.quant_tensors(spec))
    host.update(W.float_tensors(spec))
    host["router_w"] = np.zeros_like(host["router_w"])
    b = (np.random.default_rng(13).random(spec.n_experts) * 0.05).astype(np.float32)
    if pattern == "all-nan":
        b[:] = np.nan
    else:
        b[5] = np.inf
    host["router_b"] = b
    ridx, rw = oracle.topk_routing(b[None, :], k, False, True)
    want = set(ridx[0].tolist())
    if pattern == "all-nan":
        assert want == set(range(k))
    else:
        assert 5 in want and want == by_logit(b, k)
    assert np.isnan(rw).all()
    _check_every_path(gpu_ctx, spec, host, k, want, ridx, rw)


def _check_every_path(gpu_ctx, spec, host, k, want, ridx, rw):
    """The selection `want` and the oracle's weights and outputs on every device path: the
    multi-kernel routing (one token and 32), fused and multi-kernel decode, the batched path."""
    dl = W.DeviceLayer(gpu_ctx, spec, host=host)
    L = oracle.layer_from_host(host)
    try:
        # multi-kernel routing (mr_router_topk): the wave top-k, one token and 32 tokens (the
        # MFMA router and its top-k epilogue)
        for T in (1, 32):
            x = W.x_tokens(spec, T, first_token=90)
            dx = gpu_ctx.to_device(x)
            di, dw = gpu_ctx.alloc(T * k * 4), gpu_ctx.alloc(T * k * 4)
            try:
                dl.layer.router_topk(dx, T, di, dw)
                gi = di.download(np.int32).reshape(T, k)
                gw = dw.download(np.float32).reshape(T, k)
            finally:
                dx.free(), di.free(), dw.free()
            for t in range(T):
                assert set(gi[t].tolist()) == want, (T, t, gi[t], sorted(want))
                order = np.argsort(gi[t])
                ref = rw[0][np.argsort(ridx[0])]
                assert np.array_equal(np.isnan(gw[t][order]), np.isnan(ref)), (gw[t], rw[0])
                if not np.isnan(ref).any():
                    assert np.abs(gw[t][order] - ref).max() <= 1e-5, (gw[t], rw[0])
        # decode: the fused kernel and the multi-kernel path against the oracle's output
        x = W.x_tokens(spec, 2, first_token=95)
        dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(spec.hidden * 4)
        try:
            for kern in (M.DECODE_FUSED, M.DECODE_VALU):
                gpu_ctx.set_option(M.OPT_DECODE_KERNEL, kern)
                for t in range(2):
                    dl.layer.forward(dx.ptr + t * spec.hidden * 4, dy)
                    ry, oidx, _, _ = L.forward(x[t])
                    assert set(oidx[0].tolist()) == want
                    assert_close(dy.download(np.float32), ry[0], (kern, t))
        finally:
            gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
            dx.free(), dy.free()
        # the batched path (grouped GEMM for MXFP4, grouped int8 path for Q4_K): 24 tokens
        T = 24
        x = W.x_tokens(spec, T, first_token=97)
        dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(T * spec.hidden * 4)
        try:
            dl.layer.forward_batched(dx, T, dy)
            y = dy.download(np.float32).reshape(T, spec.hidden)
            ry, _, _, _ = L.forward(x)
            assert_close(y, ry, "batched")
        finally:
            dx.free(), dy.free()
    finally:
        dl.close()
