"""Layers preloaded from GGUF files (mr_gguf_layer_create) on the GPU: the same
outputs as layers built from the same bytes through mr_layer_create, the reference's
dummy-expert mask (engine.rs:628-652), f16/bf16 router weights, and the post-attention
norm weight and epsilon feeding mr_moe_forward_residual."""
import numpy as np
import pytest

import gguf_writer as G
import moe_rocm as M
import oracle
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

MX = W.LayerSpec(config=151, layer=0, ggml_type=M.GGML_MXFP4, hidden=256, inter=128, n_experts=8, top_k=2,
                 route_flags=M.ROUTE_SOFTMAX_AFTER_TOPK, act=M.ACT_SWIGLU_OAI, expert_bias=True, router_bias=True)
Q4 = W.LayerSpec(config=152, layer=0, ggml_type=M.GGML_Q4_K, hidden=512, inter=256, n_experts=16, top_k=4,
                 route_flags=M.ROUTE_NORM_TOPK, act=M.ACT_SILU, expert_bias=False, router_bias=False, sh_inter=256)
META = {id(MX): [("general.architecture", G.STR, "gpt-oss"), ("general.name", G.STR, "gpt-oss test"),
                 ("gpt-oss.expert_used_count", G.U32, 2),
                 ("gpt-oss.attention.layer_norm_rms_epsilon", G.F32, 1e-5)],
        id(Q4): [("general.architecture", G.STR, "qwen3moe"), ("general.name", G.STR, "Qwen3 test"),
                 ("qwen3moe.expert_used_count", G.U32, 4)]}


@pytest.fixture(scope="module")
def ctx():
    c = M.Context(0)
    yield c
    c.close()


def _host(spec):
    return W.quant_tensors(spec), W.float_tensors(spec)


def _oracle(spec, q, f, router_w=None, dummy_mask=None):
    return oracle.Layer(ggml_type=spec.ggml_type, hidden=spec.hidden, inter=spec.inter, n_experts=spec.n_experts,
                        top_k=spec.top_k, gate=q["gate"], up=q["up"], down=q["down"],
                        router_w=f["router_w"] if router_w is None else router_w, router_b=f["router_b"],
                        dummy_mask=dummy_mask, gate_b=f["gate_b"], up_b=f["up_b"], down_b=f["down_b"],
                        softmax_weight=spec.route_flags == M.ROUTE_SOFTMAX_AFTER_TOPK,
                        norm_topk=spec.route_flags == M.ROUTE_NORM_TOPK, act_oai=spec.act == M.ACT_SWIGLU_OAI,
                        sh_type=spec.sh_type, sh_inter=spec.sh_inter, sh_gate=q.get("sh_gate"),
                        sh_up=q.get("sh_up"), sh_down=q.get("sh_down"), sh_gate_inp=f["sh_gate_inp"])


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("spec", [MX, Q4], ids=["mxfp4-gpt-oss", "q4k-qwen3-shared"])
def test_gguf_layer_matches_api_layer(ctx, tmp_path, spec):
    q, f = _host(spec)
    path = tmp_path / "m.gguf"
    G.write(path, META[id(spec)], G.moe_layer_tensors(spec, q, f))
    dl = W.DeviceLayer(ctx, spec)  # the same bytes through mr_pack_upload / mr_layer_create
    x = W.x_tokens(spec, 3, first_token=7)
    dx, y1, y2 = ctx.to_device(x), ctx.alloc(spec.hidden * 4), ctx.alloc(spec.hidden * 4)
    with M.GgufFile(path) as g:
        L = g.layer(ctx, 0)
    try:  # the file is closed: the layer owns its device copies
        for t in range(3):
            xp = dx.ptr + t * spec.hidden * 4
            dl.layer.forward(xp, y1)
            L.forward(xp, y2)
            assert np.array_equal(y1.download(np.float32), y2.download(np.float32))
    finally:
        L.close(), dl.close()
        for b in (dx, y1, y2):
            b.free()


@pytest.mark.parametrize("router_dtype", ["f16", "bf16"])
def test_gguf_dummy_experts_and_half_router(ctx, tmp_path, router_dtype):
    spec = MX
    q, f = _host(spec)
    rw = np.array(f["router_w"], np.float32).reshape(spec.n_experts, spec.hidden)
    rw[5] = 0.25  # a padded expert: a uniform router row (masked to -inf at preload)
    f = dict(f, router_w=rw.reshape(-1))
    path = tmp_path / "d.gguf"
    G.write(path, META[id(spec)], G.moe_layer_tensors(spec, q, f, router_dtype=router_dtype))
    if router_dtype == "f16":
        rw_seen = rw.astype(np.float16).astype(np.float32)
    else:
        rw_seen = ((rw.view(np.uint32) >> 16) << 16).view(np.float32)
    mask = np.zeros(spec.n_experts, np.float32)
    mask[5] = -np.inf
    ref = _oracle(spec, q, f, router_w=rw_seen.reshape(-1), dummy_mask=mask)
    x = W.x_tokens(spec, 4, first_token=11) * np.float32(4.0)
    dx, dy = ctx.to_device(x), ctx.alloc(spec.hidden * 4)
    idx = ctx.alloc(spec.top_k * 4 * 4)
    w = ctx.alloc(spec.top_k * 4 * 4)
    with M.GgufFile(path) as g:
        L = g.layer(ctx, 0)
    try:
        L.router_topk(dx, 4, idx, w)
        gi = idx.download(np.int32).reshape(4, spec.top_k)
        assert not np.any(gi == 5)
        for t in range(4):
            L.forward(dx.ptr + t * spec.hidden * 4, dy)
            ry, ridx, _, _ = ref.forward(x[t])
            assert 5 not in ridx[0]
            assert _rel(dy.download(np.float32), ry[0]) <= 1e-3
    finally:
        L.close()
        for b in (dx, dy, idx, w):
            b.free()


def test_gguf_norm_weight_and_eps_feed_forward_residual(ctx, tmp_path):
    spec = MX
    q, f = _host(spec)
    nw = (1.0 + 0.1 * np.random.default_rng(5).standard_normal(spec.hidden)).astype(np.float32)
    path = tmp_path / "n.gguf"
    G.write(path, META[id(spec)], G.moe_layer_tensors(spec, q, f, norm_w=nw))
    h = W.x_tokens(spec, 1, first_token=3)[0] * np.float32(3.0)
    dh, dout = ctx.to_device(h), ctx.alloc(spec.hidden * 4)
    with M.GgufFile(path) as g:
        L = g.layer(ctx, 0)
    try:
        assert L.norm_w and abs(L.eps - 1e-5) < 1e-12
        L.forward_residual(dh, L.norm_w, L.eps, dout)
        ref, _, _, _ = _oracle(spec, q, f).forward_residual(h, nw, L.eps)
        err = np.abs(dout.download(np.float32).astype(np.float64) - ref[0]).max() / np.abs(ref[0] - h).max()
        assert err <= 1e-3
    finally:
        L.close()
        dh.free(), dout.free()
