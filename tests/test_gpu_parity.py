"""GPU (HIP, gfx950) vs CPU oracle parity, through the C ABI.

Bars (north star): dequantized weights and top-k indices bit-exact; layer
outputs within max relative error 1e-3, measured as
max_i |y_gpu - y_ref| / max_i |y_ref| (fp32 accumulation on both sides).
"""
import numpy as np
import pytest

import moe_rocm as M
import npref
import oracle
from moe_rocm import synth as S
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


# ---- generator and dequant ------------------------------------------------------

@pytest.mark.parametrize("ggml_type,n", [(M.GGML_MXFP4, 300_001), (M.GGML_Q4_K, 40_003)])
def test_synth_gpu_equals_host(gpu_ctx, ggml_type, n):
    seed = S.stream_seed(77, 1, 2, 3)
    buf = gpu_ctx.alloc(n * S.block_bytes(ggml_type))
    gpu_ctx.synth_blocks(ggml_type, buf, n, seed)
    got = buf.download(np.uint8, n * S.block_bytes(ggml_type))
    assert np.array_equal(got, S.blocks(ggml_type, seed, n))
    buf.free()


def test_dequant_mxfp4_bit_exact_all_codes(gpu_ctx):
    blocks = np.zeros((256, 17), dtype=np.uint8)
    blocks[:, 0] = np.arange(256)
    j = np.arange(16)
    blocks[:, 1:] = (j | ((15 - j) << 4)).astype(np.uint8)
    # a "matrix" of 256 rows x 32 columns, one block per row: every code x every exponent
    pack = M.ExpertPack.upload(gpu_ctx, M.GGML_MXFP4, blocks.reshape(-1), 1, 256, 32)
    got = pack.dequant(0).reshape(-1)
    want = oracle.dequant_mxfp4(blocks.reshape(-1), 256 * 32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    pack.close()


@pytest.mark.parametrize("ggml_type,out_f,in_f,E", [(M.GGML_MXFP4, 2880, 2880, 3),
                                                    (M.GGML_MXFP4, 90, 2880, 5),
                                                    (M.GGML_Q4_K, 768, 2048, 3),
                                                    (M.GGML_Q4_K, 2048, 512, 2)])
def test_dequant_bit_exact_random(gpu_ctx, ggml_type, out_f, in_f, E):
    per = out_f * in_f // S.block_elems(ggml_type)
    data = S.blocks(ggml_type, S.stream_seed(78, ggml_type, out_f, in_f), E * per)
    pack = M.ExpertPack.upload(gpu_ctx, ggml_type, data, E, out_f, in_f)
    mb = S.matrix_bytes(ggml_type, out_f, in_f)
    for e in range(E):
        got = pack.dequant(e).reshape(-1)
        want = oracle.dequant(ggml_type, data[e * mb:(e + 1) * mb], out_f * in_f)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), e
    pack.close()


# ---- routing -----------------------------------------------------------------------

@pytest.mark.parametrize("E,k", [(32, 4), (128, 8), (384, 10), (512, 16), (7, 7)])
@pytest.mark.parametrize("flags", [M.ROUTE_SOFTMAX_AFTER_TOPK, M.ROUTE_NORM_TOPK, 0])
def test_topk_exact_on_given_logits(gpu_ctx, E, k, flags):
    rng = np.random.default_rng(E + 1000 * k + flags)
    T = 33
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[1, 3] = logits[1, E - 1] = logits[1].max() + 0.5   # exact tie -> lower index
    logits[2, : E // 2] = -np.inf                             # masked (dummy) experts
    logits[3, :] = 0.25                                       # all equal
    d_l = gpu_ctx.to_device(logits)
    d_i = gpu_ctx.alloc(T * k * 4)
    d_w = gpu_ctx.alloc(T * k * 4)
    M.topk(gpu_ctx, d_l, T, E, k, flags, d_i, d_w)
    gi = d_i.download(np.int32).reshape(T, k)
    gw = d_w.download(np.float32).reshape(T, k)
    ri, rw = oracle.topk_routing(logits, k, bool(flags & 2), bool(flags & 1))
    assert np.array_equal(gi, ri.astype(np.int32))
    assert np.allclose(gw, rw, rtol=1e-5, atol=1e-7)


# ---- layers --------------------------------------------------------------------------

TINY_MX = W.LayerSpec(201, 0, W.GGML_MXFP4, 512, 384, 8, 2, W.ROUTE_SOFTMAX_AFTER_TOPK,
                      W.ACT_SWIGLU_OAI, True, True)
TINY_Q4 = W.LayerSpec(202, 0, W.GGML_Q4_K, 1024, 512, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                      False, False)
TINY_SH = W.LayerSpec(203, 0, W.GGML_Q4_K, 512, 256, 24, 5, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                      False, False, sh_inter=256)
TINY_Q4P = W.LayerSpec(204, 0, W.GGML_Q4_K, 512, 256, 12, 3, 0, W.ACT_SILU, False, False)  # plain softmax
# top-10 of 20 experts: the 16-slot combine of the grouped path and a ragged 16-expert router tile
TINY_MXK = W.LayerSpec(205, 0, W.GGML_MXFP4, 512, 384, 20, 10, W.ROUTE_NORM_TOPK, W.ACT_SWIGLU_OAI,
                       True, True)
# Q4_K shapes past the fixed-shape fused instantiations (I/256 <= 3, H <= 2048, slots per down
# wave within its registers): they run the streaming instantiation, units passed through the
# registers in rounds; top-16 plus a shared expert is the widest routing the fused kernels take.
WIDE_Q4 = {
    "q4k-H4096": W.LayerSpec(206, 0, W.GGML_Q4_K, 4096, 512, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, False),
    "q4k-H3072-I768": W.LayerSpec(207, 0, W.GGML_Q4_K, 3072, 768, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, False),
    "q4k-I1536-k8": W.LayerSpec(208, 0, W.GGML_Q4_K, 1024, 1536, 16, 8, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                False),
    "q4k-I1024-k7-shared": W.LayerSpec(209, 0, W.GGML_Q4_K, 2048, 1024, 32, 7, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                       False, False, sh_inter=1024),
    "q4k-k16-shared": W.LayerSpec(215, 0, W.GGML_Q4_K, 512, 256, 64, 16, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                  False, sh_inter=256),
    # a Qwen3-235B-A22B-shaped layer (H 4096, I 1536, 128 experts, top-8): two row tiles per gate/up
    # workgroup keep its grid resident
    "q4k-235b-shape": W.LayerSpec(216, 0, W.GGML_Q4_K, 4096, 1536, 128, 8, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                  False),
}
# MXFP4 layers with more than four slots (one down workgroup per row group and group of four
# slots, the last to finish combining) and with an MXFP4 shared expert
WIDE_MX = {
    "mxfp4-k3-shared": W.LayerSpec(217, 0, W.GGML_MXFP4, 512, 384, 16, 3, W.ROUTE_SOFTMAX_AFTER_TOPK,
                                   W.ACT_SWIGLU_OAI, True, True, sh_inter=384, sh_type=W.GGML_MXFP4),
    "mxfp4-k4-shared": W.LayerSpec(218, 0, W.GGML_MXFP4, 1024, 512, 32, 4, W.ROUTE_NORM_TOPK, W.ACT_SWIGLU_OAI,
                                   True, True, sh_inter=512, sh_type=W.GGML_MXFP4),
    "mxfp4-k8": W.LayerSpec(219, 0, W.GGML_MXFP4, 1024, 1024, 32, 8, W.ROUTE_SOFTMAX_AFTER_TOPK, W.ACT_SWIGLU_OAI,
                            True, True),
    "mxfp4-k16-shared": W.LayerSpec(220, 0, W.GGML_MXFP4, 512, 256, 32, 16, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                    False, sh_inter=256, sh_type=W.GGML_MXFP4),
    # 713 workgroups (17 routers, 180 row groups x 2 slot groups, 336 gate/up units): the grid
    # takes the role permutation of the dispatch slots, with slot groups and a shared expert
    "mxfp4-k6-shared-H2880": W.LayerSpec(221, 0, W.GGML_MXFP4, 2880, 1536, 64, 6, W.ROUTE_NORM_TOPK,
                                         W.ACT_SWIGLU_OAI, True, True, sh_inter=1536, sh_type=W.GGML_MXFP4),
}
# MXFP4 shared experts wider than the routed experts (4x: the Qwen2-MoE proportion; 2944, the widest a
# fused down wave takes: 23 K steps of 4 blocks): the
# fused decode kernel gives the shared slot Ish/32 gate/up units and its down wave Ish/32 K blocks;
# batches run the grouped GEMMs with the shared expert as one more group.
WIDE_SH = {
    "mxfp4-k4-shared-x4": W.LayerSpec(222, 0, W.GGML_MXFP4, 1024, 256, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                      False, False, sh_inter=1024, sh_type=W.GGML_MXFP4),
    "mxfp4-k8-shared-2944": W.LayerSpec(223, 0, W.GGML_MXFP4, 2048, 384, 64, 8, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                        False, False, sh_inter=2944, sh_type=W.GGML_MXFP4),
}
# Q4_K shared experts wider than the routed experts: the fused decode kernel runs the shared
# expert as Ish / I slots of the routed width (gate/up rows and down columns j*I .. j*I + I - 1
# of slot j, added in column order after the routed sum), in its streaming instantiation.
WIDE_SH_Q4 = {
    "q4k-k4-shared-x4": W.LayerSpec(224, 0, W.GGML_Q4_K, 512, 256, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                    False, False, sh_inter=1024),
    "q4k-k8-shared-x3-H2048": W.LayerSpec(225, 0, W.GGML_Q4_K, 2048, 512, 64, 8, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                          False, False, sh_inter=1536),
}
SPECS = {
    **WIDE_Q4,
    **WIDE_MX,
    **WIDE_SH,
    **WIDE_SH_Q4,
    "tiny-mxfp4": TINY_MX,
    "tiny-q4k-plain": TINY_Q4P,
    "tiny-q4k": TINY_Q4,
    "tiny-q4k-shared": TINY_SH,
    "tiny-mxfp4-k10": TINY_MXK,
    "C1-gpt-oss": W.gpt_oss(1, 0),
    "C3-qwen3-layer0": W.qwen3_30b(3, 0),
    "C4-coder-next-layer0": W.coder_next(4, 0),
}
# C4 layers across the range of expert counts: 260 (layer 14), 454 (layer 2) and 510 (layer 26).
# Above 448 experts all eight per-lane key columns of the fused routing are live.
C4_RANGE = {f"C4-coder-next-layer{l}-E{W.coder_next(4, l).n_experts}": W.coder_next(4, l) for l in (14, 2, 26)}


@pytest.fixture(scope="module")
def layers(gpu_ctx):
    built = {}
    yield built
    for dl, _ in built.values():
        dl.close()


def get_layer(gpu_ctx, layers, name):
    if name not in layers:
        spec = SPECS[name] if name in SPECS else C4_RANGE[name]
        dl = W.DeviceLayer(gpu_ctx, spec)
        host = dict(spec=spec)
        host.update(dl.download_quant())
        host.update(W.float_tensors(spec))
        layers[name] = (dl, host)
    return layers[name]


@pytest.mark.parametrize("name", list(SPECS))
def test_forward_decode_parity(gpu_ctx, layers, name):
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, 2)
    for t in range(2):
        dx = gpu_ctx.to_device(x[t])
        dy = gpu_ctx.alloc(spec.hidden * 4)
        dl.layer.forward(dx, dy)
        y = dy.download(np.float32)
        ry, ridx, rw, rlg = L.forward(x[t])
        # routing: GPU logits drive the same top-k unless the k-th/(k+1)-th gap is a rounding tie
        s = np.sort(rlg[0])[::-1]
        gap = s[spec.top_k - 1] - s[spec.top_k]
        if gap > 1e-5 * np.abs(rlg).max():
            assert rel_err(y, ry[0]) <= REL_TOL, (name, t, rel_err(y, ry[0]))
        dx.free(), dy.free()


@pytest.mark.parametrize("T", [8, 40])  # 40: the 16x16-tile MFMA router GEMM with ragged tiles
@pytest.mark.parametrize("name", list(SPECS))
def test_router_topk_parity(gpu_ctx, layers, name, T):
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, T, first_token=10)
    dx = gpu_ctx.to_device(x)
    di, dw, dlg = gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.n_experts * 4)
    dl.layer.router_topk(dx, T, di, dw, dlg)
    gi = di.download(np.int32).reshape(T, -1)
    gw = dw.download(np.float32).reshape(T, -1)
    glg = dlg.download(np.float32).reshape(T, -1)
    _, ridx, rw, rlg = L.forward(x)
    assert np.allclose(glg, rlg, rtol=1e-4, atol=1e-5 * np.abs(rlg).max())
    for t in range(T):
        s = np.sort(rlg[t])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg[t]).max():
            assert np.array_equal(gi[t], ridx[t].astype(np.int32)), t
            assert np.allclose(gw[t], rw[t], rtol=1e-4, atol=1e-6)
    for b in (dx, di, dw, dlg):
        b.free()


@pytest.mark.parametrize("name", ["tiny-mxfp4", "tiny-q4k", "tiny-q4k-shared", "C1-gpt-oss"])
def test_experts_given_routing_parity(gpu_ctx, layers, name):
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    L = oracle.layer_from_host(host)
    T = 3
    x = W.x_tokens(spec, T, first_token=20)
    rng = np.random.default_rng(5)
    idx = np.stack([rng.choice(spec.n_experts, spec.top_k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.05, 1.0, (T, spec.top_k)).astype(np.float32)
    dx, di, dw = gpu_ctx.to_device(x), gpu_ctx.to_device(idx), gpu_ctx.to_device(w)
    dy = gpu_ctx.alloc(T * spec.hidden * 4)
    dl.layer.experts(dx, T, di, dw, dy)
    y = dy.download(np.float32).reshape(T, -1)
    ry = L.experts(x, idx.astype(np.uint32), w)
    for t in range(T):
        assert rel_err(y[t], ry[t]) <= REL_TOL, (t, rel_err(y[t], ry[t]))
    if name.startswith("tiny"):
        fy, _, _, _ = npref.moe_forward(host, x, idx=idx, w=w)
        for t in range(T):
            assert rel_err(y[t], fy[t]) <= REL_TOL
    for b in (dx, di, dw, dy):
        b.free()


@pytest.mark.parametrize("name,T", [("tiny-mxfp4", 37), ("tiny-q4k-shared", 16), ("tiny-mxfp4-k10", 40),
                                    ("C1-gpt-oss", 64)])
def test_batched_parity(gpu_ctx, layers, name, T):
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, T, first_token=100)
    dx = gpu_ctx.to_device(x)
    dy = gpu_ctx.alloc(T * spec.hidden * 4)
    dl.layer.forward_batched(dx, T, dy)
    y = dy.download(np.float32).reshape(T, -1)
    ry, _, _, rlg = L.forward(x, n_threads=8)
    for t in range(T):
        s = np.sort(rlg[t])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg[t]).max():
            assert rel_err(y[t], ry[t]) <= REL_TOL, (t, rel_err(y[t], ry[t]))
    dx.free(), dy.free()


C5_SPEC = W.gpt_oss(5, 0, zipf_s=1.1)


@pytest.mark.parametrize("T", [1, 5, 16, 97])
def test_grouped_batched_matches_oracle_and_valu(gpu_ctx, layers, T):
    """Multi-token MXFP4 path (grouped MFMA GEMMs) on the Zipf-skewed C5 layer:
    per-token parity with the oracle and agreement with the VALU path."""
    if "C5" not in layers:
        dl = W.DeviceLayer(gpu_ctx, C5_SPEC)
        host = dict(spec=C5_SPEC)
        host.update(dl.download_quant())
        host.update(W.float_tensors(C5_SPEC))
        layers["C5"] = (dl, host)
    dl, host = layers["C5"]
    spec = dl.spec
    x = W.x_tokens(spec, T, first_token=300)
    dx = gpu_ctx.to_device(x)
    dy, dv = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
    dl.layer.forward_batched(dx, T, dy)
    gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
    try:
        dl.layer.forward_batched(dx, T, dv)
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
    y = dy.download(np.float32).reshape(T, -1)
    yv = dv.download(np.float32).reshape(T, -1)
    ry, _, _, rlg = oracle.layer_from_host(host).forward(x, n_threads=8)
    checked = 0
    for t in range(T):
        s = np.sort(rlg[t])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg[t]).max():
            assert rel_err(y[t], ry[t]) <= REL_TOL, (t, rel_err(y[t], ry[t]))
            assert rel_err(y[t], yv[t]) <= 2 * REL_TOL
            checked += 1
    assert checked >= T - 1
    for b in (dx, dy, dv):
        b.free()


def test_grouped_batched_many_tokens(gpu_ctx, layers):
    """600 tokens x top-4 = 2,400 (token, slot) pairs: the grouping kernel's two-pass path
    (more entries than stay in registers), a ragged last router tile and a long combine grid.
    Every token against the multi-kernel VALU path; the first and last 8 against the oracle."""
    if "C5" not in layers:
        dl = W.DeviceLayer(gpu_ctx, C5_SPEC)
        host = dict(spec=C5_SPEC)
        host.update(dl.download_quant())
        host.update(W.float_tensors(C5_SPEC))
        layers["C5"] = (dl, host)
    dl, host = layers["C5"]
    spec = dl.spec
    T = 600
    x = W.x_tokens(spec, T, first_token=1000)
    dx = gpu_ctx.to_device(x)
    dy, dv = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
    di, dw, dlg = gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.n_experts * 4)
    dl.layer.forward_batched(dx, T, dy)
    dl.layer.router_topk(dx, T, di, dw, dlg)
    gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
    try:
        dl.layer.forward_batched(dx, T, dv)
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
    y = dy.download(np.float32).reshape(T, -1)
    yv = dv.download(np.float32).reshape(T, -1)
    glg = dlg.download(np.float32).reshape(T, -1)
    for t in range(T):
        s = np.sort(glg[t])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(glg[t]).max():
            assert rel_err(y[t], yv[t]) <= 2 * REL_TOL, (t, rel_err(y[t], yv[t]))
    sel = np.r_[0:8, T - 8:T]
    ry, _, _, rlg = oracle.layer_from_host(host).forward(x[sel], n_threads=8)
    assert np.allclose(glg[sel], rlg, rtol=1e-4, atol=1e-5 * np.abs(rlg).max())
    for n, t in enumerate(sel):
        s = np.sort(rlg[n])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg[n]).max():
            assert rel_err(y[t], ry[n]) <= REL_TOL, (t, rel_err(y[t], ry[n]))
    for b in (dx, dy, dv, di, dw, dlg):
        b.free()


@pytest.mark.parametrize("name,T", [("mxfp4-k4-shared", 37), ("mxfp4-k16-shared", 40), ("mxfp4-k3-shared", 1),
                                    ("mxfp4-k6-shared-H2880", 70), ("mxfp4-k4-shared-x4", 33),
                                    ("mxfp4-k8-shared-2944", 24)])
def test_grouped_shared_expert_parity(gpu_ctx, layers, name, T):
    """Multi-token MXFP4 layers with an MXFP4 shared expert: the grouped GEMMs run the shared
    expert as one group of every token (weight 1, SiLU) and the combine adds it, sigmoid-gated,
    after the routed sum (layer.rs:1898-1953). Per token against the oracle and the VALU path."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    x = W.x_tokens(spec, T, first_token=400)
    dx = gpu_ctx.to_device(x)
    dy, dv = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
    gpu_ctx.profile_reset()
    gpu_ctx.set_option(M.OPT_PROFILE, 1)
    try:
        dl.layer.forward_batched(dx, T, dy)
        n_sh = gpu_ctx.profile_read("grouped_shared_gateup")[0]
        n_gu = gpu_ctx.profile_read("grouped_gateup")[0]
    finally:
        gpu_ctx.set_option(M.OPT_PROFILE, 0)
    assert (n_sh, n_gu) == (1, 1), "the grouped MXFP4 kernels did not run"
    gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
    try:
        dl.layer.forward_batched(dx, T, dv)
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
    y = dy.download(np.float32).reshape(T, -1)
    yv = dv.download(np.float32).reshape(T, -1)
    ry, _, _, rlg = oracle.layer_from_host(host).forward(x, n_threads=8)
    checked = 0
    for t in range(T):
        s = np.sort(rlg[t])[::-1]
        if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg[t]).max():
            assert rel_err(y[t], ry[t]) <= REL_TOL, (t, rel_err(y[t], ry[t]))
            assert rel_err(y[t], yv[t]) <= 2 * REL_TOL, (t, rel_err(y[t], yv[t]))
            checked += 1
    assert checked >= max(1, T - 2)
    for b in (dx, dy, dv):
        b.free()


def test_graph_replay_matches_eager(gpu_ctx, layers):
    dl, _ = get_layer(gpu_ctx, layers, "tiny-q4k-shared")
    spec = dl.spec
    dl.layer.reserve(4)
    x = W.x_tokens(spec, 1, first_token=300)
    dx = gpu_ctx.to_device(x[0])
    dy_e, dy_g = gpu_ctx.alloc(spec.hidden * 4), gpu_ctx.alloc(spec.hidden * 4)
    dl.layer.forward(dx, dy_e)
    eager = dy_e.download(np.float32)
    gpu_ctx.graph_begin()
    dl.layer.forward(dx, dy_g)
    g = gpu_ctx.graph_end()
    for rep in range(4):
        gpu_ctx.check(M.lib.mr_dev_zero(gpu_ctx.h, dy_g.ptr, spec.hidden * 4))
        g.launch()
        dl.layer.forward(dx, dy_e)  # eager work between replays
        gpu_ctx.sync()
        assert np.array_equal(dy_g.download(np.float32), eager), rep
    g.close()
    for b in (dx, dy_e, dy_g):
        b.free()


def test_batched_graph_replay_matches_eager(gpu_ctx, layers):
    """The grouped multi-token path (MFMA router, top-k, grouping, x split, grouped GEMMs with
    the h split in the epilogue, combine) captured once and replayed: every replay, with eager
    work in between, gives the eager bits (the grouping's order inside an expert's range varies
    from run to run; nothing computed depends on it)."""
    dl, _ = get_layer(gpu_ctx, layers, "tiny-mxfp4-k10")
    spec = dl.spec
    T = 40
    dl.layer.reserve(T)
    x = W.x_tokens(spec, T, first_token=700)
    dx = gpu_ctx.to_device(x)
    dy_e, dy_g = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
    dl.layer.forward_batched(dx, T, dy_e)
    eager = dy_e.download(np.float32)
    gpu_ctx.graph_begin()
    dl.layer.forward_batched(dx, T, dy_g)
    g = gpu_ctx.graph_end()
    for rep in range(4):
        gpu_ctx.check(M.lib.mr_dev_zero(gpu_ctx.h, dy_g.ptr, T * spec.hidden * 4))
        g.launch()
        dl.layer.forward_batched(dx, T, dy_e)  # eager work between replays
        gpu_ctx.sync()
        assert np.array_equal(dy_g.download(np.float32), eager), rep
        assert np.array_equal(dy_e.download(np.float32), eager), rep
    g.close()
    for b in (dx, dy_e, dy_g):
        b.free()


# ---- fused single-launch decode kernels (MXFP4 and Q4_K) ------------------------------

FUSED = ["tiny-mxfp4", "C1-gpt-oss", "tiny-q4k", "tiny-q4k-plain", "tiny-q4k-shared", "C3-qwen3-layer0",
         "C4-coder-next-layer0", *C4_RANGE, *WIDE_Q4, *WIDE_MX, *WIDE_SH, *WIDE_SH_Q4,
         "tiny-mxfp4-k10"]


@pytest.mark.parametrize("name", FUSED)
def test_fused_matches_oracle_and_valu(gpu_ctx, layers, name):
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, 4, first_token=40)
    dx = gpu_ctx.to_device(x)
    dy = gpu_ctx.alloc(spec.hidden * 4)
    try:
        for t in range(4):
            xp = dx.ptr + t * spec.hidden * 4
            gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_FUSED)
            dl.layer.forward(xp, dy)
            gpu_ctx.sync()
            yf = dy.download(np.float32)
            gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
            dl.layer.forward(xp, dy)
            yv = dy.download(np.float32)
            ry, ridx, _, rlg = L.forward(x[t])
            s = np.sort(rlg[0])[::-1]
            if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg).max():
                assert rel_err(yf, ry[0]) <= REL_TOL, (t, rel_err(yf, ry[0]))
                assert rel_err(yf, yv) <= 2 * REL_TOL
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
    dx.free(), dy.free()


@pytest.mark.parametrize("name", ["C1-gpt-oss", "C4-coder-next-layer0"])
def test_fused_repeated_launches_are_identical(gpu_ctx, layers, name):
    dl, _ = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    x = W.x_tokens(spec, 2, first_token=60)
    dx0, dx1 = gpu_ctx.to_device(x[0]), gpu_ctx.to_device(x[1])
    ys = [gpu_ctx.alloc(spec.hidden * 4) for _ in range(3)]
    dl.layer.forward(dx0, ys[0])
    dl.layer.forward(dx1, ys[1])
    ref0, ref1 = ys[0].download(np.float32), ys[1].download(np.float32)
    for rep in range(40):  # alternating inputs: every launch starts from the previous one's sync words
        dl.layer.forward(dx0 if rep % 2 == 0 else dx1, ys[2])
        got = ys[2].download(np.float32)
        assert np.array_equal(got, ref0 if rep % 2 == 0 else ref1), rep
    gpu_ctx.sync()
    for b in ys + [dx0, dx1]:
        b.free()


def _scattered_pack(ctx, ggml_type, data, n_exp, out_f, in_f):
    """The same expert matrices stored in reverse order with a 256-byte gap after each:
    offsets that are not one stride apart, so the kernels go through the offset table."""
    mb = data.nbytes // n_exp
    step = mb + 256
    buf = np.zeros(n_exp * step, np.uint8)
    offs = [(n_exp - 1 - e) * step for e in range(n_exp)]
    for e, o in enumerate(offs):
        buf[o:o + mb] = data[e * mb:(e + 1) * mb]
    return M.ExpertPack.upload(ctx, ggml_type, buf, n_exp, out_f, in_f, offsets=offs)


@pytest.mark.parametrize("name", ["tiny-mxfp4", "C1-gpt-oss", "tiny-q4k", "tiny-q4k-shared"])
def test_fused_scattered_expert_offsets(gpu_ctx, layers, name):
    """Packs with per-expert offsets (mr_pack_upload's host_offsets) give the same bits as
    the contiguous packs the other tests use (those take the uniform-stride addressing)."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    H, I, E, t = spec.hidden, spec.inter, spec.n_experts, spec.ggml_type
    packs = [_scattered_pack(gpu_ctx, t, host["gate"], E, I, H), _scattered_pack(gpu_ctx, t, host["up"], E, I, H),
             _scattered_pack(gpu_ctx, t, host["down"], E, H, I)]
    L = M.MoeLayer(gpu_ctx, *packs, router_w=dl.f["router_w"], router_b=dl.f["router_b"],
                   gate_bias=dl.f["gate_b"], up_bias=dl.f["up_b"], down_bias=dl.f["down_b"],
                   top_k=spec.top_k, route_flags=spec.route_flags, act=spec.act, alpha=spec.alpha,
                   limit=spec.limit, sh_gate=dl.sh_gate, sh_up=dl.sh_up, sh_down=dl.sh_down,
                   sh_gate_inp=dl.f["sh_gate_inp"])
    x = W.x_tokens(spec, 3, first_token=70)
    dx, y1, y2 = gpu_ctx.to_device(x), gpu_ctx.alloc(H * 4), gpu_ctx.alloc(H * 4)
    try:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_FUSED)
        for i in range(3):
            xp = dx.ptr + i * H * 4
            dl.layer.forward(xp, y1)
            L.forward(xp, y2)
            assert np.array_equal(y1.download(np.float32), y2.download(np.float32)), i
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        L.close()
        for p in packs:
            p.close()
        for b in (dx, y1, y2):
            b.free()


@pytest.mark.parametrize("name", ["tiny-mxfp4", "C1-gpt-oss"])
def test_grouped_packs_at_different_byte_offsets(gpu_ctx, layers, name):
    """Grouped MXFP4 GEMMs (multi-token path) with the gate, up and down experts starting 0, 8
    and 4 bytes further into their 16-byte pieces than in the contiguous packs (one gate/up
    work item reads gate and up rows, each at its own offset): the same bits as the contiguous
    packs."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    H, I, E, t = spec.hidden, spec.inter, spec.n_experts, spec.ggml_type

    def shifted(data, out_f, in_f, shift):
        mb = data.nbytes // E
        step = mb + 256
        buf = np.zeros(E * step + 16, np.uint8)
        offs = [(E - 1 - e) * step + shift for e in range(E)]
        for e, o in enumerate(offs):
            buf[o:o + mb] = data[e * mb:(e + 1) * mb]
        return M.ExpertPack.upload(gpu_ctx, t, buf, E, out_f, in_f, offsets=offs)

    packs = [shifted(host["gate"], I, H, 0), shifted(host["up"], I, H, 8), shifted(host["down"], H, I, 4)]
    L = M.MoeLayer(gpu_ctx, *packs, router_w=dl.f["router_w"], router_b=dl.f["router_b"],
                   gate_bias=dl.f["gate_b"], up_bias=dl.f["up_b"], down_bias=dl.f["down_b"],
                   top_k=spec.top_k, route_flags=spec.route_flags, act=spec.act, alpha=spec.alpha,
                   limit=spec.limit)
    T = 45
    x = W.x_tokens(spec, T, first_token=90)
    dx, y1, y2 = gpu_ctx.to_device(x), gpu_ctx.alloc(T * H * 4), gpu_ctx.alloc(T * H * 4)
    try:
        dl.layer.forward_batched(dx, T, y1)
        L.forward_batched(dx, T, y2)
        assert np.array_equal(y1.download(np.float32), y2.download(np.float32))
    finally:
        L.close()
        for p in packs:
            p.close()
        for b in (dx, y1, y2):
            b.free()


@pytest.mark.parametrize("name", ["tiny-mxfp4", "tiny-q4k-shared"])
def test_fused_graph_replay(gpu_ctx, layers, name):
    dl, _ = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    dl.layer.reserve(1)
    x = W.x_tokens(spec, 1, first_token=70)
    dx = gpu_ctx.to_device(x[0])
    dy_e, dy_g = gpu_ctx.alloc(spec.hidden * 4), gpu_ctx.alloc(spec.hidden * 4)
    dl.layer.forward(dx, dy_e)
    eager = dy_e.download(np.float32)
    gpu_ctx.graph_begin()
    dl.layer.forward(dx, dy_g)
    dl.layer.forward(dx, dy_g)  # two launches per replay: the epoch advances inside the graph
    g = gpu_ctx.graph_end()
    for rep in range(5):
        gpu_ctx.check(M.lib.mr_dev_zero(gpu_ctx.h, dy_g.ptr, spec.hidden * 4))
        g.launch()
        dl.layer.forward(dx, dy_e)
        gpu_ctx.sync()
        assert np.array_equal(dy_g.download(np.float32), eager), rep
    g.close()
    for b in (dx, dy_e, dy_g):
        b.free()


@pytest.mark.parametrize("name", ["C1-gpt-oss", "C3-qwen3-layer0", "mxfp4-k8", "mxfp4-k4-shared"])
def test_fused_wait_timeout_is_reported_and_recovers(gpu_ctx, layers, name):
    """A tiny spin limit (forced from the host) may make a cross-workgroup wait
    run out: the kernel still exits, mr_sync reports it, and the launches after it
    with the default limit are correct (their y rows all written again: y is cleared
    first). The MXFP4 layers with more than four slots (top-8; top-4 + shared) keep a
    per-row-group counter of down slot groups, which must stay in step through the
    failed launches."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec = dl.spec
    x = W.x_tokens(spec, 1, first_token=80)
    dx, dy = gpu_ctx.to_device(x[0]), gpu_ctx.alloc(spec.hidden * 4)
    dl.layer.forward(dx, dy)
    ref = dy.download(np.float32)
    gpu_ctx.set_option(M.OPT_WAIT_LIMIT_US, 1)
    errors = 0
    try:
        for _ in range(5):
            dl.layer.forward(dx, dy)
            try:
                gpu_ctx.sync()
            except M.MoeRocmError as e:
                assert e.status == M.MR_E_LAUNCH and "wait ran out" in e.message
                errors += 1
    finally:
        gpu_ctx.set_option(M.OPT_WAIT_LIMIT_US, 0)
    for rep in range(2):
        gpu_ctx.check(M.lib.mr_dev_zero(gpu_ctx.h, dy.ptr, spec.hidden * 4))
        dl.layer.forward(dx, dy)
        gpu_ctx.sync()
        assert np.array_equal(dy.download(np.float32), ref), rep
    print(f"forced-timeout launches reporting an error: {errors} of 5")
    dx.free(), dy.free()


# (layer, next layer) pairs: same type, MXFP4 -> Q4_K with a shared-expert gate row, Q4_K -> MXFP4
NEXT_PAIRS = [("C1-gpt-oss", "C1-gpt-oss"), ("tiny-mxfp4", "tiny-q4k-shared"),
              ("tiny-q4k-shared", "tiny-mxfp4"), ("C3-qwen3-layer0", "C4-coder-next-layer0")]


@pytest.mark.gpu
@pytest.mark.parametrize("pair", NEXT_PAIRS, ids=lambda p: f"{p[0]}->{p[1]}")
def test_next_layer_hint_keeps_results(gpu_ctx, layers, pair):
    """mr_layer_set_next only prefetches the next layer's router rows: both layers'
    outputs are bitwise the same with and without the hint, and clearing it works."""
    a, b = (get_layer(gpu_ctx, layers, n)[0] for n in pair)
    xa = gpu_ctx.to_device(W.x_tokens(a.spec, 1, first_token=90)[0])
    xb = gpu_ctx.to_device(W.x_tokens(b.spec, 1, first_token=91)[0])
    ya, yb = gpu_ctx.alloc(a.spec.hidden * 4), gpu_ctx.alloc(b.spec.hidden * 4)
    a.layer.forward(xa, ya), b.layer.forward(xb, yb)
    ref_a, ref_b = ya.download(np.float32), yb.download(np.float32)
    try:
        a.layer.set_next(b.layer)
        for _ in range(3):
            a.layer.forward(xa, ya), b.layer.forward(xb, yb)
            gpu_ctx.sync()
            assert np.array_equal(ya.download(np.float32), ref_a)
            assert np.array_equal(yb.download(np.float32), ref_b)
    finally:
        a.layer.set_next(None)
    a.layer.forward(xa, ya)
    assert np.array_equal(ya.download(np.float32), ref_a)
    for t in (xa, xb, ya, yb):
        t.free()


@pytest.mark.gpu
@pytest.mark.parametrize("name", FUSED)
def test_forward_residual_matches_oracle(gpu_ctx, layers, name):
    """mr_moe_forward_residual = h + moe(rms_norm(h)) (layer.rs:462-473, norm.rs:32-36):
    the fused kernels and the multi-kernel path against the oracle, against each other,
    and in place (h_out == h) bitwise equal to out of place."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec, H = dl.spec, dl.spec.hidden
    L = oracle.layer_from_host(host)
    rng = np.random.default_rng(1234 + H + spec.n_experts)
    h = (W.x_tokens(spec, 2, first_token=120) * np.float32(2.5)).astype(np.float32)  # un-normalised
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    eps = 1e-5
    dn, dh, dout = gpu_ctx.to_device(nw), gpu_ctx.alloc(H * 4), gpu_ctx.alloc(H * 4)
    try:
        for t in range(2):
            dh.upload(h[t])
            outs = {}
            for kname, kern in (("fused", M.DECODE_FUSED), ("valu", M.DECODE_VALU)):
                gpu_ctx.set_option(M.OPT_DECODE_KERNEL, kern)
                dl.layer.forward_residual(dh, dn, eps, dout)
                gpu_ctx.sync()
                outs[kname] = dout.download(np.float32)
            ref, _, _, rlg = L.forward_residual(h[t], nw, eps)
            moe_ref = ref[0].astype(np.float64) - h[t]
            scale = np.abs(moe_ref).max()
            s = np.sort(rlg[0])[::-1]
            if s[spec.top_k - 1] - s[spec.top_k] > 1e-5 * np.abs(rlg).max():
                for kname, out in outs.items():
                    err = np.abs(out.astype(np.float64) - ref[0]).max() / scale
                    assert err <= REL_TOL, (name, t, kname, err)
                assert np.abs(outs["fused"].astype(np.float64) - outs["valu"]).max() / scale <= 2 * REL_TOL
            # in place, fused path: the same bits as out of place
            gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_FUSED)
            dl.layer.forward_residual(dh, dn, eps, dh)
            gpu_ctx.sync()
            assert np.array_equal(dh.download(np.float32), outs["fused"])
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
    for b in (dn, dh, dout):
        b.free()


# ---- fused routing: ties and many experts ----------------------------------------------

TIE_SPECS = {
    "mxfp4-E256": W.LayerSpec(210, 0, W.GGML_MXFP4, 256, 128, 256, 4, W.ROUTE_SOFTMAX_AFTER_TOPK,
                              W.ACT_SWIGLU_OAI, True, True),
    "q4k-E300": W.LayerSpec(211, 0, W.GGML_Q4_K, 256, 256, 300, 10, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, True),
    "q4k-E100": W.LayerSpec(212, 0, W.GGML_Q4_K, 256, 256, 100, 8, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, True),
    # 512 experts: every per-lane key column live; all-equal and tied-top put more than 64 keys at or
    # above the k-th largest lane maximum, so the selection searches all columns
    "q4k-E512": W.LayerSpec(213, 0, W.GGML_Q4_K, 256, 256, 512, 10, W.ROUTE_NORM_TOPK, W.ACT_SILU, False, True),
    "q4k-E512-shared": W.LayerSpec(214, 0, W.GGML_Q4_K, 256, 256, 512, 10, W.ROUTE_NORM_TOPK, W.ACT_SILU, False,
                                   True, sh_inter=256),
}


@pytest.mark.parametrize("pattern", ["all-equal", "tied-top", "distinct"])
@pytest.mark.parametrize("name", list(TIE_SPECS))
def test_fused_routing_ties_take_lowest_index(gpu_ctx, name, pattern):
    """Router logits set through a zero router matrix and the router bias: all equal (every
    expert ties), a tied top group (every 7th expert at the maximum, the rest distinct and
    lower) and all distinct. The fused kernels must pick the oracle's experts (the largest,
    ties to the lower index; layer.rs:2346-2403) and match its output."""
    spec = TIE_SPECS[name]
    E, k = spec.n_experts, spec.top_k
    host = dict(spec=spec)
    host.update(W.quant_tensors(spec))
    host.update(W.float_tensors(spec))
    host["router_w"] = np.zeros_like(host["router_w"])
    b = np.zeros(E, np.float32)
    if pattern != "all-equal":
        b = (-1.0 - np.arange(E, dtype=np.float32) / E).astype(np.float32)[np.random.default_rng(9).permutation(E)]
    if pattern == "tied-top":
        b[::7] = 2.0
    host["router_b"] = b
    want = np.argsort(-b.astype(np.float64), kind="stable")[:k]
    dl = W.DeviceLayer(gpu_ctx, spec, host=host)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, 2, first_token=80)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(spec.hidden * 4)
    try:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_FUSED)
        for t in range(2):
            dl.layer.forward(dx.ptr + t * spec.hidden * 4, dy)
            ry, ridx, _, _ = L.forward(x[t])
            assert sorted(ridx[0].tolist()) == sorted(want.tolist())
            assert rel_err(dy.download(np.float32), ry[0]) <= REL_TOL, (t, rel_err(dy.download(np.float32), ry[0]))
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        dl.close()
        dx.free(), dy.free()


# ---- router logits out of the forward calls (mr_layer_set_logits_out) ------------------

LOGITS_OUT = ["tiny-mxfp4", "C1-gpt-oss", "tiny-q4k-shared", "C3-qwen3-layer0", "C4-coder-next-layer0",
              "mxfp4-k4-shared"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", LOGITS_OUT)
def test_logits_out_matches_router_topk(gpu_ctx, layers, name):
    """With a logits output set, the decode forward (fused and multi-kernel), its residual form
    and the batched forward write the router logits the reference reads back after the GPU MoE
    (layer.rs:879-905): equal to mr_router_topk's on the same input (bitwise on the batched path,
    which runs that router; within 1e-4 on the fused kernels' own router), and to the oracle's.
    The outputs y are bitwise the same with and without the logits output; a call of more
    tokens than the output holds is refused; clearing it stops the writes."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec, H, E = dl.spec, dl.spec.hidden, dl.spec.n_experts
    L = oracle.layer_from_host(host)
    T = 20
    x = W.x_tokens(spec, T, first_token=130)
    dx, dx1 = gpu_ctx.to_device(x), gpu_ctx.to_device(x[0])
    dy, dyr = gpu_ctx.alloc(T * H * 4), gpu_ctx.alloc(T * H * 4)
    dlg, rlg = gpu_ctx.alloc(T * E * 4), gpu_ctx.alloc(T * E * 4)
    di, dw = gpu_ctx.alloc(T * spec.top_k * 4), gpu_ctx.alloc(T * spec.top_k * 4)
    nan = np.full(T * E, np.nan, np.float32)
    try:
        dl.layer.router_topk(dx, T, di, dw, rlg)
        router = rlg.download(np.float32).reshape(T, E)
        _, _, _, olg = L.forward(x)
        assert np.allclose(router, olg, rtol=1e-4, atol=1e-5 * np.abs(olg).max())
        for kname, kern in (("fused", M.DECODE_FUSED), ("valu", M.DECODE_VALU)):
            gpu_ctx.set_option(M.OPT_DECODE_KERNEL, kern)
            try:
                dl.layer.forward(dx1, dyr)
                ref_y = dyr.download(np.float32, H)
                dl.layer.set_logits_out(dlg, T)
                dlg.upload(nan)
                dl.layer.forward(dx1, dy)
                gpu_ctx.sync()
                got = dlg.download(np.float32)
                assert np.array_equal(dy.download(np.float32, H), ref_y), kname
                assert np.allclose(got[:E], router[0], rtol=1e-4, atol=1e-5 * np.abs(router[0]).max()), kname
                assert np.all(np.isnan(got[E:])), kname  # one row only
            finally:
                dl.layer.set_logits_out(None)
                gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        # the batched forward runs mr_router_topk's router: the same bits
        dl.layer.set_logits_out(dlg, T)
        dlg.upload(nan)
        dl.layer.forward_batched(dx, T, dy)
        gpu_ctx.sync()
        assert np.array_equal(dlg.download(np.float32).reshape(T, E), router)
        with pytest.raises(M.MoeRocmError) as ei:
            dl.layer.set_logits_out(dlg, T - 1)
            dl.layer.forward_batched(dx, T, dy)
        assert ei.value.status == M.MR_E_INVAL and "logits output" in ei.value.message
        # cleared: a forward leaves the array alone
        dl.layer.set_logits_out(None)
        dlg.upload(nan)
        dl.layer.forward(dx1, dy)
        gpu_ctx.sync()
        assert np.all(np.isnan(dlg.download(np.float32)))
    finally:
        dl.layer.set_logits_out(None)
        for b in (dx, dx1, dy, dyr, dlg, rlg, di, dw):
            b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["C1-gpt-oss", "C3-qwen3-layer0"])
def test_logits_out_residual_and_graph(gpu_ctx, layers, name):
    """The residual decode forward writes the logits of rms_norm(h) (the oracle's), and a graph
    captured with the logits output set writes each replay's logits (new h uploaded between
    replays, every replay checked)."""
    dl, host = get_layer(gpu_ctx, layers, name)
    spec, H, E = dl.spec, dl.spec.hidden, dl.spec.n_experts
    L = oracle.layer_from_host(host)
    rng = np.random.default_rng(77 + E)
    h = (W.x_tokens(spec, 3, first_token=140) * np.float32(2.5)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    eps = 1e-5
    dn, dh, dout, dlg = gpu_ctx.to_device(nw), gpu_ctx.alloc(H * 4), gpu_ctx.alloc(H * 4), gpu_ctx.alloc(E * 4)
    dl.layer.reserve(1)
    dl.layer.set_logits_out(dlg, 1)
    try:
        dh.upload(h[0])
        dl.layer.forward_residual(dh, dn, eps, dout)
        gpu_ctx.sync()
        _, _, _, rlg = L.forward_residual(h[0], nw, eps)
        got = dlg.download(np.float32)
        assert np.allclose(got, rlg[0], rtol=1e-4, atol=1e-5 * np.abs(rlg).max())
        gpu_ctx.graph_begin()
        dl.layer.forward_residual(dh, dn, eps, dout)
        g = gpu_ctx.graph_end()
        for t in (1, 2, 0):
            dh.upload(h[t])
            dlg.upload(np.full(E, np.nan, np.float32))
            g.launch()
            gpu_ctx.sync()
            _, _, _, rlg = L.forward_residual(h[t], nw, eps)
            got = dlg.download(np.float32)
            assert np.allclose(got, rlg[0], rtol=1e-4, atol=1e-5 * np.abs(rlg).max()), t
        g.close()
    finally:
        dl.layer.set_logits_out(None)
        for b in (dn, dh, dout, dlg):
            b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("pair", [("C1-gpt-oss", "C1-gpt-oss"), ("tiny-mxfp4", "tiny-q4k-shared"),
                                  ("C3-qwen3-layer0", "C4-coder-next-layer0")], ids=lambda p: f"{p[0]}->{p[1]}")
def test_norm_hint_keeps_results(gpu_ctx, layers, pair):
    """mr_layer_set_norm only lets the layer before prefetch the norm weights: both layers'
    residual outputs are bitwise the same with and without the hints (next layer and norm
    weights), and clearing them works."""
    a, b = (get_layer(gpu_ctx, layers, n)[0] for n in pair)
    if a.spec.hidden != b.spec.hidden:
        pytest.skip("the chained layers share the hidden size")
    H = a.spec.hidden
    rng = np.random.default_rng(17 + H)
    nw = (1.0 + 0.1 * rng.standard_normal((2, H))).astype(np.float32)
    dnw = gpu_ctx.to_device(nw)
    h0 = (W.x_tokens(a.spec, 1, first_token=150)[0] * np.float32(2.0)).astype(np.float32)
    dh = gpu_ctx.alloc(H * 4)

    def run():
        dh.upload(h0)
        a.layer.forward_residual(dh, dnw.ptr, 1e-5, dh)
        b.layer.forward_residual(dh, dnw.ptr + H * 4, 1e-5, dh)
        gpu_ctx.sync()
        return dh.download(np.float32)

    ref = run()
    try:
        a.layer.set_next(b.layer)
        b.layer.set_norm(dnw.ptr + H * 4)
        a.layer.set_norm(dnw.ptr)
        for _ in range(3):
            assert np.array_equal(run(), ref)
    finally:
        a.layer.set_next(None)
        a.layer.set_norm(None), b.layer.set_norm(None)
    assert np.array_equal(run(), ref)
    dnw.free(), dh.free()
