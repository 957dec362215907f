"""Edge cases of the C ABI on the GPU: scratch growth after a graph was captured, and NaN
router logits (ranked below every number on every path)."""
import numpy as np
import pytest

import moe_rocm as M
import oracle
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_graph_survives_scratch_growth(gpu_ctx):
    """A graph captured while the context scratch was sized for one token keeps working after
    a larger batched call grows the scratch (the superseded allocation is kept until the
    context is destroyed, since the graph still addresses it)."""
    spec = W.LayerSpec(220, 0, W.GGML_MXFP4, 512, 384, 8, 2, W.ROUTE_SOFTMAX_AFTER_TOPK,
                       W.ACT_SWIGLU_OAI, True, True)
    ctx = M.Context(0)  # a fresh context: its scratch starts at this layer's one-token size
    dl = W.DeviceLayer(ctx, spec)
    try:
        dl.layer.reserve(1)
        x = W.x_tokens(spec, 64, first_token=5)
        dx1, dy_e, dy_g = ctx.to_device(x[0]), ctx.alloc(spec.hidden * 4), ctx.alloc(spec.hidden * 4)
        dl.layer.forward(dx1, dy_e)
        eager = dy_e.download(np.float32)
        ctx.graph_begin()
        dl.layer.forward(dx1, dy_g)
        g = ctx.graph_end()
        g.launch()
        ctx.sync()
        assert np.array_equal(dy_g.download(np.float32), eager)
        # 64 tokens: the scratch grows (new allocation); the graph still points at the old one
        dxb, dyb = ctx.to_device(x), ctx.alloc(64 * spec.hidden * 4)
        dl.layer.forward_batched(dxb, 64, dyb)
        for _ in range(3):
            ctx.check(M.lib.mr_dev_zero(ctx.h, dy_g.ptr, spec.hidden * 4))
            g.launch()
            dl.layer.forward(dx1, dy_e)  # eager work on the new scratch in between
            ctx.sync()
            assert np.array_equal(dy_g.download(np.float32), eager)
            assert np.array_equal(dy_e.download(np.float32), eager)
        g.close()
        for b in (dx1, dy_e, dy_g, dxb, dyb):
            b.free()
    finally:
        dl.close()
        ctx.close()


def _hip_free_bytes() -> int:
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_scratch_growth_without_capture_frees_and_doubles(gpu_ctx):
    """Token counts that creep up one at a time, with no graph captured: the scratch grows to
    at least twice its token capacity each time, so only a few allocations are made, and a
    superseded allocation is freed (device memory in use ends near one scratch, not the sum of
    every size seen). Results match the oracle throughout."""
    spec = W.LayerSpec(223, 0, W.GGML_MXFP4, 512, 384, 64, 4, W.ROUTE_SOFTMAX_AFTER_TOPK,
                       W.ACT_SWIGLU_OAI, True, True)
    host = W.host_layer(spec)
    ctx = M.Context(0)  # a fresh context: no graph captured, scratch starts empty
    dl = W.DeviceLayer(ctx, spec, host=host)
    n_max = 96
    try:
        x = W.x_tokens(spec, n_max, first_token=7)
        ref, _, _, _ = oracle.layer_from_host(host).forward(x)
        dxb, dyb = ctx.to_device(x), ctx.alloc(n_max * spec.hidden * 4)
        ctx.sync()
        free0 = _hip_free_bytes()
        for T in range(1, n_max + 1):
            dl.layer.forward_batched(dxb, T, dyb)
            if T in (1, 2, 3, 17, 64, n_max):
                got = dyb.download(np.float32, T * spec.hidden).reshape(T, spec.hidden)
                assert rel_err(got, ref[:T]) < REL_TOL, T
        ctx.sync()
        used = free0 - _hip_free_bytes()
        # a scratch for 128 tokens of this shape is about 2 MiB (12 KiB per token plus fixed
        # parts); keeping every superseded allocation would hold over 60 MiB
        print(f"device memory held after growing to {n_max} tokens: {used / 2**20:.1f} MiB")
        assert used < 24 << 20, used
        dxb.free(), dyb.free()
    finally:
        dl.close()
        ctx.close()


NAN_SPECS = {
    "mxfp4-E32": W.LayerSpec(221, 0, W.GGML_MXFP4, 512, 256, 32, 4, W.ROUTE_SOFTMAX_AFTER_TOPK,
                             W.ACT_SWIGLU_OAI, True, True),
    "q4k-E300-softmax-after": W.LayerSpec(222, 0, W.GGML_Q4_K, 256, 256, 300, 10, W.ROUTE_SOFTMAX_AFTER_TOPK,
                                          W.ACT_SILU, False, True),
}


@pytest.mark.parametrize("name", list(NAN_SPECS))
@pytest.mark.parametrize("kernel", ["fused", "valu"])
def test_nan_logits_rank_below_every_number(gpu_ctx, name, kernel):
    """Router logits set through a zero router matrix and the bias, with NaN at the experts
    that would otherwise rank first: no path selects a NaN expert while numbers remain,
    and the output matches the oracle (which applies the same rule)."""
    spec = NAN_SPECS[name]
    E, k = spec.n_experts, spec.top_k
    host = W.host_layer(spec)
    host["router_w"] = np.zeros_like(host["router_w"])
    b = (-1.0 - np.arange(E, dtype=np.float32) / E)[np.random.default_rng(3).permutation(E)].astype(np.float32)
    top = np.argsort(-b, kind="stable")[:3]
    b[top] = np.nan
    host["router_b"] = b
    finite = np.where(~np.isnan(b))[0]
    want = sorted(finite[np.argsort(-b[finite], kind="stable")[:k]].tolist())
    dl = W.DeviceLayer(gpu_ctx, spec, host=host)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, 1, first_token=9)
    dx, dy = gpu_ctx.to_device(x[0]), gpu_ctx.alloc(spec.hidden * 4)
    try:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_FUSED if kernel == "fused" else M.DECODE_VALU)
        dl.layer.forward(dx, dy)
        gpu_ctx.sync()
        ry, ridx, _, _ = L.forward(x)
        assert sorted(ridx[0].tolist()) == want
        y = dy.download(np.float32)
        assert np.all(np.isfinite(y))
        assert rel_err(y, ry[0]) <= REL_TOL
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        dl.close()
        dx.free(), dy.free()


def test_probe_read_reads_every_byte(gpu_ctx):
    """mr_probe_read (the plain-stream ceiling of bench.py --probe) folds every 32-bit word of
    the buffer into the per-workgroup sinks: their XOR is the XOR of the whole buffer, for a
    grid that divides the buffer evenly and one that leaves a ragged tail, at every load depth."""
    rng = np.random.default_rng(11)
    data = rng.integers(0, 2**32, size=(1 << 20) // 4 + 4 * 37, dtype=np.uint32)
    want = np.bitwise_xor.reduce(data)
    d = gpu_ctx.to_device(data)
    for n_wg in (64, 548):
        for depth in (4, 8, 16):
            sink = gpu_ctx.alloc(n_wg * 4)
            gpu_ctx.probe_read(d, data.nbytes, n_wg, sink, depth=depth)
            got = np.bitwise_xor.reduce(sink.download(np.uint32))
            assert got == want, (n_wg, depth)
            sink.free()
    gpu_ctx.probe_empty(576)
    gpu_ctx.sync()
    d.free()


def _tile_probe_xor(data: np.ndarray, rb: int, n_tiles: int, n_wg: int, steps: int = 3, npc: int = 15) -> int:
    """XOR of the 16-byte pieces mr_probe_tiles reads (every lane's four pieces of every chunk of
    every tile its wave streams), restated on the host."""
    words = data.view(np.uint32)
    acc = 0
    lane = np.arange(64)
    cbytes = 68 * steps
    nc = (rb + cbytes - 1) // cbytes
    for it in range((16 * npc + 63) // 64):
        q = it * 64 + lane
        row = np.minimum(q // npc, 15)
        pc = np.minimum(q - row * npc, npc - 1)
        for t in range(n_tiles):
            base = t * 16 * rb
            a = base & 15
            rowa = a + row * rb
            lastr = (rowa + rb - 1) & ~15
            for c in range(nc):
                off = np.minimum(((rowa + cbytes * c) & ~15) + 16 * pc, lastr) + (base - a)
                for o in off:
                    acc ^= int(np.bitwise_xor.reduce(words[o // 4:o // 4 + 4]))
    return acc


def test_probe_tiles_reads_the_gateup_pattern(gpu_ctx):
    """mr_probe_tiles (the fused kernel's gate/up access pattern, bench.py --probe) folds exactly
    the pieces that pattern reads, at every depth and for grids smaller and larger than the tile
    count."""
    rng = np.random.default_rng(12)
    rb, n_tiles = 1530, 10
    data = rng.integers(0, 2**32, size=(n_tiles * 16 * rb + 64) // 4, dtype=np.uint32)
    want = _tile_probe_xor(data, rb, n_tiles, 0)
    d = gpu_ctx.to_device(data)
    for n_wg in (2, 5):
        for depth in (2, 4, 8, 0x106, 0x10C, 0x117):
            w = want if depth < 0x100 else _tile_probe_xor(data, rb, n_tiles, 0, depth - 0x100,
                                                             {6: 27, 12: 53, 23: 99}[depth - 0x100])
            sink = gpu_ctx.alloc(n_wg * 4)
            gpu_ctx.probe_tiles(d, rb, n_tiles, n_wg, sink, depth=depth)
            got = int(np.bitwise_xor.reduce(sink.download(np.uint32)))
            assert got == w, (n_wg, depth)
            sink.free()
    d.free()
