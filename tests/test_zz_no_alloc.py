"""mr_moe_forward_batched_noalloc (static per-GPU scratch, no allocation) against
mr_moe_forward_batched, through the C ABI: two calls in a row, the second with fewer
tokens, each bit-identical to the allocating entry point (the same kernels run on the
same inputs). Also: a call whose scratch would not fit is refused with MR_E_INVAL."""
import ctypes as C

import numpy as np
import pytest

import moe_rocm as M
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

SPECS = {
    # MXFP4: the grouped MFMA path (pair lists, images, per-pair outputs in the scratch)
    "mxfp4-grouped": W.LayerSpec(230, 0, W.GGML_MXFP4, 512, 384, 20, 10, W.ROUTE_NORM_TOPK, W.ACT_SWIGLU_OAI,
                                 True, True),
    # Q4_K with a shared expert: the grouped Q4_K MFMA path (pair lists, images, shared rows)
    "q4k-shared-grouped": W.LayerSpec(231, 0, W.GGML_Q4_K, 512, 256, 24, 5, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                      False, False, sh_inter=256),
    # MXFP4 with an MXFP4 shared expert twice as wide: the grouped path's shared group (its h
    # images, down rows and sigmoid gates in the scratch)
    "mxfp4-shared-grouped": W.LayerSpec(232, 0, W.GGML_MXFP4, 512, 384, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                                        False, False, sh_inter=768, sh_type=W.GGML_MXFP4),
    "C1-gpt-oss": W.gpt_oss(1, 0),
}
TOKENS = {"mxfp4-grouped": (96, 17), "q4k-shared-grouped": (64, 9), "mxfp4-shared-grouped": (80, 21),
          "C1-gpt-oss": (200, 33)}
# Layers run with MR_OPT_DECODE_KERNEL = MR_DECODE_VALU, which sends both entry points down the
# VALU path (activations [T, k, I] and shared activations [T, Ish + 1] in the scratch)
VALU = {"q4k-shared-valu": "q4k-shared-grouped", "mxfp4-valu": "mxfp4-grouped"}


@pytest.mark.parametrize("name", list(SPECS) + list(VALU))
def test_noalloc_matches_batched(gpu_ctx, name):
    base = VALU.get(name, name)
    spec = SPECS[base]
    dl = W.DeviceLayer(gpu_ctx, spec)
    if name in VALU:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
    try:
        for call, T in enumerate(TOKENS[base]):  # the second call has fewer tokens
            x = W.x_tokens(spec, T, first_token=40 * call)
            dx = gpu_ctx.to_device(x)
            dy_ref, dy = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
            gpu_ctx.check(M.lib.mr_moe_forward_batched(gpu_ctx.h, dl.layer.h, dx.ptr, T, dy_ref.ptr))
            gpu_ctx.check(M.lib.mr_dev_zero(gpu_ctx.h, dy.ptr, T * spec.hidden * 4))
            gpu_ctx.check(M.lib.mr_moe_forward_batched_noalloc(gpu_ctx.h, dl.layer.h, dx.ptr, T, dy.ptr))
            gpu_ctx.sync()
            ref = dy_ref.download(np.float32)
            got = dy.download(np.float32)
            assert np.all(np.isfinite(got))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (name, call, T)
            for b in (dx, dy_ref, dy):
                b.free()
    finally:
        gpu_ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_AUTO)
        dl.close()


def test_noalloc_refuses_what_does_not_fit(gpu_ctx):
    spec = W.gpt_oss(1, 0)
    dl = W.DeviceLayer(gpu_ctx, spec)
    try:
        T = 2000  # about 200 MB of scratch at this shape, beyond the 64 MiB array
        dx, dy = gpu_ctx.alloc(T * spec.hidden * 4), gpu_ctx.alloc(T * spec.hidden * 4)
        rc = M.lib.mr_moe_forward_batched_noalloc(gpu_ctx.h, dl.layer.h, dx.ptr, T, dy.ptr)
        assert rc == M.MR_E_INVAL
        assert b"static scratch holds" in C.string_at(M.lib.mr_last_error(gpu_ctx.h))
        gpu_ctx.sync()  # nothing was launched; the context stays usable
        dx.free(), dy.free()
    finally:
        dl.close()
