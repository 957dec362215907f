"""C-ABI checks that run without a GPU: the library loads, exports every
function include/moe_rocm.h (and the bench-support header moe_rocm_bench.h) declares, and rejects invalid arguments with the
documented status codes on a host-only context (MR_DEVICE_NONE)."""
import re
from pathlib import Path

import numpy as np
import pytest

import moe_rocm as M
from moe_rocm import synth as S

HEADER = Path(__file__).resolve().parent.parent / "include" / "moe_rocm.h"
BENCH_HEADER = HEADER.with_name("moe_rocm_bench.h")


def declared_functions(headers=(HEADER, BENCH_HEADER)):
    names = []
    for h in headers:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_bench_support_stays_out_of_the_drop_in_header():
    core = declared_functions((HEADER,))
    for n in ("mr_synth_blocks", "mr_probe_read", "mr_probe_empty", "mr_probe_tiles", "mr_probe_touch",
              "mr_probe_flags"):
        assert n not in core and n in declared_functions((BENCH_HEADER,))


def test_header_declares_core_entry_points():
    names = declared_functions()
    for n in ("mr_ctx_create", "mr_router_topk", "mr_moe_forward", "mr_moe_forward_batched",
              "mr_moe_experts", "mr_dequant", "mr_pack_upload", "mr_layer_create"):
        assert n in names


def test_library_exports_every_declared_symbol():
    missing = [n for n in declared_functions() if not hasattr(M.lib, n)]
    assert not missing, missing
    # the Python binding wraps every declared function
    assert set(declared_functions()) <= set(M.exported_symbols())


def test_status_strings():
    assert M.lib.mr_status_string(M.MR_OK) == b"ok"
    assert M.lib.mr_status_string(M.MR_E_INVAL) == b"invalid argument"
    assert M.lib.mr_status_string(-99) == b"unknown status"


@pytest.fixture
def hctx():
    ctx = M.Context(M.DEVICE_NONE)
    yield ctx
    ctx.close()


def test_ctx_create_rejects_bad_device():
    with pytest.raises(M.MoeRocmError) as ei:
        M.Context(-7)
    assert ei.value.status == M.MR_E_INVAL


def test_host_only_ctx_device_calls_return_nodev(hctx):
    with pytest.raises(M.MoeRocmError) as ei:
        hctx.sync()
    assert ei.value.status == M.MR_E_NODEV
    with pytest.raises(M.MoeRocmError) as ei:
        hctx.alloc(16)
    assert ei.value.status == M.MR_E_NODEV


def _mx_pack(ctx, E=4, out_f=64, in_f=128):
    data = S.mxfp4_blocks(1, E * out_f * in_f // 32)
    return M.ExpertPack.upload(ctx, M.GGML_MXFP4, data, E, out_f, in_f)


def test_pack_validation(hctx):
    data = np.zeros(4 * 64 * 4 * 17, dtype=np.uint8)
    with pytest.raises(M.MoeRocmError) as ei:
        M.ExpertPack.upload(hctx, 7, data, 4, 64, 128)
    assert ei.value.status == M.MR_E_UNSUPPORTED
    with pytest.raises(M.MoeRocmError) as ei:
        M.ExpertPack.upload(hctx, M.GGML_MXFP4, data, 4, 64, 100)  # not a multiple of 32
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.ExpertPack.upload(hctx, M.GGML_MXFP4, data, 5, 64, 128)  # 5 experts do not fit
    assert ei.value.status == M.MR_E_INVAL and "exceeds" in ei.value.message
    with pytest.raises(M.MoeRocmError) as ei:
        M.ExpertPack.upload(hctx, M.GGML_Q4_K, np.zeros(144 * 64, np.uint8), 1, 64, 128)  # in % 256
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.ExpertPack.upload(hctx, M.GGML_Q4_K, np.zeros(144 * 65, np.uint8), 1, 64, 256,
                            offsets=[2])  # unaligned Q4_K offset
    assert ei.value.status == M.MR_E_INVAL
    p = M.ExpertPack.upload(hctx, M.GGML_MXFP4, data, 4, 64, 128,
                            offsets=[0, 4352, 8704, 13056])  # explicit native offsets
    p.close()


def test_layer_validation(hctx):
    g, u, d = _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 128, 64)
    rw = 0x1000  # any non-NULL address: a host-only context never dereferences it
    kw = dict(router_w=rw, route_flags=M.ROUTE_SOFTMAX_AFTER_TOPK, act=M.ACT_SWIGLU_OAI)
    L = M.MoeLayer(hctx, g, u, d, top_k=2, **kw)
    L.close()
    for bad_k in (0, 5, 17):
        with pytest.raises(M.MoeRocmError) as ei:
            M.MoeLayer(hctx, g, u, d, top_k=bad_k, **kw)
        assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, g, top_k=2, **kw)  # down has the wrong shape
    assert ei.value.status == M.MR_E_INVAL and "down pack" in ei.value.message
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, router_w=None, route_flags=1, act=1)
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, router_w=rw, route_flags=8, act=1)
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, router_w=rw, route_flags=1, act=5)
    assert ei.value.status == M.MR_E_INVAL
    # a shared expert needs all three packs with matching shapes
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, sh_gate=g, **kw)
    assert ei.value.status == M.MR_E_INVAL
    sg = _mx_pack(hctx, 1, 32, 128)
    su = _mx_pack(hctx, 1, 32, 128)
    sd = _mx_pack(hctx, 1, 128, 32)
    L = M.MoeLayer(hctx, g, u, d, top_k=2, sh_gate=sg, sh_up=su, sh_down=sd, **kw)
    L.close()
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, sh_gate=sg, sh_up=su, sh_down=sg, **kw)
    assert ei.value.status == M.MR_E_INVAL


def test_compute_calls_validate_then_need_device(hctx):
    g, u, d = _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 128, 64)
    L = M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1000, route_flags=1, act=1)
    with pytest.raises(M.MoeRocmError) as ei:
        L.forward(None, 0x2000)
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        L.forward(0x1000, 0x2000)
    assert ei.value.status == M.MR_E_NODEV
    # zero tokens is a no-op, even without a device
    L.forward_batched(0x1000, 0, 0x2000)
    with pytest.raises(M.MoeRocmError) as ei:
        M.topk(hctx, 0x1000, 1, 600, 4, 1, 0x2000, 0x3000)  # E > 512
    assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        M.topk(hctx, 0x1000, 1, 32, 17, 1, 0x2000, 0x3000)  # k > 16
    assert ei.value.status == M.MR_E_INVAL
    # expert out of range is caught before the device check
    assert M.lib.mr_dequant(hctx.h, g.h, 9, 0x1000) == M.MR_E_INVAL
    assert M.lib.mr_dequant(hctx.h, g.h, 3, 0x1000) == M.MR_E_NODEV


def test_matrix_bytes():
    assert M.matrix_bytes(M.GGML_MXFP4, 2880, 2880) == 4_406_400
    assert M.matrix_bytes(M.GGML_Q4_K, 768, 2048) == 884_736
    assert M.matrix_bytes(M.GGML_Q4_K, 2048, 512) == 589_824
    assert M.matrix_bytes(99, 1, 1) == 0


def test_set_next_validation(hctx):
    g, u, d = _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 128, 64)
    L1 = M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1000, route_flags=1, act=1)
    L2 = M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x2000, route_flags=1, act=1)
    L1.set_next(L2)  # a hint: no device work, valid on a host-only context
    L1.set_next(L1)  # a layer may follow itself (one-layer loops)
    L1.set_next(None)
    assert M.lib.mr_layer_set_next(None, None) == M.MR_E_INVAL
    other = M.Context(M.DEVICE_NONE)
    try:
        g2, u2, d2 = _mx_pack(other, 4, 64, 128), _mx_pack(other, 4, 64, 128), _mx_pack(other, 4, 128, 64)
        L3 = M.MoeLayer(other, g2, u2, d2, top_k=2, router_w=0x3000, route_flags=1, act=1)
        with pytest.raises(M.MoeRocmError) as ei:
            L1.set_next(L3)
        assert ei.value.status == M.MR_E_INVAL and "different contexts" in ei.value.message
        L3.close()
    finally:
        other.close()


def test_forward_residual_validation(hctx):
    g, u, d = _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 128, 64)
    L = M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1000, route_flags=1, act=1)
    for args in ((None, 0x2000, 1e-5, 0x3000), (0x1000, None, 1e-5, 0x3000), (0x1000, 0x2000, 1e-5, None),
                 (0x1000, 0x2000, -1.0, 0x3000), (0x1000, 0x2000, float("nan"), 0x3000)):
        with pytest.raises(M.MoeRocmError) as ei:
            L.forward_residual(*args)
        assert ei.value.status == M.MR_E_INVAL
    with pytest.raises(M.MoeRocmError) as ei:
        L.forward_residual(0x1000, 0x2000, 1e-6, 0x1000)  # valid (in place): needs a device
    assert ei.value.status == M.MR_E_NODEV


def test_alignment_is_checked_before_the_device(hctx):
    """Kernels read activations and router rows as 16-byte vectors and index/weight arrays
    as 4-byte words: every entry point rejects misaligned pointers with MR_E_INVAL."""
    g, u, d = _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 64, 128), _mx_pack(hctx, 4, 128, 64)
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1004, route_flags=1, act=1)
    assert ei.value.status == M.MR_E_INVAL and "16-byte" in ei.value.message
    with pytest.raises(M.MoeRocmError) as ei:
        M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1000, down_bias=0x2008, route_flags=1, act=1)
    assert ei.value.status == M.MR_E_INVAL
    L = M.MoeLayer(hctx, g, u, d, top_k=2, router_w=0x1000, route_flags=1, act=1)
    calls = [
        lambda: L.forward(0x1004, 0x2000),
        lambda: L.forward_batched(0x1008, 3, 0x2000),
        lambda: L.forward_batched(0x1000, 3, 0x2004),
        lambda: L.experts(0x1004, 2, 0x2000, 0x3000, 0x4000),
        lambda: L.experts(0x1000, 2, 0x2002, 0x3000, 0x4000),
        lambda: L.router_topk(0x100c, 2, 0x2000, 0x3000),
        lambda: L.router_topk(0x1000, 2, 0x2000, 0x3001),
        lambda: M.topk(hctx, 0x1002, 1, 32, 4, 1, 0x2000, 0x3000),
    ]
    for i, call in enumerate(calls):
        with pytest.raises(M.MoeRocmError) as ei:
            call()
        assert ei.value.status == M.MR_E_INVAL, i
    with pytest.raises(M.MoeRocmError) as ei:  # aligned: validation passes, then no device
        L.forward_batched(0x1000, 3, 0x2000)
    assert ei.value.status == M.MR_E_NODEV
    L.close()
