"""The dump consumer (python -m moe_rocm.dump) end to end on the GPU: a two-layer GGUF model and
a DUMP_ACTIVATIONS directory in the reference's format whose routing records are the oracle's
top_k_routing (layer.rs:2346-2403) of the dumped inputs; the consumer rebuilds the layers from the
GGUF file (mr_gguf_layer_create), routes the dumped inputs with mr_router_topk and must agree on
every token, and must report a planted wrong index."""
from dataclasses import replace

import numpy as np
import pytest

import dump_writer as DW
import gguf_writer as G
import moe_rocm as M
import oracle
from moe_rocm import dump as D
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

SPEC = W.LayerSpec(config=171, layer=0, ggml_type=M.GGML_MXFP4, hidden=256, inter=128, n_experts=16, top_k=4,
                   route_flags=M.ROUTE_SOFTMAX_AFTER_TOPK, act=M.ACT_SWIGLU_OAI, expert_bias=True, router_bias=True)
META = [("general.architecture", G.STR, "gpt-oss"), ("general.name", G.STR, "gpt-oss dump test"),
        ("gpt-oss.expert_used_count", G.U32, 4), ("gpt-oss.attention.layer_norm_rms_epsilon", G.F32, 1e-5)]


def test_dump_consumer_agrees_with_the_oracles_routing(gpu_ctx, tmp_path):
    specs = [replace(SPEC, layer=l) for l in range(2)]
    tensors, floats = [], []
    for l, s in enumerate(specs):
        q, f = W.quant_tensors(s), W.float_tensors(s)
        tensors += G.moe_layer_tensors(s, q, f, layer=l)
        floats.append(f)
    model = tmp_path / "m.gguf"
    G.write(model, META, tensors)
    dump = tmp_path / "dump"
    dump.mkdir()
    DW.write_meta(dump, SPEC.hidden, SPEC.top_k, SPEC.n_experts, 2)
    for l, s in enumerate(specs):
        for call in range(2):  # two forward calls appended
            x = (W.x_tokens(s, 24, first_token=100 * call) * np.float32(3.0)).astype(np.float32)
            rw = floats[l]["router_w"].reshape(s.n_experts, s.hidden)
            lg = np.stack([oracle.f32_matvec(rw, x[t]) for t in range(x.shape[0])])
            lg = (lg + floats[l]["router_b"]).astype(np.float32)
            idx, w = oracle.topk_routing(lg, s.top_k, normalize=False, softmax_weight=True)
            DW.append(dump, l, x, idx, w)
    assert D.main(["--gguf", str(model), "--dump", str(dump)]) == 0
    # plant a wrong expert in token 5 of layer 1
    dl = D.read_layer(dump, 1)
    bad = dl.idx.copy()
    bad[5, 0] = next(e for e in range(SPEC.n_experts) if e not in set(bad[5].tolist()))
    (dump / "layer_01_hidden.bin").unlink()
    (dump / "layer_01_routing.bin").unlink()
    DW.append(dump, 1, dl.hidden, bad, dl.w)
    g = M.GgufFile(model)
    layer = g.layer(gpu_ctx, 1)
    try:
        rep = D.check_routing(gpu_ctx, layer, D.read_layer(dump, 1))
    finally:
        layer.close()
        g.close()
    assert rep["tokens"] == 48 and rep["mismatch"] == 1 and rep["first_mismatches"][0]["token"] == 5
    assert rep["match"] + rep["tie_ambiguous"] == 47
