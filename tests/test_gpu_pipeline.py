"""The benchmark's timed decode pipeline against the oracle.

bench.py times moe_rocm.workloads.DecodeStack: distinct GPT-OSS-shape (C2) layers,
each linked to the next with mr_layer_set_next in a ring (the last to the first), one
captured HIP graph per token holding that token's layer launches, replayed in token
order. These tests build the same object on four distinct C2 layers, replay the token
graphs twice, and compare every layer's output of every token with the oracle
(max relative error 1e-3; layer.rs:756-1980 with the reference's CPU arithmetic).
"""
import numpy as np
import pytest

import oracle
from moe_rocm import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
N_LAYERS, N_TOKENS = 4, 3


def _oracle_layers(stack):
    out = []
    for dl in stack.layers:
        host = dict(spec=dl.spec)
        host.update(dl.download_quant())
        host.update(W.float_tensors(dl.spec))
        out.append(oracle.layer_from_host(host))
    return out


def _tie_ambiguous(logits, k):
    s = np.sort(logits)[::-1]
    return s[k - 1] - s[k] <= 1e-5 * np.abs(logits).max()


@pytest.mark.parametrize("residual", [False, True], ids=["forward", "forward_residual"])
def test_timed_pipeline_matches_oracle(gpu_ctx, residual):
    specs = W.config_layers(2)[:N_LAYERS]
    stack = W.DecodeStack(gpu_ctx, specs, residual=residual)
    try:
        xs = stack.inputs(N_TOKENS, first_token=500)
        stack.load(xs)
        stack.capture()
        assert len(stack.graphs) == N_TOKENS
        orc = _oracle_layers(stack)
        ref, scale, skip = {}, {}, set()
        for t in range(N_TOKENS):
            for li, L in enumerate(orc):
                if residual:
                    y, _, _, lg = L.forward_residual(xs[t, li], stack.norm_w[li], stack.eps, n_threads=8)
                    scale[t, li] = np.abs(y[0].astype(np.float64) - xs[t, li]).max()
                else:
                    y, _, _, lg = L.forward(xs[t, li], n_threads=8)
                    scale[t, li] = np.abs(y[0]).max()
                ref[t, li] = y[0]
                if _tie_ambiguous(lg[0], specs[li].top_k):
                    skip.add((t, li))
        assert len(skip) < N_TOKENS * N_LAYERS // 2
        for rep in range(2):  # every token graph replayed twice, in decode order
            for t in range(N_TOKENS):
                stack.run(t)
                gpu_ctx.sync()
                y = stack.outputs()
                for li in range(N_LAYERS):
                    if (t, li) in skip:
                        continue
                    err = float(np.abs(y[li].astype(np.float64) - ref[t, li]).max() / scale[t, li])
                    assert err <= REL_TOL, (rep, t, li, err)
    finally:
        stack.close()


def test_chained_pipeline_matches_eager_chain_and_oracle(gpu_ctx):
    """bench.py --decode chain: one hidden state per token carried through four C2 layers in
    place (mr_moe_forward_residual per layer), the layers in a set_next ring, one graph per
    token. The replayed graphs must leave exactly the bits of the same chain run eagerly;
    each layer of the eager chain is then compared with the oracle on its own input (the
    chain amplifies rounding differences from layer to layer, so whole-chain errors of two
    correct implementations are not comparable)."""
    specs = W.config_layers(2)[:N_LAYERS]
    stack = W.ChainStack(gpu_ctx, specs)
    H = stack.H
    try:
        h0 = stack.inputs(N_TOKENS, first_token=700)
        stack.load(h0)
        stack.capture()
        for t in range(N_TOKENS):
            stack.run(t)
        gpu_ctx.sync()
        got = stack.outputs()
        orc = _oracle_layers(stack)
        buf = gpu_ctx.alloc(H * 4)
        try:
            for t in range(N_TOKENS):
                buf.upload(h0[t])
                for li, dl in enumerate(stack.layers):
                    hin = buf.download(np.float32)
                    dl.layer.forward_residual(buf, stack.d_nw.ptr + li * H * 4, stack.eps, buf)
                    out = buf.download(np.float32).astype(np.float64)
                    ref, _, _, lg = orc[li].forward_residual(hin, stack.norm_w[li], stack.eps, n_threads=8)
                    if not _tie_ambiguous(lg[0], specs[li].top_k):
                        err = np.abs(out - ref[0]).max() / np.abs(ref[0].astype(np.float64) - hin).max()
                        assert err <= REL_TOL, (t, li, err)
                assert np.array_equal(buf.download(np.float32), got[t]), t
        finally:
            buf.free()
    finally:
        stack.close()
