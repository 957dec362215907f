"""The configured workloads and builders for their synthetic layers.

Each LayerSpec describes one MoE layer; host_layer() produces its tensors as
numpy arrays (small shapes, tests), device_layer() builds it on the GPU with
the quantized blocks generated in place by mr_synth_blocks (identical bytes to
host_layer) and the float tensors generated here.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import synth as S

GGML_Q4_K, GGML_MXFP4 = 12, 39
ROUTE_SOFTMAX_AFTER_TOPK, ROUTE_NORM_TOPK = 1, 2
ACT_SILU, ACT_SWIGLU_OAI = 0, 1


@dataclass(frozen=True)
class LayerSpec:
    config: int               # workload id (1..5; 100+ for test shapes)
    layer: int
    ggml_type: int
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    route_flags: int
    act: int
    expert_bias: bool         # ffn_{gate,up,down}_exps.bias present (GPT-OSS)
    router_bias: bool         # ffn_gate_inp.bias present (GPT-OSS)
    sh_inter: int = 0         # shared expert intermediate (0 = none)
    sh_type: int = GGML_Q4_K
    zipf_s: float = 0.0       # router skew: logit_e += ln p_e, p_e ~ rank^-s
    alpha: float = 1.702
    limit: float = 7.0

    @property
    def mxfp4(self) -> bool:
        return self.ggml_type == GGML_MXFP4

    def seed(self, tensor: int, sub: int = 0) -> int:
        return S.stream_seed(self.config, self.layer, tensor, sub)

    def weight_bytes_per_token(self) -> int:
        """Algorithmic bytes one decode token moves through this layer: the k
        selected experts' quantized weights and biases, the router (+bias),
        the shared expert, x read once and y written once."""
        H, I, k, E = self.hidden, self.inter, self.top_k, self.n_experts
        t = self.ggml_type
        b = k * (2 * S.matrix_bytes(t, I, H) + S.matrix_bytes(t, H, I))
        if self.expert_bias:
            b += k * (2 * I + H) * 4
        b += E * H * 4 + (E * 4 if self.router_bias else 0)
        if self.sh_inter:
            b += 2 * S.matrix_bytes(self.sh_type, self.sh_inter, H) + S.matrix_bytes(self.sh_type, H, self.sh_inter)
            b += H * 4  # shared gate_inp
        b += 2 * H * 4
        return b

    def flops_per_token(self) -> int:
        H, I, k, E = self.hidden, self.inter, self.top_k, self.n_experts
        f = 2 * E * H + k * 2 * (3 * H * I)
        if self.sh_inter:
            f += 2 * 3 * H * self.sh_inter + 2 * H
        return f


def batched_bytes(spec: LayerSpec, n_tokens: int) -> int:
    """Algorithmic bytes of one batched forward: every expert's weights and biases
    (each read once), router weights/bias, x read once, y written once."""
    H, I, E = spec.hidden, spec.inter, spec.n_experts
    t = spec.ggml_type
    b = E * (2 * S.matrix_bytes(t, I, H) + S.matrix_bytes(t, H, I))
    if spec.expert_bias:
        b += E * (2 * I + H) * 4
    b += E * H * 4 + (E * 4 if spec.router_bias else 0)
    b += 2 * n_tokens * H * 4
    return b


def gpt_oss(config: int, layer: int, **kw) -> LayerSpec:
    base = LayerSpec(config, layer, GGML_MXFP4, 2880, 2880, 32, 4, ROUTE_SOFTMAX_AFTER_TOPK,
                     ACT_SWIGLU_OAI, True, True)
    return replace(base, **kw)


def qwen3_30b(config: int, layer: int, **kw) -> LayerSpec:
    base = LayerSpec(config, layer, GGML_Q4_K, 2048, 768, 128, 8, ROUTE_NORM_TOPK, ACT_SILU,
                     False, False)
    return replace(base, **kw)


def coder_next_experts_per_layer(n_layers: int = 48) -> list[int]:
    """E_l ~ U{256..512} per layer (experts_per_layer pruning metadata, config.rs:376-379)."""
    return [int(v) for v in S.uniform_int(S.stream_seed(4, 0, S.T_EXPERTS_PER_LAYER, 0), n_layers, 256, 512)]


def coder_next(config: int, layer: int, n_experts: int | None = None, **kw) -> LayerSpec:
    if n_experts is None:
        n_experts = coder_next_experts_per_layer()[layer]
    base = LayerSpec(config, layer, GGML_Q4_K, 2048, 512, n_experts, 10, ROUTE_NORM_TOPK, ACT_SILU,
                     False, False, sh_inter=512, sh_type=GGML_Q4_K)
    return replace(base, **kw)


def config_layers(config: int) -> list[LayerSpec]:
    """All layers of a configured workload (C1..C5)."""
    if config == 1:
        # one layer shape; 8 independently seeded instances (3.4 GB) are cycled so the
        # 256 MB Infinity Cache cannot serve repeats
        return [gpt_oss(1, l) for l in range(8)]
    if config == 2:
        return [gpt_oss(2, l) for l in range(24)]
    if config == 3:
        return [qwen3_30b(3, l) for l in range(48)]
    if config == 4:
        epl = coder_next_experts_per_layer()
        return [coder_next(4, l, n_experts=epl[l]) for l in range(48)]
    if config == 5:
        return [gpt_oss(5, 0, zipf_s=1.1)]
    raise ValueError(config)


CONFIG_TOKENS = {1: 1, 2: 256, 3: 1, 4: 1, 5: 512}
CONFIG_NAMES = {
    1: "gpt-oss-20b-shape, 1 MoE layer, 1 decode token (MXFP4, top-4/32)",
    2: "gpt-oss-20b-shape, 24-layer MoE stack, batch-1 decode of 256 tokens (MXFP4, top-4/32)",
    3: "qwen3-30b-a3b-shape, 48-layer MoE stack, batch-1 decode (Q4_K, top-8/128)",
    4: "qwen3-coder-next-80b-shape pruned, 48 layers, top-10 + shared expert (Q4_K, E_l in [256,512])",
    5: "gpt-oss-20b-shape batched/prefill, 512 tokens, Zipf(1.1)-skewed routing (MXFP4)",
}


def zipf_log_p(spec: LayerSpec) -> np.ndarray:
    """ln p_e with p_e proportional to rank_e^-s over a seeded rank permutation."""
    E = spec.n_experts
    keys = S.draws(spec.seed(S.T_ZIPF), 0, E)
    rank = np.empty(E, dtype=np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(1, E + 1)
    p = rank.astype(np.float64) ** (-spec.zipf_s)
    p /= p.sum()
    return np.log(p)


def float_tensors(spec: LayerSpec) -> dict[str, np.ndarray | None]:
    """Router, biases and shared gate: float32 by Box-Muller."""
    H, I, E = spec.hidden, spec.inter, spec.n_experts
    t: dict[str, np.ndarray | None] = {}
    t["router_w"] = S.normal(spec.seed(S.T_ROUTER_W), E * H, 0.02)
    rb = S.normal(spec.seed(S.T_ROUTER_B), E, 0.01) if spec.router_bias else None
    if spec.zipf_s:
        base = rb.astype(np.float64) if rb is not None else np.zeros(E)
        rb = (base + zipf_log_p(spec)).astype(np.float32)
    t["router_b"] = rb
    if spec.expert_bias:
        t["gate_b"] = S.normal(spec.seed(S.T_GATE_B), E * I, 0.01)
        t["up_b"] = S.normal(spec.seed(S.T_UP_B), E * I, 0.01)
        t["down_b"] = S.normal(spec.seed(S.T_DOWN_B), E * H, 0.01)
    else:
        t["gate_b"] = t["up_b"] = t["down_b"] = None
    t["sh_gate_inp"] = S.normal(spec.seed(S.T_SH_GATE_INP), H, 0.02) if spec.sh_inter else None
    return t


def _n_blocks(ggml_type: int, rows: int, cols: int) -> int:
    return rows * cols // S.block_elems(ggml_type)


def quant_tensors(spec: LayerSpec) -> dict[str, np.ndarray | None]:
    """Stacked expert tensors [E][out][in] in native block layout (host)."""
    H, I, E, t = spec.hidden, spec.inter, spec.n_experts, spec.ggml_type
    q: dict[str, np.ndarray | None] = {
        "gate": S.blocks(t, spec.seed(S.T_GATE), E * _n_blocks(t, I, H)),
        "up": S.blocks(t, spec.seed(S.T_UP), E * _n_blocks(t, I, H)),
        "down": S.blocks(t, spec.seed(S.T_DOWN), E * _n_blocks(t, H, I)),
    }
    if spec.sh_inter:
        st, Is = spec.sh_type, spec.sh_inter
        q["sh_gate"] = S.blocks(st, spec.seed(S.T_SH_GATE), _n_blocks(st, Is, H))
        q["sh_up"] = S.blocks(st, spec.seed(S.T_SH_UP), _n_blocks(st, Is, H))
        q["sh_down"] = S.blocks(st, spec.seed(S.T_SH_DOWN), _n_blocks(st, H, Is))
    else:
        q["sh_gate"] = q["sh_up"] = q["sh_down"] = None
    return q


def x_tokens(spec: LayerSpec, n_tokens: int, first_token: int = 0) -> np.ndarray:
    """Layer input activations x ~ N(0,1), one stream per (layer, token)."""
    return np.stack([S.normal(spec.seed(S.T_X, first_token + i), spec.hidden, 1.0)
                     for i in range(n_tokens)])


def host_layer(spec: LayerSpec) -> dict:
    d = dict(spec=spec)
    d.update(quant_tensors(spec))
    d.update(float_tensors(spec))
    return d


class DeviceLayer:
    """A LayerSpec materialised on the GPU behind the C ABI."""

    def __init__(self, ctx, spec: LayerSpec, host: dict | None = None):
        import moe_rocm as M

        self.spec, self.ctx = spec, ctx
        H, I, E, t = spec.hidden, spec.inter, spec.n_experts, spec.ggml_type
        self._bufs = []

        def quant(name, tensor_id, ggml_type, n_exp, out_f, in_f):
            nb = n_exp * _n_blocks(ggml_type, out_f, in_f)
            nbytes = nb * S.block_bytes(ggml_type)
            buf = ctx.alloc(nbytes + 64)
            if host is not None:
                buf.upload(host[name])
            else:
                ctx.synth_blocks(ggml_type, buf, nb, spec.seed(tensor_id))
            self._bufs.append(buf)
            return M.ExpertPack.wrap(ctx, ggml_type, buf, nbytes, n_exp, out_f, in_f)

        self.gate = quant("gate", S.T_GATE, t, E, I, H)
        self.up = quant("up", S.T_UP, t, E, I, H)
        self.down = quant("down", S.T_DOWN, t, E, H, I)
        if spec.sh_inter:
            st, Is = spec.sh_type, spec.sh_inter
            self.sh_gate = quant("sh_gate", S.T_SH_GATE, st, 1, Is, H)
            self.sh_up = quant("sh_up", S.T_SH_UP, st, 1, Is, H)
            self.sh_down = quant("sh_down", S.T_SH_DOWN, st, 1, H, Is)
        else:
            self.sh_gate = self.sh_up = self.sh_down = None
        ft = float_tensors(spec) if host is None else {k: host[k] for k in
                                                        ("router_w", "router_b", "gate_b", "up_b", "down_b", "sh_gate_inp")}
        self.f = {k: (ctx.to_device(v) if v is not None else None) for k, v in ft.items()}
        self.layer = M.MoeLayer(
            ctx, self.gate, self.up, self.down, router_w=self.f["router_w"], router_b=self.f["router_b"],
            gate_bias=self.f["gate_b"], up_bias=self.f["up_b"], down_bias=self.f["down_b"],
            top_k=spec.top_k, route_flags=spec.route_flags, act=spec.act, alpha=spec.alpha,
            limit=spec.limit, sh_gate=self.sh_gate, sh_up=self.sh_up, sh_down=self.sh_down,
            sh_gate_inp=self.f["sh_gate_inp"])

    def download_quant(self) -> dict:
        """The device-resident quantized tensors as numpy (for the oracle)."""
        out = {}
        for name in ("gate", "up", "down", "sh_gate", "sh_up", "sh_down"):
            pack = getattr(self, name)
            if pack is None:
                out[name] = None
                continue
            i = ["gate", "up", "down", "sh_gate", "sh_up", "sh_down"].index(name)
            buf = self._bufs[i]
            n = pack.n_experts * S.matrix_bytes(pack.type, pack.out_features, pack.in_features)
            out[name] = buf.download(np.uint8, n)
        return out

    def close(self):
        self.layer.close()
        for p in (self.gate, self.up, self.down, self.sh_gate, self.sh_up, self.sh_down):
            if p is not None:
                p.close()
        for b in self._bufs:
            b.free()
        for b in self.f.values():
            if b is not None:
                b.free()



def norm_weights(n_layers: int, hidden: int) -> np.ndarray:
    """Synthetic post-attention RMSNorm weights, one vector per layer: 1 + 0.1 N(0,1)."""
    rng = np.random.default_rng(20261201)
    return (1.0 + 0.1 * rng.standard_normal((n_layers, hidden))).astype(np.float32)


class DecodeStack:
    """The batch-1 decode pipeline the benchmark times: the layers of a stack on the GPU,
    each linked to the one that runs after it (mr_layer_set_next; the last layer to the
    first, where the next token starts), the inputs x[token][layer] resident in HBM, and
    one HIP graph per token holding that token's layer launches in order. Layer l of
    token t reads x[t][l] and writes y[l] (mr_moe_forward), or with residual=True writes
    y[l] = x[t][l] + moe(rms_norm(x[t][l])) (mr_moe_forward_residual)."""

    def __init__(self, ctx, specs, *, residual: bool = False, prefetch_hint: bool = True):
        self.ctx, self.specs, self.residual = ctx, list(specs), residual
        self.layers = [DeviceLayer(ctx, s) for s in self.specs]
        for dl in self.layers:
            dl.layer.reserve(1)
        n = len(self.layers)
        if prefetch_hint:
            for li, dl in enumerate(self.layers):
                dl.layer.set_next(self.layers[(li + 1) % n].layer)
        self.H = self.specs[0].hidden
        self.eps = 1e-5
        self.norm_w = norm_weights(n, self.H) if residual else None
        self.d_nw = ctx.to_device(self.norm_w) if residual else None
        if residual and prefetch_hint:  # each layer's norm weights, read ahead by the layer before
            for li, dl in enumerate(self.layers):
                dl.layer.set_norm(self.d_nw.ptr + li * self.H * 4)
        self.d_x = self.d_y = None
        self.graphs: list = []

    @property
    def n_layers(self) -> int:
        return len(self.layers)

    def inputs(self, n_tokens: int, first_token: int = 0) -> np.ndarray:
        """x[token][layer] ~ N(0,1), one stream per (layer, token)."""
        xs = np.empty((n_tokens, self.n_layers, self.H), dtype=np.float32)
        for li, s in enumerate(self.specs):
            xs[:, li, :] = x_tokens(s, n_tokens, first_token)
        return xs

    def load(self, xs: np.ndarray) -> None:
        """Uploads the inputs and clears the outputs y[layer]."""
        for b in (self.d_x, self.d_y):
            if b is not None:
                b.free()
        self.n_tokens = xs.shape[0]
        self.d_x = self.ctx.to_device(np.ascontiguousarray(xs, dtype=np.float32))
        self.d_y = self.ctx.zeros((self.n_layers, self.H))
        self.ctx.sync()

    def x_ptr(self, t: int, li: int) -> int:
        return self.d_x.ptr + ((t * self.n_layers + li) * self.H) * 4

    def y_ptr(self, li: int) -> int:
        return self.d_y.ptr + li * self.H * 4

    def enqueue_token(self, t: int) -> None:
        for li, dl in enumerate(self.layers):
            if self.residual:
                dl.layer.forward_residual(self.x_ptr(t, li), self.d_nw.ptr + li * self.H * 4, self.eps,
                                          self.y_ptr(li))
            else:
                dl.layer.forward(self.x_ptr(t, li), self.y_ptr(li))

    def capture(self) -> None:
        """One graph per loaded token."""
        self.close_graphs()
        for t in range(self.n_tokens):
            self.ctx.graph_begin()
            self.enqueue_token(t)
            self.graphs.append(self.ctx.graph_end())

    def run(self, t: int) -> None:
        if self.graphs:
            self.graphs[t].launch()
        else:
            self.enqueue_token(t)

    def outputs(self) -> np.ndarray:
        return self.d_y.download(np.float32).reshape(self.n_layers, self.H)

    def close_graphs(self) -> None:
        for g in self.graphs:
            g.close()
        self.graphs = []

    def close(self) -> None:
        self.close_graphs()
        for b in (self.d_x, self.d_y, self.d_nw):
            if b is not None:
                b.free()
        for dl in self.layers:
            dl.close()


class ChainStack(DecodeStack):
    """Decode with the hidden state carried from layer to layer: token t starts from h[t] and
    every layer applies h <- h + moe_l(rms_norm(h, norm_w[l])) in place with one
    mr_moe_forward_residual (layer.rs:462-473 per layer), so each layer reads what the
    previous one wrote and the layer order is enforced by the data. Layers are linked in a
    ring as in DecodeStack; one HIP graph per token."""

    def __init__(self, ctx, specs, *, prefetch_hint: bool = True):
        super().__init__(ctx, specs, residual=True, prefetch_hint=prefetch_hint)

    def inputs(self, n_tokens: int, first_token: int = 0) -> np.ndarray:
        """h[token] ~ N(0,1) (the first layer's input stream)."""
        return x_tokens(self.specs[0], n_tokens, first_token)

    def load(self, xs: np.ndarray) -> None:
        """Uploads h[token] into the buffers the chain updates in place (kept: h0)."""
        for b in (self.d_x, self.d_y):
            if b is not None:
                b.free()
        self.h0 = np.ascontiguousarray(xs, dtype=np.float32)
        self.n_tokens = self.h0.shape[0]
        self.d_x = self.ctx.to_device(self.h0)
        self.d_y = None
        self.ctx.sync()

    def h_ptr(self, t: int) -> int:
        return self.d_x.ptr + t * self.H * 4

    def enqueue_token(self, t: int) -> None:
        h = self.h_ptr(t)
        for li, dl in enumerate(self.layers):
            dl.layer.forward_residual(h, self.d_nw.ptr + li * self.H * 4, self.eps, h)

    def outputs(self) -> np.ndarray:
        """h[token] after the whole stack."""
        return self.d_x.download(np.float32).reshape(self.n_tokens, self.H)
