"""The reference's activation dumps, read and checked against this library.

moe-stream writes them when DUMP_ACTIVATIONS=<dir> is set (model/layer.rs:1036-1083), appending
on every forward call:
  meta.json              {"hidden_dim": H, "top_k": k, "n_experts": E, "n_layers": L}
  layer_LL_hidden.bin    f32[H] per token, little-endian: the MoE input of layer LL
                         (the hidden state after the post-attention norm)
  layer_LL_routing.bin   per token: u32[k] expert indices, then f32[k] routing weights (LE)
so a dump taken from a real model is a golden record of routing on real activations. This module
reads it and replays the dumped inputs through a layer built from the same model file
(mr_gguf_layer_create), comparing the selected experts exactly and the weights to 1e-5.

    python -m moe_rocm.dump --gguf model.gguf --dump <dir> [--layers 0,1,...]

prints one JSON report and exits 1 when a token's routing differs. A token whose k-th and
(k+1)-th logits (this library's, f32) lie within 1e-5 of the largest is tie-ambiguous: the two
sides may rank its experts differently within rounding, and it is reported, not counted.
"""
from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass
from pathlib import Path

import numpy as np


@dataclass
class DumpLayer:
    layer: int
    hidden: np.ndarray  # [N, H] f32
    idx: np.ndarray     # [N, k] u32, the reference's rank order
    w: np.ndarray       # [N, k] f32

    @property
    def n_tokens(self) -> int:
        return self.hidden.shape[0]


def read_meta(d) -> dict:
    meta = json.loads((Path(d) / "meta.json").read_text())
    for key in ("hidden_dim", "top_k", "n_experts", "n_layers"):
        if not isinstance(meta.get(key), int) or meta[key] <= 0:
            raise ValueError(f"meta.json: {key} missing or not a positive integer")
    return meta


def layers_present(d) -> list[int]:
    out = []
    for p in sorted(Path(d).glob("layer_*_hidden.bin")):
        s = p.name[len("layer_"):-len("_hidden.bin")]
        if s.isdigit() and (Path(d) / f"layer_{s}_routing.bin").exists():
            out.append(int(s))
    return sorted(out)


def read_layer(d, layer: int, meta: dict | None = None) -> DumpLayer:
    meta = meta or read_meta(d)
    H, k = meta["hidden_dim"], meta["top_k"]
    hb = (Path(d) / f"layer_{layer:02d}_hidden.bin").read_bytes()
    rb = (Path(d) / f"layer_{layer:02d}_routing.bin").read_bytes()
    if len(hb) % (4 * H):
        raise ValueError(f"layer {layer}: hidden file of {len(hb)} bytes is not a whole number of f32[{H}] rows")
    if len(rb) % (8 * k):
        raise ValueError(f"layer {layer}: routing file of {len(rb)} bytes is not a whole number of "
                         f"(u32[{k}], f32[{k}]) records")
    n = len(hb) // (4 * H)
    if len(rb) // (8 * k) != n:
        raise ValueError(f"layer {layer}: {n} hidden rows but {len(rb) // (8 * k)} routing records")
    hidden = np.frombuffer(hb, dtype="<f4").reshape(n, H).astype(np.float32)
    rec = np.frombuffer(rb, dtype="<u4").reshape(n, 2 * k)
    return DumpLayer(layer, hidden, rec[:, :k].astype(np.uint32), rec[:, k:].copy().view(np.float32))


def check_routing(ctx, layer, dump: DumpLayer, chunk: int = 4096, tie_rel: float = 1e-5) -> dict:
    """Routing of the dumped inputs through `layer` (mr_router_topk) against the dump."""
    H, k = dump.hidden.shape[1], dump.idx.shape[1]
    E = layer.n_experts
    if layer.hidden != H or layer.top_k != k:
        raise ValueError(f"layer {dump.layer}: model has hidden {layer.hidden}, top_k {layer.top_k}; "
                         f"dump has {H}, {k}")
    match, ambiguous, mismatch, max_werr = 0, [], [], 0.0
    for t0 in range(0, dump.n_tokens, chunk):
        x = dump.hidden[t0:t0 + chunk]
        T = x.shape[0]
        dx, di, dw, dl = ctx.to_device(x), ctx.alloc(T * k * 4), ctx.alloc(T * k * 4), ctx.alloc(T * E * 4)
        try:
            layer.router_topk(dx, T, di, dw, dl)
            gi = di.download(np.int32).reshape(T, k)
            gw = dw.download(np.float32).reshape(T, k)
            lg = dl.download(np.float32).reshape(T, E)
        finally:
            for b in (dx, di, dw, dl):
                b.free()
        for r in range(T):
            t = t0 + r
            s = np.sort(lg[r])[::-1]
            if k < E and s[k - 1] - s[k] <= tie_rel * np.abs(lg[r]).max():
                ambiguous.append(t)
                continue
            ref_i, ref_w = dump.idx[t].astype(np.int64), dump.w[t]
            if set(ref_i.tolist()) != set(gi[r].astype(np.int64).tolist()):
                mismatch.append({"token": t, "ref": ref_i.tolist(), "got": gi[r].tolist()})
                continue
            order_ref, order_got = np.argsort(ref_i), np.argsort(gi[r])
            werr = float(np.abs(ref_w[order_ref].astype(np.float64) - gw[r][order_got]).max())
            if werr > 1e-5 * max(1.0, float(np.abs(ref_w).max())) + 1e-6:
                mismatch.append({"token": t, "ref_w": ref_w.tolist(), "got_w": gw[r].tolist()})
                continue
            max_werr = max(max_werr, werr)
            match += 1
    return {"layer": dump.layer, "tokens": dump.n_tokens, "match": match, "tie_ambiguous": len(ambiguous),
            "mismatch": len(mismatch), "first_mismatches": mismatch[:20], "max_weight_err": max_werr}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gguf", required=True, help="the model file the dump was taken from")
    ap.add_argument("--dump", required=True, help="the DUMP_ACTIVATIONS directory")
    ap.add_argument("--layers", default="", help="comma-separated layer indices (default: every dumped layer)")
    ap.add_argument("--device", type=int, default=0)
    a = ap.parse_args(argv)
    from . import Context, GgufFile

    meta = read_meta(a.dump)
    layers = [int(s) for s in a.layers.split(",") if s] if a.layers else layers_present(a.dump)
    ctx = Context(a.device)
    reports, bad = [], 0
    with GgufFile(a.gguf) as g:
        for li in layers:
            layer = g.layer(ctx, li, top_k=meta["top_k"])
            try:
                rep = check_routing(ctx, layer, read_layer(a.dump, li, meta))
            finally:
                layer.close()
            bad += rep["mismatch"]
            reports.append(rep)
    ctx.close()
    print(json.dumps({"dump": str(a.dump), "gguf": str(a.gguf), "meta": meta, "layers": reports}))
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
