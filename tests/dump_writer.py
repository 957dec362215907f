"""Writes activation dumps in the reference's DUMP_ACTIVATIONS format (model/layer.rs:1036-1083):
meta.json written once as the reference formats it, then per forward call the layer's hidden rows
(f32 LE) appended to layer_LL_hidden.bin and per token u32[k] indices + f32[k] weights (LE)
appended to layer_LL_routing.bin. Test data, not product code."""
from pathlib import Path

import numpy as np


def write_meta(d, hidden_dim: int, top_k: int, n_experts: int, n_layers: int) -> None:
    p = Path(d) / "meta.json"
    if not p.exists():
        p.write_text(f'{{"hidden_dim":{hidden_dim},"top_k":{top_k},"n_experts":{n_experts},"n_layers":{n_layers}}}')


def append(d, layer: int, hidden: np.ndarray, idx: np.ndarray, w: np.ndarray) -> None:
    d = Path(d)
    with open(d / f"layer_{layer:02d}_hidden.bin", "ab") as f:
        f.write(np.ascontiguousarray(hidden, dtype="<f4").tobytes())
    with open(d / f"layer_{layer:02d}_routing.bin", "ab") as f:
        for t in range(idx.shape[0]):
            f.write(np.ascontiguousarray(idx[t], dtype="<u4").tobytes())
            f.write(np.ascontiguousarray(w[t], dtype="<f4").tobytes())
