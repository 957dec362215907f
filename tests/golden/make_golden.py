#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/.

Two kinds of fixture are written:

* reference_kats.json: the known-answer values that the reference's own unit
  tests hold for this path, as data with the file:line each comes from
  (moe-stream-core/src/gguf/dequant.rs:808-837, ops/activation.rs:67-81,
  model/train.rs:1151-1184).
* layer_<name>.npz: small MoE layers with every input stored explicitly
  (native GGUF block bytes, router, biases, shared expert, x) and the expected
  outputs computed by the independent float64 numpy restatement in
  tests/npref.py: router logits, top-k indices and weights, the layer output y,
  and the bit patterns of the first rows of expert 0's dequantized gate matrix.

The fixtures are checked in; this script regenerates them byte-identically
(seeded counter-based generator). Run it from anywhere:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "moe-stream_amd"))
sys.path.insert(0, str(ROOT / "tests"))

from moe_rocm import synth as S  # noqa: E402
from moe_rocm import workloads as W  # noqa: E402

import npref  # noqa: E402

# Layers small enough to store; shapes cover both routing modes, both block
# formats, expert biases and the sigmoid-gated shared expert.
GOLDEN_SPECS = {
    # GPT-OSS semantics: raw-logit top-k then softmax over k, OAI SwiGLU, biases
    "mxfp4_oai": W.LayerSpec(901, 0, W.GGML_MXFP4, 64, 96, 6, 2, W.ROUTE_SOFTMAX_AFTER_TOPK,
                             W.ACT_SWIGLU_OAI, True, True),
    # Qwen semantics: softmax over all experts, top-k, renormalised, SiLU
    "q4k_qwen": W.LayerSpec(902, 0, W.GGML_Q4_K, 256, 256, 3, 2, W.ROUTE_NORM_TOPK,
                            W.ACT_SILU, False, False),
    # Coder-Next semantics: + always-on shared expert with sigmoid gate
    "q4k_shared": W.LayerSpec(903, 0, W.GGML_Q4_K, 256, 256, 2, 2, W.ROUTE_NORM_TOPK,
                              W.ACT_SILU, False, False, sh_inter=256),
}
N_TOKENS = 3
DEQUANT_ROWS = 8  # rows of expert 0's gate matrix stored as dequantized bit patterns

SPEC_FIELDS = ("config", "layer", "ggml_type", "hidden", "inter", "n_experts", "top_k",
               "route_flags", "act", "expert_bias", "router_bias", "sh_inter", "sh_type")


def reference_kats() -> dict:
    q4k = np.zeros(144, dtype=np.uint8)
    q4k[0:2] = (0x00, 0x3C)   # d = 1.0
    q4k[4:8] = 1              # scales[0..4] = 1 (6-bit scales of sub-blocks 0..3)
    return {
        "fp16_to_f32": {"source": "moe-stream-core/src/gguf/dequant.rs:808-816",
                        "cases": [[0x3C00, 1.0], [0x0000, 0.0], [0xBC00, -1.0]]},
        "q4k_single_block": {"source": "moe-stream-core/src/gguf/dequant.rs:818-837",
                             "block_hex": q4k.tobytes().hex(), "index": 0, "expected": 0.0},
        "silu_and_mul": {"source": "moe-stream-core/src/ops/activation.rs:67-81",
                         "gate": [1.0, -1.0, 2.0, 0.0], "up": [1.0, 1.0, 1.0, 1.0],
                         "checks": [[0, 0.7311, 0.01], [1, -0.2689, 0.01], [3, 0.0, 0.001]]},
        "swiglu_oai": {"source": "moe-stream-core/src/model/train.rs:1151-1184",
                       "gate": [1.0, -1.0, 5.0, 10.0], "up": [0.5, -0.5, 2.0, 3.0],
                       "alpha": 1.702, "limit": 7.0, "checks": [[3, 28.0, 0.5]]},
    }


def layer_fixture(spec: W.LayerSpec) -> dict:
    host = W.host_layer(spec)
    x = W.x_tokens(spec, N_TOKENS)
    y, idx, w, logits = npref.moe_forward(host, x)
    nb = S.matrix_bytes(spec.ggml_type, DEQUANT_ROWS, spec.hidden)
    deq = npref.dequant(spec.ggml_type, host["gate"][:nb], DEQUANT_ROWS * spec.hidden).astype(np.float32)
    out = {"spec": np.array([int(getattr(spec, f)) for f in SPEC_FIELDS], dtype=np.int64),
           "alpha_limit": np.array([spec.alpha, spec.limit], dtype=np.float32),
           "x": x.astype(np.float32), "y": y.astype(np.float64), "idx": idx.astype(np.int32),
           "w": np.asarray(w, dtype=np.float64), "logits": logits.astype(np.float64),
           "gate0_dequant_bits": deq.view(np.uint32)}
    for k in ("gate", "up", "down", "sh_gate", "sh_up", "sh_down", "router_w", "router_b",
              "gate_b", "up_b", "down_b", "sh_gate_inp"):
        if host[k] is not None:
            out[k] = host[k]
    return out


def load_layer(path: Path):
    """Read a layer fixture back into (host dict as workloads.host_layer builds it, npz)."""
    z = np.load(path, allow_pickle=False)
    vals = dict(zip(SPEC_FIELDS, (int(v) for v in z["spec"])))
    for b in ("expert_bias", "router_bias"):
        vals[b] = bool(vals[b])
    al = z["alpha_limit"]
    spec = W.LayerSpec(**vals, alpha=float(al[0]), limit=float(al[1]))
    host = {"spec": spec}
    for k in ("gate", "up", "down", "sh_gate", "sh_up", "sh_down", "router_w", "router_b",
              "gate_b", "up_b", "down_b", "sh_gate_inp"):
        host[k] = z[k] if k in z.files else None
    return host, z


def main() -> None:
    (HERE / "reference_kats.json").write_text(json.dumps(reference_kats(), indent=1) + "\n")
    for name, spec in GOLDEN_SPECS.items():
        np.savez(HERE / f"layer_{name}.npz", **layer_fixture(spec))
        print(f"wrote layer_{name}.npz")


if __name__ == "__main__":
    main()
