"""Minimal GGUF v3 writer for the reader tests (test infrastructure).

Writes the container as the GGUF format describes it (all little-endian): magic
"GGUF", version, tensor count (u64), metadata count (u64); metadata entries (gguf
string key, u32 value type, value; arrays as element type u32 + count u64 +
elements); tensor infos (name, n_dims u32, dims u64 innermost first, ggml type u32,
offset u64 relative to the data section); padding to `alignment`; tensor data, each
tensor at an aligned offset.
"""
from __future__ import annotations

import struct

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def build(metadata: list[tuple[str, int, object]], tensors: list[tuple[str, int, tuple, bytes]],
          alignment: int = 32, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    """metadata: (key, type, value); tensors: (name, ggml_type, dims innermost first, data)."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, v in metadata:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offs, rel = [], 0
    for _, _, _, data in tensors:
        offs.append(rel)
        rel = (rel + len(data) + alignment - 1) // alignment * alignment
    for (name, gtype, dims, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, off)
    start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + bytes(start - len(head)))
    for (_, _, _, data), off in zip(tensors, offs):
        if len(out) < start + off:
            out += bytes(start + off - len(out))
        out += data
    return bytes(out)


def write(path, metadata, tensors, **kw) -> int:
    data = build(metadata, tensors, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return len(data)


def f32(a) -> bytes:
    return np.ascontiguousarray(a, dtype=np.float32).tobytes()


def moe_layer_tensors(spec, quant: dict, floats: dict, layer: int = 0, norm_w=None,
                      router_dtype: str = "f32") -> list:
    """The tensors of one MoE layer under the reference's names (layer.rs:806-837,
    1130-1135, 1898-1953): stacked experts [E, out, in] as GGUF dims [in, out, E]."""
    H, I, E = spec.hidden, spec.inter, spec.n_experts
    p = f"blk.{layer}."
    t = [(p + "ffn_gate_exps.weight", spec.ggml_type, (H, I, E), quant["gate"].tobytes()),
         (p + "ffn_up_exps.weight", spec.ggml_type, (H, I, E), quant["up"].tobytes()),
         (p + "ffn_down_exps.weight", spec.ggml_type, (I, H, E), quant["down"].tobytes())]
    rw = np.asarray(floats["router_w"], np.float32)
    if router_dtype == "f32":
        t.append((p + "ffn_gate_inp.weight", 0, (H, E), f32(rw)))
    elif router_dtype == "f16":
        t.append((p + "ffn_gate_inp.weight", 1, (H, E), rw.astype(np.float16).tobytes()))
    else:  # bf16: the upper half of each f32 (round toward zero)
        t.append((p + "ffn_gate_inp.weight", 30, (H, E), (rw.view(np.uint32) >> 16).astype(np.uint16).tobytes()))
    for key, name, dims in (("router_b", "ffn_gate_inp.bias", (E,)), ("gate_b", "ffn_gate_exps.bias", (I, E)),
                            ("up_b", "ffn_up_exps.bias", (I, E)), ("down_b", "ffn_down_exps.bias", (H, E))):
        if floats.get(key) is not None:
            t.append((p + name, 0, dims, f32(floats[key])))
    if spec.sh_inter:
        Ish = spec.sh_inter
        t += [(p + "ffn_gate_shexp.weight", spec.sh_type, (H, Ish), quant["sh_gate"].tobytes()),
              (p + "ffn_up_shexp.weight", spec.sh_type, (H, Ish), quant["sh_up"].tobytes()),
              (p + "ffn_down_shexp.weight", spec.sh_type, (Ish, H), quant["sh_down"].tobytes())]
        if floats.get("sh_gate_inp") is not None:
            t.append((p + "ffn_gate_inp_shexp.weight", 0, (H,), f32(floats["sh_gate_inp"])))
    if norm_w is not None:
        t.append((p + "post_attention_norm.weight", 0, (H,), f32(norm_w)))
    return t
