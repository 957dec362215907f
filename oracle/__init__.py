"""ctypes wrapper of the CPU oracle (libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py -- never by the product package.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "libmoe_oracle.so"

GGML_Q4_K, GGML_MXFP4 = 12, 39


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    return C.CDLL(str(LIB_PATH))


_lib = _load()
_vp, _sz, _u32, _f32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_float


class OrLayer(C.Structure):
    _fields_ = [
        ("type", C.c_int), ("hidden", _u32), ("inter", _u32), ("n_experts", _u32), ("top_k", _u32),
        ("gate", _vp), ("up", _vp), ("down", _vp),
        ("gate_b", _vp), ("up_b", _vp), ("down_b", _vp),
        ("router_w", _vp), ("router_b", _vp), ("dummy_mask", _vp),
        ("softmax_weight", C.c_int), ("norm_topk", C.c_int), ("act_oai", C.c_int),
        ("alpha", _f32), ("limit", _f32),
        ("sh_type", C.c_int), ("sh_inter", _u32),
        ("sh_gate", _vp), ("sh_up", _vp), ("sh_down", _vp), ("sh_gate_inp", _vp),
    ]


_SIGS = {
    "or_fp16_to_f32": (_f32, [C.c_uint16]),
    "or_e8m0_to_f32_half": (_f32, [C.c_uint8]),
    "or_dequant_mxfp4": (None, [_vp, _sz, _vp]),
    "or_mxfp4_matvec": (None, [_vp, _vp, _sz, _sz, _vp, C.c_int]),
    "or_mxfp4_matmul": (None, [_vp, _vp, _sz, _sz, _sz, _vp, C.c_int]),
    "or_get_scale_min_k4": (None, [C.c_int, _vp, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]),
    "or_dequant_q4k": (None, [_vp, _sz, _vp]),
    "or_f32_matvec": (None, [_vp, _vp, _sz, _sz, _vp]),
    "or_topk_routing": (None, [_vp, _sz, _sz, _sz, C.c_int, C.c_int, _vp, _vp]),
    "or_swiglu_oai1": (_f32, [_f32, _f32, _f32, _f32]),
    "or_silu_mul1": (_f32, [_f32, _f32]),
    "or_sigmoid1": (_f32, [_f32]),
    "or_rms_norm": (None, [_vp, _vp, _sz, _sz, _f32, _vp]),
    "or_matrix_bytes": (C.c_uint64, [C.c_int, C.c_uint64, C.c_uint64]),
    "or_moe_forward": (C.c_int, [C.POINTER(OrLayer), _vp, _sz, _vp, _vp, _vp, _vp, C.c_int]),
    "or_moe_experts": (C.c_int, [C.POINTER(OrLayer), _vp, _sz, _vp, _vp, _vp, C.c_int]),
}
for _n, (_r, _a) in _SIGS.items():
    _f = getattr(_lib, _n)
    _f.restype, _f.argtypes = _r, _a


def _p(a):
    return None if a is None else a.ctypes.data


def fp16_to_f32(h: int) -> float:
    return float(_lib.or_fp16_to_f32(h))


def e8m0_to_f32_half(e: int) -> float:
    return float(_lib.or_e8m0_to_f32_half(e))


def dequant_mxfp4(blocks: np.ndarray, n_elements: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n_elements, dtype=np.float32)
    _lib.or_dequant_mxfp4(blocks.ctypes.data, n_elements, out.ctypes.data)
    return out


def dequant_q4k(blocks: np.ndarray, n_elements: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n_elements, dtype=np.float32)
    _lib.or_dequant_q4k(blocks.ctypes.data, n_elements, out.ctypes.data)
    return out


def dequant(ggml_type: int, blocks: np.ndarray, n_elements: int) -> np.ndarray:
    return dequant_mxfp4(blocks, n_elements) if ggml_type == GGML_MXFP4 else dequant_q4k(blocks, n_elements)


def get_scale_min_k4(j: int, q: np.ndarray) -> tuple[int, int]:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sc, m = C.c_uint8(), C.c_uint8()
    _lib.or_get_scale_min_k4(j, q.ctypes.data, C.byref(sc), C.byref(m))
    return sc.value, m.value


def mxfp4_matvec(w: np.ndarray, x: np.ndarray, out_f: int, in_f: int, n_threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(out_f, dtype=np.float32)
    _lib.or_mxfp4_matvec(w.ctypes.data, x.ctypes.data, out_f, in_f, y.ctypes.data, n_threads)
    return y


def mxfp4_matmul(w: np.ndarray, x: np.ndarray, out_f: int, in_f: int, n_threads: int = 1) -> np.ndarray:
    """x [T, in_f] -> y [T, out_f] (or_mxfp4_matmul, dequant.rs:705-721)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_f)
    y = np.empty((x.shape[0], out_f), dtype=np.float32)
    _lib.or_mxfp4_matmul(w.ctypes.data, x.ctypes.data, x.shape[0], out_f, in_f, y.ctypes.data, n_threads)
    return y


def f32_matvec(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[0], dtype=np.float32)
    _lib.or_f32_matvec(w.ctypes.data, x.ctypes.data, w.shape[0], w.shape[1], y.ctypes.data)
    return y


def topk_routing(logits: np.ndarray, k: int, normalize: bool, softmax_weight: bool):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), dtype=np.uint32)
    w = np.empty((T, k), dtype=np.float32)
    _lib.or_topk_routing(logits.ctypes.data, T, E, k, int(normalize), int(softmax_weight),
                         idx.ctypes.data, w.ctypes.data)
    return idx, w


def swiglu_oai(g: float, u: float, alpha: float = 1.702, limit: float = 7.0) -> float:
    return float(_lib.or_swiglu_oai1(g, u, alpha, limit))


def silu_mul(g: float, u: float) -> float:
    return float(_lib.or_silu_mul1(g, u))


def sigmoid(x: float) -> float:
    return float(_lib.or_sigmoid1(x))


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """ops/norm.rs:32-36 over the last axis (or_rms_norm)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    width = x.shape[-1]
    out = np.empty_like(x)
    _lib.or_rms_norm(x.ctypes.data, w.ctypes.data, x.size // width, width, eps, out.ctypes.data)
    return out


class Layer:
    """Host-side copy of one MoE layer for the oracle (numpy arrays)."""

    def __init__(self, *, ggml_type, hidden, inter, n_experts, top_k, gate, up, down, router_w,
                 router_b=None, dummy_mask=None, gate_b=None, up_b=None, down_b=None,
                 softmax_weight=False, norm_topk=True, act_oai=False, alpha=1.702, limit=7.0,
                 sh_type=GGML_Q4_K, sh_inter=0, sh_gate=None, sh_up=None, sh_down=None,
                 sh_gate_inp=None):
        def u8(a):
            return None if a is None else np.ascontiguousarray(a, dtype=np.uint8)

        def f32(a):
            return None if a is None else np.ascontiguousarray(a, dtype=np.float32)

        self.arrays = dict(gate=u8(gate), up=u8(up), down=u8(down), router_w=f32(router_w),
                           router_b=f32(router_b), dummy_mask=f32(dummy_mask), gate_b=f32(gate_b),
                           up_b=f32(up_b), down_b=f32(down_b), sh_gate=u8(sh_gate), sh_up=u8(sh_up),
                           sh_down=u8(sh_down), sh_gate_inp=f32(sh_gate_inp))
        a = self.arrays
        self.s = OrLayer(
            type=ggml_type, hidden=hidden, inter=inter, n_experts=n_experts, top_k=top_k,
            gate=_p(a["gate"]), up=_p(a["up"]), down=_p(a["down"]),
            gate_b=_p(a["gate_b"]), up_b=_p(a["up_b"]), down_b=_p(a["down_b"]),
            router_w=_p(a["router_w"]), router_b=_p(a["router_b"]), dummy_mask=_p(a["dummy_mask"]),
            softmax_weight=int(softmax_weight), norm_topk=int(norm_topk), act_oai=int(act_oai),
            alpha=alpha, limit=limit, sh_type=sh_type, sh_inter=sh_inter,
            sh_gate=_p(a["sh_gate"]), sh_up=_p(a["sh_up"]), sh_down=_p(a["sh_down"]),
            sh_gate_inp=_p(a["sh_gate_inp"]))
        self.hidden, self.inter, self.n_experts, self.top_k = hidden, inter, n_experts, top_k

    def forward(self, x: np.ndarray, n_threads: int = 1):
        """Returns (y [T,H], idx [T,k], w [T,k], logits [T,E])."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.hidden)
        T = x.shape[0]
        y = np.empty((T, self.hidden), dtype=np.float32)
        idx = np.empty((T, self.top_k), dtype=np.uint32)
        w = np.empty((T, self.top_k), dtype=np.float32)
        lg = np.empty((T, self.n_experts), dtype=np.float32)
        rc = _lib.or_moe_forward(C.byref(self.s), x.ctypes.data, T, y.ctypes.data, idx.ctypes.data,
                                 w.ctypes.data, lg.ctypes.data, n_threads)
        if rc != 0:
            raise MemoryError("oracle allocation failed")
        return y, idx, w, lg

    def forward_residual(self, h: np.ndarray, norm_w: np.ndarray, eps: float, n_threads: int = 1):
        """The MoE block of a decoder layer (layer.rs:462-473): residual + moe(rms_norm(h)).
        Returns (h_out, idx, w, logits)."""
        h = np.ascontiguousarray(h, dtype=np.float32).reshape(-1, self.hidden)
        y, idx, w, lg = self.forward(rms_norm(h, norm_w, eps), n_threads)
        return h + y, idx, w, lg

    def experts(self, x: np.ndarray, idx: np.ndarray, w: np.ndarray, n_threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.hidden)
        T = x.shape[0]
        idx = np.ascontiguousarray(idx, dtype=np.uint32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        y = np.zeros((T, self.hidden), dtype=np.float32)
        rc = _lib.or_moe_experts(C.byref(self.s), x.ctypes.data, T, idx.ctypes.data, w.ctypes.data,
                                 y.ctypes.data, n_threads)
        if rc != 0:
            raise MemoryError("oracle allocation failed")
        return y


def layer_from_host(host: dict) -> Layer:
    """Oracle view of a synthetic layer built by moe_rocm.workloads.host_layer."""
    spec = host["spec"]
    return Layer(
        ggml_type=spec.ggml_type, hidden=spec.hidden, inter=spec.inter, n_experts=spec.n_experts,
        top_k=spec.top_k, gate=host["gate"], up=host["up"], down=host["down"],
        router_w=host["router_w"], router_b=host["router_b"], gate_b=host["gate_b"],
        up_b=host["up_b"], down_b=host["down_b"],
        softmax_weight=bool(spec.route_flags & 1), norm_topk=bool(spec.route_flags & 2),
        act_oai=spec.act == 1, alpha=spec.alpha, limit=spec.limit, sh_type=spec.sh_type,
        sh_inter=spec.sh_inter, sh_gate=host.get("sh_gate"), sh_up=host.get("sh_up"),
        sh_down=host.get("sh_down"), sh_gate_inp=host.get("sh_gate_inp"))
