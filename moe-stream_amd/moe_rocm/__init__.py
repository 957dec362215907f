"""moe_rocm -- Python binding of the MI355X MoE expert-FFN engine (libmoe_rocm.so).

A thin ctypes layer over the C ABI in include/moe_rocm.h. There is no fallback:
if the HIP library is missing, importing this package raises. Device buffers
are plain device addresses owned by DeviceBuffer objects; numpy arrays are
copied in and out explicitly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

from . import synth  # noqa: F401  (re-exported)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MOE_ROCM_LIB", PKG_DIR / "libmoe_rocm.so"))

MR_OK = 0
MR_E_INVAL, MR_E_NOMEM, MR_E_NODEV, MR_E_LAUNCH, MR_E_UNSUPPORTED = -1, -2, -3, -4, -5
GGML_Q4_K, GGML_MXFP4 = 12, 39
ROUTE_SOFTMAX_AFTER_TOPK, ROUTE_NORM_TOPK = 1, 2
ACT_SILU, ACT_SWIGLU_OAI = 0, 1
DEVICE_NONE = -1
OPT_DECODE_KERNEL = 1
OPT_PROFILE = 2
OPT_WAIT_LIMIT_US = 3
DECODE_AUTO, DECODE_VALU, DECODE_FUSED = 0, 1, 2

if not LIB_PATH.exists():
    raise ImportError(
        f"libmoe_rocm.so not found at {LIB_PATH}: build it with "
        "`python -m moe_rocm.build` (hipcc, gfx950) -- there is no CPU fallback")

_lib = C.CDLL(str(LIB_PATH))

_vp, _u32, _u64, _i32, _f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_float


class GgufTensor(C.Structure):
    _fields_ = [("ggml_type", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("data_offset", C.c_uint64), ("nbytes", C.c_uint64)]


class GgufLayerOpts(C.Structure):
    _fields_ = [("top_k", C.c_uint32), ("route_flags", C.c_int32), ("act", C.c_int32),
                ("alpha", C.c_float), ("limit", C.c_float)]


class LayerDesc(C.Structure):
    _fields_ = [
        ("gate", _vp), ("up", _vp), ("down", _vp),
        ("gate_bias", _vp), ("up_bias", _vp), ("down_bias", _vp),
        ("router_w", _vp), ("router_b", _vp), ("dummy_mask", _vp),
        ("sh_gate", _vp), ("sh_up", _vp), ("sh_down", _vp), ("sh_gate_inp", _vp),
        ("top_k", _u32), ("route_flags", _u32), ("act", _u32),
        ("alpha", _f32), ("limit", _f32),
    ]


_SIGS = {
    "mr_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "mr_ctx_destroy": (None, [_vp]),
    "mr_last_error": (C.c_char_p, [_vp]),
    "mr_status_string": (C.c_char_p, [C.c_int]),
    "mr_ctx_device": (C.c_int, [_vp]),
    "mr_ctx_set_stream": (C.c_int, [_vp, _vp]),
    "mr_ctx_stream": (_vp, [_vp]),
    "mr_ctx_set_option": (C.c_int, [_vp, C.c_int, C.c_int]),
    "mr_sync": (C.c_int, [_vp]),
    "mr_dev_alloc": (C.c_int, [_vp, _u64, C.POINTER(_vp)]),
    "mr_dev_free": (C.c_int, [_vp, _vp]),
    "mr_upload": (C.c_int, [_vp, _vp, _vp, _u64]),
    "mr_download": (C.c_int, [_vp, _vp, _vp, _u64]),
    "mr_dev_zero": (C.c_int, [_vp, _vp, _u64]),
    "mr_pack_upload": (C.c_int, [_vp, C.c_int, _vp, _u64, _u32, _u32, _u32, _vp, C.POINTER(_vp)]),
    "mr_pack_wrap": (C.c_int, [_vp, C.c_int, _vp, _u64, _u32, _u32, _u32, _vp, C.POINTER(_vp)]),
    "mr_pack_destroy": (None, [_vp]),
    "mr_matrix_bytes": (_u64, [C.c_int, _u64, _u64]),
    "mr_dequant": (C.c_int, [_vp, _vp, _u32, _vp]),
    "mr_layer_create": (C.c_int, [_vp, C.POINTER(LayerDesc), C.POINTER(_vp)]),
    "mr_layer_destroy": (None, [_vp]),
    "mr_layer_set_next": (C.c_int, [_vp, _vp]),
    "mr_layer_set_norm": (C.c_int, [_vp, _vp]),
    "mr_layer_set_logits_out": (C.c_int, [_vp, _vp, C.c_uint32]),
    "mr_reserve": (C.c_int, [_vp, _vp, _u32]),
    "mr_router_topk": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "mr_topk": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp]),
    "mr_moe_experts": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "mr_moe_forward": (C.c_int, [_vp, _vp, _vp, _vp]),
    "mr_moe_forward_residual": (C.c_int, [_vp, _vp, _vp, _vp, _f32, _vp]),
    "mr_moe_forward_batched": (C.c_int, [_vp, _vp, _vp, _u32, _vp]),
    "mr_moe_forward_batched_residual": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _f32, _vp]),
    "mr_probe_read": (C.c_int, [_vp, _vp, _u64, _u32, _u32, _vp]),
    "mr_probe_empty": (C.c_int, [_vp, _u32]),
    "mr_probe_flags": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "mr_probe_tiles": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "mr_probe_touch": (C.c_int, [_vp, _vp, _u64, _u32, _vp]),
    "mr_moe_forward_batched_noalloc": (C.c_int, [_vp, _vp, _vp, _u32, _vp]),
    "mr_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "mr_gguf_close": (None, [_vp]),
    "mr_gguf_n_tensors": (_u64, [_vp]),
    "mr_gguf_tensor_name": (C.c_char_p, [_vp, _u64]),
    "mr_gguf_tensor_info": (C.c_int, [_vp, C.c_char_p, C.POINTER(GgufTensor)]),
    "mr_gguf_tensor_data": (C.c_int, [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(_u64)]),
    "mr_gguf_meta_u32": (C.c_int, [_vp, C.c_char_p, C.POINTER(_u32)]),
    "mr_gguf_meta_f32": (C.c_int, [_vp, C.c_char_p, C.POINTER(_f32)]),
    "mr_gguf_meta_str": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(_u64)]),
    "mr_gguf_meta_u32_array": (C.c_int, [_vp, C.c_char_p, _vp, _u64, C.POINTER(_u64)]),
    "mr_gguf_upload_experts": (C.c_int, [_vp, _vp, C.c_char_p, C.POINTER(_vp)]),
    "mr_gguf_layer_create": (C.c_int, [_vp, _vp, _u32, C.POINTER(GgufLayerOpts), C.POINTER(_vp),
                                       C.POINTER(_vp), C.POINTER(_f32)]),
    "mr_graph_begin": (C.c_int, [_vp]),
    "mr_graph_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "mr_graph_launch": (C.c_int, [_vp, _vp]),
    "mr_graph_destroy": (None, [_vp]),
    "mr_timer_start": (C.c_int, [_vp]),
    "mr_timer_stop": (C.c_int, [_vp, C.POINTER(_f32)]),
    "mr_synth_blocks": (C.c_int, [_vp, C.c_int, _vp, _u64, _u64]),
    "mr_profile_read": (C.c_int, [_vp, C.c_char_p, C.POINTER(_u64), C.POINTER(C.c_double)]),
    "mr_profile_reset": (C.c_int, [_vp]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

lib = _lib


class MoeRocmError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


def _ptr(obj) -> int | None:
    """Device address of a DeviceBuffer / int / None."""
    if obj is None:
        return None
    if isinstance(obj, DeviceBuffer):
        return obj.ptr
    if isinstance(obj, int):
        return obj
    raise TypeError(f"expected DeviceBuffer, int address or None, got {type(obj)}")


class Context:
    """One HIP device + one stream (mr_ctx)."""

    def __init__(self, device: int = 0):
        h = _vp()
        rc = _lib.mr_ctx_create(device, C.byref(h))
        if rc != MR_OK:
            raise MoeRocmError(rc, _lib.mr_last_error(None).decode())
        self.h = h.value
        self.device = device
        self._keep: list = []

    def check(self, rc: int) -> None:
        if rc != MR_OK:
            raise MoeRocmError(rc, _lib.mr_last_error(self.h).decode())

    @property
    def last_error(self) -> str:
        return _lib.mr_last_error(self.h).decode()

    def close(self) -> None:
        if getattr(self, "h", None):
            _lib.mr_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sync(self) -> None:
        self.check(_lib.mr_sync(self.h))

    def set_option(self, option: int, value: int) -> None:
        self.check(_lib.mr_ctx_set_option(self.h, option, value))

    # -- memory ---------------------------------------------------------------
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, max(arr.nbytes, 4))
        buf.upload(arr)
        return buf

    def zeros(self, shape, dtype=np.float32) -> "DeviceBuffer":
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        buf = DeviceBuffer(self, max(n, 4))
        self.check(_lib.mr_dev_zero(self.h, buf.ptr, (max(n, 4) + 3) // 4 * 4))
        return buf

    # -- timing ----------------------------------------------------------------
    def timer_start(self) -> None:
        self.check(_lib.mr_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = _f32()
        self.check(_lib.mr_timer_stop(self.h, C.byref(ms)))
        return float(ms.value)

    def profile_read(self, kernel: str) -> tuple[int, float]:
        n, ms = _u64(), C.c_double()
        self.check(_lib.mr_profile_read(self.h, kernel.encode(), C.byref(n), C.byref(ms)))
        return int(n.value), float(ms.value)

    def profile_reset(self) -> None:
        self.check(_lib.mr_profile_reset(self.h))

    # -- graphs ----------------------------------------------------------------
    def graph_begin(self) -> None:
        self.check(_lib.mr_graph_begin(self.h))

    def graph_end(self) -> "Graph":
        g = _vp()
        self.check(_lib.mr_graph_end(self.h, C.byref(g)))
        return Graph(self, g.value)

    def probe_read(self, src, nbytes: int, n_workgroups: int, sink, depth: int = 8) -> None:
        self.check(_lib.mr_probe_read(self.h, _ptr(src), nbytes, n_workgroups, depth, _ptr(sink)))

    def probe_tiles(self, src, row_bytes: int, n_tiles: int, n_workgroups: int, sink, depth: int = 2) -> None:
        self.check(_lib.mr_probe_tiles(self.h, _ptr(src), row_bytes, n_tiles, n_workgroups, depth, _ptr(sink)))

    def probe_touch(self, src, nbytes: int, stride: int, sink) -> None:
        self.check(_lib.mr_probe_touch(self.h, _ptr(src), nbytes, stride, _ptr(sink)))

    def probe_empty(self, n_workgroups: int) -> None:
        self.check(_lib.mr_probe_empty(self.h, n_workgroups))

    def probe_flags(self, words, wg_a: int, wg_b: int, n_round_trips: int, result) -> None:
        self.check(_lib.mr_probe_flags(self.h, _ptr(words), wg_a, wg_b, n_round_trips, _ptr(result)))

    def synth_blocks(self, ggml_type: int, dst: "DeviceBuffer", n_blocks: int, seed: int,
                     offset: int = 0) -> None:
        self.check(_lib.mr_synth_blocks(self.h, ggml_type, dst.ptr + offset, n_blocks,
                                        seed & 0xFFFFFFFFFFFFFFFF))


class Graph:
    def __init__(self, ctx: Context, h: int):
        self.ctx, self.h = ctx, h

    def launch(self) -> None:
        self.ctx.check(_lib.mr_graph_launch(self.ctx.h, self.h))

    def close(self) -> None:
        if self.h:
            _lib.mr_graph_destroy(self.h)
            self.h = None


class DeviceBuffer:
    def __init__(self, ctx: Context, nbytes: int):
        p = _vp()
        ctx.check(_lib.mr_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.ctx, self.ptr, self.nbytes = ctx, p.value, nbytes

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        self.ctx.check(_lib.mr_upload(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes))

    def download(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        self.ctx.check(_lib.mr_download(self.ctx.h, out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx.check(_lib.mr_dev_free(self.ctx.h, self.ptr))
            self.ptr = 0


class ExpertPack:
    """One projection of all experts of a layer in native GGUF layout (mr_pack)."""

    def __init__(self, ctx: Context, h: int, ggml_type: int, n_experts: int, out_f: int, in_f: int,
                 keep=None):
        self.ctx, self.h = ctx, h
        self.type, self.n_experts, self.out_features, self.in_features = ggml_type, n_experts, out_f, in_f
        self._keep = keep

    @classmethod
    def upload(cls, ctx: Context, ggml_type: int, data: np.ndarray, n_experts: int, out_f: int,
               in_f: int, offsets=None) -> "ExpertPack":
        data = np.ascontiguousarray(data, dtype=np.uint8)
        h = _vp()
        offs = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.uint64)
        ctx.check(_lib.mr_pack_upload(ctx.h, ggml_type, data.ctypes.data, data.nbytes, n_experts,
                                      out_f, in_f, None if offs is None else offs.ctypes.data,
                                      C.byref(h)))
        return cls(ctx, h.value, ggml_type, n_experts, out_f, in_f,
                   keep=data if ctx.device == DEVICE_NONE else None)

    @classmethod
    def wrap(cls, ctx: Context, ggml_type: int, dev: "DeviceBuffer | int", nbytes: int,
             n_experts: int, out_f: int, in_f: int, offsets=None) -> "ExpertPack":
        h = _vp()
        offs = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.uint64)
        ctx.check(_lib.mr_pack_wrap(ctx.h, ggml_type, _ptr(dev), nbytes, n_experts, out_f, in_f,
                                    None if offs is None else offs.ctypes.data, C.byref(h)))
        return cls(ctx, h.value, ggml_type, n_experts, out_f, in_f, keep=dev)

    def dequant(self, expert: int) -> np.ndarray:
        out = DeviceBuffer(self.ctx, self.out_features * self.in_features * 4)
        self.ctx.check(_lib.mr_dequant(self.ctx.h, self.h, expert, out.ptr))
        arr = out.download(np.float32).reshape(self.out_features, self.in_features)
        out.free()
        return arr

    def close(self) -> None:
        if self.h:
            _lib.mr_pack_destroy(self.h)
            self.h = None


class MoeLayer:
    """One MoE layer (mr_layer): packs, biases, router, optional shared expert."""

    def __init__(self, ctx: Context, gate: ExpertPack, up: ExpertPack, down: ExpertPack, *,
                 router_w, top_k: int, route_flags: int, act: int, alpha: float = 1.702,
                 limit: float = 7.0, router_b=None, dummy_mask=None, gate_bias=None,
                 up_bias=None, down_bias=None, sh_gate: ExpertPack | None = None,
                 sh_up: ExpertPack | None = None, sh_down: ExpertPack | None = None,
                 sh_gate_inp=None):
        d = LayerDesc()
        d.gate, d.up, d.down = gate.h, up.h, down.h
        d.gate_bias, d.up_bias, d.down_bias = _ptr(gate_bias), _ptr(up_bias), _ptr(down_bias)
        d.router_w, d.router_b, d.dummy_mask = _ptr(router_w), _ptr(router_b), _ptr(dummy_mask)
        d.sh_gate = sh_gate.h if sh_gate else None
        d.sh_up = sh_up.h if sh_up else None
        d.sh_down = sh_down.h if sh_down else None
        d.sh_gate_inp = _ptr(sh_gate_inp)
        d.top_k, d.route_flags, d.act, d.alpha, d.limit = top_k, route_flags, act, alpha, limit
        h = _vp()
        ctx.check(_lib.mr_layer_create(ctx.h, C.byref(d), C.byref(h)))
        self.ctx, self.h, self.desc = ctx, h.value, d
        self.hidden, self.inter = gate.in_features, gate.out_features
        self.n_experts, self.top_k = gate.n_experts, top_k
        self._refs = (gate, up, down, router_w, router_b, dummy_mask, gate_bias, up_bias,
                      down_bias, sh_gate, sh_up, sh_down, sh_gate_inp)
        self._next = None

    def set_next(self, nxt: "MoeLayer | None") -> None:
        """Prefetch hint: `nxt` runs after this layer (mr_layer_set_next); results do not change."""
        self.ctx.check(_lib.mr_layer_set_next(self.h, nxt.h if nxt is not None else None))
        self._next = nxt  # keeps the next layer alive while this one may prefetch it

    def set_norm(self, norm_w) -> None:
        """Prefetch hint: the norm weights (device buffer or address) passed to this layer's
        residual forwards (mr_layer_set_norm); results do not change."""
        self.ctx.check(_lib.mr_layer_set_norm(self.h, _ptr(norm_w)))

    def set_logits_out(self, logits, max_tokens: int = 1) -> None:
        """Forward calls also write their router logits [T, E] f32 to the device buffer
        `logits` (mr_layer_set_logits_out); None clears it."""
        ptr = None if logits is None else logits.ptr
        self.ctx.check(_lib.mr_layer_set_logits_out(self.h, ptr, 0 if logits is None else max_tokens))

    def reserve(self, max_tokens: int) -> None:
        self.ctx.check(_lib.mr_reserve(self.ctx.h, self.h, max_tokens))

    def router_topk(self, x, n_tokens: int, idx, w, logits=None) -> None:
        self.ctx.check(_lib.mr_router_topk(self.ctx.h, self.h, _ptr(x), n_tokens, _ptr(idx),
                                           _ptr(w), _ptr(logits)))

    def experts(self, x, n_tokens: int, idx, w, y) -> None:
        self.ctx.check(_lib.mr_moe_experts(self.ctx.h, self.h, _ptr(x), n_tokens, _ptr(idx),
                                           _ptr(w), _ptr(y)))

    def forward(self, x, y) -> None:
        self.ctx.check(_lib.mr_moe_forward(self.ctx.h, self.h, _ptr(x), _ptr(y)))

    def forward_residual(self, h, norm_w, eps: float, h_out) -> None:
        """h_out = h + moe(rms_norm(h, norm_w, eps)) (mr_moe_forward_residual); h_out may be h."""
        self.ctx.check(_lib.mr_moe_forward_residual(self.ctx.h, self.h, _ptr(h), _ptr(norm_w), eps,
                                                    _ptr(h_out)))

    def forward_batched(self, x, n_tokens: int, y) -> None:
        self.ctx.check(_lib.mr_moe_forward_batched(self.ctx.h, self.h, _ptr(x), n_tokens, _ptr(y)))

    def forward_batched_residual(self, h, n_tokens: int, norm_w, eps: float, h_out) -> None:
        """mr_moe_forward_batched_residual: h_out[t] = h[t] + moe(rms_norm(h[t]))."""
        self.ctx.check(_lib.mr_moe_forward_batched_residual(self.ctx.h, self.h, _ptr(h), n_tokens, _ptr(norm_w),
                                                            eps, _ptr(h_out)))

    def forward_batched_noalloc(self, x, n_tokens: int, y) -> None:
        """mr_moe_forward_batched_noalloc: the same result with the static per-GPU scratch
        (no allocation; calls that overlap on one GPU race)."""
        self.ctx.check(_lib.mr_moe_forward_batched_noalloc(self.ctx.h, self.h, _ptr(x), n_tokens, _ptr(y)))

    def close(self) -> None:
        if self.h:
            _lib.mr_layer_destroy(self.h)
            self.h = None
            self._next = None


def _gguf_check(rc: int) -> None:
    if rc != MR_OK:
        raise MoeRocmError(rc, _lib.mr_last_error(None).decode(errors="replace"))


class GgufFile:
    """A memory-mapped GGUF file (mr_gguf_open; GgufReader, gguf/reader.rs)."""

    def __init__(self, path):
        h = _vp()
        _gguf_check(_lib.mr_gguf_open(str(path).encode(), C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            _lib.mr_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor_names(self) -> list[str]:
        n = _lib.mr_gguf_n_tensors(self.h)
        return [_lib.mr_gguf_tensor_name(self.h, i).decode() for i in range(n)]

    def info(self, name: str) -> dict:
        t = GgufTensor()
        _gguf_check(_lib.mr_gguf_tensor_info(self.h, name.encode(), C.byref(t)))
        return dict(ggml_type=t.ggml_type, dims=tuple(t.dims[: t.n_dims]), data_offset=t.data_offset,
                    nbytes=t.nbytes)

    def data(self, name: str) -> np.ndarray:
        p, n = _vp(), _u64()
        _gguf_check(_lib.mr_gguf_tensor_data(self.h, name.encode(), C.byref(p), C.byref(n)))
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value)).copy()

    def meta_u32(self, key: str) -> int:
        v = _u32()
        _gguf_check(_lib.mr_gguf_meta_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_f32(self, key: str) -> float:
        v = _f32()
        _gguf_check(_lib.mr_gguf_meta_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str:
        p, n = C.c_void_p(), _u64()
        _gguf_check(_lib.mr_gguf_meta_str(self.h, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value).decode() if n.value else ""

    def meta_u32_array(self, key: str) -> list[int]:
        n = _u64()
        _gguf_check(_lib.mr_gguf_meta_u32_array(self.h, key.encode(), None, 0, C.byref(n)))
        out = np.zeros(n.value, dtype=np.uint32)
        _gguf_check(_lib.mr_gguf_meta_u32_array(self.h, key.encode(), out.ctypes.data, n.value, C.byref(n)))
        return out.tolist()

    def layer(self, ctx: "Context", index: int, *, top_k: int = 0, route_flags: int = -1, act: int = -1,
              alpha: float = 0.0, limit: float = 0.0) -> "MoeLayer":
        """mr_gguf_layer_create: the MoE layer `index`, owning its device copies; the
        returned layer's `norm_w` (device pointer or None) and `eps` feed forward_residual."""
        o = GgufLayerOpts(top_k=top_k, route_flags=route_flags, act=act, alpha=alpha, limit=limit)
        h, nw, eps = _vp(), _vp(), _f32()
        ctx.check(_lib.mr_gguf_layer_create(ctx.h, self.h, index, C.byref(o), C.byref(h), C.byref(nw),
                                            C.byref(eps)))
        L = MoeLayer.__new__(MoeLayer)
        L.ctx, L.h, L.desc, L._refs, L._next = ctx, h.value, None, (), None
        gate = self.info(f"blk.{index}.ffn_gate_exps.weight")
        L.hidden, L.inter, L.n_experts = gate["dims"][0], gate["dims"][1], gate["dims"][2]
        L.top_k = top_k or self.meta_u32(f"{self.meta_str('general.architecture')}.expert_used_count")
        L.norm_w, L.eps = nw.value, eps.value
        return L


def topk(ctx: Context, logits, n_tokens: int, n_experts: int, top_k: int, flags: int, idx, w) -> None:
    ctx.check(_lib.mr_topk(ctx.h, _ptr(logits), n_tokens, n_experts, top_k, flags, _ptr(idx), _ptr(w)))


def matrix_bytes(ggml_type: int, rows: int, cols: int) -> int:
    return int(_lib.mr_matrix_bytes(ggml_type, rows, cols))


def exported_symbols() -> list[str]:
    return sorted(_SIGS)
