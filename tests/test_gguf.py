"""GGUF reader (mr_gguf_*; gguf/reader.rs) on files written by tests/gguf_writer.py:
header, metadata of every value type, tensor index and data views, the data-section
alignment, and the error cases GgufReader::open rejects. Host only."""
import struct

import numpy as np
import pytest

import gguf_writer as G
import moe_rocm as M
from moe_rocm import workloads as W

TINY = W.LayerSpec(config=150, layer=0, ggml_type=M.GGML_MXFP4, hidden=256, inter=128, n_experts=8, top_k=2,
                   route_flags=M.ROUTE_SOFTMAX_AFTER_TOPK, act=M.ACT_SWIGLU_OAI, expert_bias=True,
                   router_bias=True)


def _meta_all():
    return [("general.architecture", G.STR, "gpt-oss"), ("general.name", G.STR, "tiny test"),
            ("k.u8", G.U8, 200), ("k.i8", G.I8, -5), ("k.u16", G.U16, 60000), ("k.i16", G.I16, -300),
            ("k.u32", G.U32, 4000000000), ("k.i32", G.I32, 77), ("k.f32", G.F32, 1.5),
            ("k.bool", G.BOOL, 1), ("k.u64", G.U64, 123456789), ("k.i64", G.I64, -9),
            ("k.f64", G.F64, 0.25), ("k.arr", G.ARR, (G.U32, [256, 384, 512])),
            ("k.nested", G.ARR, (G.ARR, [(G.STR, ["a", "bc"]), (G.STR, [])])),
            ("gpt-oss.expert_used_count", G.U32, 2), ("gpt-oss.attention.layer_norm_rms_epsilon", G.F32, 1e-5)]


def _tensors():
    rng = np.random.default_rng(3)
    q = W.quant_tensors(TINY)
    t = [("a.f32", 0, (5, 3), G.f32(rng.standard_normal(15))),
         ("b.f16", 1, (7,), rng.standard_normal(7).astype(np.float16).tobytes()),
         ("blk.0.ffn_gate_exps.weight", M.GGML_MXFP4, (256, 128, 8), q["gate"].tobytes()),
         ("c.q4k", M.GGML_Q4_K, (512, 2), bytes(range(256)) * 2 + bytes(32) + bytes(4 * 144 - 544))]
    return t


@pytest.fixture
def gfile(tmp_path):
    path = tmp_path / "t.gguf"
    G.write(path, _meta_all(), _tensors())
    with M.GgufFile(path) as g:
        yield g


def test_tensor_index_and_data(gfile):
    tens = _tensors()
    assert gfile.tensor_names() == [t[0] for t in tens]
    raw = {"a.f32": 15 * 4, "b.f16": 7 * 2, "blk.0.ffn_gate_exps.weight": 8 * 128 * 256 // 32 * 17,
           "c.q4k": 4 * 144}
    prev_end = 0
    for name, gtype, dims, data in tens:
        info = gfile.info(name)
        assert info["ggml_type"] == gtype and info["dims"] == dims
        assert info["nbytes"] == raw[name] == len(data)
        assert info["data_offset"] % 32 == 0 and info["data_offset"] >= prev_end
        prev_end = info["data_offset"] + info["nbytes"]
        assert gfile.data(name).tobytes() == data


def test_metadata_getters(gfile):
    assert gfile.meta_str("general.architecture") == "gpt-oss"
    assert gfile.meta_u32("k.u8") == 200 and gfile.meta_u32("k.u16") == 60000
    assert gfile.meta_u32("k.u32") == 4000000000 and gfile.meta_u32("k.i32") == 77
    assert gfile.meta_u32("k.u64") == 123456789  # as_u32 truncates u64 (reader.rs:170-179)
    assert gfile.meta_f32("k.f32") == 1.5 and gfile.meta_f32("k.f64") == 0.25
    assert gfile.meta_u32_array("k.arr") == [256, 384, 512]
    for key, getter in (("k.i8", gfile.meta_u32), ("k.bool", gfile.meta_u32), ("k.f32", gfile.meta_u32),
                        ("k.u32", gfile.meta_f32), ("k.u32", gfile.meta_str), ("missing", gfile.meta_u32),
                        ("k.nested", gfile.meta_u32_array)):
        with pytest.raises(M.MoeRocmError) as ei:
            getter(key)
        assert ei.value.status == M.MR_E_INVAL


def test_alignment_from_metadata(tmp_path):
    path = tmp_path / "a.gguf"
    G.write(path, [("general.alignment", G.U32, 256)], [("x", 0, (3,), G.f32([1, 2, 3])),
                                                        ("y", 0, (1,), G.f32([4]))], alignment=256)
    with M.GgufFile(path) as g:
        assert g.info("x")["data_offset"] % 256 == 0 and g.info("y")["data_offset"] % 256 == 0
        assert np.frombuffer(g.data("y").tobytes(), np.float32)[0] == 4.0


def _open_err(path):
    with pytest.raises(M.MoeRocmError) as ei:
        M.GgufFile(path)
    return ei.value


def test_open_errors(tmp_path):
    good = G.build(_meta_all(), _tensors())
    cases = {
        "magic": (G.build([], [], magic=b"GGUX"), M.MR_E_INVAL, "magic"),
        "version1": (G.build([], [], version=1), M.MR_E_UNSUPPORTED, "version"),
        "version4": (G.build([], [], version=4), M.MR_E_UNSUPPORTED, "version"),
        "truncated_header": (good[:40], M.MR_E_INVAL, "end of file"),
        "iq_type": (G.build([], [("t", 16, (256,), bytes(66))]), M.MR_E_UNSUPPORTED, "quant type"),
        "too_many_meta": (b"GGUF" + struct.pack("<IQQ", 3, 0, 1000001), M.MR_E_INVAL, "metadata count"),
        "too_many_tensors": (b"GGUF" + struct.pack("<IQQ", 3, 1000001, 0), M.MR_E_INVAL, "tensor count"),
        "bad_value_type": (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + G._str("k") + struct.pack("<I", 13),
                           M.MR_E_INVAL, "metadata type"),
        "empty": (b"", M.MR_E_INVAL, "empty"),
    }
    for name, (data, code, text) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        e = _open_err(p)
        assert e.status == code and text in e.message, (name, e.status, e.message)
    e = _open_err(tmp_path / "does-not-exist.gguf")
    assert e.status == M.MR_E_INVAL


def test_tensor_data_bounds(tmp_path):
    data = G.build([], [("x", 0, (64,), G.f32(np.arange(64)))])
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[:-16])  # the index parses, the data runs past the end of the file
    with M.GgufFile(p) as g:
        assert g.info("x")["nbytes"] == 256
        with pytest.raises(M.MoeRocmError) as ei:
            g.data("x")
        assert ei.value.status == M.MR_E_INVAL and "out of bounds" in ei.value.message
        with pytest.raises(M.MoeRocmError) as ei:
            g.data("nope")
        assert ei.value.status == M.MR_E_INVAL and "not found" in ei.value.message


def test_layer_create_needs_device(tmp_path):
    """Layer preload on a host-only context: the expert packs upload (host copies), the
    first device buffer fails with MR_E_NODEV, and everything made so far is released."""
    q, f = W.quant_tensors(TINY), W.float_tensors(TINY)
    p = tmp_path / "layer.gguf"
    G.write(p, _meta_all(), G.moe_layer_tensors(TINY, q, f))
    ctx = M.Context(M.DEVICE_NONE)
    try:
        with M.GgufFile(p) as g:
            with pytest.raises(M.MoeRocmError) as ei:
                g.layer(ctx, 0)
            assert ei.value.status == M.MR_E_NODEV
            with pytest.raises(M.MoeRocmError) as ei:
                g.layer(ctx, 3)  # no such layer
            assert ei.value.status == M.MR_E_INVAL and "not found" in ei.value.message
    finally:
        ctx.close()
