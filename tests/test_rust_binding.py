"""The Rust FFI crate (moe-stream_amd/rust/moe-rocm-sys) against include/moe_rocm.h.

No Rust toolchain exists in this image, so the crate cannot be compiled here; these tests
read both files as text and check that the crate declares every function, struct and
constant of the header with the same parameter types (C -> Rust by the usual FFI mapping),
the same field order and the same values. A header change that the binding misses fails
here.
"""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "moe_rocm.h"
CRATE = ROOT / "moe-stream_amd" / "rust" / "moe-rocm-sys"
LIB_RS = CRATE / "src" / "lib.rs"

BASE = {"int": "c_int", "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32", "float": "f32",
        "double": "f64", "void": "c_void", "char": "c_char"}


def _strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", " ", s, flags=re.S)


def c_to_rust(ctype: str) -> str:
    """`const T**` -> `*mut *const T` and so on (const binds to the innermost pointee)."""
    t = " ".join(ctype.replace("*", " * ").split())
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    parts = t.split()
    base, stars = parts[0], parts[1:]
    assert all(p == "*" for p in stars), ctype
    base = BASE.get(base, base)
    if not stars:
        return base
    out = ("*const " if const else "*mut ") + base
    for _ in stars[1:]:
        out = "*mut " + out
    return out


def header_functions():
    s = _strip_c_comments(HEADER.read_text())
    s = re.sub(r"#.*", "", s)
    s = re.sub(r"typedef struct \w+ \{.*?\} \w+;", "", s, flags=re.S)
    funcs = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(mr_\w+)\s*\(([^)]*)\)\s*;", s):
        ret = " ".join(m.group(1).split())
        params = []
        for p in [p.strip() for p in m.group(3).split(",") if p.strip()]:
            if p == "void":
                continue
            # drop the parameter name (last identifier not part of the type)
            pm = re.match(r"(.*?[\s\*])(\w+)$", p)
            params.append(c_to_rust(pm.group(1)))
        funcs[m.group(2)] = (c_to_rust(ret) if ret != "void" else None, params)
    return funcs


def rust_functions():
    s = LIB_RS.read_text()
    block = s[s.index('extern "C" {'):]
    funcs = {}
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        params = []
        for p in [p.strip() for p in m.group(2).split(",") if p.strip()]:
            name, ty = p.split(":", 1)
            params.append(" ".join(ty.split()))
        ret = " ".join(m.group(4).split()) if m.group(4) else None
        funcs[m.group(1)] = (ret, params)
    return funcs


def header_structs():
    s = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \1;", s, flags=re.S):
        fields = []
        for decl in [d.strip() for d in m.group(2).split(";") if d.strip()]:
            dm = re.match(r"(.*?[\s\*])(\w+(?:\s*\[\d+\])?(?:\s*,\s*\w+)*)$", decl)
            ty = dm.group(1)
            for name in [n.strip() for n in dm.group(2).split(",")]:
                am = re.match(r"(\w+)\s*\[(\d+)\]", name)
                if am:
                    fields.append((am.group(1), f"[{c_to_rust(ty)}; {am.group(2)}]"))
                else:
                    fields.append((name, c_to_rust(ty)))
        out[m.group(1)] = fields
    return out


def rust_structs():
    s = LIB_RS.read_text()
    out = {}
    for m in re.finditer(r"pub struct (\w+) \{(.*?)\n\}", s, flags=re.S):
        fields = re.findall(r"pub (\w+): ([^,\n]+),", m.group(2))
        if fields:
            out[m.group(1)] = [(n, " ".join(t.split())) for n, t in fields]
    return out


def _c_int(v: str) -> int:
    v = v.strip().strip("()")
    v = re.sub(r"(?<=\d)(ull|ul|u)\b", "", v)
    return int(eval(v, {"__builtins__": {}}))  # header literals: ints, shifts, unary minus


def header_constants():
    s = HEADER.read_text()
    out = {}
    for m in re.finditer(r"#define (MR_\w+) +(\(?-?[\w <]+\)?)", s):
        try:
            out[m.group(1)] = _c_int(m.group(2))
        except Exception:
            pass
    return out


def rust_constants():
    s = LIB_RS.read_text()
    return {m.group(1): int(eval(m.group(2), {"__builtins__": {}}))
            for m in re.finditer(r"pub const (MR_\w+): \w+ = ([^;]+);", s)}


def test_crate_files_and_links_key():
    cargo = (CRATE / "Cargo.toml").read_text()
    assert re.search(r'^links = "moe_rocm"$', cargo, flags=re.M)
    assert re.search(r'^name = "moe-rocm-sys"$', cargo, flags=re.M)
    build = (CRATE / "build.rs").read_text()
    assert "cargo:rustc-link-lib=dylib=moe_rocm" in build and "cargo:rustc-link-search" in build


def test_every_header_function_is_declared_with_its_types():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 50
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (ret, params) in h.items():
        assert r[name] == (ret, params), (name, r[name], (ret, params))


def test_structs_match_field_by_field():
    h, r = header_structs(), rust_structs()
    assert set(h) == {"mr_layer_desc", "mr_gguf_tensor", "mr_gguf_layer_opts"}
    for name, fields in h.items():
        assert r.get(name) == fields, (name, r.get(name), fields)


def test_constants_have_the_header_values():
    h, r = header_constants(), rust_constants()
    for name in ("MR_OK", "MR_E_INVAL", "MR_E_LAUNCH", "MR_GGML_Q4_K", "MR_GGML_MXFP4", "MR_DECODE_FUSED",
                 "MR_OPT_WAIT_LIMIT_US", "MR_STATIC_SCRATCH_BYTES", "MR_ROUTE_NORM_TOPK", "MR_ACT_SWIGLU_OAI"):
        assert name in h, name
    missing = sorted(set(h) - set(r))
    assert not missing, missing
    for name, v in h.items():
        assert r[name] == v, (name, r[name], v)


@pytest.mark.parametrize("ctype,rust", [("const float*", "*const f32"), ("mr_ctx**", "*mut *mut mr_ctx"),
                                        ("const char**", "*mut *const c_char"), ("void*", "*mut c_void"),
                                        ("uint64_t", "u64"), ("const mr_layer*", "*const mr_layer")])
def test_type_mapping(ctype, rust):
    assert c_to_rust(ctype) == rust
