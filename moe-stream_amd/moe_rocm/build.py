"""Build libmoe_rocm.so (the C-ABI library) for gfx950 with hipcc, in-tree.

Usage: python moe-stream_amd/moe_rocm/build.py [--trace], or moe_rocm.build.build().
--trace builds the same library with the fused decode kernel's phase timestamps compiled in
(MR_FUSED_TRACE; read by `bench.py --trace`) as moe_rocm/trace/libmoe_rocm.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
LIB_PATH = PKG_DIR / "libmoe_rocm.so"
OBJ_DIR = PKG_DIR.parent / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


EXTRA_FLAGS = os.environ.get("MOE_ROCM_EXTRA_FLAGS", "").split()
TRACE_LIB = PKG_DIR / "trace" / "libmoe_rocm.so"


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *EXTRA_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *HIP_FLAGS, *EXTRA_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: Path | None = None, obj_dir: Path | None = None, trace: bool = False) -> Path:
    global OBJ_DIR, EXTRA_FLAGS
    if trace:
        EXTRA_FLAGS = [*EXTRA_FLAGS, "-DMR_FUSED_TRACE"]
        obj_dir = obj_dir or OBJ_DIR / "trace"
        out = out or TRACE_LIB
    if obj_dir is not None:
        OBJ_DIR = obj_dir
    lib_path = out or LIB_PATH
    lib_path.parent.mkdir(parents=True, exist_ok=True)
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path}")
    return lib_path


if __name__ == "__main__":
    build(verbose=True, trace="--trace" in sys.argv[1:])
    sys.exit(0)
