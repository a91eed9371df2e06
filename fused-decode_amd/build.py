"""Build libfused_decode_hip.so for gfx950 from csrc/*.hip with hipcc, and the
CPython binding of its C ABI (csrc/fdcall.c) with the host C compiler.

Usage: python fused-decode_amd/build.py [--jobs N]

Both land next to the Python package (fused_decode/), where fused_decode._lib
loads them. Each .hip file is compiled to an object in _build/ (git-ignored)
and the objects are linked into one shared library. The binding needs only
Python's headers and the C ABI header: it dlopens the library at run time.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
BUILD = HERE / "_build"
LIB_NAME = "libfused_decode_hip.so"
OUT = HERE / "fused_decode" / LIB_NAME
BINDING_OUT = HERE / "fused_decode" / ("_fdcall" + sysconfig.get_config_var("EXT_SUFFIX"))
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


# Packed-FP32 instructions are disabled for every device compile: the kernels
# rely on plain float32 VALU ops only.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def compile_one(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{errs}")
    if errs.strip():
        print(errs, file=sys.stderr)
    return obj


def build(jobs: int = 4) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objects = list(pool.map(compile_one, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    build_binding()
    return OUT


def build_binding() -> Path:
    """The CPython extension fused_decode._fdcall (plain C, no torch)."""
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler found for the Python binding (set CC)")
    tmp = BINDING_OUT.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", "-Werror", f"-I{sysconfig.get_paths()['include']}",
           f"-I{INCLUDE}", str(CSRC / "fdcall.c"), "-ldl", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building the Python binding failed:\n{proc.stderr}")
    os.replace(tmp, BINDING_OUT)
    return BINDING_OUT


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args()
    print(build(args.jobs))


if __name__ == "__main__":
    main()
