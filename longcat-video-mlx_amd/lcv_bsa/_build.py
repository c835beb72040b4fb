"""Build recipe for liblcv_bsa.so, the gfx950 C-ABI library.

Compiles every ``csrc/*.hip`` translation unit with hipcc for gfx950 (in
parallel), then links one shared library next to this file.  The library links
against the HIP runtime that ships inside the installed torch wheel, so a
process that imports torch and then loads the library has exactly one HIP
runtime (a second copy from /opt/rocm cannot coexist with torch's).

Usage:  python -m lcv_bsa._build   (or ``__graft_entry__.build()``)
"""

from __future__ import annotations

import concurrent.futures as _fut
import importlib.util
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
REPO_DIR = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "liblcv_bsa.so"
OBJ_DIR = PKG_DIR.parent / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def torch_lib_dir() -> Path:
    """Directory holding torch's bundled libamdhip64.so (without importing torch)."""
    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        raise RuntimeError("torch is not installed; it provides the HIP runtime to link against")
    lib = Path(spec.origin).parent / "lib"
    if not (lib / "libamdhip64.so").exists():
        raise RuntimeError(f"{lib}/libamdhip64.so not found (a ROCm build of torch is required)")
    return lib


def sources() -> list[Path]:
    return sorted(SRC_DIR.glob("*.hip"))


def _compile(src: Path, hipcc: str) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{SRC_DIR}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the GPU feature
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all kernels and link liblcv_bsa.so; returns its path."""
    hipcc = _hipcc()
    tlib = torch_lib_dir()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with _fut.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [
        hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC",
        *[str(o) for o in objs],
        f"-L{tlib}", "-lamdhip64", f"-Wl,-rpath,{tlib}",
        "-o", str(tmp),
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
