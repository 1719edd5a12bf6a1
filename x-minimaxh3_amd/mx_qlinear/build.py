"""Build recipe for libmx_qlinear.so (hipcc, gfx950 only).

``python -m mx_qlinear.build`` (with ``x-minimaxh3_amd`` on ``sys.path``) or
``build()`` compiles every ``csrc/*.hip`` translation unit in parallel and links
them into ``mx_qlinear/libmx_qlinear.so``. hipcc cross-compiles without a GPU.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libmx_qlinear.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Every fp32 expression rounds exactly as written (no implicit multiply-add fusion).
    "-ffp-contract=off",
    # Packed fp32 VALU instructions are kept out of all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    # The 65,536-entry GELU table is evaluated at compile time.
    "-fconstexpr-steps=100000000",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = pathlib.Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; ROCm is required to build libmx_qlinear.so")
    return found


# Per-source compiler flags (none needed at present; the hook stays for per-kernel tuning).
FILE_FLAGS: dict[str, list[str]] = {}


def _compile(src: pathlib.Path, extra: list[str]) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> pathlib.Path:
    """Compile all HIP sources and link libmx_qlinear.so; returns its path."""
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, extra_flags=sys.argv[1:])
