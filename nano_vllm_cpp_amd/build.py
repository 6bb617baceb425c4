"""Builds libnvf_ops.so (the HIP kernels + C ABI) in-tree for gfx950.

Every .hip file under csrc/ is compiled by hipcc to an object in _build/ and
linked into lib/libnvf_ops.so.  `python -m nano_vllm_cpp_amd.build` runs it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libnvf_ops.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NVF_OFFLOAD_ARCH", "gfx950")

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # hipcc -O3 forms packed-fp32 ops from plain float code; keep them off.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln]
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + "\n".join(msgs))
    if msgs:
        print("\n".join(msgs), file=sys.stderr)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    _run([HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every csrc/*.hip and links lib/libnvf_ops.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
