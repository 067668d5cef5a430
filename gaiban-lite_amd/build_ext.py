"""Build recipe for the gfx950 HIP library behind ``include/dsv4moe.h``.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 into one shared library,
``libdsv4moe.so``, next to this file (in-tree, so it travels with the source
tree to the GPU host).  No torch extension machinery: the library exposes a
plain C ABI and the Python host code binds it with ctypes.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
BUILD_DIR = HERE / "_build"
LIB_NAME = "libdsv4moe.so"
LIB_PATH = HERE / LIB_NAME

ARCH = os.environ.get("DSV4MOE_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed fp32 VALU ops stay disabled (the compiler may not emit them).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE division and square root in the router's fixed operation sequence.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # MFMA accumulators in ordinary VGPRs: the kernels rescale them with VALU
    # FMAs once per K group, which AGPR accumulators would turn into extra
    # v_accvgpr moves per element.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources and link ``libdsv4moe.so``; returns its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        # the host pass warns about the device-only target feature; keep real diagnostics
        diag = "\n".join(
            line for line in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops" not in line and "warning: feature flag" not in line
        )
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{diag}")
        if verbose and diag.strip():
            print(diag, flush=True)
        return obj

    workers = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(compile_one, zip(srcs, objs)))

    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
