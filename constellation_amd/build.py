"""Builds libcx_moe.so (HIP, gfx950) in-tree with hipcc.

    python -m constellation_amd.build            # the library (build())
    python -m constellation_amd.build --kbench   # the kernel micro-benchmark only

The library build does not depend on the micro-benchmark: build() compiles
libcx_moe.so alone, build_kbench() the stand-alone cx_kbench program.

Every HIP file is compiled with packed-fp32 code generation disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops) and the generator with
contraction off, so its arithmetic is bit-reproducible against the CPU
definition.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcx_moe.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("CX_OFFLOAD_ARCH", "gfx950")

SOURCES = {
    "cx_runtime.hip": [],
    "cx_expert.hip": [],
    "cx_route.hip": [],
    "cx_gen.hip": ["-ffp-contract=off"],
}

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
]


def _compile(name: str, extra: list[str]) -> Path:
    src = CSRC / name
    obj = BUILD / (Path(name).stem + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {name}")
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines()
            if "packed-fp32-ops" not in ln and ln.strip()]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


KBENCH_SRC = PKG / "kbench" / "kbench.hip"
KBENCH = PKG / "kbench" / "cx_kbench"


def build_kbench(verbose: bool = False) -> Path:
    """The kernel micro-benchmark (constellation_amd/kbench): a stand-alone
    program that compiles the library's kernels and times single launches."""
    tmp = KBENCH.with_suffix(".tmp")
    cmd = [HIPCC, *COMMON, "-o", str(tmp), str(KBENCH_SRC)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed for kbench.hip")
    os.replace(tmp, KBENCH)
    if verbose:
        print(f"built {KBENCH}")
    return KBENCH


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libcx_moe.so failed")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    if "--kbench" in sys.argv[1:]:
        build_kbench(verbose=True)
    else:
        build(verbose=True)
