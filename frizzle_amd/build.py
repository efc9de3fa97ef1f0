"""Builds the HIP backend, libfrizzle_hip.so, in-tree for gfx950.

    python -m frizzle_amd.build

Each .hip source under csrc/ compiles with hipcc, and each host-only .cpp
source with g++, to an object in _build/ (in parallel); then all link into
frizzle_amd/libfrizzle_hip.so. The flags keep every
rounding point where the sources write it: -ffp-contract=off (no multiply-add
is fused unless the source calls fma) and packed FP32 math off.
"""
import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libfrizzle_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# The prefill products keep their matrix accumulators in ordinary vector
# registers, which the totals are added from.
FILE_FLAGS = {"gemv.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    return obj


CXX = os.environ.get("CXX", "g++")
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def _compile_host(src: Path) -> Path:
    """Host-only sources (the GGUF reader and its C ABI)."""
    obj = BUILD / (src.stem + ".host.o")
    r = subprocess.run([CXX, *CXX_FLAGS, "-c", str(src), "-o", str(obj)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed on {src.name}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    host = sorted(CSRC.glob("*.cpp"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources)) + list(ex.map(_compile_host, host))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
