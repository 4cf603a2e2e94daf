"""Build libalveare_q4.so (HIP kernels + C ABI) for gfx950, in-tree.

    python -m alveare_amd.build          # or alveare_amd.build.build()

Each csrc/*.hip compiles to an object with hipcc, then one shared library is
linked next to this file. Packed-FP32 instructions are disabled for the device
code (``-Xclang -target-feature -Xclang -packed-fp32-ops``); hipcc's host pass
warns that it does not know the feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libalveare_q4.so")
# The reference runtime's C++ registry interface over LIB (alveare::NpuRegistry)
# and the program that drives it in the tests.
NPU_SRC = os.path.join(HERE, "cpp", "npu_registry.cpp")
NPU_LIB = os.path.join(HERE, "libalveare_npu.so")
CHECK_SRC = os.path.join(ROOT, "tests", "cpp", "npu_registry_check.cpp")
CHECK_BIN = os.path.join(HERE, "npu_registry_check")
ARCH = os.environ.get("ALV_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_adapter(verbose)
    build_probe(verbose)
    return LIB


PROBE_SRC = os.path.join(ROOT, "measure", "read_probe.hip")
PROBE_LIB = os.path.join(ROOT, "measure", "libalveare_probe.so")


def build_probe(verbose: bool = True) -> str:
    """The benchmark's streaming-read probe, a library of its own
    (measure/libalveare_probe.so), not part of libalveare_q4.so."""
    tmp = PROBE_LIB + ".tmp"
    cmd = [_hipcc(), *HIPCC_FLAGS, "-shared", PROBE_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC}:\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB}")
    return PROBE_LIB


def _run(cmd: list[str], what: str) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr}")


def build_adapter(verbose: bool = True) -> str:
    """libalveare_npu.so (alveare::NpuRegistry over libalveare_q4.so) and, when
    the tests are present, the program that drives it."""
    # Host code only (the HIP runtime API, no kernels): the system C++ compiler.
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cxx = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(HERE, "cpp"), "-I", os.path.join(ROOT, "include"), "-I", os.path.join(rocm, "include")]
    link = ["-L", HERE, "-L", os.path.join(rocm, "lib"), "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(rocm, "lib")]
    tmp = NPU_LIB + ".tmp"
    _run([*cxx, "-fPIC", "-shared", NPU_SRC, "-o", tmp, *link, "-lalveare_q4", "-lamdhip64"], "adapter build")
    os.replace(tmp, NPU_LIB)
    if os.path.exists(CHECK_SRC):
        tmp = CHECK_BIN + ".tmp"
        _run([*cxx, CHECK_SRC, "-o", tmp, *link, "-lalveare_npu", "-lalveare_q4", "-lamdhip64"], "adapter check build")
        os.replace(tmp, CHECK_BIN)
    if verbose:
        print(f"built {NPU_LIB}")
    return NPU_LIB


if __name__ == "__main__":
    build()
