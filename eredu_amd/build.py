"""Builds the gfx950 kernel library ``eredu_amd/_lib/liberedu_hip.so`` in-tree.

``python -m eredu_amd.build`` (or ``__graft_entry__.build()``) compiles every
``eredu_amd/csrc/*.hip`` with hipcc for gfx950 and links one shared library
whose exported symbols are the C ABI of ``include/eredu_hip.h``.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ_DIR = os.path.join(PKG, "_build")
LIB_DIR = os.path.join(PKG, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "liberedu_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: no implicit a*b+c fusion, so every expression rounds as
# written (FMAs in the kernels are explicit fmaf calls).  Packed FP32 ops are
# disabled for the device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in res.stderr.splitlines() if ln.strip() and noise not in ln]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compile all kernels and link the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "4")), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build (the C ABI's
# argument checks, error state and planners; device code is built as usual).
# Each sanitizer flag applies to the host compilation only.
SAN_DIR = os.path.join(OBJ_DIR, "asan")
SAN_LIB = os.path.join(SAN_DIR, "liberedu_hip_asan.so")
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=all",
             "-Xarch_host", "-fno-omit-frame-pointer"]


def _compile_sanitized(src: str) -> str:
    obj = os.path.join(SAN_DIR, os.path.basename(src).replace(".hip", ".o"))
    flags = [f for f in HIP_FLAGS if f != "-O3"] + ["-O1", "-g"]
    res = subprocess.run([HIPCC, *flags, *SAN_FLAGS, "-c", src, "-o", obj], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc (sanitized host) failed for {src}:\n{res.stderr}")
    return obj


def build_host_sanitized() -> str:
    """Builds ``_build/asan/liberedu_hip_asan.so`` (only when a source is newer
    than it) and returns its path.  Load it with clang's ASan runtime preloaded
    (``sanitizer_runtime()``) and ``EREDU_AMD_LIB`` pointing at it."""
    os.makedirs(SAN_DIR, exist_ok=True)
    srcs = sources()
    newest = max(os.path.getmtime(f) for f in srcs + [os.path.join(ROOT, "include", "eredu_hip.h")] +
                 [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hpp")])
    if os.path.exists(SAN_LIB) and os.path.getmtime(SAN_LIB) > newest:
        return SAN_LIB
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        objs = list(ex.map(_compile_sanitized, srcs))
    tmp = SAN_LIB + ".tmp"
    res = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *SAN_FLAGS, "-o", tmp, *objs],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link (sanitized host) failed:\n{res.stderr}")
    os.replace(tmp, SAN_LIB)
    return SAN_LIB


def sanitizer_runtime() -> str:
    """Path of the ASan runtime of hipcc's clang (to preload into a process
    that loads the sanitized library)."""
    clang = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "lib", "llvm", "bin", "clang")
    if not os.path.exists(clang):
        clang = "/opt/rocm/llvm/bin/clang"
    res = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return res.stdout.strip()


if __name__ == "__main__":
    build()
