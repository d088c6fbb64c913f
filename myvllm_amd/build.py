"""In-tree build of libgdn_hip.so (gfx950) with hipcc.

Objects go to ``myvllm_amd/_build/``; the shared library to
``myvllm_amd/lib/libgdn_hip.so`` (written to a temporary name and renamed, so a
process that already loaded the old library is not disturbed).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIBNAME = "libgdn_hip.so"
SOURCES = [
    "gdn_decode.hip",
    "gdn_decode_fused.hip",
    "gdn_prefill.hip",
    "causal_conv1d.hip",
    "gdn_norm.hip",
    "attention.hip",
    "hbm_copy.hip",
    "gdn_capi.cpp",
]

ARCH = "gfx950"
# Per-source flags.  attention.hip: keep MFMA accumulators in architectural
# VGPRs; with the default AGPR form the D=256 prefill tile (128 accumulator
# registers) was shuttled between AGPRs and VGPRs on every key tile.
SOURCE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
# Packed-FP32 VALU ops are disabled for all device code (they are generated
# from plain float2 arithmetic at -O3 otherwise).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libgdn_hip.so)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in res.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def library_path() -> str:
    return os.path.join(LIBDIR, LIBNAME)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source for gfx950 and link the shared library; returns its path."""
    hipcc = _hipcc()
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    out = library_path()
    tmp = out + f".tmp{os.getpid()}"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


ASAN_LIBNAME = "libgdn_hip_asan.so"
# Host-only AddressSanitizer for the C-ABI layer: every -fsanitize flag goes
# after -Xarch_host, so the device code of the kernels is built as usual.
ASAN_HOST_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
                   "-Xarch_host", "-shared-libsan"]


def asan_runtime() -> str:
    """The compiler's shared AddressSanitizer runtime (to preload into a host
    process that loads the instrumented library)."""
    res = subprocess.run([_hipcc(), "--print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE,
                         stderr=subprocess.DEVNULL, text=True)
    path = res.stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        raise RuntimeError("the AddressSanitizer runtime libclang_rt.asan-x86_64.so was not found")
    return path


def build_asan(verbose: bool = False) -> str:
    """libgdn_hip_asan.so: gdn_capi.cpp (argument validation, the C ABI)
    compiled with host AddressSanitizer, linked with the kernels' objects of
    the last build(); returns its path.  Load it through MYVLLM_AMD_LIB with
    asan_runtime() preloaded."""
    hipcc = _hipcc()
    objs = []
    for src in SOURCES:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        if src == "gdn_capi.cpp":
            obj = os.path.join(OBJDIR, "gdn_capi_asan.o")
            _run([hipcc, *COMMON_FLAGS, *ASAN_HOST_FLAGS, "-g", "-c", os.path.join(CSRC, src), "-o", obj], verbose)
        elif not os.path.exists(obj):
            raise RuntimeError(f"{obj} is missing: run build() first")
        objs.append(obj)
    out = os.path.join(LIBDIR, ASAN_LIBNAME)
    tmp = out + f".tmp{os.getpid()}"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *ASAN_HOST_FLAGS, "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_asan(verbose="-v" in sys.argv) if "--asan" in sys.argv else build(verbose="-v" in sys.argv))
