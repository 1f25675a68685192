"""Builds libspectra_hip.so in-tree with hipcc for gfx950 (no torch headers needed), then the
thin PyTorch extension _spectra_torch.so over its C ABI (torch.ops.spectra_hip.*).

    python -m spectra_amd._build            # compile + link both
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(PKG, "_obj")
LIB = os.path.join(PKG, "libspectra_hip.so")
TORCH_OPS_LIB = os.path.join(PKG, "_spectra_torch.so")
TORCH_OPS_SOURCE = "torch_ops.cpp"
SOURCES = ["api.hip", "quant.hip", "dequant.hip", "gemv.hip", "gemv_f16.hip", "gemv_bf16.hip", "gemv_stream_f16.hip", "gemv_stream_bf16.hip", "gemv_rows_plain.hip", "gemv_rows_pro.hip", "gemv_rows_lm.hip", "gemv_rows_multi_f16.hip", "gemv_rows_multi_bf16.hip", "gemm.hip", "prefill.hip", "skinny.hip", "outliers.hip", "decode.hip", "measure.hip"]
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # every float op rounds where it is written (bit-exact quantizer/dequant)
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    # hand-written packed-fp32 forms are avoided on this pool; keep the compiler off them too
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return cand


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-8000:]}")
    return obj


def build_torch_ops(verbose: bool = True) -> str:
    """The operator registration (csrc/torch_ops.cpp): host C++ only, compiled with the host
    compiler against the installed torch's headers and linked to libspectra_hip.so, which it
    finds next to itself (rpath $ORIGIN)."""
    import torch

    tdir = os.path.dirname(os.path.abspath(torch.__file__))
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler (g++) for the torch operator library")
    tmp = TORCH_OPS_LIB + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           f"-I{tdir}/include", f"-I{tdir}/include/torch/csrc/api/include", f"-I{INCLUDE}", "-I/opt/rocm/include",
           os.path.join(CSRC, TORCH_OPS_SOURCE),
           f"-L{tdir}/lib", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", f"-L{PKG}", "-lspectra_hip",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tdir}/lib", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch operator library failed to build:\n{r.stderr[-8000:]}")
    os.replace(tmp, TORCH_OPS_LIB)
    if verbose:
        print(f"built {TORCH_OPS_LIB}")
    return TORCH_OPS_LIB


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-8000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
