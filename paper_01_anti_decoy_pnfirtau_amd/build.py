"""Build libpnfx.so (the gfx950 HIP kernels behind the C ABI in include/pnfx.h) and
_pnfx_torch.so (the torch.library registration of the pnfx ops over that ABI).

    python -m paper_01_anti_decoy_pnfirtau_amd.build

Compiles every ``csrc/*.hip`` with hipcc for gfx950 into ``_build/`` (in
parallel), then links ``libpnfx.so`` next to this file.  Packed-FP32 VALU
instructions are disabled for all device code.  ``csrc/torch_ops.cpp`` is host
code: g++ compiles it against torch's headers into ``_pnfx_torch.so``, which
finds ``libpnfx.so`` beside itself.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libpnfx.so")
TORCH_LIB = os.path.join(PKG, "_pnfx_torch.so")
INCLUDE = os.path.join(os.path.dirname(PKG), "include")
ARCH = os.environ.get("PNFX_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def _torch_paths() -> tuple[str, str, bool]:
    import torch

    root = os.path.dirname(torch.__file__)
    return os.path.join(root, "include"), os.path.join(root, "lib"), torch._C._GLIBCXX_USE_CXX11_ABI


def build_torch_ops(verbose: bool = True) -> str:
    """Compile csrc/torch_ops.cpp (host code) into _pnfx_torch.so, linked to libpnfx.so."""
    inc, libdir, abi = _torch_paths()
    tmp = TORCH_LIB + ".tmp%d" % os.getpid()
    cmd = ["g++", "-O2", "-fPIC", "-shared", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={int(abi)}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-I{inc}",
           f"-I{os.path.join(inc, 'torch', 'csrc', 'api', 'include')}", "-I/opt/rocm/include",
           os.path.join(CSRC, "torch_ops.cpp"), "-o", tmp, f"-L{PKG}", "-lpnfx", f"-L{libdir}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for torch_ops.cpp:\n{r.stdout}{r.stderr}")
    os.replace(tmp, TORCH_LIB)
    if verbose:
        print(f"built {TORCH_LIB}")
    return TORCH_LIB


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + 1)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.check_call(cmd)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    build()
