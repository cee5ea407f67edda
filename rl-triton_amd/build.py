"""Build the two in-tree libraries of the rl_triton package.

    python rl-triton_amd/build.py            # compile what is older than its sources
    python rl-triton_amd/build.py --force    # always compile

  librl_triton_amd.so   the gfx950 HIP kernels and their C ABI (include/rl_triton_amd.h),
                        hipcc, cross-compiled for gfx950 on a machine without a GPU
  _rlk_torch.so         the PyTorch-ROCm extension module over that C ABI
                        (csrc/rlk_torch.cpp), host code only, g++ against torch's headers
  librlk_stream_ceiling.so
                        the benchmark's streaming-ceiling kernel (csrc/bench/,
                        include/rlk_stream_ceiling.h); not used by the package

Both land next to the Python package (rl-triton_amd/rl_triton/), which loads them from
its own directory.
"""
from __future__ import annotations

import argparse
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB = os.path.join(HERE, "rl_triton", "librl_triton_amd.so")
EXT = os.path.join(HERE, "rl_triton", "_rlk_torch.so")
EXT_SRC = os.path.join(CSRC, "rlk_torch.cpp")
CEILING = os.path.join(HERE, "rl_triton", "librlk_stream_ceiling.so")
CEILING_SRC = os.path.join(CSRC, "bench", "stream_ceiling.hip")
ARCH = os.environ.get("RLK_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    # no packed-FP32 (v_pk_*_f32) code generation
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # every atomic here is issued by one lane; the wave-aggregating rewrite would consume
    # the ticket right after issuing it and stall the coordinator on it
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall", "-Wno-unused-result",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def deps() -> list[str]:
    return sources() + sorted(glob.glob(os.path.join(CSRC, "*.hpp"))) + [
        os.path.join(INCLUDE, "rl_triton_amd.h"), os.path.abspath(__file__)]


def up_to_date(target: str, inputs: list[str]) -> bool:
    if not os.path.exists(target):
        return False
    t = os.path.getmtime(target)
    return all(os.path.getmtime(d) <= t for d in inputs)


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib(force: bool = True, verbose: bool = False) -> str:
    if not force and up_to_date(LIB, deps()):
        return LIB
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    _run([hipcc, *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *sources(), "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_ceiling(force: bool = True, verbose: bool = False) -> str:
    inputs = [CEILING_SRC, os.path.join(INCLUDE, "rlk_stream_ceiling.h"), os.path.abspath(__file__)]
    if not force and up_to_date(CEILING, inputs):
        return CEILING
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = CEILING + ".tmp"
    _run([hipcc, *FLAGS, f"-I{INCLUDE}", CEILING_SRC, "-o", tmp], verbose)
    os.replace(tmp, CEILING)
    return CEILING


def build_ext(force: bool = True, verbose: bool = False) -> str:
    """_rlk_torch.so: a CPython extension module (no pybind11) linked against torch's
    libraries and against librl_triton_amd.so, found next to it at run time."""
    inputs = [EXT_SRC, os.path.join(INCLUDE, "rl_triton_amd.h"), os.path.abspath(__file__), LIB]
    if not force and up_to_date(EXT, inputs):
        return EXT
    import sysconfig

    import torch
    from torch.utils import cpp_extension
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    incs = [sysconfig.get_paths()["include"], INCLUDE,
            *cpp_extension.include_paths(device_type="cuda")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = EXT + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{i}" for i in incs], EXT_SRC, "-o", tmp,
           f"-L{torch_lib}", f"-L{os.path.dirname(LIB)}",
           "-ltorch_python", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10_hip", "-lc10",
           "-l:librl_triton_amd.so", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, EXT)
    return EXT


def build(force: bool = True, verbose: bool = False) -> list[str]:
    return [build_lib(force, verbose), build_ext(force, verbose), build_ceiling(force, verbose)]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    for path in build(force=a.force, verbose=a.verbose):
        print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
