"""Build recipe for the package's native libraries (run from __graft_entry__.build()).

  librw_rocm.so   hipcc, gfx950 only: csrc/rw_rocm.hip (+ rw_kernels.hpp) and
                  the host-only model loader csrc/rw_model.cpp
  _rw_quant*.so   g++: the C++ mirror of the reference's quant API
                  (host/rw_quant.cpp) with its pybind11 binding

Every GPU translation unit is compiled with packed-FP32 instructions
disabled and without FP contraction (the kernels call fma explicitly where
they want one, so results do not depend on what the compiler fuses), and
with the leading kernel arguments preloaded into SGPRs at wave launch
(gfx950 kernarg preloading; the code object keeps the prologue that loads
them itself where the firmware does not preload): a wave's first scalar
loads of its arguments leave the start of every launch, which the decoder's
chains of small launches and the encoder's 256-launch step feel.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

LIB_ROCM = os.path.join(HERE, "librw_rocm.so")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_rocm(extra: list[str] | None = None) -> str:
    srcs = [os.path.join(CSRC, "rw_rocm.hip"), os.path.join(CSRC, "rw_model.cpp")]
    tmp = LIB_ROCM + ".tmp"
    _run([HIPCC, *HIP_FLAGS, *(extra or []), f"-I{INCLUDE}", f"-I{CSRC}", *srcs, "-o", tmp])
    os.replace(tmp, LIB_ROCM)
    return LIB_ROCM


def host_ext_path() -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(HERE, "_rw_quant" + suffix)


def build_host() -> str:
    import pybind11

    out = host_ext_path()
    tmp = out + ".tmp"
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        f"-I{INCLUDE}", f"-I{HOST}", f"-I{pybind11.get_include()}",
        f"-I{sysconfig.get_paths()['include']}",
        os.path.join(HOST, "rw_quant.cpp"), os.path.join(HOST, "py_quant.cpp"),
        "-o", tmp,
        f"-L{HERE}", "-lrw_rocm", "-Wl,-rpath,$ORIGIN",
    ])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_rocm()
    if os.path.exists(os.path.join(HOST, "py_quant.cpp")):
        build_host()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
