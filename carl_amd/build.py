"""Build the native parts of carl_amd in-tree.

    python carl_amd/build.py          # engine + Python binding
    python carl_amd/build.py --oracle # also the CPU oracle (test infrastructure)

(Run by path: importing the carl_amd package needs the extension built here.)

Outputs (next to this file):
  libcarl_amd.so   HIP engine for gfx950 + C-ABI (include/carl_amd.h)
  _carl*.so        pybind11 module exposing carl_amd._carl.Env
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("CARL_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: every + - * / is one IEEE binary32 operation (the CPU
# model of the same physics is compiled the same way).  Packed FP32 math is
# disabled for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, cwd=ROOT)


def engine_path() -> Path:
    return PKG / "libcarl_amd.so"


def binding_path() -> Path:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return PKG / f"_carl{suffix}"


def build_engine() -> Path:
    out = engine_path()
    hipcc = str(ROCM / "bin" / "hipcc")
    _run([hipcc, *HIP_FLAGS, "-shared", "-o", str(out),
          str(CSRC / "engine.hip"), str(CSRC / "arena.cpp")])
    return out


def build_binding() -> Path:
    import pybind11

    out = binding_path()
    py_inc = sysconfig.get_paths()["include"]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          "-D__HIP_PLATFORM_AMD__", f"-I{py_inc}", f"-I{pybind11.get_include()}",
          f"-I{ROCM / 'include'}", str(CSRC / "binding.cpp"),
          f"-L{PKG}", "-lcarl_amd", f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(out)])
    return out


def build_oracle() -> Path:
    _run(["make", "-C", str(ROOT / "oracle"), "-B"])
    return ROOT / "oracle" / "liboracle.so"


def main(argv: list[str]) -> None:
    build_engine()
    build_binding()
    if "--oracle" in argv:
        build_oracle()


if __name__ == "__main__":
    main(sys.argv[1:])
