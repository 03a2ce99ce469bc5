"""In-tree build of the MoE expert path for MI355X (gfx950).

Two artefacts, both next to this file:

* ``libnanotitan_moe.so`` — the C ABI (``include/nanotitan_moe.h``): every HIP
  kernel, compiled by ``hipcc --offload-arch=gfx950``. No torch dependency.
* ``_nanotitan_hip.so`` — the PyTorch-ROCm extension module exposing the
  reference op surface (``csrc/torch_ext.cpp``: the pybind module and the
  ``torch.ops.nanotitan`` op library, whose CPU kernels are
  ``csrc/cpu_ops.cpp``), compiled by ``g++`` against torch's headers and
  linked to the C ABI library through ``$ORIGIN``.

Plain compiler invocations (no hipify, no cpp_extension JIT), so the built
files travel with the source tree. ``python -m nanotitan_amd.build`` rebuilds
both.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB = PKG / "libnanotitan_moe.so"
EXT = PKG / "_nanotitan_hip.so"

HIP_SOURCES = ["library.hip", "router.hip", "dispatch.hip", "combine.hip", "grouped_gemm.hip"]
OFFLOAD_ARCH = "gfx950"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

# Packed FP32 VALU ops are disabled for every HIP translation unit: hipcc
# would otherwise emit v_pk_{add,mul,fma}_f32 from ordinary float code.
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        # Drop hipcc's host-pass notice about the packed-fp32 target feature.
        err = "\n".join(
            ln for ln in proc.stderr.splitlines() if "packed-fp32-ops" not in ln
        )
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def _hipcc() -> str:
    cand = ROCM / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build_library(verbose: bool = False) -> Path:
    """Compile every .hip source for gfx950 and link libnanotitan_moe.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    # Generated sources (lookup tables) go to the build folder.
    _run([sys.executable, str(CSRC / "gen_gelu_table.py"), str(BUILD_DIR / "gelu_table_bf16.inc")],
         verbose)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{BUILD_DIR}", "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_extension(verbose: bool = False) -> Path:
    """Compile the torch extension module against the C ABI library."""
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # The CPU kernels' ordered fp32 sums must round each product before
        # the add, as the HIP kernels do.
        "-ffp-contract=off",
        str(CSRC / "torch_ext.cpp"),
        str(CSRC / "cpu_ops.cpp"),
        "-o",
        str(EXT.with_suffix(".so.tmp")),
        f"-I{INCLUDE}",
        *[f"-I{p}" for p in include_paths()],
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{ROCM / 'include'}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_nanotitan_hip",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-L{p}" for p in library_paths()],
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        f"-L{PKG}",
        "-lnanotitan_moe",
        "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd, verbose)
    os.replace(EXT.with_suffix(".so.tmp"), EXT)
    return EXT


def build_all(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(f"built {LIB.name} and {EXT.name}")
