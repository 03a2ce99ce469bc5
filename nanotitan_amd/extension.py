"""Loaders for the native MoE path.

``get_hip_extension()`` plays the role of the reference's
``get_cuda_extension()`` (src/model/cuda_extension.py:5-14): it returns the
compiled op module and raises ``RuntimeError`` when it has not been built.
There is no CPU fallback anywhere on this path.

torch is imported first on purpose: torch ships its own HIP runtime
(``libamdhip64.so.7``), and the native libraries must bind to that same
runtime rather than load a second copy.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path
from types import ModuleType

import torch  # noqa: F401  (binds the HIP runtime before the native libraries load)

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libnanotitan_moe.so"
EXT_PATH = PKG / "_nanotitan_hip.so"


@lru_cache
def get_hip_extension() -> ModuleType:
    """The PyTorch-ROCm extension module with the reference op surface."""
    try:
        from nanotitan_amd import _nanotitan_hip
    except ImportError as exc:
        raise RuntimeError(
            "The nanoTitan HIP extension is not built "
            f"({EXT_PATH.name} / {LIB_PATH.name} missing or unloadable). "
            "Run `python -m nanotitan_amd.build` before selecting moe_backend='hip'."
        ) from exc
    return _nanotitan_hip


def load_op_library():
    """``torch.ops.nanotitan``: the op library the extension module registers
    on load (HIP kernels for GPU tensors, C++ kernels for CPU tensors, shape
    functions for meta tensors). Raises RuntimeError when it is not built."""
    get_hip_extension()
    return torch.ops.nanotitan
