"""ctypes binding of the C ABI in ``include/nanotitan_moe.h``.

This is the binding a non-torch host (or a test that wants to exercise the
boundary itself) uses: raw device pointers, sizes and a ``hipStream_t``.
``EXPORTS`` lists every symbol the header declares, with its ctypes
signature; ``load()`` checks that the library exports all of them.
"""

from __future__ import annotations

import ctypes
from ctypes import c_char_p, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from functools import lru_cache

from nanotitan_amd.extension import LIB_PATH

NT_F32, NT_F64, NT_F16, NT_BF16 = 0, 1, 2, 3
NT_OK = 0
NT_ERR_INVALID_ARG = 1
NT_ERR_DTYPE = 2
NT_ERR_TOO_MANY_EXPERTS = 3
NT_ERR_WORKSPACE = 4
NT_ERR_LAUNCH = 5
NT_ERR_TOO_LARGE = 6
NT_ERR_SCRATCH = 7
NT_MAX_EXPERTS = 1024
NT_NOALLOC_SCRATCH_BYTES = 4 << 20

_P = c_void_p  # any device pointer, hipStream_t included

EXPORTS: dict[str, tuple[object, list[object]]] = {
    "nt_strerror": (c_char_p, [c_int]),
    "nt_version": (c_int, []),
    "nt_stream_copy": (c_int, [_P, _P, c_size_t, c_int32, _P]),
    "nt_stream_fill": (c_int, [_P, c_size_t, c_uint32, _P]),
    "nt_stream_read": (c_int, [_P, c_size_t, _P, _P]),
    "nt_dispatch_workspace_bytes": (c_size_t, [c_int64, c_int32, c_int32, c_int64, c_int]),
    "nt_count_experts": (
        c_int,
        [_P, _P, c_int64, c_int32, c_int32, _P, _P, c_size_t, _P],
    ),
    "nt_pack_tokens": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P,
         c_size_t, _P],
    ),
    "nt_dispatch": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P, _P,
         c_size_t, _P],
    ),
    "nt_dispatch_counted": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P, _P,
         c_size_t, _P],
    ),
    "nt_dispatch_noalloc": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "nt_dispatch_block_tokens": (c_int32, [c_int64, c_int32, c_int64, c_int]),
    "nt_combine_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "nt_combine_tokens": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_combine_inv": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, c_int, _P, _P],
    ),
    "nt_combine_backward": (
        c_int,
        [c_int, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P],
    ),
    "nt_combine_backward_inv": (
        c_int,
        [c_int, _P, _P, _P, c_int, _P, c_int64, c_int32, c_int64, _P, _P, _P],
    ),
    "nt_pack_backward": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, c_int64, c_int64, c_int32, c_int64, _P, _P, _P, c_size_t,
         _P],
    ),
    "nt_pack_backward_inv": (
        c_int,
        [c_int, _P, _P, _P, c_int64, c_int32, c_int64, _P, _P, _P],
    ),
    "nt_pack_backward_inv_route": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, c_int64, c_int32, c_int64, c_int32, _P, _P, _P, _P],
    ),
    "nt_route_topk": (c_int, [_P, c_int64, c_int32, c_int32, _P, _P, _P, _P]),
    "nt_route_topk_count": (
        c_int,
        [_P, c_int64, c_int32, c_int32, _P, _P, _P, c_int32, _P, _P],
    ),
    "nt_route_topk_backward": (c_int, [_P, _P, _P, c_int64, c_int32, c_int32, _P, _P]),
    "nt_grouped_gemm_workspace_bytes": (c_size_t, [c_int, c_int32, c_int64, c_int64, c_int64]),
    "nt_grouped_gemm": (
        c_int,
        [c_int, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_gelu": (
        c_int,
        [c_int, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dx_gelu": (
        c_int,
        [c_int, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_swiglu": (
        c_int,
        [c_int, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dx_swiglu": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dx2": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dx": (
        c_int,
        [c_int, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dw": (
        c_int,
        [c_int, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dw_dx": (
        c_int,
        [c_int, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, c_size_t, _P],
    ),
    "nt_grouped_gemm_dw_dx_gelu": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, c_size_t,
         _P],
    ),
    "nt_grouped_gemm_dw_dx_swiglu": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P, _P,
         c_size_t, _P],
    ),
    "nt_grouped_gemm_dw_dx2": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, _P, _P, _P,
         c_size_t, _P],
    ),
}


class NativeError(RuntimeError):
    """A C-ABI call returned a status other than NT_OK."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


@lru_cache
def load() -> ctypes.CDLL:
    """Open libnanotitan_moe.so and attach signatures; raise if anything is missing."""
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m nanotitan_amd.build`")
    lib = ctypes.CDLL(str(LIB_PATH))
    missing = [name for name in EXPORTS if not hasattr(lib, name)]
    if missing:
        raise RuntimeError(f"{LIB_PATH.name} lacks exports: {missing}")
    for name, (res, args) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise NativeError on failure."""
    lib = load()
    code = getattr(lib, name)(*args)
    if code != NT_OK:
        raise NativeError(name, code, lib.nt_strerror(code).decode())


def dtype_code(dtype) -> int:
    import torch

    return {
        torch.float32: NT_F32,
        torch.float64: NT_F64,
        torch.float16: NT_F16,
        torch.bfloat16: NT_BF16,
    }[dtype]


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None for an empty tensor)."""
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def current_stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream
