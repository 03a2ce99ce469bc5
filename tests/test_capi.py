"""The C ABI boundary on the CPU: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the GPU."""

import re

import pytest

from nanotitan_amd import capi
from tests.conftest import ROOT

HEADER = ROOT / "include" / "nanotitan_moe.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nt_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    syms = declared_symbols()
    for name in ("nt_count_experts", "nt_pack_tokens", "nt_combine_tokens", "nt_combine_backward",
                 "nt_pack_backward", "nt_grouped_gemm", "nt_grouped_gemm_dx",
                 "nt_grouped_gemm_dw", "nt_dispatch", "nt_strerror"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    syms = declared_symbols()
    assert set(syms) == set(capi.EXPORTS), "capi.EXPORTS out of sync with the header"
    for name in syms:
        assert hasattr(lib, name), name


def test_strerror_and_version():
    lib = capi.load()
    assert lib.nt_strerror(capi.NT_OK) == b"success"
    assert b"workspace" in lib.nt_strerror(capi.NT_ERR_WORKSPACE)
    assert lib.nt_strerror(12345) == b"unknown status code"
    assert lib.nt_version() >= 100


def test_dispatch_block_tokens():
    """The router's count blocks follow the pack's: 64 tokens per block for rows up to
    1 KiB, 32 for wider rows, fewer when that leaves under 512 blocks of long rows."""
    lib = capi.load()
    bt = lib.nt_dispatch_block_tokens
    assert bt(30720, 2, 4096, capi.NT_BF16) == 32
    assert bt(30720, 2, 512, capi.NT_BF16) == 64
    assert bt(30720, 2, 1024, capi.NT_F32) < bt(30720, 2, 256, capi.NT_BF16)
    assert bt(4096, 2, 512, capi.NT_F32) == 8  # C1: 512 blocks of 2 KiB rows
    assert bt(100, 32, 8, capi.NT_F32) * 32 <= 2048
    assert bt(100, 0, 8, capi.NT_F32) == 0
    assert bt(100, 2, 8, 99) == 0


def test_workspace_sizes_are_sane():
    lib = capi.load()
    assert lib.nt_dispatch_workspace_bytes(30720, 2, 8, 512, capi.NT_BF16) > 0
    assert lib.nt_dispatch_workspace_bytes(-1, 2, 8, 512, capi.NT_BF16) == 0
    assert lib.nt_combine_workspace_bytes(61440, 30720) >= 4 * (61440 + 2 * 30720)


@pytest.mark.parametrize(
    "fn,args,code",
    [
        ("nt_grouped_gemm", (99, None, None, None, 8, 16, 8, 8, None, None, 0, None),
         capi.NT_ERR_DTYPE),
        ("nt_grouped_gemm", (capi.NT_BF16, None, None, None, 0, 16, 8, 8, None, None, 0, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_grouped_gemm_dw", (capi.NT_BF16, None, None, None, 2000, 16, 8, 8, None, None, 0,
                                None), capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_count_experts", (None, None, 10, 2, 4, None, None, 0, None), capi.NT_ERR_INVALID_ARG),
        ("nt_count_experts", (None, None, 10, 2, 1025, None, None, 0, None),
         capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_pack_tokens", (7, None, None, None, 4, 2, 8, 3, None, None, None, None, None, None,
                            None, 0, None), capi.NT_ERR_DTYPE),
        ("nt_combine_tokens", (capi.NT_F32, None, None, None, 4, 2, 8, None, None, 0, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_combine_inv", (capi.NT_F32, None, None, None, 4, 0, 8, capi.NT_F32, None, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_pack_backward_inv", (capi.NT_BF16, None, None, None, -3, 2, 8, None, None, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_route_topk_count", (None, 8, 4, 2, None, None, None, 0, None, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_route_topk_count", (None, 8, 4, 5, None, None, None, 16, None, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_route_topk_count", (None, 8, 1025, 2, None, None, None, 16, None, None),
         capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_route_topk_count", (None, 8, 4, 2, None, None, None, 24, None, None),
         capi.NT_ERR_INVALID_ARG),  # block size not a power of two
        ("nt_route_topk", (None, 8, 1025, 2, None, None, None, None), capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_grouped_gemm_dw_dx", (99, None, None, None, None, 8, 16, 8, 8, None, None, None, 0,
                                   None), capi.NT_ERR_DTYPE),
        ("nt_grouped_gemm_dw_dx_gelu", (capi.NT_BF16, None, None, None, None, None, 8, 16, 8, 8,
                                        None, None, None, 0, None), capi.NT_ERR_INVALID_ARG),
        ("nt_route_topk_backward", (None, None, None, 8, 1025, 2, None, None),
         capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_route_topk_backward", (None, None, None, 8, 64, 33, None, None),
         capi.NT_ERR_INVALID_ARG),
        ("nt_dispatch_counted", (capi.NT_BF16, None, None, None, 8, 2, 16, 1025, None, None,
                                 None, None, None, None, None, None, 0, None),
         capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_pack_backward_inv_route", (99, None, None, None, None, None, 8, 2, 16, 8, None,
                                        None, None, None), capi.NT_ERR_DTYPE),
        ("nt_pack_backward_inv_route", (capi.NT_BF16, None, None, None, None, None, 8, 2, 16,
                                        1025, None, None, None, None),
         capi.NT_ERR_TOO_MANY_EXPERTS),
        ("nt_pack_backward_inv_route", (capi.NT_BF16, None, None, None, None, None, 8, 33, 16,
                                        64, None, None, None, None), capi.NT_ERR_INVALID_ARG),
        ("nt_pack_backward_inv_route", (capi.NT_BF16, None, None, None, None, None, 8, 4, 16, 3,
                                        None, None, None, None), capi.NT_ERR_INVALID_ARG),  # k > E
        ("nt_pack_backward_inv_route", (capi.NT_BF16, None, None, None, None, None, 8, 2, 16, 8,
                                        None, None, None, None), capi.NT_ERR_INVALID_ARG),  # nulls
    ],
)
def test_argument_errors_return_codes(fn, args, code):
    lib = capi.load()
    assert getattr(lib, fn)(*args) == code


C_HOST = r"""
#include <stdio.h>
#include "nanotitan_moe.h"

/* The GELU-FFN layer sequence of the integration guide, compiled against the
   header only (never called here: there is no GPU on this machine). */
int layer(const float* logits, const void* X, int64_t T, int32_t E, int32_t k, int64_t d,
          int64_t f, const void* W_up, const void* W_down, float* gates, int32_t* topk,
          int32_t* counts, int32_t* offsets, void* packed_X, int32_t* token_id,
          int32_t* expert, float* packed_w, int32_t* inv, void* act, void* g, void* y,
          void* out, void* ws, size_t ws_bytes, hipStream_t stream) {
  int32_t TB = nt_dispatch_block_tokens(T, k, d, NT_BF16);
  int rc = nt_route_topk_count(logits, T, E, k, gates, topk, NULL, TB, (int32_t*)ws, stream);
  if (rc == NT_OK)
    rc = nt_dispatch_counted(NT_BF16, X, gates, topk, T, k, d, E, counts, offsets, packed_X,
                             token_id, expert, packed_w, inv, ws, ws_bytes, stream);
  if (rc == NT_OK)
    rc = nt_grouped_gemm_gelu(NT_BF16, packed_X, offsets, W_up, E, T * k, d, f, act, g, NULL, 0,
                              stream);
  if (rc == NT_OK)
    rc = nt_grouped_gemm(NT_BF16, act, offsets, W_down, E, T * k, f, d, y, NULL, 0, stream);
  if (rc == NT_OK) rc = nt_combine_inv(NT_BF16, y, inv, packed_w, T, k, d, NT_BF16, out, stream);
  return rc;
}

int main(void) {
  printf("%d|%s|%zu\n", nt_version(), nt_strerror(NT_ERR_WORKSPACE),
         nt_dispatch_workspace_bytes(30720, 2, 8, 512, NT_BF16));
  return 0;
}
"""


def test_plain_c_host_compiles_links_and_runs(tmp_path):
    """A C99 host (gcc, no HIP compiler, no C++) compiles against the header,
    links libnanotitan_moe.so and calls its host-only functions; the layer
    sequence of the integration guide type-checks against the header."""
    import shutil
    import subprocess
    from pathlib import Path

    gcc = shutil.which("gcc")
    rocm_inc = Path("/opt/rocm/include")
    if gcc is None or not (rocm_inc / "hip").is_dir():
        pytest.skip("gcc or the HIP headers are not available")
    src = tmp_path / "host.c"
    src.write_text(C_HOST)
    lib_dir = ROOT / "nanotitan_amd"
    exe = tmp_path / "host"
    cmd = [gcc, "-std=c99", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{rocm_inc}",
           f"-I{ROOT / 'include'}", str(src), f"-L{lib_dir}", "-lnanotitan_moe",
           f"-Wl,-rpath,{lib_dir}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.strip()
    version, message, ws = out.split("|")
    assert int(version) == capi.load().nt_version()
    assert message == capi.load().nt_strerror(capi.NT_ERR_WORKSPACE).decode()
    assert int(ws) == capi.load().nt_dispatch_workspace_bytes(30720, 2, 8, 512, capi.NT_BF16)
