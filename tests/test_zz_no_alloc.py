"""nt_dispatch_noalloc through the C ABI: the same outputs as nt_dispatch (the
entry point it is a variant of), bit for bit, on two calls in a row with the
second smaller (the scratch keeps the first call's contents), and the
documented error for sizes beyond its fixed scratch."""

import numpy as np
import pytest
import torch

from nanotitan_amd import capi
from nanotitan_amd.capi import call, current_stream, dtype_code, ptr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return capi.load()


def _outputs(T, k, E, d, dtype):
    A = T * k
    i32 = dict(dtype=torch.int32, device="cuda")
    return dict(
        counts=torch.full((E,), -7, **i32),
        offsets=torch.full((E + 1,), -7, **i32),
        packed_X=torch.zeros(A, d, dtype=dtype, device="cuda"),
        token_id=torch.full((A,), -7, **i32),
        expert=torch.full((A,), -7, **i32),
        packed_w=torch.zeros(A, dtype=torch.float32, device="cuda"),
        inv=torch.full((T, k), -7, **i32),
    )


def _args(o):
    return [ptr(o["counts"]), ptr(o["offsets"]), ptr(o["packed_X"]), ptr(o["token_id"]),
            ptr(o["expert"]), ptr(o["packed_w"]), ptr(o["inv"])]


def _inputs(T, k, E, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, d, generator=g).to(dtype).cuda()
    logits = torch.randn(T, E, generator=g)
    w, topk = torch.softmax(logits, -1).topk(k, dim=-1)
    return X, w.contiguous().cuda(), topk.to(torch.int32).contiguous().cuda()


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_dispatch_matches_dispatch_twice(lib, dtype):
    s = current_stream()
    dc = dtype_code(dtype)
    # Each call after the first is smaller than one before it (fewer tokens,
    # experts or columns): it must not depend on what those left in the
    # scratch. 128 experts over 1024 and 313 token blocks take the separate
    # histogram scan (above 8192 entries); the others sum the histogram
    # inside the pack.
    for T, k, E, d, seed in [(65536, 8, 128, 256, 3), (30720, 2, 8, 512, 1),
                             (20000, 8, 128, 128, 4), (3001, 8, 64, 256, 2)]:
        X, w, topk = _inputs(T, k, E, d, dtype, seed)
        print(f"[no-alloc] T={T} k={k} E={E} d={d} {dtype}", flush=True)
        ref = _outputs(T, k, E, d, dtype)
        nb = lib.nt_dispatch_workspace_bytes(T, k, E, d, dc)
        assert 0 < nb <= capi.NT_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        call("nt_dispatch", dc, ptr(X), ptr(w), ptr(topk), T, k, d, E, *_args(ref), ptr(ws), nb, s)
        got = _outputs(T, k, E, d, dtype)
        call("nt_dispatch_noalloc", dc, ptr(X), ptr(w), ptr(topk), T, k, d, E, *_args(got), s)
        torch.cuda.synchronize()
        for name in ref:
            assert torch.equal(_bits(got[name]), _bits(ref[name])), name
        # and the closed forms: counts = bincount, offsets = their exclusive scan
        want = np.bincount(topk.cpu().numpy().ravel(), minlength=E)
        assert np.array_equal(got["counts"].cpu().numpy(), want)
        assert np.array_equal(got["offsets"].cpu().numpy(), np.concatenate([[0], np.cumsum(want)]))


def test_noalloc_dispatch_rejects_sizes_beyond_scratch(lib):
    # 2**20 tokens x 1024 experts at 1 KiB rows need about 64 MiB of histogram.
    T, k, E, d = 1 << 20, 2, 1024, 512
    dc = capi.NT_BF16
    assert lib.nt_dispatch_workspace_bytes(T, k, E, d, dc) > capi.NT_NOALLOC_SCRATCH_BYTES
    z = torch.zeros(1, device="cuda")
    code = lib.nt_dispatch_noalloc(dc, ptr(z), ptr(z), ptr(z), T, k, d, E, ptr(z), ptr(z), ptr(z),
                                   ptr(z), ptr(z), ptr(z), ptr(z), current_stream())
    assert code == capi.NT_ERR_SCRATCH
    assert b"scratch" in lib.nt_strerror(code)
