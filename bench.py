"""MoE-layer forward+backward throughput on one MI355X (the BASELINE.json metric).

A step is one pass of the hot path over one batch: from router logits,
fp32 softmax / stable top-k / renorm, fused count + offsets + pack, grouped
GEMM up with the GELU in its epilogue, grouped GEMM down, combine
(activation dtype out), then the full backward to dX, dlogits, dW_up and
dW_down (the GELU backward fused into the down projection's dX GEMM). Inputs
are resident in HBM before the timed region. Headline workload: config C2
(30720 tokens, d=512, E=8, top-2, FFN 512->2048->512, bf16), synthetic seeded
data, random-init weights.

Prints ONE JSON line:

* ``value``: tokens/s over K timed steps with only the step's own launches
  on the stream, after W warmup steps launched the same way. The headline
  runs right after the other GPU legs below, the last of which are C4's
  layer steps (its inputs already resident), so its steps start on a device
  at its working clocks, as in a training loop that runs layer after layer:
  measured step by step on MI355X, C2 steps that follow 200 ms of idle GPU
  (or memory-bound work) run 10-25% slower for their first 10-20 steps
  while the clocks ramp, and steps that follow GEMM work do not.
* ``roofline``: the dominant kernel family (the grouped GEMMs): algorithmic
  FLOPs per launch (2*A*K*N) over the average launch duration, measured with
  HIP events on the launch stream around every launch in a second timed pass
  over the same K steps (the event markers slow the step by a few percent, so
  that pass does not feed ``value``).
* ``kernels``: the HBM-bound kernels inside those steps (warm: at C2 the
  working set fits the 256 MB Infinity Cache). ``kernels_cold``: the same
  kernels standalone, each launch preceded by a full read of a 512 MB scratch
  buffer outside the events, so their operands come from HBM; median over
  the repetitions.
  ``copy_ceiling``: the library's own 16-byte streaming copy under the same
  cold rule, at about the HBM kernels' sizes, the achievable bandwidth they
  are measured against, and beside it a write-only fill and a read-only pass
  of the same byte counts (the ceilings of write- and read-dominated mixes).
* ``configs``: the other BASELINE.json configs (C1, C3, C4, C5) through the
  same measurement with fewer steps: ms/step, tokens/s, GEMM TF/s and its
  fraction of the roof, the HBM kernels in the layer and cold.
* ``cpu_baseline``: the CPU restatement of the reference torch path on the
  headline inputs, all of them when 1 warmup + 3 timed iterations fit the
  budget (C2 does), else their first tokens (rank 0, N=1 only); and
  ``configs.C1.cpu_baseline``: the same on C1 (fp32, the reference CPU
  path's config), 2 warmup + 5 timed iterations.

Headline and C1 inputs are drawn on the CPU with a seeded generator and
copied to the GPU, so the CPU baselines run on the same bits; the other
configs are drawn on the GPU (no CPU run uses them).

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 50] [--config 2]
       [--ffn gelu|swiglu] [--configs all|none|1,3,...]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from bench_profiles import kernel_source_hash  # noqa: E402

METRIC = "MoE layer fwd+bwd tokens/sec (1×MI355X); pack/combine HBM GB/s; GEMM MFMA %"
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {torch.bfloat16: 2500.0, torch.float16: 2500.0, torch.float32: 157.3}
# Read between cold timings: twice the Infinity Cache. A read leaves the
# caches holding clean, unrelated lines; a write would leave dirty lines whose
# write-back lands inside the next timed kernel (measured: C4 combine 5.0 ->
# 3.4 TB/s, the 400 MB copy 5.5 -> 3.8 TB/s).
SCRATCH_BYTES = 512 << 20

# name: (dtype, T, d, E, k, f, weight std, logit std)
WORKLOADS = {
    1: ("C1", torch.float32, 4096, 512, 8, 2, 2048, 0.02, 1.0),
    2: ("C2", torch.bfloat16, 30720, 512, 8, 2, 2048, 0.02, 1.0),
    3: ("C3", torch.bfloat16, 30720, 512, 64, 8, 256, 0.02, 1.0),
    4: ("C4", torch.bfloat16, 16384, 4096, 8, 2, 14336, 0.01, 1.0),
    5: ("C5", torch.float16, 65536, 2048, 128, 8, 768, 0.02, 2.0),
}
SEED = 1234


def make_workload(cfg_id: int, device: str, seed: int = SEED, draw: str = "cpu"):
    """Synthetic inputs of config C<cfg_id>: X, logits (with the config's edits),
    weights, dY. ``draw="cpu"``: drawn with a CPU generator, then copied to
    ``device`` (the same bits on every device); ``draw="device"``: drawn on
    ``device`` directly (faster for the large configs)."""
    name, dtype, T, d, E, k, f, wstd, lstd = WORKLOADS[cfg_id]
    gdev = "cpu" if draw == "cpu" else device
    g = torch.Generator(device=gdev).manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=gdev)

    X = randn(T, d).to(dtype)
    logits = randn(T, E) * lstd
    if cfg_id == 3:  # Zipf(1.2) expert popularity as a log-prior bias
        z = torch.tensor([(i + 1) ** -1.2 for i in range(E)], dtype=torch.float64)
        perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed))
        logits += torch.log(z[perm] / z.sum()).float().to(gdev)
    if cfg_id == 5:  # 16 dead experts, 1% of tokens with all live logits tied
        cg = torch.Generator().manual_seed(seed)
        dead = torch.randperm(E, generator=cg)[:16]
        ties = torch.randperm(T, generator=cg)[: math.ceil(T / 100)]
        live = torch.ones(E, dtype=torch.bool)
        live[dead] = False
        logits[ties.to(gdev).unsqueeze(1), live.nonzero().squeeze(1).to(gdev).unsqueeze(0)] = 0.0
        logits[:, dead.to(gdev)] = float("-inf")
    W_up = (randn(E, d, f) * wstd).to(dtype)
    W_down = (randn(E, f, d) * wstd).to(dtype)
    dY = randn(T, d).to(dtype)
    wl = dict(name=name, dtype=dtype, T=T, d=d, E=E, k=k, f=f, X=X, logits=logits,
              W_up=W_up, W_down=W_down, dY=dY, seed=seed, draw=draw)
    for key in ("X", "logits", "W_up", "W_down", "dY"):
        wl[key] = wl[key].to(device)
    return wl


# Algorithmic bytes of the HBM-bound kernels (each tensor touched once):
# dispatch reads X, the ids and gates and writes the packed rows, ids and
# gates; combine reads the packed rows, gates and the inverse map and writes
# [T,d]; combine backward reads dY once and the packed rows, writes dy and
# dw; pack backward reads the packed grads, gate grads and inverse map and
# writes dX and dw.
def hbm_bytes(kind, T, d, A, b, b_out=None, b_grad=None, E=None):
    if kind == "dispatch":
        return T * d * b + A * d * b + 8.0 * A + 12.0 * A
    if kind == "combine_fwd":
        return A * d * b + 8.0 * A + T * d * (b if b_out is None else b_out)
    if kind == "combine_bwd":
        return T * d * (b if b_grad is None else b_grad) + 2.0 * A * d * b + 12.0 * A
    if kind == "pack_bwd":
        return A * d * b + T * d * b + 12.0 * A
    if kind == "pack_bwd_route":  # no dw; reads gates and ids, writes dlogits [T,E] f32
        return A * d * b + T * d * b + 16.0 * A + 4.0 * T * E
    raise ValueError(kind)


class LaunchTimer:
    """Wraps the native module: HIP events around selected ops on the current stream."""

    FAMILIES = {
        "grouped_gemm_kernel": "gemm",
        "grouped_gemm_gelu": "gemm",
        "bwd_grouped_gemm_dX_kernel": "gemm",
        "bwd_grouped_gemm_dX_gelu": "gemm",
        "bwd_grouped_gemm_dW_kernel": "gemm",
        "bwd_grouped_gemm_dW_dX": "gemm",
        "bwd_grouped_gemm_dW_dX_gelu": "gemm",
        "grouped_gemm_swiglu": "gemm",
        "bwd_grouped_gemm_dX_swiglu": "gemm",
        "bwd_grouped_gemm_dW_dX_swiglu": "gemm",
        "bwd_grouped_gemm_dW_dX2": "gemm",
        "bwd_grouped_gemm_dX2": "gemm",
        "dispatch_tokens": "dispatch",
        "dispatch_tokens_counted": "dispatch",
        "combine_inv": "combine_fwd",
        "combine_backward_inv": "combine_bwd",
        "pack_backward_inv": "pack_bwd",
        "pack_backward_inv_route": "pack_bwd",
    }

    def __init__(self, ext):
        self._ext = ext
        self.active = False
        self.records = []  # (family, name, start_event, end_event, work, launches)

    def __getattr__(self, name):
        fn = getattr(self._ext, name)
        fam = self.FAMILIES.get(name)
        if fam is None:
            return fn

        def timed(*args):
            if not self.active:
                return fn(*args)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            out = fn(*args)
            e.record()
            self.records.append((fam, name, s, e, self._work(name, args), self._launches(name)))
            return out

        return timed

    @staticmethod
    def _launches(name):
        """GEMMs inside one call (the paired dW + dX calls hold two, which may
        run side by side: the pair's span is their joint time). SwiGLU: the
        gate|value forward and the two-part dX (reduction over gate and value)
        count as two GEMMs each, the dW_gate + two-part dX pair as three."""
        if name in ("bwd_grouped_gemm_dW_dX", "bwd_grouped_gemm_dW_dX_gelu", "grouped_gemm_swiglu",
                    "bwd_grouped_gemm_dW_dX_swiglu", "bwd_grouped_gemm_dX2"):
            return 2
        return 3 if name == "bwd_grouped_gemm_dW_dX2" else 1

    @staticmethod
    def _work(name, args):
        """Algorithmic work of one launch: FLOPs for GEMMs, bytes otherwise."""
        if name in ("grouped_gemm_kernel", "grouped_gemm_gelu"):
            X, _off, W = args
            return 2.0 * X.shape[0] * X.shape[1] * W.shape[2]
        if name in ("bwd_grouped_gemm_dX_kernel", "bwd_grouped_gemm_dX_gelu"):
            W, _off, G = args[:3]
            return 2.0 * G.shape[0] * W.shape[1] * W.shape[2]
        if name == "grouped_gemm_swiglu":  # X [A,d], W_gate, W_val [E,d,f]
            X, _off, Wg = args[:3]
            return 2 * 2.0 * X.shape[0] * X.shape[1] * Wg.shape[2]
        if name == "bwd_grouped_gemm_dX_swiglu":  # W_out [E,f,d], dy [A,d]
            W, _off, G = args[:3]
            return 2.0 * G.shape[0] * W.shape[1] * W.shape[2]
        if name == "bwd_grouped_gemm_dW_dX_swiglu":  # hidden [A,f], dy [A,d]
            h, _W, _off, G = args[:4]
            return 2 * 2.0 * h.shape[0] * h.shape[1] * G.shape[1]
        if name in ("bwd_grouped_gemm_dW_dX2", "bwd_grouped_gemm_dX2"):
            # two-part dX over the gate|value reduction (+ dW_gate when paired)
            Wg = args[1] if name == "bwd_grouped_gemm_dW_dX2" else args[0]
            dg = args[-2]
            E, d, f = Wg.shape
            return (3 if name == "bwd_grouped_gemm_dW_dX2" else 2) * 2.0 * dg.shape[0] * d * f
        if name == "bwd_grouped_gemm_dW_kernel":
            X, _off, G = args
            return 2.0 * X.shape[0] * X.shape[1] * G.shape[1]
        if name in ("bwd_grouped_gemm_dW_dX", "bwd_grouped_gemm_dW_dX_gelu"):
            X, _W, _off, G = args[:4]
            return 2 * 2.0 * X.shape[0] * X.shape[1] * G.shape[1]
        if name in ("dispatch_tokens", "dispatch_tokens_counted"):
            X, _w, topk = args[:3]
            return hbm_bytes("dispatch", X.shape[0], X.shape[1], topk.numel(), X.element_size())
        if name == "combine_inv":
            y, inv, _w, out_dtype = args
            ob = torch.empty(0, dtype=out_dtype).element_size()
            return hbm_bytes("combine_fwd", inv.shape[0], y.shape[1], y.shape[0],
                             y.element_size(), b_out=ob)
        if name == "combine_backward_inv":
            y, inv, _w, dY = args
            return hbm_bytes("combine_bwd", inv.shape[0], y.shape[1], y.shape[0],
                             y.element_size(), b_grad=dY.element_size())
        if name == "pack_backward_inv":
            dpX, _dpw, inv = args
            return hbm_bytes("pack_bwd", inv.shape[0], dpX.shape[1], dpX.shape[0],
                             dpX.element_size())
        if name == "pack_backward_inv_route":
            dpX, _dpw, inv, _gates, _topk, E = args
            return hbm_bytes("pack_bwd_route", inv.shape[0], dpX.shape[1], dpX.shape[0],
                             dpX.element_size(), E=E)
        return 0.0

    def summary(self):
        out = {}
        for fam, name, s, e, work, launches in self.records:
            ms = s.elapsed_time(e)
            r = out.setdefault(fam, {"launches": 0, "ms": 0.0, "work": 0.0})
            r["launches"] += launches
            r["ms"] += ms
            r["work"] += work
        return out


class _GeluFFN(torch.nn.Module):
    """Up -> GELU -> down experts on the fused grouped GEMMs (the layer's GeluExpertFFN)."""

    def __init__(self, W_up, W_down):
        super().__init__()
        self.W_up = W_up
        self.W_down = W_down

    def forward(self, packed_X, offsets):
        from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn

        return grouped_gelu_ffn_fn(packed_X, self.W_up, self.W_down, offsets)


class _SwiGLUFFN(torch.nn.Module):
    """The reference's ExpertFFN (src/model/feed_fwd.py:102-112): silu(X W_gate) * (X W_val), then W_out."""

    def __init__(self, W_gate, W_val, W_out):
        super().__init__()
        self.W_gate, self.W_val, self.W_out = W_gate, W_val, W_out

    def forward(self, packed_X, offsets):
        from nanotitan_amd.moe_ops import swiglu_ffn_fn

        return swiglu_ffn_fn(packed_X, self.W_gate, self.W_val, self.W_out, offsets)


def gemm_roof(wl):
    """Roof of the config's grouped GEMMs: the dense MFMA peak of its dtype,
    or HBM bandwidth x arithmetic intensity when that is lower (C3). The
    intensity is the up-projection's 2*A*d*f over (A*d + E*d*f + A*f) bytes."""
    A, d, f, E = wl["T"] * wl["k"], wl["d"], wl["f"], wl["E"]
    b = torch.empty(0, dtype=wl["dtype"]).element_size()
    ai = 2.0 * A * d * f / ((A * d + E * d * f + A * f) * b)
    peak = PEAK_TFLOPS[wl["dtype"]]
    hbm_roof = ai * PEAK_HBM_GBS / 1e3
    return dict(peak_tflops=peak, intensity_flop_per_byte=round(ai, 1),
                roof_tflops=round(min(peak, hbm_roof), 1),
                bound="mfma" if peak <= hbm_roof else "hbm")


def run_layer(timer, wl, steps, warmup, ffn_kind):
    """Warmup, then K timed steps without markers, then K steps with HIP
    events around every launch. Returns the timings and per-family records."""
    from nanotitan_amd.layer import moe_forward_from_logits

    W_up = wl["W_up"].detach().requires_grad_(True)
    W_down = wl["W_down"].detach().requires_grad_(True)
    W_val = None
    ffn = _GeluFFN(W_up, W_down)
    if ffn_kind == "swiglu":  # W_up serves as W_gate and W_down as W_out
        g = torch.Generator(device="cuda").manual_seed(4321)
        std = WORKLOADS[int(wl["name"][1])][7]
        W_val = (torch.randn(W_up.shape, generator=g, device="cuda") * std).to(wl["dtype"])
        W_val.requires_grad_(True)
        ffn = _SwiGLUFFN(W_up, W_val, W_down)

    def step():
        x = wl["X"].detach().requires_grad_(True)
        logits = wl["logits"].detach().requires_grad_(True)
        out, _counts, _gates = moe_forward_from_logits(x, logits, ffn, wl["E"], wl["k"])
        out.backward(wl["dY"])
        W_up.grad = W_down.grad = None
        if W_val is not None:
            W_val.grad = None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    timer.records.clear()
    timer.active = True
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed_events = time.perf_counter() - t1
    timer.active = False
    fams = timer.summary()
    timer.records.clear()
    return elapsed, elapsed_events, fams


def family_report(fams, wl):
    """GEMM TF/s against the roof, HBM kernels' GB/s against 8 TB/s."""
    kernels = {}
    for fam, r in fams.items():
        avg_ms = r["ms"] / r["launches"]
        per = r["work"] / r["launches"]
        if fam == "gemm":
            roof = gemm_roof(wl)
            tf = per / avg_ms / 1e9
            kernels[fam] = {"avg_ms": round(avg_ms, 4), "tflops": round(tf, 2),
                            "frac_of_peak": round(tf / roof["peak_tflops"], 4),
                            "frac_of_roof": round(tf / roof["roof_tflops"], 4), **roof}
        else:
            gbs = per / (avg_ms * 1e-3) / 1e9
            kernels[fam] = {"avg_ms": round(avg_ms, 4), "GB_s": round(gbs, 1),
                            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": per}
    return kernels


_SINK = {}


def _flush(scratch):
    """Read all of `scratch` with the library's streaming read (evicts the
    L2s and the Infinity Cache; no temporaries, nothing written)."""
    from nanotitan_amd.extension import get_hip_extension

    dev = scratch.device
    if dev not in _SINK:
        _SINK[dev] = torch.zeros(1, dtype=torch.int32, device=dev)
    get_hip_extension().stream_read(scratch, _SINK[dev])


def _cold_median(fn, scratch, reps):
    """Median device time of fn() (HIP events on the current stream), each
    launch preceded by a full read of `scratch` outside the events."""
    times = []
    for _ in range(reps):
        _flush(scratch)
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return statistics.median(times)


def cold_hbm_kernels(ext, wl, scratch, reps=10):
    """The layer's HBM-bound kernels standalone on this config's routing, cold."""
    T, d, E, k = wl["T"], wl["d"], wl["E"], wl["k"]
    A = T * k
    b = torch.empty(0, dtype=wl["dtype"]).element_size()
    X, dY = wl["X"], wl["dY"]
    gates, topk = ext.route_topk(wl["logits"].contiguous(), k)
    _c, _o, packed_X, _tid, _ex, packed_w, inv = ext.dispatch_tokens(X, gates, topk, E)
    y = packed_X  # expert outputs: any [A,d] rows of the activation dtype
    cases = {
        "dispatch": (lambda: ext.dispatch_tokens(X, gates, topk, E),
                     hbm_bytes("dispatch", T, d, A, b)),
        "combine_fwd": (lambda: ext.combine_inv(y, inv, packed_w, wl["dtype"]),
                        hbm_bytes("combine_fwd", T, d, A, b)),
        "combine_bwd": (lambda: ext.combine_backward_inv(y, inv, packed_w, dY),
                        hbm_bytes("combine_bwd", T, d, A, b)),
        "pack_bwd": (lambda: ext.pack_backward_inv(y, packed_w, inv),
                     hbm_bytes("pack_bwd", T, d, A, b)),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        fn()  # first launch (code object load, allocator) outside the timing
        ms = _cold_median(fn, scratch, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 1), "GB_s": round(gbs, 1),
                     "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes}
    return out


def copy_ceiling(ext, scratch, reps=10):
    """The library's streaming copy (nt_stream_copy), cold, at about the
    bytes the HBM kernels move (C1: 25 and 42 MB, C2: 95 and 158 MB, C4:
    400 MB, C5: 2.4 GB):
    GB/s of bytes read + written. Short copies do not reach the long ones'
    rate (launch fill and drain), so each kernel compares with its size.
    Beside it, at the same byte counts, the write-only fill (nt_stream_fill:
    the ceiling of a kernel that mostly writes, like the dispatch's k copies
    of each row) and the read-only pass (nt_stream_read)."""
    out = {}
    for label, moved in (("moved_25MB", 25e6), ("moved_42MB", 42e6), ("moved_95MB", 95e6),
                         ("moved_158MB", 158e6), ("moved_400MB", 400e6), ("moved_2400MB", 2400e6)):
        n = int(moved // 2) // 16 * 16
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        ext.stream_copy(dst, src)
        ms = _cold_median(lambda: ext.stream_copy(dst, src), scratch, reps)
        gbs = 2.0 * n / (ms * 1e-3) / 1e9
        out[label] = {"us": round(ms * 1e3, 1), "GB_s": round(gbs, 1),
                      "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
        del src, dst
        buf = torch.empty(2 * n, dtype=torch.uint8, device="cuda")
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        for kind, fn in (("write", lambda: ext.stream_fill(buf, 0)),
                         ("read", lambda: ext.stream_read(buf, sink))):
            fn()
            ms = _cold_median(fn, scratch, reps)
            gbs = 2.0 * n / (ms * 1e-3) / 1e9
            out[label.replace("moved", kind)] = {"us": round(ms * 1e3, 1), "GB_s": round(gbs, 1),
                                                 "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
        del buf
    torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(wl_cpu, budget_s: float = 20.0, warmup: int = 1, max_iters: int = 3):
    """The reference torch CPU path (oracle restatement) on the same inputs
    the GPU ran (drawn on the CPU): the whole workload when `warmup` +
    `max_iters` iterations fit in about budget_s (C2: 1 + 3, C1: 2 + 5, as
    planned for the baseline), else its first tokens, sized to ~budget_s."""
    from oracle import moe_oracle as O

    host_cores = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", host_cores))
    torch.set_num_threads(max(1, min(host_cores, cap)))
    k, T0 = wl_cpu["k"], wl_cpu["T"]
    weights = {"up": wl_cpu["W_up"], "down": wl_cpu["W_down"]}

    def layer(T):
        O.moe_layer_torch(wl_cpu["X"][:T], wl_cpu["logits"][:T], weights, k, ffn="gelu",
                          dY=wl_cpu["dY"][:T])

    # Size the sample from a 256-token probe so that warmup + timed
    # iterations stay near budget_s (fp16 on the CPU is slow at C5).
    T = min(T0, 256)
    layer(T)
    t0 = time.perf_counter()
    layer(T)
    per_token = (time.perf_counter() - t0) / T
    fit = budget_s / (warmup + max_iters) / per_token
    T = T0 if fit >= T0 else int(max(256, fit) // 256 * 256)
    print(f"bench.py: cpu_baseline {wl_cpu['name']} sample {T} tokens "
          f"(~{per_token * T:.2f} s per iteration)", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for _ in range(warmup):
        layer(T)
    first = (time.perf_counter() - t0) / max(warmup, 1)
    iters = max(1, min(max_iters, int(budget_s / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(iters):
        layer(T)
    dt = (time.perf_counter() - t0) / iters
    return {
        "value": T / dt,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "host_cores": host_cores,
        "thread_cap": os.environ.get("OMP_NUM_THREADS"),
        "kind": "port",
        "tokens": T,
        "sample": f"{wl_cpu['name']} inputs (seed {wl_cpu['seed']}, drawn on the CPU, "
                  f"the same bits the GPU ran): "
                  + (f"all {T0} tokens" if T == T0 else f"first {T} of {T0} tokens")
                  + f", {wl_cpu['dtype']}, "
                  f"{warmup} warmup + {iters} timed fwd+bwd iterations on {torch.get_num_threads()} "
                  f"threads of {host_cores} host cores (thread cap OMP_NUM_THREADS="
                  f"{os.environ.get('OMP_NUM_THREADS', 'unset')}); host CPU: {cpu_model()}; "
                  f"torch {torch.__version__}",
    }


def profile_fields(wl, ffn_kind):
    """HBM traffic and MFMA busy fraction of the GEMMs from the committed
    rocprofv3 counter summaries (profiles/*.json, written by bench_profiles.py),
    tagged with the commit whose kernels they were measured on and marked
    stale when the kernel sources have changed since."""
    out = {}
    if ffn_kind != "gelu":
        return out
    prof = ROOT / "profiles" / f"traffic_{wl['name'].lower()}.json"
    if prof.exists():
        js = json.loads(prof.read_text())
        fams_t = js.get("families", {})
        # GEMM launches of one step: up (fused GELU), down, and the backward's
        # down dX (fused GELU backward), up dX and two dW, either as paired
        # launches (dW + dX in one kernel, two GEMMs each) or one by one;
        # traffic per GEMM averaged over the six.
        per_step = {"gemm_fwd_gelu": 1, "gemm_fwd": 1, "gemm_pair_dw_dx_gelu": 1,
                    "gemm_pair_dw_dx": 1}
        if not all(f in fams_t for f in per_step):
            per_step = {"gemm_fwd_gelu": 1, "gemm_fwd": 1, "gemm_dx_gelu": 1, "gemm_dx": 1,
                        "gemm_dw": 2}
        if all(f in fams_t for f in per_step):
            n = 6
            out["traffic"] = round(sum(fams_t[f]["bytes"] * c for f, c in per_step.items()) / n)
            out["traffic_algorithmic"] = round(
                sum(fams_t[f]["algorithmic_bytes"] * c for f, c in per_step.items()) / n)
            out["traffic_source"] = source_note(prof, js)
    mf = ROOT / "profiles" / f"mfma_{wl['name'].lower()}.json"
    if mf.exists():
        js = json.loads(mf.read_text())
        fam_m = js.get("families", {})
        t_all = sum(v["launches"] * v["avg_us"] for v in fam_m.values())
        if t_all > 0:
            def tw(key):
                return sum(v[key] * v["launches"] * v["avg_us"] for v in fam_m.values()) / t_all
            out["mfma_busy_frac"] = round(tw("mfma_busy_frac"), 4)
            out["clock_ghz"] = round(tw("clock_ghz"), 3)
            out["mfma_source"] = source_note(mf, js)
    return out


def source_note(path, js):
    """Where a profile figure comes from, and whether the kernel sources it
    was measured on are the ones this run executes."""
    same = js.get("source_hash") == kernel_source_hash(ROOT)
    return (f"profiles/{path.name}, kernels of commit {js.get('commit', 'unrecorded')}"
            f"{'' if same else ' (kernel sources changed since: stale)'}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--configs", default="all",
                    help="secondary configs to measure as well: all, none, or ids like 1,3,4")
    ap.add_argument("--config-steps", type=int, default=20)
    ap.add_argument("--config-warmup", type=int, default=10)
    ap.add_argument("--cold-reps", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--ffn", choices=["gelu", "swiglu"], default="gelu",
                    help="expert FFN: the configs' up->GELU->down (headline) or the reference's "
                         "SwiGLU ExpertFFN")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run 5 device copies of 1 GiB (HBM counter calibration) and exit")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            f"bench.py: --gpus {args.gpus} requested, but this build measures one MI355X only; "
            "the MoE expert path runs on a single GPU here (multi-GPU expert parallelism is "
            "not built). Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    import nanotitan_amd.moe_ops as moe_ops
    from nanotitan_amd.extension import get_hip_extension

    ext = get_hip_extension()

    if args.copy_probe:
        nbytes = 1 << 30
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            ext.stream_copy(dst, src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes,
                          "launches": 5}), flush=True)
        return

    timer = LaunchTimer(ext)
    moe_ops.get_hip_extension = lambda: timer

    torch.manual_seed(0)
    wl_cpu = make_workload(args.config, "cpu", draw="cpu")

    # The other GPU legs (cold-cache kernel timings, copy ceilings, the other
    # configs) run first and the headline last.
    scratch = torch.ones(SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    # The headline inputs stay resident from here on, so that its warmup
    # follows the last GPU leg with no host-side copy in between.
    wl = {k: (v.to("cuda") if isinstance(v, torch.Tensor) else v) for k, v in wl_cpu.items()}
    kernels_cold = cold_hbm_kernels(ext, wl, scratch, args.cold_reps)
    ceiling = copy_ceiling(ext, scratch, args.cold_reps)

    configs = {}
    cpu_configs = {}
    if args.configs != "none":
        ids = sorted(WORKLOADS) if args.configs == "all" else [int(c) for c in args.configs.split(",")]
        # C4 (the GEMM-heaviest) last, and each config's cold kernel timings
        # before its layer steps: the headline then follows layer steps.
        ids = sorted(ids, key=lambda c: (c == 4, c))
        for cid in ids:
            if cid == args.config:
                continue
            # C1 (the CPU path's own config, 4096 tokens) is drawn on the CPU,
            # so its CPU baseline runs on the bits the GPU ran.
            if cid == 1:
                w_cpu = make_workload(cid, "cpu", draw="cpu")
                w2 = {k: (v.to("cuda") if isinstance(v, torch.Tensor) else v)
                      for k, v in w_cpu.items()}
                cpu_configs[w2["name"]] = w_cpu
            else:
                w2 = make_workload(cid, "cuda", draw="device")
            cold2 = cold_hbm_kernels(ext, w2, scratch, args.cold_reps)
            e2, ee2, f2 = run_layer(timer, w2, args.config_steps, args.config_warmup, args.ffn)
            rep = family_report(f2, w2)
            configs[w2["name"]] = {
                "workload": f"{w2['T']} tokens x d={w2['d']}, E={w2['E']}, top-{w2['k']}, "
                            f"FFN {w2['d']}->{w2['f']}->{w2['d']}, {w2['dtype']}",
                "tokens_per_s": round(w2["T"] * args.config_steps / e2, 1),
                "ms_per_step": round(e2 / args.config_steps * 1e3, 4),
                "steps": args.config_steps,
                "warmup": args.config_warmup,
                "gemm": rep.pop("gemm", None),
                "hbm_in_layer": rep,
                "hbm_cold": cold2,
            }
            del w2
            if cid != ids[-1]:  # no cache release (hipFree calls, an idle GPU) before the headline
                torch.cuda.empty_cache()
    del scratch

    elapsed, elapsed_events, fams = run_layer(timer, wl, args.steps, args.warmup, args.ffn)

    ms_per_step = elapsed / args.steps * 1e3
    tokens_per_s = wl["T"] * args.steps / elapsed
    gemm = fams.get("gemm", {"launches": 0, "ms": 0.0, "work": 0.0})
    peak = PEAK_TFLOPS[wl["dtype"]]
    achieved = (gemm["work"] / (gemm["ms"] * 1e-3) / 1e12) if gemm["ms"] > 0 else 0.0
    roofline = {
        "bound": "mfma",
        "kernel": "grouped GEMM (fwd, dX, dW launches)",
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "traffic": None,
        "flops_per_launch": gemm["work"] / max(gemm["launches"], 1),
        "avg_launch_ms": gemm["ms"] / max(gemm["launches"], 1),
        "timing": f"HIP events around each launch, second pass of the {args.steps} steps "
                  f"({elapsed_events / args.steps * 1e3:.4f} ms/step with the events); a paired "
                  f"dW + dX call counts as two launches over its joint span",
    }
    roofline.update(profile_fields(wl, args.ffn))
    kernels = family_report(fams, wl)
    del wl
    torch.cuda.empty_cache()

    name, dtype_, T, d, E, k, f, _ws, _ls = WORKLOADS[args.config]
    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype_],
        "data": "synthetic (seeded N(0,1) activations/logits, N(0,std^2) random-init expert "
                "weights; headline drawn on the CPU)",
        "config": {
            "workload": f"{name}: MoE layer fwd+bwd, {T} tokens x d={d}, E={E}, top-{k}, "
                        f"FFN {d}->{f}->{d} "
                        + ("GELU" if args.ffn == "gelu" else "SwiGLU (reference ExpertFFN)"),
            "tokens": T,
            "d_model": d,
            "num_experts": E,
            "top_k": k,
            "ffn": f,
            "parallelism": "single-gpu",
        },
        "roofline": roofline,
        "kernels": kernels,
        "kernels_cold": kernels_cold,
        "copy_ceiling": ceiling,
        "configs": configs,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl_cpu, args.cpu_budget)
        for name, w_cpu in cpu_configs.items():  # C1: 2 warmup + 5 timed iterations
            configs[name]["cpu_baseline"] = cpu_baseline(w_cpu, args.cpu_budget, warmup=2,
                                                         max_iters=5)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
