"""MoE-layer forward+backward throughput on one MI355X (the BASELINE.json metric).

A step is one pass of the hot path over one batch: from router logits,
fp32 softmax / stable top-k / renorm, fused count + offsets + pack, grouped
GEMM up with the GELU in its epilogue, grouped GEMM down, combine
(activation dtype out), then the full backward to dX, dlogits, dW_up and
dW_down (the GELU backward fused into the down projection's dX GEMM). Inputs are resident in HBM
before the timed region. Default workload: config C2 (30720 tokens, d=512,
E=8, top-2, FFN 512->2048->512, bf16), synthetic seeded data, random-init
weights.

Prints ONE JSON line. ``value`` times K steps with only the step's own
launches on the stream, after W warmup steps launched the same way (the
GPU's clocks settle over the first ~20 back-to-back steps; the default W
is past that). ``roofline`` is for the dominant kernel family (the
grouped GEMMs): algorithmic FLOPs per launch (2*A*K*N) over the average
launch duration, measured with HIP events on the launch stream around every
launch in a second timed pass over the same K steps (the event markers
slow the step by a few percent, so that pass does not feed ``value``). ``cpu_baseline`` times the CPU restatement of the reference
torch path on a bounded token sample (rank 0, N=1 only).

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 50] [--config 2] [--ffn gelu|swiglu]

``--ffn swiglu`` runs the reference's SwiGLU ExpertFFN in place of the
configs' GELU FFN (a secondary figure; the headline is the GELU FFN).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE layer fwd+bwd tokens/sec (1×MI355X); pack/combine HBM GB/s; GEMM MFMA %"
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {torch.bfloat16: 2500.0, torch.float16: 2500.0, torch.float32: 157.3}

# name: (dtype, T, d, E, k, f, weight std, logit std)
WORKLOADS = {
    1: ("C1", torch.float32, 4096, 512, 8, 2, 2048, 0.02, 1.0),
    2: ("C2", torch.bfloat16, 30720, 512, 8, 2, 2048, 0.02, 1.0),
    3: ("C3", torch.bfloat16, 30720, 512, 64, 8, 256, 0.02, 1.0),
    4: ("C4", torch.bfloat16, 16384, 4096, 8, 2, 14336, 0.01, 1.0),
    5: ("C5", torch.float16, 65536, 2048, 128, 8, 768, 0.02, 2.0),
}


def make_workload(cfg_id: int, device: str, seed: int = 1234, T: int | None = None):
    """Synthetic inputs of config C<cfg_id>: X, logits (with the config's edits), weights, dY."""
    name, dtype, T0, d, E, k, f, wstd, lstd = WORKLOADS[cfg_id]
    T = T0 if T is None else T
    g = torch.Generator(device=device).manual_seed(seed)
    X = torch.randn(T, d, generator=g, device=device).to(dtype)
    logits = torch.randn(T, E, generator=g, device=device) * lstd
    if cfg_id == 3:  # Zipf(1.2) expert popularity as a log-prior bias
        z = torch.tensor([(i + 1) ** -1.2 for i in range(E)], dtype=torch.float64)
        perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed))
        logits += torch.log(z[perm] / z.sum()).float().to(device)
    if cfg_id == 5:  # 16 dead experts, 1% of tokens with all live logits tied
        cg = torch.Generator().manual_seed(seed)
        dead = torch.randperm(E, generator=cg)[:16]
        ties = torch.randperm(T, generator=cg)[: math.ceil(T / 100)]
        live = torch.ones(E, dtype=torch.bool)
        live[dead] = False
        logits[ties.to(device).unsqueeze(1), live.nonzero().squeeze(1).to(device).unsqueeze(0)] = 0.0
        logits[:, dead.to(device)] = float("-inf")
    W_up = (torch.randn(E, d, f, generator=g, device=device) * wstd).to(dtype)
    W_down = (torch.randn(E, f, d, generator=g, device=device) * wstd).to(dtype)
    dY = torch.randn(T, d, generator=g, device=device).to(dtype)
    return dict(name=name, dtype=dtype, T=T, d=d, E=E, k=k, f=f, X=X, logits=logits,
                W_up=W_up, W_down=W_down, dY=dY)


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
    }

    def __init__(self, ext):
        self._ext = ext
        self.active = False
        self.records = []  # (family, name, start_event, end_event, work)

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
            # read X once, write packed rows, ids/gates
            X, w, topk = args[:3]
            T, d = X.shape
            A = topk.numel()
            b = X.element_size()
            return T * d * b + A * d * b + 8.0 * A + 12.0 * A
        if name == "combine_inv":  # read packed rows + gates/inv, write [T,d] in out dtype
            y, inv, w, out_dtype = args
            A, d = y.shape
            T = inv.shape[0]
            ob = torch.empty(0, dtype=out_dtype).element_size()
            return A * d * y.element_size() + 8.0 * A + T * d * ob
        if name == "combine_backward_inv":  # read dY once, y; write dy, dw
            y, inv, w, dY = args
            A, d = y.shape
            T = inv.shape[0]
            return T * d * dY.element_size() + 2.0 * A * d * y.element_size() + 12.0 * A
        if name == "pack_backward_inv":  # read dpX, dpw, inv; write dX, dw
            dpX, dpw, inv = args
            A, d = dpX.shape
            T = inv.shape[0]
            return A * d * dpX.element_size() + T * d * dpX.element_size() + 12.0 * A
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


def gpu_step(wl, W_up, W_down, ffn):
    from nanotitan_amd.layer import moe_forward_from_logits

    x = wl["X"].detach().requires_grad_(True)
    logits = wl["logits"].detach().requires_grad_(True)
    out, _counts, _probs = moe_forward_from_logits(x, logits, ffn, wl["E"], wl["k"])
    out.backward(wl["dY"])
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


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg_id: int, budget_s: float = 20.0):
    """The reference torch CPU path (oracle restatement) on a bounded token sample."""
    from oracle import moe_oracle as O

    name, dtype, T0, d, E, k, f, wstd, lstd = WORKLOADS[cfg_id]
    cores = os.cpu_count() or 1
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)

    def layer(wl):
        weights = {"up": wl["W_up"], "down": wl["W_down"]}
        O.moe_layer_torch(wl["X"], wl["logits"], weights, k, ffn="gelu", dY=wl["dY"])

    # Size the sample from a 256-token probe so that warmup + timed
    # iterations stay near budget_s (fp16 on the CPU is slow at C5).
    T = min(T0, 256)
    probe = make_workload(cfg_id, "cpu", seed=99, T=T)
    layer(probe)
    t0 = time.perf_counter()
    layer(probe)
    per_token = (time.perf_counter() - t0) / T
    T = int(min(T0, 4096, max(256, budget_s / 4 / per_token)) // 256 * 256)
    print(f"bench.py: cpu_baseline sample {T} tokens (~{per_token * T:.1f} s per iteration)",
          file=sys.stderr, flush=True)
    if T == probe["T"]:
        wl, first = probe, per_token * T  # the probe runs were the warmup
    else:
        wl = make_workload(cfg_id, "cpu", seed=99, T=T)
        t0 = time.perf_counter()
        layer(wl)  # warmup
        first = time.perf_counter() - t0
    iters = max(1, min(3, int(budget_s / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(iters):
        layer(wl)
    dt = (time.perf_counter() - t0) / iters
    return {
        "value": T / dt,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{name} routing and widths, first {T} of {T0} tokens, {dtype}, "
                  f"1 warmup + {iters} timed fwd+bwd iterations; host CPU: {cpu_model()}; "
                  f"torch {torch.__version__}",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--ffn", choices=["gelu", "swiglu"], default="gelu",
                    help="expert FFN: the configs' up->GELU->down (headline) or the reference's "
                         "SwiGLU ExpertFFN")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run 5 device copies of 1 GiB (HBM counter calibration) and exit")
    args = ap.parse_args()

    if args.copy_probe:
        nbytes = 1 << 30
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes,
                          "launches": 5}), flush=True)
        return

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
    timer = LaunchTimer(ext)
    moe_ops.get_hip_extension = lambda: timer

    torch.manual_seed(0)
    wl = make_workload(args.config, "cuda")
    W_up = wl["W_up"].detach().requires_grad_(True)
    W_down = wl["W_down"].detach().requires_grad_(True)
    ffn = _GeluFFN(W_up, W_down)
    W_val = None
    if args.ffn == "swiglu":  # W_up serves as W_gate and W_down as W_out
        std = WORKLOADS[args.config][7]
        g = torch.Generator(device="cuda").manual_seed(4321)
        W_val = (torch.randn(W_up.shape, generator=g, device="cuda") * std).to(wl["dtype"])
        W_val.requires_grad_(True)
        ffn = _SwiGLUFFN(W_up, W_val, W_down)

    for _ in range(args.warmup):
        gpu_step(wl, W_up, W_down, ffn)
        W_up.grad = W_down.grad = None
        if W_val is not None:
            W_val.grad = None
    torch.cuda.synchronize()

    # Headline: K steps with nothing but the step's own launches on the stream.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        gpu_step(wl, W_up, W_down, ffn)
        W_up.grad = W_down.grad = None
        if W_val is not None:
            W_val.grad = None
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # Per-launch timing: the same K steps again, with a HIP event pair around
    # every kernel-family launch on the launch stream. The event markers add
    # a few percent to the step, so this pass does not feed `value`.
    timer.active = True
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        gpu_step(wl, W_up, W_down, ffn)
        W_up.grad = W_down.grad = None
        if W_val is not None:
            W_val.grad = None
    torch.cuda.synchronize()
    elapsed_events = time.perf_counter() - t1
    timer.active = False

    ms_per_step = elapsed / args.steps * 1e3
    tokens_per_s = wl["T"] * args.steps / elapsed
    fams = timer.summary()
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
    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE
    # (calibrated on a device copy), committed with the profile summaries.
    prof = ROOT / "profiles" / f"traffic_{wl['name'].lower()}.json"
    if prof.exists() and args.ffn == "gelu":
        fams_t = json.loads(prof.read_text()).get("families", {})
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
            roofline["traffic"] = round(sum(fams_t[f]["bytes"] * c for f, c in per_step.items()) / n)
            roofline["traffic_algorithmic"] = round(
                sum(fams_t[f]["algorithmic_bytes"] * c for f, c in per_step.items()) / n)
            roofline["traffic_source"] = f"profiles/{prof.name}"
    # MFMA busy fraction and running clock of the GEMMs, from a rocprofv3
    # counter pass (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x 1024
    # SIMDs) committed with the profile summaries; time-weighted over the
    # GEMM families of a step.
    mf = ROOT / "profiles" / f"mfma_{wl['name'].lower()}.json"
    if mf.exists() and args.ffn == "gelu":
        fam_m = json.loads(mf.read_text())
        t_all = sum(v["launches"] * v["avg_us"] for v in fam_m.values())
        if t_all > 0:
            def tw(key):
                return sum(v[key] * v["launches"] * v["avg_us"] for v in fam_m.values()) / t_all
            roofline["mfma_busy_frac"] = round(tw("mfma_busy_frac"), 4)
            roofline["clock_ghz"] = round(tw("clock_ghz"), 3)
            roofline["mfma_source"] = f"profiles/{mf.name}"
    kernels = {}
    for fam, r in fams.items():
        avg_ms = r["ms"] / r["launches"]
        per = r["work"] / r["launches"]
        if fam == "gemm":
            kernels[fam] = {"avg_ms": round(avg_ms, 4), "tflops": round(per / avg_ms / 1e9, 2)}
        else:
            gbs = per / (avg_ms * 1e-3) / 1e9
            kernels[fam] = {"avg_ms": round(avg_ms, 4), "GB_s": round(gbs, 1),
                            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": per}

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
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[wl["dtype"]],
        "data": "synthetic (seeded N(0,1) activations/logits, N(0,std^2) random-init expert weights)",
        "config": {
            "workload": f"{wl['name']}: MoE layer fwd+bwd, {wl['T']} tokens x d={wl['d']}, "
                        f"E={wl['E']}, top-{wl['k']}, FFN {wl['d']}->{wl['f']}->{wl['d']} "
                        + ("GELU" if args.ffn == "gelu" else "SwiGLU (reference ExpertFFN)"),
            "tokens": wl["T"],
            "d_model": wl["d"],
            "num_experts": wl["E"],
            "top_k": wl["k"],
            "ffn": wl["f"],
            "parallelism": "single-gpu",
        },
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.config, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
