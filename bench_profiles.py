"""Summarise rocprofv3 runs of ``bench.py`` into ``profiles/``.

``bench.py`` adds HBM traffic (``roofline.traffic``) and the GEMMs' MFMA busy
fraction to its JSON line from the summaries this script writes:

- ``profiles/traffic_c<N>.json`` and ``profiles/moe_layer_c<N>_hbm_traffic.md``
  from one ``--pmc FETCH_SIZE`` and one ``--pmc WRITE_SIZE`` pass of a config,
  each scaled by what the same counter reads for the 1 GiB copy of
  ``bench.py --copy-probe``;
- ``profiles/mfma_c<N>.json`` and ``profiles/grouped_gemm_mfma_util.md`` from a
  ``--pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_*
  SQ_BUSY_CYCLES`` pass;
- ``profiles/moe_layer_c<N>_kernel_trace.md`` from a ``--kernel-trace --stats``
  pass, with the bench line that run printed.

Every JSON records the commit it was measured on and ``source_hash``, a hash of
the kernel sources (``kernel_source_hash``); ``bench.py`` recomputes the hash
and reports whether the profile still matches the code it runs.

Usage, after the profiling runs (``rocprofv3 ... -d <dir>/<pass> -o c<N> --
python3 bench.py --config N ...``) have written their CSVs under ``<dir>``::

    python bench_profiles.py --config 4 --dir gpurun_out/prof_c4 \\
        --copy-dir gpurun_out/prof_copy --commit $(git rev-parse --short HEAD)
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import hashlib
import json
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PROFILES = ROOT / "profiles"

# (title, T, d, E, k, f, bytes per element, MFMA-ops counter) of each config.
CONFIGS = {
    1: ("C1 (fp32, 4096 tokens, d=512, E=8, top-2, FFN 512->2048->512 GELU)",
        4096, 512, 8, 2, 2048, 4, None),
    2: ("C2 (bf16, 30720 tokens, d=512, E=8, top-2, FFN 512->2048->512 GELU)",
        30720, 512, 8, 2, 2048, 2, "SQ_INSTS_VALU_MFMA_MOPS_BF16"),
    3: ("C3 (bf16, 30720 tokens, d=512, E=64 Zipf-skewed, top-8, FFN 512->256->512 GELU)",
        30720, 512, 64, 8, 256, 2, "SQ_INSTS_VALU_MFMA_MOPS_BF16"),
    4: ("C4 (bf16, 16384 tokens, d=4096, E=8, top-2, FFN 4096->14336->4096 GELU)",
        16384, 4096, 8, 2, 14336, 2, "SQ_INSTS_VALU_MFMA_MOPS_BF16"),
    5: ("C5 (fp16, 65536 tokens, d=2048, E=128 with 16 dead, top-8, FFN 2048->768->2048 GELU)",
        65536, 2048, 128, 8, 768, 2, "SQ_INSTS_VALU_MFMA_MOPS_F16"),
}

XCDS = 8
SIMDS = 1024
COPY_BYTES = 1 << 30  # bench.py --copy-probe moves 1 GiB per launch


def kernel_source_hash(root: Path = ROOT) -> str:
    """sha256 over the kernel sources and the C ABI header (sorted paths)."""
    h = hashlib.sha256()
    files = sorted(list((root / "nanotitan_amd" / "csrc").glob("*")) +
                   list((root / "include").glob("*.h")))
    for p in files:
        if p.is_file():
            h.update(p.relative_to(root).as_posix().encode())
            h.update(p.read_bytes())
    return h.hexdigest()[:16]


def family(name: str) -> str:
    """Kernel family of a demangled kernel name."""
    if "route_topk_hist" in name:
        return "router_fwd_count"
    if "route_topk_backward" in name:
        return "router_bwd"
    if "route_topk" in name:
        return "router_fwd"
    if "scan_kernel" in name and "token_scan" not in name:
        return "dispatch_scan"
    if "hist_kernel" in name and "radix" not in name:
        return "dispatch_hist"
    if "pack_rows_kernel" in name:
        return "dispatch_pack"
    if "combine_bwd_inv" in name:
        return "combine_bwd"
    if "combine_inv_kernel" in name:
        return "combine_fwd"
    if "pack_bwd_inv" in name:
        return "pack_bwd"
    if "dw_reduce" in name:
        return "gemm_dw_reduce"
    if "zero_i32" in name:
        return "gemm_pair_counters"
    if "gelu_elementwise" in name:
        return "gelu_elementwise"
    m = re.search(r"gg_pair_kernel<[^,]+, (\d+)", name)
    if m:
        return "gemm_pair_dw_dx_gelu" if m.group(1) == "2" else "gemm_pair_dw_dx"
    m = re.search(r"gg_f32_mfma_kernel<(\d+), (\d+)>", name)
    if m:
        return {"0": "gemm_fwd", "1": "gemm_dx", "2": "gemm_dw"}[m.group(1)]
    m = re.search(r"gg_generic_kernel<[^,]+, (\d+)>", name)
    if m:
        return {"0": "gemm_fwd", "1": "gemm_dx", "2": "gemm_dw"}[m.group(1)]
    m = re.search(r"gg_mfma_kernel<([^>]*)>", name)
    if m:
        a = [x.strip() for x in m.group(1).split(",")]
        op, epi = a[1], a[8]
        if op == "0":
            return "gemm_fwd_gelu" if epi == "1" else "gemm_fwd"
        if op == "1":
            return "gemm_dx_gelu" if epi != "0" else "gemm_dx"
        return "gemm_dw"
    if "at::" in name:
        return "torch"
    return "other"


def algorithmic(cfg_id: int):
    """Algorithmic bytes (each tensor touched once) and FLOPs per launch."""
    _, T, d, E, k, f, b, _ = CONFIGS[cfg_id]
    A = T * k
    nbytes = {
        "combine_bwd": T * d * b + 2 * A * d * b + 12 * A,
        "combine_fwd": A * d * b + 8 * A + T * d * b,
        "dispatch_pack": T * d * b + A * d * b + 20 * A,
        # the layer's launches also write the router's gradient (no dw)
        "pack_bwd": A * d * b + T * d * b + 16 * A + 4 * T * E,
        "gemm_fwd_gelu": (A * d + E * d * f + 2 * A * f) * b,
        "gemm_fwd": (A * f + E * f * d + A * d) * b,
        "gemm_pair_dw_dx_gelu": (3 * A * f + A * d + 2 * E * f * d) * b,
        "gemm_pair_dw_dx": (2 * A * d + A * f + 2 * E * d * f) * b,
        "gemm_dx_gelu": (A * d + E * f * d + 2 * A * f) * b,
        "gemm_dx": (A * f + E * d * f + A * d) * b,
        "gemm_dw": (A * f + A * d + E * f * d) * b,
    }
    one = 2 * A * d * f
    flops = {"gemm_fwd_gelu": one, "gemm_fwd": one, "gemm_dx_gelu": one, "gemm_dx": one,
             "gemm_dw": one, "gemm_pair_dw_dx_gelu": 2 * one, "gemm_pair_dw_dx": 2 * one}
    return nbytes, flops


def _find(d: Path, suffix: str) -> Path:
    hits = sorted(glob.glob(f"{d}/**/*{suffix}", recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return Path(hits[0])


def counters(d: Path):
    """Per-dispatch counter sums, durations (ns) and kernel names."""
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names = {}
    with open(_find(d, "counter_collection.csv")) as fh:
        for r in csv.DictReader(fh):
            did = int(r["Dispatch_Id"])
            per[did][r["Counter_Name"]] += float(r["Counter_Value"])
            per[did]["_ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
            names[did] = r["Kernel_Name"]
    return per, names


def _stamp(js: dict, commit: str) -> dict:
    js["commit"] = commit
    js["source_hash"] = kernel_source_hash()
    return js


def traffic(cfg_id: int, d: Path, copy_dir: Path, commit: str) -> None:
    title = CONFIGS[cfg_id][0]
    cf, _ = counters(copy_dir / "copy_fetch")
    cw, _ = counters(copy_dir / "copy_write")
    fetch_copy = max(v["FETCH_SIZE"] for v in cf.values()) * 1024
    write_copy = max(v["WRITE_SIZE"] for v in cw.values()) * 1024
    fs, ws = COPY_BYTES / fetch_copy, COPY_BYTES / write_copy
    fe, names_f = counters(d / "fetch")
    wr, names_w = counters(d / "write")
    fam = collections.defaultdict(lambda: {"launches": 0, "read": 0.0, "write": 0.0})
    for did, v in fe.items():
        r = fam[family(names_f[did])]
        r["launches"] += 1
        r["read"] += v["FETCH_SIZE"] * 1024 * fs
    for did, v in wr.items():
        fam[family(names_w[did])]["write"] += v["WRITE_SIZE"] * 1024 * ws
    alg, _ = algorithmic(cfg_id)
    js = {"fetch_scale": fs, "write_scale": ws, "families": {}}
    c = f"c{cfg_id}"
    run = f"python3 bench.py --config {cfg_id} --configs none --steps 2 --warmup 1 --no-cpu-baseline"
    lines = [
        f"# HBM traffic per launch — MoE layer fwd+bwd, {title}", "",
        f"Measured on the kernels of commit `{commit}` (kernel source hash "
        f"`{kernel_source_hash()}`). Commands (run from the repository root on one MI355X; "
        "each counter in its own pass):", "", "```",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {d}/fetch -o {c} -- {run}",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {d}/write -o {c} -- {run}",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {copy_dir}/copy_fetch -o copy -- "
        "python3 bench.py --copy-probe",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {copy_dir}/copy_write -o copy -- "
        "python3 bench.py --copy-probe",
        "```", "",
        f"Calibration: the 1 GiB device copy of `bench.py --copy-probe` reads "
        f"{fetch_copy / 1024:,.0f} KiB of FETCH_SIZE and writes {write_copy / 1024:,.0f} KiB of "
        f"WRITE_SIZE per launch, so FETCH_SIZE is scaled by {fs:.3f} and WRITE_SIZE by {ws:.3f}.",
        "",
        "| kernel family | launches | read MB | write MB | total MB | algorithmic MB | total / algorithmic |",
        "|---|---:|---:|---:|---:|---:|---:|"]
    for k in sorted(fam):
        r = fam[k]
        n = r["launches"]
        rd, wt = r["read"] / n, r["write"] / n
        a = alg.get(k)
        js["families"][k] = {"launches": n, "read_bytes": rd, "write_bytes": wt,
                             "bytes": rd + wt, "algorithmic_bytes": a}
        ratio = f"{(rd + wt) / a:.2f}" if a else "—"
        amb = f"{a / 1e6:,.1f}" if a else "—"
        lines.append(f"| {k} | {n} | {rd / 1e6:,.1f} | {wt / 1e6:,.1f} | {(rd + wt) / 1e6:,.1f} "
                     f"| {amb} | {ratio} |")
    lines += ["", "FETCH_SIZE and WRITE_SIZE count traffic below the L2 (Infinity Cache and HBM). "
              "Per-launch figures average the launches of the run (warmup and timed steps)."]
    (PROFILES / f"moe_layer_{c}_hbm_traffic.md").write_text("\n".join(lines) + "\n")
    (PROFILES / f"traffic_{c}.json").write_text(json.dumps(_stamp(js, commit), indent=1) + "\n")


def mfma(cfg_id: int, d: Path, commit: str) -> None:
    mops = CONFIGS[cfg_id][7]
    per, names = counters(d / "mfma")
    _, flops = algorithmic(cfg_id)
    fam = collections.defaultdict(
        lambda: {"n": 0, "busy": 0.0, "active": 0.0, "mops": 0.0, "ns": 0.0})
    for did, v in per.items():
        k = family(names[did])
        if k not in flops:
            continue
        r = fam[k]
        r["n"] += 1
        r["busy"] += v["SQ_VALU_MFMA_BUSY_CYCLES"]
        r["active"] += v["GRBM_GUI_ACTIVE"]
        r["mops"] += v[mops]
        r["ns"] += v["_ns"]
    out = {}
    for k, r in sorted(fam.items()):
        active = r["active"] / XCDS  # rocprofv3 sums GRBM_GUI_ACTIVE over the XCDs
        out[k] = {"launches": r["n"],
                  "mfma_busy_frac": r["busy"] / (active * SIMDS),
                  "mfma_flops_per_launch": r["mops"] * 512 / r["n"],
                  "algorithmic_flops": flops[k],
                  "gui_active_cycles_per_xcd": active / r["n"],
                  "avg_us": r["ns"] / r["n"] / 1e3,
                  "clock_ghz": active / r["ns"],
                  "tflops": flops[k] * r["n"] / r["ns"] / 1e3}
    js = {"families": out}
    (PROFILES / f"mfma_c{cfg_id}.json").write_text(json.dumps(_stamp(js, commit), indent=1) + "\n")
    mfma_table()


def mfma_table() -> None:
    """profiles/grouped_gemm_mfma_util.md from every profiles/mfma_c*.json."""
    lines = ["# MFMA utilisation of the grouped GEMMs", "",
             "Commands (run from the repository root on one MI355X; one counter pass per config):",
             "", "```"]
    rows = []
    for p in sorted(PROFILES.glob("mfma_c*.json")):
        cfg_id = int(p.stem[len("mfma_c"):])
        js = json.loads(p.read_text())
        mops = CONFIGS[cfg_id][7]
        lines.append(f"rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE {mops} "
                     f"SQ_BUSY_CYCLES --output-format csv -d gpurun_out/prof_c{cfg_id}/mfma "
                     f"-o c{cfg_id} -- python3 bench.py --config {cfg_id} --configs none "
                     "--steps 2 --warmup 1 --no-cpu-baseline")
        for k, v in js["families"].items():
            rows.append(
                f"| C{cfg_id} | `{js['commit']}` | {k} | {v['launches']} | {v['avg_us']:,.1f} "
                f"| {v['tflops']:,.0f} | {v['tflops'] / 25:.1f} | {100 * v['mfma_busy_frac']:.1f}% "
                f"| {v['clock_ghz']:.2f} | "
                f"{v['mfma_flops_per_launch'] / v['algorithmic_flops']:.4f} |")
    lines += ["```", "",
              "Per launch, averaged over the run's launches (counter runs serialise the "
              "dispatches):", "",
              "- `MFMA busy` = Σ `SQ_VALU_MFMA_BUSY_CYCLES` ÷ (`GRBM_GUI_ACTIVE` per XCD × 1024 "
              "SIMDs); rocprofv3 reports `GRBM_GUI_ACTIVE` summed over the 8 XCDs.",
              "- `clock` = `GRBM_GUI_ACTIVE` per XCD ÷ the dispatch's duration: the shader "
              "clock the kernel ran at.",
              "- `TF/s` = algorithmic 2·A·K·N per GEMM ÷ duration; `% of 2.5 PF` uses the "
              "nominal dense bf16/fp16 peak.",
              "- `MFMA FLOPs / algorithmic` = `SQ_INSTS_VALU_MFMA_MOPS_*` × 512 ÷ Σ 2·A·K·N: "
              "work on zero-padded tile rows at expert boundaries.", "",
              "| config | commit | GEMM family | launches | avg µs | TF/s | % of 2.5 PF | MFMA busy "
              "| clock GHz | MFMA FLOPs / algorithmic |",
              "|---|---|---|---:|---:|---:|---:|---:|---:|---:|", *rows, "",
              "Families: `gemm_fwd_gelu` up-projection with the GELU epilogue; `gemm_fwd` "
              "down-projection; `gemm_dx_gelu` down-projection dX with the GELU backward; "
              "`gemm_dx` up-projection dX; `gemm_dw` a dW launch; `gemm_pair_*` one launch "
              "running a dW and a dX side by side (two GEMMs' FLOPs)."]
    (PROFILES / "grouped_gemm_mfma_util.md").write_text("\n".join(lines) + "\n")


def kernel_trace(cfg_id: int, d: Path, commit: str, steps: int, bench_log: Path,
                 cmd: str) -> None:
    title = CONFIGS[cfg_id][0]
    with open(_find(d / "kt", "kernel_stats.csv")) as fh:
        rows = list(csv.DictReader(fh))
    lines = [f"# Kernel trace — MoE layer fwd+bwd, {title}", "",
             f"Measured on the kernels of commit `{commit}` (kernel source hash "
             f"`{kernel_source_hash()}`). Command (run from the repository root on one MI355X):",
             "", "```", cmd, "```", "",
             f"{steps} layer steps. Per-kernel statistics from the `--stats` summary "
             "(`kernel_stats.csv`):", "",
             "| kernel | family | calls | avg µs | total % |", "|---|---|---:|---:|---:|"]
    total = gemm = 0.0
    _, flops = algorithmic(cfg_id)
    gemm_flops = 0.0
    for r in rows:
        fam = family(r["Name"])
        ns = float(r["TotalDurationNs"])
        # torch kernels (input set-up, the cold-cache scratch reads) and the
        # copy probe are bench.py's own, not the layer's
        if fam not in ("torch", "other"):
            total += ns
        if fam in flops:
            gemm += ns
            gemm_flops += flops[fam] * int(r["Calls"])
        if float(r["Percentage"]) >= 0.01:
            lines.append(f"| `{r['Name'][:100]}` | {fam} | {r['Calls']} | "
                         f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    lines += ["", f"Layer kernel time per step: {total / steps / 1e3:,.0f} µs (every family but "
              f"`torch` and `other`, {steps} steps; the standalone cold-cache timings of the HBM "
              f"kernels add a few launches); grouped GEMMs {gemm / steps / 1e3:,.0f} µs at "
              f"{gemm_flops / gemm / 1e3:,.0f} TF/s."]
    line = next((ln for ln in bench_log.read_text().splitlines()
                 if ln.startswith('{"metric"')), None)
    if line:
        b = json.loads(line)
        rb = b["roofline"]
        lines += ["", "The same run's `bench.py` line: "
                  f"{b['value']:,.0f} {b['unit']}, {b['ms_per_step']} ms per step; "
                  f"`roofline.achieved` {rb['achieved']:,.1f} {rb['unit']} (HIP events around "
                  f"each launch, average launch {rb['avg_launch_ms'] * 1e3:,.1f} µs)."]
    (PROFILES / f"moe_layer_c{cfg_id}_kernel_trace.md").write_text("\n".join(lines) + "\n")


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", type=int, required=True, choices=sorted(CONFIGS))
    ap.add_argument("--dir", type=Path, required=True,
                    help="folder holding the kt/, fetch/, write/, mfma/ rocprofv3 outputs")
    ap.add_argument("--copy-dir", type=Path, help="folder with copy_fetch/ and copy_write/")
    ap.add_argument("--commit", required=True, help="commit whose kernels were profiled")
    ap.add_argument("--steps", type=int, default=30, help="layer steps of the kernel trace run")
    ap.add_argument("--kt-cmd", default="", help="the kernel trace command, for the summary")
    args = ap.parse_args()
    if (args.dir / "kt").exists():
        kernel_trace(args.config, args.dir, args.commit, args.steps, args.dir / "kt.log",
                     args.kt_cmd)
    if (args.dir / "fetch").exists() and (args.dir / "write").exists() and args.copy_dir:
        traffic(args.config, args.dir, args.copy_dir, args.commit)
    if (args.dir / "mfma").exists():
        mfma(args.config, args.dir, args.commit)


if __name__ == "__main__":
    main()
