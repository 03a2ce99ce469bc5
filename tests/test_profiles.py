"""The profile summaries bench.py reads (calibrated traffic, MFMA busy cycles) are well formed.

bench.py adds ``roofline.traffic`` from ``profiles/traffic_<cfg>.json`` and
``roofline.mfma_busy_frac`` / ``clock_ghz`` from ``profiles/mfma_<cfg>.json``;
these checks keep those files consistent with what it looks up.
"""

import json
from pathlib import Path

import pytest

PROFILES = Path(__file__).resolve().parent.parent / "profiles"

# GEMM launches of one layer step, paired (dW + dX in one launch) or one by one.
PAIRED = {"gemm_fwd_gelu", "gemm_fwd", "gemm_pair_dw_dx_gelu", "gemm_pair_dw_dx"}
SEPARATE = {"gemm_fwd_gelu", "gemm_fwd", "gemm_dx_gelu", "gemm_dx", "gemm_dw"}
HBM_KERNELS = {"dispatch_pack", "combine_fwd", "combine_bwd", "pack_bwd"}


@pytest.mark.parametrize("path", sorted(PROFILES.glob("traffic_c*.json")), ids=lambda p: p.name)
def test_traffic_profile(path):
    js = json.loads(path.read_text())
    assert 1.0 <= js["fetch_scale"] <= 4.0 and 0.5 <= js["write_scale"] <= 2.0
    fams = js["families"]
    assert PAIRED <= fams.keys() or SEPARATE <= fams.keys()
    for name in HBM_KERNELS:
        f = fams[name]
        assert f["launches"] > 0
        assert f["bytes"] == pytest.approx(f["read_bytes"] + f["write_bytes"])
        # a gather/scatter moves each byte once: measured within 10% of algorithmic
        assert f["bytes"] == pytest.approx(f["algorithmic_bytes"], rel=0.1)
    for name in (PAIRED | SEPARATE) & fams.keys():
        f = fams[name]
        assert f["bytes"] >= 0.9 * f["algorithmic_bytes"] > 0


@pytest.mark.parametrize("path", sorted(PROFILES.glob("mfma_c*.json")), ids=lambda p: p.name)
def test_mfma_profile(path):
    js = json.loads(path.read_text())
    assert PAIRED <= js.keys() or SEPARATE <= js.keys()
    for name, f in js.items():
        assert name.startswith("gemm_")
        assert 0.0 < f["mfma_busy_frac"] <= 1.0
        assert 1.0 < f["clock_ghz"] < 2.6  # MI355X peak engine clock is 2.4 GHz
        # MFMA work = algorithmic FLOPs plus tile padding at expert boundaries
        assert 1.0 <= f["mfma_flops_per_launch"] / f["algorithmic_flops"] < 1.1
        assert f["avg_us"] > 0 and f["launches"] > 0


def test_bench_reads_the_profiles():
    """The headline config (C2) and the MFMA-utilisation config (C4) have both profile files."""
    names = {p.stem.split("_")[1] for p in PROFILES.glob("mfma_c*.json")}
    assert {"c2", "c4"} <= names
    assert (PROFILES / "traffic_c2.json").exists() and (PROFILES / "traffic_c4.json").exists()
