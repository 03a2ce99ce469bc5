"""The profile summaries bench.py reads (calibrated traffic, MFMA busy cycles) are well formed,
record the commit they were measured on, and were measured on the kernel sources in this tree.

bench.py adds ``roofline.traffic`` from ``profiles/traffic_<cfg>.json`` and
``roofline.mfma_busy_frac`` / ``clock_ghz`` from ``profiles/mfma_<cfg>.json``
(both written by bench_profiles.py); these checks keep those files consistent
with what it looks up and flag summaries left behind by a kernel change.
"""

import json
import subprocess
from pathlib import Path

import pytest

from bench_profiles import family, kernel_source_hash

ROOT = Path(__file__).resolve().parent.parent
PROFILES = ROOT / "profiles"

# GEMM launches of one layer step, paired (dW + dX in one launch) or one by one.
PAIRED = {"gemm_fwd_gelu", "gemm_fwd", "gemm_pair_dw_dx_gelu", "gemm_pair_dw_dx"}
SEPARATE = {"gemm_fwd_gelu", "gemm_fwd", "gemm_dx_gelu", "gemm_dx", "gemm_dw"}
HBM_KERNELS = {"dispatch_pack", "combine_fwd", "combine_bwd", "pack_bwd"}


def _provenance(js):
    assert len(js["commit"]) >= 7
    assert js["source_hash"] == kernel_source_hash(ROOT), \
        "kernel sources changed since this profile was measured: profile again"
    git = ROOT / ".git"
    if git.exists():
        r = subprocess.run(["git", "-C", str(ROOT), "cat-file", "-e", js["commit"] + "^{commit}"],
                           capture_output=True)
        assert r.returncode == 0, f"commit {js['commit']} is not in this repository"


@pytest.mark.parametrize("path", sorted(PROFILES.glob("traffic_c*.json")), ids=lambda p: p.name)
def test_traffic_profile(path):
    js = json.loads(path.read_text())
    _provenance(js)
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
    _provenance(js)
    fams = js["families"]
    assert PAIRED <= fams.keys() or SEPARATE <= fams.keys()
    for name, f in fams.items():
        assert name.startswith("gemm_")
        assert 0.0 < f["mfma_busy_frac"] <= 1.0
        assert 1.0 < f["clock_ghz"] < 2.6  # MI355X peak engine clock is 2.4 GHz
        # MFMA work = algorithmic FLOPs plus tile padding at expert boundaries
        assert 1.0 <= f["mfma_flops_per_launch"] / f["algorithmic_flops"] < 1.1
        assert f["avg_us"] > 0 and f["launches"] > 0


def test_kernel_families():
    """The summariser names every kernel the layer launches."""
    assert family("void nt::gg_mfma_kernel<nt::bf16, 0, 256, 256, 2, 4, 64, 2, 1, false>"
                  "(nt::GemmArgs)") == "gemm_fwd_gelu"
    assert family("void nt::gg_mfma_kernel<nt::bf16, 1, 256, 256, 2, 4, 64, 2, 2, false>"
                  "(nt::GemmArgs)") == "gemm_dx_gelu"
    assert family("void nt::gg_pair_kernel<nt::bf16, 2, false>(nt::GemmArgs, nt::GemmArgs, int, "
                  "int*)") == "gemm_pair_dw_dx_gelu"
    assert family("void nt::(anonymous namespace)::gg_f32_mfma_kernel<2, 0>(nt::GemmArgs)") \
        == "gemm_dw"
    assert family("void nt::pack_rows_kernel<HIP_vector_type<unsigned int, 4u> >(...)") \
        == "dispatch_pack"
    assert family("void nt::combine_bwd_inv_kernel<nt::bf16, nt::bf16, 8, 2>(...)") == "combine_bwd"
