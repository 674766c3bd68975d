"""bench.py's byte accounting and its refusal of more than one GPU (CPU only).

The algorithmic bytes per step are the denominators of every roofline figure
bench.py reports; they must reproduce the per-configuration totals of the
scope table (route + dispatch + combine GB: C2 0.471, C3 1.287, C4 8.969,
C5 7.149), which follow the traffic each stage cannot avoid: x read by the
router and again by the permute, each routed row written once and read once.
"""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [REPO, os.path.join(REPO, "ernie-evolve-results_amd")]

import bench  # noqa: E402
from moe_route.configs import CONFIGS  # noqa: E402


@pytest.mark.parametrize("name,total_gb,route_gb,dispatch_gb,combine_gb", [
    ("C2", 0.471, 0.068, 0.202, 0.202),
    ("C3", 1.287, 0.077, 0.605, 0.605),
    ("C4", 8.969, 0.509, 4.230, 4.230),
    ("C5", 7.149, 0.509, 2.410, 4.230),
])
def test_algorithmic_bytes_match_the_scope_table(name, total_gb, route_gb, dispatch_gb,
                                                 combine_gb):
    ab = bench.algorithmic_bytes(CONFIGS[name])
    # the table quotes GB to three decimals
    assert ab["route"] / 1e9 == pytest.approx(route_gb, abs=0.001)
    assert ab["gather"] / 1e9 == pytest.approx(dispatch_gb, abs=0.001)
    assert ab["combine"] / 1e9 == pytest.approx(combine_gb, abs=0.001)
    total = ab["route"] + ab["gather"] + ab["combine"]
    assert total / 1e9 == pytest.approx(total_gb, abs=0.001)


def test_route_bytes_count_an_fp32_weight_whole():
    """C1's router weight is fp32 (split into bf16 hi/lo on the device): its
    E*H*4 bytes are read, twice the bf16 weight's."""
    c1 = CONFIGS["C1"]
    ab = bench.algorithmic_bytes(c1)
    assert ab["route"] == (c1.T * c1.H * 2 + c1.E * c1.H * 4 + c1.T * c1.E * 4
                           + c1.T * c1.k * 8)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=REPO)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""
