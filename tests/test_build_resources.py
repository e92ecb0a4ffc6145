"""Register / scratch budget of the gfx950 kernels, from the resource report
the build writes next to the library (hipcc -Rpass-analysis=kernel-resource-usage).

A kernel that spills to scratch, or a streaming kernel that drops below four
workgroups per CU, loses a large share of its HBM bandwidth; this catches it
on the CPU, at build time.
"""
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPORT = os.path.join(ROOT, "vindexllm_amd", "lib", "kernel_resources.json")


@pytest.fixture(scope="module")
def report():
    if not os.path.exists(REPORT):
        pytest.skip("library not built (run __graft_entry__.build())")
    with open(REPORT) as f:
        return json.load(f)


def _find(report, short):
    hits = {k: v for k, v in report.items() if f"{short}E" in k or f"{short}I" in k}
    assert hits, f"{short} missing from the build report"
    return hits


def test_no_kernel_spills_to_scratch(report):
    assert report, "empty build report"
    bad = {k: v["scratch"] for k, v in report.items() if v.get("scratch", 0) != 0}
    assert not bad, f"kernels using scratch: {bad}"


@pytest.mark.parametrize("kernel", ["k_topk_vec", "k_greedy"])
def test_streaming_kernels_keep_four_workgroups_per_cu(report, kernel):
    for name, v in _find(report, kernel).items():
        assert v["occupancy"] >= 4, (name, v)
        assert v["lds"] * 4 <= 160 * 1024, (name, v)
