"""CPU checks of the compiled kernels' resources, from the compiler remarks the build
records (``vllm-mach_amd/_build/kernel_resources.json``):

* no kernel uses scratch memory.  A scratch reload is a vector memory load; vector
  loads complete in issue order, so waiting for one also waits for every weight load
  or global->LDS copy issued before it, which drains the streaming and copy pipelines
  (a run-time-indexed lane-offset array in scratch once cost the grouped wide GEMM 20 %);
* every kernel's static LDS fits one CU (160 KiB);
* the grouped wide GEMM fits two workgroups per CU (its schedule relies on the second
  workgroup covering each tile's prologue and epilogue).
"""
import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REPORT = ROOT / "vllm-mach_amd" / "_build" / "kernel_resources.json"
LDS_PER_CU = 160 * 1024


@pytest.fixture(scope="module")
def resources():
    if not REPORT.exists():
        pytest.skip("no build report (run __graft_entry__.build() first)")
    data = json.loads(REPORT.read_text())
    assert data, "empty build report"
    return data


def test_remark_parser():
    sys.path.insert(0, str(ROOT / "vllm-mach_amd"))
    try:
        import build
    finally:
        sys.path.pop(0)
    text = "\n".join([
        "x.hip:5:1: remark: Function Name: _Z1kv [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     TotalSGPRs: 33 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     VGPRs: 38 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     Occupancy [waves/SIMD]: 8 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:5:1: remark:     LDS Size [bytes/block]: 4096 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build.parse_resource_remarks(text) == {
        "_Z1kv": {"sgpr": 33, "vgpr": 38, "scratch": 12, "occupancy": 8, "lds": 4096}}


def test_every_kernel_reported(resources):
    for name in ("gemm_wide_kernel", "gemm_stream_kernel", "gemm_stream_grouped_kernel", "quant_mxfp8_kernel",
                 "swiglu_mxfp8_kernel", "gemm_kernel"):
        assert any(name in k for k in resources), name
    for k, v in resources.items():
        assert {"vgpr", "scratch", "lds", "occupancy"} <= set(v), k


def test_no_kernel_uses_scratch(resources):
    offenders = {k: v["scratch"] for k, v in resources.items() if v["scratch"] != 0}
    assert not offenders, offenders


def test_static_lds_fits_a_cu(resources):
    over = {k: v["lds"] for k, v in resources.items() if v["lds"] > LDS_PER_CU}
    assert not over, over


def test_grouped_wide_gemm_fits_two_workgroups_per_cu(resources):
    # gemm_wide_kernel<fmt, MT, NT, BLOCK = false, GROUPED = true, WM = 1>
    grouped = {k: v for k, v in resources.items() if "gemm_wide_kernel" in k and "Lb0ELb1ELi1E" in k}
    assert grouped
    for k, v in grouped.items():
        assert 2 * v["lds"] <= LDS_PER_CU, (k, v["lds"])
        assert v["occupancy"] >= 2 and v["vgpr"] + v.get("agpr", 0) <= 256, (k, v)
