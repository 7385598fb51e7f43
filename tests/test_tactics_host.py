"""CPU checks of the per-shape GEMM tactic table (``vllm_mach_amd.tactics``) and the
library's override registry (``mxl_set_gemm_config``): the packaged table's contract, its
registration and filtering, and what the plan query reports with entries registered.

The reference's counterpart checks its frozen projection table and that an eligible rank
registers each row once (tests/native_mxfp6/test_moe_projection.py)."""
import json
from pathlib import Path

import pytest
import torch

LIB = Path(__file__).resolve().parents[1] / "vllm-mach_amd" / "libmxlinear.so"


@pytest.fixture
def tac(pkg):
    if not LIB.exists():
        pytest.skip("libmxlinear.so not built")
    return pkg.tactics


def _host_plans():
    # the plans a table records are those of a 256-CU device; the host planner assumes 256
    return not torch.cuda.is_available() or torch.cuda.get_device_properties(0).multi_processor_count == 256


def test_packaged_table_contract(tac):
    from vllm_mach_amd import _lib
    t = tac.load_table()
    assert t["config_abi"] == _lib.query("mxl_gemm_config_abi")
    assert t["cu_count"] == 256
    keys = [(e["m"], e["n"], e["k"], e["w_fmt"], e["block"]) for e in t["entries"]]
    assert len(keys) == len(set(keys))
    # every shape the sweep was asked for has its entry
    assert set(keys) == set(tac.BENCH_SHAPES) | set(tac.REFERENCE_SHAPES)
    for e in t["entries"]:
        assert set(e["config"]) == set(tac.FIELDS)
        assert e["us"] <= e["auto_us"]  # the entry is the cost model's plan or a faster one


def test_cost_model_within_three_percent_on_benchmark_prefill(tac):
    """The planner's own choice at the benchmark configurations' prefill sizes (c2, c3, c4 at
    M >= 128) measured within 3 % of the best swept configuration."""
    t = tac.load_table()
    rows = [e for e in t["entries"] if e["m"] >= 128 and (e["n"], e["k"]) in ((2560, 9216), (18432, 2560),
                                                                            (17408, 5120))]
    assert len(rows) == 8
    worst = max(e["auto_us"] / e["us"] for e in rows)
    assert worst <= 1.03, worst


def test_prepare_registers_each_row_once_and_plans_follow(tac):
    from vllm_mach_amd import _lib
    t = tac.load_table()
    assert tac.installed() == 0
    assert tac.prepare() == len(t["entries"])
    assert tac.installed() == len(t["entries"])
    if _host_plans():
        for e in t["entries"]:
            assert tac.plan_name(e["m"], e["n"], e["k"], e["w_fmt"], e["block"]) == e["plan"], e
    # an explicit option bypasses the table
    e = t["entries"][0]
    forced = _lib.GemmOptions(kernel=2)
    assert _lib.plan_name("mxl_gemm_plan_name", e["m"], e["n"], e["k"], e["w_fmt"], e["block"],
                          options=forced).startswith("gemm_kernel<")
    # registering again replaces, it does not add
    assert tac.prepare() == len(t["entries"]) and tac.installed() == len(t["entries"])
    tac.clear()
    assert tac.installed() == 0
    if _host_plans():
        for e in t["entries"]:
            assert tac.plan_name(e["m"], e["n"], e["k"], e["w_fmt"], e["block"]) == e["auto_plan"], e


def test_prepare_filters_by_problem_and_mode(tac):
    t = tac.load_table()
    # the model's dense problems as warmup.collect_problems keys them
    problems = [("Mxfp8LinearKernel", 2560, 9216, 0, ()), ("BlockFp8LinearKernel", 18432, 2560, None, ())]
    want = sum(1 for e in t["entries"] if (e["n"], e["k"], e["w_fmt"], e["block"]) in
               ((2560, 9216, 0, 0), (18432, 2560, 0, 1)))
    assert want == 12
    assert tac.prepare(problems) == want and tac.installed() == want
    tac.clear()
    assert tac.prepare(problems, mode="off") == 0 and tac.installed() == 0
    with pytest.raises(ValueError, match="mode"):
        tac.prepare(mode="sometimes")
    bad = dict(t, config_abi=t["config_abi"] + 1)
    with pytest.raises(RuntimeError, match="config ABI"):
        tac.prepare(table=bad)
    assert tac.installed() == 0


def test_registry_refuses_what_does_not_run(tac):
    from vllm_mach_amd import _lib
    opts = _lib.GemmOptions(kernel=0)  # weight streaming: at most 16 rows
    with pytest.raises(_lib.MxlError, match="do not run"):
        _lib.call("mxl_set_gemm_config", 512, 2560, 9216, 0, 0, _lib.options_ptr(opts))
    with pytest.raises(_lib.MxlError, match="unknown weight format"):
        _lib.call("mxl_set_gemm_config", 512, 2560, 9216, 9, 0, _lib.options_ptr(_lib.GemmOptions()))
    with pytest.raises(_lib.MxlError, match="invalid options"):
        _lib.call("mxl_set_gemm_config", 512, 2560, 9216, 0, 0, _lib.options_ptr(_lib.GemmOptions(tile_n=3)))
    with pytest.raises(_lib.MxlError, match="NULL"):
        _lib.call("mxl_set_gemm_config", 512, 2560, 9216, 0, 0, None)
    assert tac.installed() == 0
    # the registered split changes the workspace the shape needs
    base = _lib.query("mxl_gemm_workspace_bytes_ex", 512, 2560, 9216, 0, 0, None)
    _lib.call("mxl_set_gemm_config", 512, 2560, 9216, 0, 0,
              _lib.options_ptr(_lib.GemmOptions(kernel=1, tile_n=1, splits=4)))
    assert _lib.query("mxl_gemm_workspace_bytes_ex", 512, 2560, 9216, 0, 0, None) == 4 * 512 * 2560 * 4 != base


def test_table_is_plain_json(tac):
    # the table is data: JSON with the fields the loader reads, nothing executable
    text = tac.TABLE.read_text()
    t = json.loads(text)
    assert set(t) >= {"config_abi", "device", "cu_count", "measured", "method", "entries"}
