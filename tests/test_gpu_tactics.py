"""GPU checks of registered per-shape GEMM configs: a call whose options leave the tuning
automatic runs the registered plan -- bit-identical to the same options passed explicitly,
within the GEMM bar of the oracle -- and the cost model's plan again once cleared; the
packaged table registers on an MI355X and its plans run.  (The reference registers its
measured projection table before warmup: src/vllm_mach/mxfp6/moe_projection.py:35-105.)"""
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


def _mx_case(pkg, oracle_mod, dev, M, N, K, fmt, seed):
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, seed)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, seed + 1)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    return a, sa, tiled, tiled_s, ref


@pytest.mark.parametrize("M,N,K,fmt,config", [
    (128, 2048, 2048, 0, dict(kernel=1, splits=2, tile_n=1, tile_m=0, hybrid=0, waves=4)),
    (96, 1536, 2048, 2, dict(kernel=4, splits=0, tile_n=0, tile_m=0, hybrid=0, waves=0)),
    (64, 1024, 1280, 3, dict(kernel=1, splits=1, tile_n=2, tile_m=4, hybrid=0, waves=4)),
    (256, 640, 1024, 0, dict(kernel=2, splits=1, tile_n=0, tile_m=0, hybrid=0, waves=0)),
])
def test_registered_config_is_the_plan_that_runs(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, config):
    from vllm_mach_amd import _lib
    ops, tac = pkg.ops, pkg.tactics
    monkeypatch.setattr(ops, "_tuning", None)
    a, sa, tiled, tiled_s, ref = _mx_case(pkg, oracle_mod, dev, M, N, K, fmt, 71 + M + N)
    auto_plan = tac.plan_name(M, N, K, fmt, 0)
    y_auto = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    with ops.tuning(**{k: (bool(v) if k == "hybrid" else v) for k, v in config.items()}):
        y_forced = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    table = {"config_abi": _lib.query("mxl_gemm_config_abi"),
             "cu_count": torch.cuda.get_device_properties(dev).multi_processor_count,
             "entries": [dict(m=M, n=N, k=K, w_fmt=fmt, block=0, config=config)]}
    assert tac.prepare(table=table, mode="on") == 1
    assert tac.plan_name(M, N, K, fmt, 0) == tac.plan_name(M, N, K, fmt, 0, config)
    y_reg = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    y_reg2 = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    assert torch.equal(y_reg, y_forced) and torch.equal(y_reg2, y_forced)
    _check(y_reg.float().cpu().numpy(), ref)
    # another M of the same weights is not the registered shape
    assert tac.plan_name(M + 16, N, K, fmt, 0) == tac.plan_name(M + 16, N, K, fmt, 0)
    tac.clear()
    assert tac.plan_name(M, N, K, fmt, 0) == auto_plan
    assert torch.equal(torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None), y_auto)


def test_registered_block_fp8_config(pkg, oracle_mod, dev, monkeypatch):
    from vllm_mach_amd import _lib
    ops, tac = pkg.ops, pkg.tactics
    monkeypatch.setattr(ops, "_tuning", None)
    M, N, K = 64, 1024, 1280
    g = torch.Generator().manual_seed(5)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    config = dict(kernel=1, splits=2, tile_n=1, tile_m=0, hybrid=0, waves=4)
    with ops.tuning(kernel=1, splits=2, tile_n=1, waves=4):
        y_forced = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    _lib.call("mxl_set_gemm_config", M, N, K, 0, 1, _lib.options_ptr(pkg.tactics.options_of(config)))
    y_reg = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    assert torch.equal(y_reg, y_forced)
    rq, rs = oracle_mod.quant_block_fp8(x)
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    _check(y_reg.float().cpu().numpy(), ref)
    tac.clear()


def test_packaged_table_registers_and_runs(pkg, oracle_mod, dev, monkeypatch):
    """The packaged table on this device: every entry registers, and a W6A8 projection entry
    (the reference's table shapes) runs its recorded plan within the bar."""
    ops, tac = pkg.ops, pkg.tactics
    monkeypatch.setattr(ops, "_tuning", None)
    t = tac.load_table()
    if torch.cuda.get_device_properties(dev).multi_processor_count != t["cu_count"]:
        pytest.skip("the packaged table was measured on a 256-CU MI355X")
    assert tac.prepare(mode="on") == len(t["entries"])
    e = next(e for e in t["entries"] if (e["m"], e["n"], e["k"]) == (64, 2048, 256))
    assert tac.plan_name(64, 2048, 256, e["w_fmt"], 0) == e["plan"]
    a, sa, tiled, tiled_s, ref = _mx_case(pkg, oracle_mod, dev, 64, 2048, 256, e["w_fmt"], 404)
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, 2048, 256, e["w_fmt"], None)
    _check(y.float().cpu().numpy(), ref)
    tac.clear()
