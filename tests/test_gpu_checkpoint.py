"""Checkpoints on disk -> loaded layers on the GPU -> outputs against the oracle.

Each case writes a synthetic safetensors checkpoint and a config.json in one of the
three formats the path accepts (compressed-tensors MXFP8, Quark OCP-MX FP6, block-FP8
``weight_scale_inv``), derives the layer's scheme from the config, loads a merged
gate/up layer (two shards of different widths) or routed experts through the vLLM
loading sequence, and checks the forward pass against the oracle's GEMM on the
concatenated checkpoint tensors to the GEMM bar (relative Frobenius <= 1e-3, max
element <= 1e-2 max|ref|).  Expert layers are also checked bit-exact against the
same experts packed directly."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from test_gpu_gemm import _act, _check
from test_gpu_moe import _moe_case

pytestmark = pytest.mark.gpu

_CONFIGS = {
    "mxfp8": {"quant_method": "compressed-tensors", "format": "mxfp8-quantized", "ignore": ["lm_head"],
              "config_groups": {"group_0": {
                  "format": "mxfp8-quantized", "targets": ["Linear"],
                  "weights": {"num_bits": 8, "type": "float", "strategy": "group", "group_size": 32,
                              "symmetric": True, "dynamic": False, "scale_dtype": "torch.uint8"},
                  "input_activations": {"num_bits": 8, "type": "float", "strategy": "group", "group_size": 32,
                                        "symmetric": True, "dynamic": True, "scale_dtype": "torch.uint8"}}}},
    "fp6_e3m2": None, "fp6_e2m3": None,
    "fp8_block": {"quant_method": "fp8", "activation_scheme": "dynamic", "weight_block_size": [128, 128]},
}
for _d in ("fp6_e3m2", "fp6_e2m3"):
    _CONFIGS[_d] = {"quant_method": "quark", "exclude": ["lm_head"], "global_quant_config": {
        "weight": dict(dtype=_d, group_size=32, qscheme="per_group", scale_format="e8m0",
                       is_dynamic=False, symmetric=True),
        "input_tensors": dict(dtype="fp8_e4m3", group_size=32, qscheme="per_group", scale_format="e8m0",
                              is_dynamic=True, symmetric=True)}}
_FMT = {"mxfp8": 0, "fp6_e2m3": 2, "fp6_e3m2": 3}


def _write(tmp_path, fmt_name, tensors):
    save_file(tensors, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": _CONFIGS[fmt_name]}))


def _block_fp8(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    wb = (torch.randn(N, K, generator=g) * 0.02).reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    return (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn), sb


@pytest.mark.parametrize("fmt_name", ["mxfp8", "fp6_e3m2", "fp6_e2m3", "fp8_block"])
@pytest.mark.parametrize("M", [3, 200])
def test_loaded_merged_linear_matches_oracle(pkg, oracle_mod, dev, tmp_path, fmt_name, M):
    K, widths = 640, (256, 384)                 # K % 512 != 0: a partial last super-tile
    shards = ["model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"]
    tensors, codes, scales, biases = {}, [], [], []
    for i, (name, n) in enumerate(zip(shards, widths)):
        if fmt_name == "fp8_block":
            wq, sb = _block_fp8(n, K, 50 + i)
            tensors[f"{name}.weight"] = wq
            # fp8/linear.py:120-123 prefers weight_scale_inv and falls back to weight_scale
            tensors[f"{name}.weight_scale_inv" if i == 0 else f"{name}.weight_scale"] = sb
            codes.append(wq.view(torch.uint8).numpy()); scales.append(sb.numpy())
        else:
            g = torch.Generator().manual_seed(60 + i)
            w = (torch.randn(n, K, generator=g) * 0.03).bfloat16()
            fmt = _FMT[fmt_name]
            c, s = oracle_mod.quant_mxfp8(w, 0) if fmt == 0 else oracle_mod.quant_mxfp6(w, fmt)
            stored = torch.from_numpy(c).view(torch.float8_e4m3fn) if fmt == 0 else \
                torch.from_numpy(oracle_mod.pack_fp6(c))
            tensors[f"{name}.weight"] = stored
            tensors[f"{name}.weight_scale"] = torch.from_numpy(s)
            codes.append(c); scales.append(s)
        if M == 3:
            b = torch.randn(n, generator=torch.Generator().manual_seed(70 + i)).bfloat16()
            tensors[f"{name}.bias"] = b
            biases.append(b)
    _write(tmp_path, fmt_name, tensors)

    key = pkg.linear_quant_key(pkg.quant_config_of(tmp_path), "model.layers.0.mlp.gate_up_proj", shards)
    assert key is not None
    layer = pkg.load_linear(pkg.SafetensorsCheckpoint(tmp_path), "model.layers.0.mlp.gate_up_proj", key,
                            shards=shards, device=dev)
    assert layer.mxl_shape == (sum(widths), K)
    x = _act(M, K, 80 + M)
    y = layer(x.to(dev)).float().cpu()

    wc, ws = np.concatenate(codes), np.concatenate(scales)
    if fmt_name == "fp8_block":
        rq, rs = oracle_mod.quant_block_fp8(x)
        ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wc, ws))
    else:
        rc, rs = oracle_mod.quant_mxfp8(x, 0)
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, _FMT[fmt_name])))
    if biases:
        ref = (torch.from_numpy(ref).bfloat16() + torch.cat(biases)).float().numpy()
    _check(y.numpy(), ref)


def test_load_rejects_mismatched_checkpoint(pkg, oracle_mod, dev, tmp_path):
    """A tensor whose dtype is not the scheme's (bf16 codes under MXFP8) is an error."""
    tensors = {"p.weight": torch.zeros(128, 128, dtype=torch.bfloat16),
               "p.weight_scale": torch.zeros(128, 4, dtype=torch.uint8)}
    _write(tmp_path, "mxfp8", tensors)
    with pytest.raises(ValueError, match="does not match"):
        pkg.load_linear(pkg.SafetensorsCheckpoint(tmp_path), "p", pkg.linear.MXFP8_STATIC, device=dev)


@pytest.mark.parametrize("fmt_name", ["fp6_e3m2", "fp6_e2m3"])
def test_loaded_experts_match_oracle(pkg, oracle_mod, dev, tmp_path, fmt_name):
    E, H, I, T, topk = 4, 256, 128, 9, 2
    fmt = _FMT[fmt_name]
    c13, s13, c2, s2, x, wts, ids = _moe_case(oracle_mod, E, H, I, T, topk, 4242, fmt)
    tensors = {}
    for e in range(E):
        base = f"model.layers.0.mlp.experts.{e}"
        for name, rows in (("gate_proj", slice(0, I)), ("up_proj", slice(I, 2 * I))):
            tensors[f"{base}.{name}.weight"] = torch.from_numpy(oracle_mod.pack_fp6(c13[e][rows]))
            tensors[f"{base}.{name}.weight_scale"] = torch.from_numpy(np.ascontiguousarray(s13[e][rows]))
        tensors[f"{base}.down_proj.weight"] = torch.from_numpy(oracle_mod.pack_fp6(c2[e]))
        tensors[f"{base}.down_proj.weight_scale"] = torch.from_numpy(s2[e])
    _write(tmp_path, fmt_name, tensors)
    key = pkg.moe_quant_key(pkg.quant_config_of(tmp_path), "model.layers.0.mlp")
    layer = pkg.load_moe(pkg.SafetensorsCheckpoint(tmp_path), "model.layers.0.mlp", E, key, device=dev)
    xd, wd, idd = x.to(dev), wts.to(dev), ids.to(dev)
    got = layer(xd, wd, idd)

    # the same experts packed directly (no checkpoint): identical kernels, identical bits
    direct = pkg.Mxfp6Experts(fmt=fmt)
    w1, w2 = direct.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    assert torch.equal(got, direct(xd, w1, w2, wd, idd))
    ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(x, c13, s13, c2, s2, wts.numpy(), ids.numpy(), fmt))
    rel = np.linalg.norm(got.float().cpu().numpy() - ref) / np.linalg.norm(ref)
    assert rel < 1e-2, rel
