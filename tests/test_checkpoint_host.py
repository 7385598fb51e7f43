"""Checkpoint formats on the host: scheme recognition from HF quantization configs, the
safetensors reader, and where the vLLM-style loaders put each shard (no GPU needed).

The Quark scheme dicts are the ones the reference's own admission tests use
(tests/native_mxfp6/test_dense_prep_cpu.py:12-16, tests/test_attention_segments_cpu.py:9);
the compressed-tensors dict has the fields prepare_model.py:665-681 writes; the block-FP8
dict has vLLM's Fp8Config fields that fp8/linear.py serves (weight_block_size 128x128,
dynamic activations)."""
import json

import pytest
import torch
from safetensors.torch import save_file


def _ct_config(ignore=("lm_head",), **weight_overrides):
    rule = {"actorder": None, "block_structure": None, "group_size": 32, "num_bits": 8, "observer_kwargs": {},
            "scale_dtype": "torch.uint8", "strategy": "group", "symmetric": True, "type": "float", "zp_dtype": None}
    return {"quant_method": "compressed-tensors", "format": "mxfp8-quantized",
            "config_groups": {"group_0": {
                "format": "mxfp8-quantized", "targets": ["Linear"],
                "weights": {**rule, "dynamic": False, **weight_overrides},
                "input_activations": {**rule, "dynamic": True}}},
            "ignore": list(ignore)}


def _quark_config(wdtype="fp6_e3m2", exclude=("lm_head",), **act_overrides):
    weight = dict(dtype=wdtype, group_size=32, qscheme="per_group", scale_format="e8m0",
                  is_dynamic=False, symmetric=True)
    act = dict(dtype="fp8_e4m3", group_size=32, qscheme="per_group", scale_format="e8m0",
               is_dynamic=True, symmetric=True)
    act.update(act_overrides)
    return {"quant_method": "quark", "global_quant_config": {"weight": weight, "input_tensors": act},
            "exclude": list(exclude)}


def _fp8_config(**kw):
    cfg = {"quant_method": "fp8", "activation_scheme": "dynamic", "weight_block_size": [128, 128],
           "fmt": "e4m3", "ignored_layers": ["model.layers.0.mlp.down_proj"]}
    cfg.update(kw)
    return cfg


def test_compressed_tensors_mxfp8(pkg):
    L = pkg.linear
    cfg = _ct_config(ignore=("lm_head", "re:.*linear_attn\\.in_proj_[ab]$"))
    assert pkg.linear_quant_key(cfg, "model.layers.3.mlp.down_proj") == L.MXFP8_STATIC
    assert pkg.linear_quant_key(cfg, "lm_head") is None
    assert pkg.linear_quant_key(cfg, "model.layers.0.linear_attn.in_proj_a") is None
    assert pkg.linear_quant_key(cfg, "model.layers.0.linear_attn.in_proj_qkvz") == L.MXFP8_STATIC
    # near misses stay with upstream
    assert pkg.linear_quant_key(_ct_config(group_size=16), "x.down_proj") is None
    assert pkg.linear_quant_key(_ct_config(dynamic=True), "x.down_proj") is None
    assert pkg.linear_quant_key(_ct_config(num_bits=4), "x.down_proj") is None


def test_merged_layer_shards_must_agree(pkg):
    cfg = _ct_config(ignore=("model.layers.0.mlp.gate_proj",))
    with pytest.raises(ValueError, match="quantized differently"):
        pkg.linear_quant_key(cfg, "model.layers.0.mlp.gate_up_proj",
                             ["model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"])
    cfg = _ct_config(ignore=("model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"))
    assert pkg.linear_quant_key(cfg, "model.layers.0.mlp.gate_up_proj",
                                ["model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"]) is None


def test_quark_ocp_mx_fp6(pkg):
    L = pkg.linear
    cfg = _quark_config(exclude=("lm_head", "*mlp.gate"))
    assert pkg.linear_quant_key(cfg, "model.layers.1.self_attn.o_proj") == L.MXFP6_E3M2_STATIC
    assert pkg.linear_quant_key(cfg, "model.layers.1.mlp.gate") is None
    assert pkg.linear_quant_key(cfg, "model.layers.1.mlp.gate_up_proj") == L.MXFP6_E3M2_STATIC
    assert pkg.linear_quant_key(_quark_config("fp6_e2m3"), "a.b") == L.MXFP6_E2M3_STATIC
    assert pkg.moe_quant_key(cfg, "model.layers.1.mlp") == L.MXFP6_E3M2_STATIC
    # per-tensor or static activations, fp4 weights: not this path
    assert pkg.linear_quant_key(_quark_config(qscheme="per_tensor"), "a.b") is None
    assert pkg.linear_quant_key(_quark_config(is_dynamic=False), "a.b") is None
    assert pkg.linear_quant_key(_quark_config("fp4"), "a.b") is None
    # a per-layer override wins over the global scheme
    over = dict(cfg, layer_quant_config={"*.o_proj": {"weight": None, "input_tensors": None}})
    assert pkg.linear_quant_key(over, "model.layers.1.self_attn.o_proj") is None
    assert pkg.linear_quant_key(over, "model.layers.1.self_attn.qkv_proj") == L.MXFP6_E3M2_STATIC


def test_block_fp8(pkg):
    L = pkg.linear
    assert pkg.linear_quant_key(_fp8_config(), "model.layers.1.mlp.down_proj") == L.FP8_BLOCK128
    assert pkg.linear_quant_key(_fp8_config(), "model.layers.0.mlp.down_proj") is None
    assert pkg.linear_quant_key(_fp8_config(weight_block_size=[128, 64]), "a") is None
    assert pkg.linear_quant_key(_fp8_config(activation_scheme="static"), "a") is None
    assert pkg.linear_quant_key(_fp8_config(weight_block_size=None), "a") is None
    assert pkg.moe_quant_key(_fp8_config(), "a") is None
    assert pkg.linear_quant_key({"quant_method": "gptq"}, "a") is None
    assert pkg.linear_quant_key(None, "a") is None


def test_quant_config_of_reads_text_config(pkg, tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"text_config": {"quantization_config": _fp8_config()}}))
    assert pkg.quant_config_of(tmp_path)["quant_method"] == "fp8"
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "x"}))
    assert pkg.quant_config_of(tmp_path) is None


def test_reader_single_and_sharded(pkg, tmp_path):
    a = {"m.a.weight": torch.arange(12, dtype=torch.uint8).view(3, 4),
         "m.a.weight_scale": torch.full((3, 1), 127, dtype=torch.uint8)}
    b = {"m.b.weight": torch.randn(2, 8).to(torch.float8_e4m3fn),
         "m.b.weight_scale_inv": torch.ones(1, 1)}
    save_file(a, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(b, str(tmp_path / "model-00002-of-00002.safetensors"))
    ck = pkg.SafetensorsCheckpoint(tmp_path)
    assert ck.keys() == sorted(list(a) + list(b))
    assert ck.info("m.b.weight") == (torch.float8_e4m3fn, (2, 8))
    assert torch.equal(ck.get("m.a.weight"), a["m.a.weight"])
    assert torch.equal(ck.get("m.b.weight").view(torch.uint8), b["m.b.weight"].view(torch.uint8))
    with pytest.raises(KeyError):
        ck.get("m.c.weight")
    one = pkg.SafetensorsCheckpoint(tmp_path / "model-00001-of-00002.safetensors")
    assert "m.a.weight" in one and "m.b.weight" not in one
    # an index must agree with its shards
    index = {"metadata": {}, "weight_map": {**{k: "model-00001-of-00002.safetensors" for k in a},
                                            **{k: "model-00002-of-00002.safetensors" for k in b}}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    assert pkg.SafetensorsCheckpoint(tmp_path).keys() == ck.keys()
    index["weight_map"]["m.a.weight"] = "model-00002-of-00002.safetensors"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(ValueError, match="index"):
        pkg.SafetensorsCheckpoint(tmp_path)


def test_reader_rejects_duplicates_and_other_files(pkg, tmp_path):
    t = {"w": torch.zeros(2, dtype=torch.uint8)}
    save_file(t, str(tmp_path / "a.safetensors"))
    save_file(t, str(tmp_path / "b.safetensors"))
    with pytest.raises(ValueError, match="appears in"):
        pkg.SafetensorsCheckpoint(tmp_path)
    (tmp_path / "w.bin").write_bytes(b"\0" * 16)
    with pytest.raises(ValueError, match="not a .safetensors"):
        pkg.SafetensorsCheckpoint(tmp_path / "w.bin")
    (tmp_path / "empty").mkdir()
    with pytest.raises(ValueError, match="no safetensors"):
        pkg.SafetensorsCheckpoint(tmp_path / "empty")


@pytest.mark.parametrize("key", ["mxfp8_e4m3_static", "mxfp6_e2m3_static", "fp8_e4m3_block128"])
def test_merged_partitions_land_in_their_rows(pkg, key):
    """gate (128 rows) then up (256 rows): each shard's codes and scales go to its own rows."""
    L = pkg.linear
    layer = torch.nn.Module()
    L.MxLinearMethod(key).create_weights(layer, 256, [128, 256], 256, 384, torch.bfloat16, device="cpu")
    sname = "weight_scale_inv" if key == L.FP8_BLOCK128 else "weight_scale"
    w, s = layer.weight, getattr(layer, sname)
    parts = []
    for i, rows in enumerate((128, 256)):
        wi = torch.full((rows, w.shape[1]), i + 1, dtype=torch.uint8)
        si = (torch.full((rows // 128, 2), float(i + 2)) if key == L.FP8_BLOCK128
              else torch.full((rows, 8), 100 + i, dtype=torch.uint8))
        w.weight_loader(w, wi.view(w.dtype), i)
        s.weight_loader(s, si, i)
        parts.append((wi, si))
    assert torch.equal(w.data.view(torch.uint8), torch.cat([p[0] for p in parts]))
    assert torch.equal(s.data, torch.cat([p[1] for p in parts]))
    with pytest.raises(ValueError, match="does not match"):
        w.weight_loader(w, parts[0][0].view(w.dtype), 1)     # 128 rows into the 256-row shard
    with pytest.raises(ValueError, match="partitions"):
        w.weight_loader(w, parts[0][0].view(w.dtype), 2)
    with pytest.raises(ValueError, match="does not match"):
        s.weight_loader(s, parts[0][1].double(), 0)          # a dtype change is not converted


def test_qkv_shard_names_and_caller_loader(pkg):
    L = pkg.linear
    layer = torch.nn.Module()
    L.MxLinearMethod(L.MXFP8_STATIC).create_weights(layer, 128, [256, 128, 128], 128, 512, torch.bfloat16,
                                                    device="cpu")
    v = torch.full((128, 128), 7, dtype=torch.uint8).view(torch.float8_e4m3fn)
    layer.weight.weight_loader(layer.weight, v, "v")
    assert (layer.weight.data.view(torch.uint8)[384:] == 7).all()
    marker = object()
    other = torch.nn.Module()
    L.MxLinearMethod(L.MXFP8_STATIC).create_weights(other, 128, [128], 128, 128, torch.bfloat16, device="cpu",
                                                    weight_loader=marker)
    assert other.weight.weight_loader is marker and other.weight_scale.weight_loader is marker
    with pytest.raises(ValueError, match="multiples of 128"):
        L.MxLinearMethod(L.FP8_BLOCK128).create_weights(torch.nn.Module(), 128, [64, 128], 128, 192,
                                                        torch.bfloat16, device="cpu")


def test_moe_expert_loader(pkg):
    E, H, I = 3, 256, 128
    method = pkg.Mxfp6MoEMethod()
    layer = torch.nn.Module()
    method.create_weights(layer, E, H, I, torch.bfloat16, device="cpu")
    assert tuple(layer.w13_weight.shape) == (E, 2 * I, H * 3 // 4)
    assert tuple(layer.w2_weight_scale.shape) == (E, H, I // 32)
    for e in range(E):
        for shard, val in (("w1", 10), ("w3", 20)):
            p = layer.w13_weight
            p.weight_loader(p, torch.full((I, H * 3 // 4), val + e, dtype=torch.uint8), "w", shard, e)
            p = layer.w13_weight_scale
            p.weight_loader(p, torch.full((I, H // 32), val + e, dtype=torch.uint8), "s", shard, e)
        p = layer.w2_weight
        p.weight_loader(p, torch.full((H, I * 3 // 4), 30 + e, dtype=torch.uint8), "w", "w2", e)
    for e in range(E):
        assert (layer.w13_weight.data[e, :I] == 10 + e).all() and (layer.w13_weight.data[e, I:] == 20 + e).all()
        assert (layer.w13_weight_scale.data[e, I:] == 20 + e).all()
        assert (layer.w2_weight.data[e] == 30 + e).all()
    p = layer.w2_weight
    with pytest.raises(ValueError, match="outside"):
        p.weight_loader(p, torch.zeros((H, I * 3 // 4), dtype=torch.uint8), "w", "w2", E)
    with pytest.raises(ValueError, match="loads w13"):
        p.weight_loader(p, torch.zeros((I, I * 3 // 4), dtype=torch.uint8), "w", "w1", 0)
    with pytest.raises(ValueError, match="unknown expert shard"):
        p.weight_loader(p, torch.zeros((H, I * 3 // 4), dtype=torch.uint8), "w", "w4", 0)
    with pytest.raises(ValueError, match="divisible by 128"):
        method.create_weights(torch.nn.Module(), E, H, 96, torch.bfloat16, device="cpu")
