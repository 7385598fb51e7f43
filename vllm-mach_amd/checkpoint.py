"""On-disk formats of the quantized linear path, and loading them into MFMA-native layers.

Three checkpoint formats reach the path (the formats the reference's loaders accept):

* compressed-tensors MXFP8 (``quant_method: compressed-tensors``, ``format:
  mxfp8-quantized``; src/vllm_mach/mxfp8/prepare_model.py:665-681): ``<layer>.weight``
  F8_E4M3 [N, K] and ``<layer>.weight_scale`` U8 E8M0 [N, K/32] (key rule
  prepare_model.py:632-633), layers named in ``ignore`` stay bf16;
* Quark OCP-MX FP6 (``quant_method: quark``, ``global_quant_config`` weight
  ``fp6_e3m2``/``fp6_e2m3`` per_group 32 e8m0 static, input fp8_e4m3 per_group 32 e8m0
  dynamic; src/vllm_mach/runtime/attention.py:25-45): ``<layer>.weight`` U8 [N, 3K/4]
  (four 6-bit codes in three bytes, src/vllm_mach/mxfp6/dense.py:61-80) and
  ``<layer>.weight_scale`` U8 [N, K/32]; routed experts as per-expert tensors stacked
  into ``w13_weight``/``w2_weight`` (mxfp6/profile/runtime.patch:207-250);
* block-FP8 (``quant_method: fp8``, ``weight_block_size: [128, 128]``, dynamic
  activations): ``<layer>.weight`` F8_E4M3 [N, K] and fp32 ``<layer>.weight_scale_inv``
  (or ``weight_scale``) [ceil(N/128), K/128] (src/vllm_mach/fp8/linear.py:120-134).

``linear_quant_key`` / ``moe_quant_key`` read the HF ``quantization_config`` and name the
scheme for one layer (None: not quantized by a scheme this path serves).
``SafetensorsCheckpoint`` reads shards through safetensors only -- nothing in a
checkpoint is unpickled or executed.  ``load_linear`` / ``load_moe`` drive the vLLM
loading sequence (``create_weights`` -> ``weight_loader`` per checkpoint tensor ->
``process_weights_after_loading``) and return ready layers in the tiled layout.
"""
from __future__ import annotations

import fnmatch
import json
import re
from pathlib import Path
from typing import Iterable, Optional, Sequence, Union

import torch

from . import linear as L
from . import ops
from .moe import Mxfp6MoEMethod

_FP6_KEYS = {"fp6_e3m2": L.MXFP6_E3M2_STATIC, "fp6_e2m3": L.MXFP6_E2M3_STATIC}
_FP6_FMT = {L.MXFP6_E3M2_STATIC: ops.E3M2, L.MXFP6_E2M3_STATIC: ops.E2M3}


# ------------------------------------------------------------ quantization config

def _matches(name: str, pattern: str) -> bool:
    """``re:<regex>`` (compressed-tensors), a shell wildcard (Quark), else an exact name."""
    if pattern.startswith("re:"):
        return re.match(pattern[3:], name) is not None
    if any(c in pattern for c in "*?["):
        return fnmatch.fnmatchcase(name, pattern)
    return name == pattern


def _excluded(prefix: str, patterns: Iterable[str], shards: Optional[Sequence[str]]) -> bool:
    """A merged layer (``shards`` = its checkpoint prefixes) is excluded only if all of its
    shards are; a disagreement is an error, as in vLLM's fused-layer skip check."""
    patterns = list(patterns or ())
    names = list(shards) if shards else [prefix]
    hits = [any(_matches(n, p) for p in patterns) for n in names]
    if any(hits) and not all(hits):
        raise ValueError(f"shards of {prefix} are quantized differently: {dict(zip(names, hits))}")
    return all(hits)


def _mxfp8_rule(rule: dict, dynamic: bool) -> bool:
    return (isinstance(rule, dict) and rule.get("num_bits") == 8 and rule.get("type") == "float"
            and rule.get("strategy") == "group" and rule.get("group_size") == 32
            and rule.get("symmetric", True) is True and bool(rule.get("dynamic")) is dynamic)


def _compressed_tensors_key(qc: dict, prefix: str, shards) -> Optional[str]:
    if _excluded(prefix, qc.get("ignore", ()), shards):
        return None
    for group in (qc.get("config_groups") or {}).values():
        targets = group.get("targets", ())
        if not any(t == "Linear" or _matches(prefix, t) for t in targets):
            continue
        fmt = group.get("format", qc.get("format"))
        if (fmt == "mxfp8-quantized" and _mxfp8_rule(group.get("weights"), False)
                and _mxfp8_rule(group.get("input_activations"), True)):
            return L.MXFP8_STATIC
        return None
    return None


def _quark_scheme(qc: dict, prefix: str) -> Optional[dict]:
    for pattern, cfg in (qc.get("layer_quant_config") or {}).items():
        if _matches(prefix, pattern):
            return cfg
    return qc.get("global_quant_config")


def _quark_key(qc: dict, prefix: str, shards) -> Optional[str]:
    if _excluded(prefix, qc.get("exclude", ()), shards):
        return None
    scheme = _quark_scheme(qc, prefix)
    if not isinstance(scheme, dict):
        return None
    w, a = scheme.get("weight"), scheme.get("input_tensors")
    if not isinstance(w, dict) or not isinstance(a, dict):
        return None
    ok_w = (w.get("dtype") in _FP6_KEYS and w.get("group_size") == 32 and w.get("qscheme") == "per_group"
            and w.get("scale_format") == "e8m0" and w.get("is_dynamic") is False and w.get("symmetric") is True)
    ok_a = (a.get("dtype") == "fp8_e4m3" and a.get("group_size") == 32 and a.get("qscheme") == "per_group"
            and a.get("scale_format") == "e8m0" and a.get("is_dynamic") is True and a.get("symmetric") is True)
    return _FP6_KEYS[w["dtype"]] if ok_w and ok_a else None


def _fp8_key(qc: dict, prefix: str, shards) -> Optional[str]:
    ignored = list(qc.get("ignored_layers") or ()) + list(qc.get("modules_to_not_convert") or ())
    if _excluded(prefix, ignored, shards):
        return None
    if (list(qc.get("weight_block_size") or ()) == [128, 128] and qc.get("activation_scheme") == "dynamic"
            and qc.get("fmt", "e4m3") == "e4m3"):
        return L.FP8_BLOCK128
    return None


def linear_quant_key(quant_config: Optional[dict], prefix: str,
                     shards: Optional[Sequence[str]] = None) -> Optional[str]:
    """Weight quant key for the linear layer at ``prefix`` under an HF ``quantization_config``
    (a config.json's ``quantization_config`` object), or None when the layer is excluded or
    its scheme is not one of this path's.  ``shards`` lists a merged layer's checkpoint
    prefixes (q/k/v, gate/up)."""
    if not quant_config:
        return None
    method = quant_config.get("quant_method")
    if method == "compressed-tensors":
        return _compressed_tensors_key(quant_config, prefix, shards)
    if method == "quark":
        return _quark_key(quant_config, prefix, shards)
    if method == "fp8":
        return _fp8_key(quant_config, prefix, shards)
    return None


def moe_quant_key(quant_config: Optional[dict], prefix: str) -> Optional[str]:
    """Quant key of the routed experts under ``prefix`` (Quark OCP-MX FP6 only: the reference's
    W6A8 MoE admission, tests/native_mxfp6/test_moe_quant_admission_cpu.py:35-60)."""
    key = linear_quant_key(quant_config, prefix) if (quant_config or {}).get("quant_method") == "quark" else None
    return key if key in _FP6_FMT else None


def quant_config_of(model_dir: Union[str, Path]) -> Optional[dict]:
    """The ``quantization_config`` of a model directory's config.json (or its text_config)."""
    cfg = json.loads((Path(model_dir) / "config.json").read_text())
    for section in (cfg, cfg.get("text_config") or {}):
        if isinstance(section.get("quantization_config"), dict):
            return section["quantization_config"]
    return None


# ------------------------------------------------------------ safetensors reading

_ST_DTYPES = {"F8_E4M3": torch.float8_e4m3fn, "U8": torch.uint8, "F32": torch.float32,
              "BF16": torch.bfloat16, "F16": torch.float16, "I32": torch.int32, "I64": torch.int64}


def _header(path: Path) -> dict:
    with open(path, "rb") as f:
        size = int.from_bytes(f.read(8), "little")
        if size <= 0 or size > 100 << 20:
            raise ValueError(f"{path}: invalid safetensors header length {size}")
        head = json.loads(f.read(size))
    head.pop("__metadata__", None)
    return head


class SafetensorsCheckpoint:
    """Read-only view of a ``.safetensors`` file or a directory of shards.

    A directory with one ``*.safetensors.index.json`` is read through its ``weight_map``;
    otherwise every ``*.safetensors`` in it is scanned and a key present in two shards is
    an error.  Headers are parsed as JSON and tensors are read by safetensors' own loader.
    """

    def __init__(self, path: Union[str, Path]):
        from safetensors import safe_open  # noqa: F401  (fail early when it is missing)
        root = Path(path)
        self._where: dict[str, Path] = {}
        self._meta: dict[str, dict] = {}
        if root.is_file():
            if root.suffix != ".safetensors":
                raise ValueError(f"{root} is not a .safetensors file")
            files = [root]
            index = None
        else:
            indices = sorted(root.glob("*.safetensors.index.json"))
            if len(indices) > 1:
                raise ValueError(f"{root} holds more than one safetensors index")
            index = json.loads(indices[0].read_text())["weight_map"] if indices else None
            files = sorted({root / f for f in index.values()}) if index else sorted(root.glob("*.safetensors"))
            if not files:
                raise ValueError(f"{root} holds no safetensors shards")
        for f in files:
            if f.suffix != ".safetensors" or not f.is_file():
                raise ValueError(f"shard {f} is missing or not a .safetensors file")
            for key, item in _header(f).items():
                if key in self._where:
                    raise ValueError(f"tensor {key} appears in {self._where[key].name} and {f.name}")
                if index is not None and Path(index.get(key, "")).name != f.name:
                    raise ValueError(f"tensor {key} in {f.name} is not where the index places it")
                self._where[key] = f
                self._meta[key] = item
        if index is not None and set(index) - set(self._where):
            raise ValueError(f"index names tensors absent from its shards: {sorted(set(index) - set(self._where))[:4]}")

    def keys(self) -> list[str]:
        return sorted(self._where)

    def __contains__(self, key: str) -> bool:
        return key in self._where

    def info(self, key: str) -> tuple[torch.dtype, tuple[int, ...]]:
        """(torch dtype, shape) from the header, without reading the data."""
        if key not in self._meta:
            raise KeyError(f"checkpoint has no tensor {key}")
        item = self._meta[key]
        if item["dtype"] not in _ST_DTYPES:
            raise ValueError(f"{key}: unsupported safetensors dtype {item['dtype']}")
        return _ST_DTYPES[item["dtype"]], tuple(item["shape"])

    def get(self, key: str, device: Union[str, torch.device, None] = None) -> torch.Tensor:
        from safetensors import safe_open
        self.info(key)
        dev = "cpu" if device is None else str(torch.device(device))
        with safe_open(str(self._where[key]), framework="pt", device=dev) as f:
            return f.get_tensor(key)


# ------------------------------------------------------------ loading layers

class QuantizedLinear(torch.nn.Module):
    """A linear layer in the tiled layout: ``forward`` is the quant method's ``apply``."""

    def __init__(self, method: L.MxLinearMethod):
        super().__init__()
        self.quant_method = method
        self.bias: Optional[torch.Tensor] = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.quant_method.apply(self, x, self.bias)


def _scale_name(ckpt: SafetensorsCheckpoint, prefix: str, key: str) -> str:
    if key != L.FP8_BLOCK128:
        return "weight_scale"
    # fp8/linear.py:120-123: weight_scale_inv first, weight_scale otherwise
    return "weight_scale_inv" if f"{prefix}.weight_scale_inv" in ckpt else "weight_scale"


def load_linear(ckpt: SafetensorsCheckpoint, prefix: str, quant_key: str,
                shards: Optional[Sequence[str]] = None, device: Union[str, torch.device, None] = None,
                method: Optional[L.MxLinearMethod] = None) -> QuantizedLinear:
    """Build the layer at ``prefix`` from checkpoint tensors and prepare it for the GPU.

    ``shards`` lists the checkpoint prefixes merged along N, in order (e.g. gate_proj then
    up_proj for a gate_up layer); by default the layer is the single tensor at ``prefix``.
    A ``<shard>.bias`` (bf16) is loaded when every shard has one.
    """
    names = list(shards) if shards else [prefix]
    method = method or L.MxLinearMethod(quant_key)
    widths, ks = [], set()
    for name in names:
        dtype, shape = ckpt.info(f"{name}.weight")
        if len(shape) != 2:
            raise ValueError(f"{name}.weight must be two-dimensional, got {shape}")
        widths.append(shape[0])
        ks.add(shape[1] * 4 // 3 if quant_key in _FP6_FMT else shape[1])
        if quant_key in _FP6_FMT and shape[1] % 3:
            raise ValueError(f"{name}.weight: packed FP6 width {shape[1]} is not a multiple of 3")
    if len(ks) != 1:
        raise ValueError(f"shards of {prefix} disagree on K: {sorted(ks)}")
    k = ks.pop()
    layer = QuantizedLinear(method)
    method.create_weights(layer, k, widths, k, sum(widths), torch.bfloat16, device=device)
    scale_param = "weight_scale_inv" if quant_key == L.FP8_BLOCK128 else "weight_scale"
    for i, name in enumerate(names):
        shard = None if len(names) == 1 else i
        w = layer.weight
        w.weight_loader(w, ckpt.get(f"{name}.weight", device), shard)
        s = getattr(layer, scale_param)
        s.weight_loader(s, ckpt.get(f"{name}.{_scale_name(ckpt, name, quant_key)}", device), shard)
    if all(f"{name}.bias" in ckpt for name in names):
        bias = torch.cat([ckpt.get(f"{name}.bias", device) for name in names])
        if bias.dtype != torch.bfloat16:
            raise ValueError(f"{prefix}: bias must be bf16, got {bias.dtype}")
        layer.bias = bias
    method.process_weights_after_loading(layer)
    return layer


class QuantizedExperts(torch.nn.Module):
    """Routed experts in the tiled layout: ``forward(x, topk_weights, topk_ids)``."""

    def __init__(self, method: Mxfp6MoEMethod):
        super().__init__()
        self.quant_method = method

    def forward(self, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        return self.quant_method.apply(self, x, topk_weights, topk_ids)


def load_moe(ckpt: SafetensorsCheckpoint, prefix: str, num_experts: int, quant_key: str,
             device: Union[str, torch.device, None] = None,
             expert_names: tuple[str, str, str] = ("gate_proj", "up_proj", "down_proj")) -> QuantizedExperts:
    """Routed experts ``<prefix>.experts.<e>.<gate|up|down>.weight`` (+ ``.weight_scale``),
    stacked through vLLM's expert loader (gate -> w1, up -> w3, down -> w2)."""
    if quant_key not in _FP6_FMT:
        raise ValueError(f"routed experts load packed MXFP6 only, not {quant_key}")
    gate, up, down = expert_names
    _, gshape = ckpt.info(f"{prefix}.experts.0.{gate}.weight")
    _, dshape = ckpt.info(f"{prefix}.experts.0.{down}.weight")
    inter, hidden = gshape[0], dshape[0]
    method = Mxfp6MoEMethod(_FP6_FMT[quant_key])
    layer = QuantizedExperts(method)
    method.create_weights(layer, num_experts, hidden, inter, torch.bfloat16, device=device)
    for e in range(num_experts):
        for name, shard in ((gate, "w1"), (up, "w3"), (down, "w2")):
            base = f"{prefix}.experts.{e}.{name}"
            for suffix, param_name in (("weight", "_weight"), ("weight_scale", "_weight_scale")):
                param = getattr(layer, ("w13" if shard != "w2" else "w2") + param_name)
                param.weight_loader(param, ckpt.get(f"{base}.{suffix}", device), f"{base}.{suffix}", shard, e)
    method.process_weights_after_loading(layer)
    return layer
