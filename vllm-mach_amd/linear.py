"""vLLM quantization surface for the MI355X quantized linear layers.

Two levels mirror the reference's drop-in boundary:

* kernel classes with vLLM's LinearKernel contract -- ``is_supported``,
  ``can_implement``, ``process_weights_after_loading``, ``apply_weights`` --
  the level the reference plugs into (src/vllm_mach/mxfp6/dense.py:160-214,
  src/vllm_mach/mxfp6/dense_mxfp8.py:114-162, src/vllm_mach/fp8/linear.py:157-216);
* ``MxLinearMethod``, a ``LinearMethodBase``-shaped method
  (``create_weights`` / ``process_weights_after_loading`` / ``apply``) that
  owns the checkpoint parameters and delegates to a kernel, for callers that
  plug in one level higher.

Importing this module does not touch the GPU; the HIP library is loaded on
the first call that needs it.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import ops

# quant keys (vLLM spells these kMxfp8Dynamic, kMxfp6E3M2Static, ...)
MXFP8_DYNAMIC = "mxfp8_e4m3_dynamic"
MXFP8_STATIC = "mxfp8_e4m3_static"
MXFP6_E3M2_STATIC = "mxfp6_e3m2_static"
MXFP6_E2M3_STATIC = "mxfp6_e2m3_static"
FP8_BLOCK128 = "fp8_e4m3_block128"

_FP6_FORMAT = {MXFP6_E3M2_STATIC: ops.E3M2, MXFP6_E2M3_STATIC: ops.E2M3}


def is_mi355x_available(device: Optional[int] = None) -> tuple[bool, Optional[str]]:
    """Fail-closed device admission: a gfx950 GPU and a loadable library."""
    try:
        if not torch.cuda.is_available():
            return False, "no HIP device"
        from . import _lib
        dev = torch.cuda.current_device() if device is None else device
        ok = _lib.query("mxl_device_supported", dev)
        if ok != 1:
            return False, f"device {dev} is not gfx950"
        return True, None
    except Exception as error:  # noqa: BLE001 - admission must fail closed
        return False, f"mach_amd runtime unavailable: {error}"


def _replace(layer: torch.nn.Module, name: str, value: torch.Tensor) -> None:
    setattr(layer, name, torch.nn.Parameter(value, requires_grad=False))


_QKV_SHARDS = {"q": 0, "k": 1, "v": 2}


def load_partition(param: torch.nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id=None) -> None:
    """Copy one checkpoint tensor into a parameter made by ``MxLinearMethod.create_weights``.

    ``loaded_shard_id`` None loads the whole parameter; an index (or ``"q"``/``"k"``/``"v"``)
    loads partition ``i`` of a merged layer (gate/up, q/k/v) into rows
    ``sum(widths[:i]) / r`` .. of the parameter, r being the output rows one entry covers
    (1 for codes and E8M0 scales, 128 for block-FP8 scales), as vLLM's merged-column
    loaders do.  Shape and dtype must match exactly: a checkpoint in another format is an
    error, never a silent conversion.
    """
    widths = param.mxl_logical_widths
    rows = param.mxl_rows_per_entry
    target = param.data
    if loaded_shard_id is not None:
        idx = _QKV_SHARDS.get(loaded_shard_id, loaded_shard_id)
        if not isinstance(idx, int) or not 0 <= idx < len(widths):
            raise ValueError(f"shard {loaded_shard_id!r} is not one of {len(widths)} partitions")
        start = sum(widths[:idx])
        target = target.narrow(0, start // rows, (widths[idx] + rows - 1) // rows)
    if loaded_weight.dtype != target.dtype or tuple(loaded_weight.shape) != tuple(target.shape):
        raise ValueError(f"checkpoint tensor {loaded_weight.dtype}{tuple(loaded_weight.shape)} does not match "
                         f"parameter slice {target.dtype}{tuple(target.shape)}")
    target.copy_(loaded_weight)


def _flatten(x: torch.Tensor, k: int) -> torch.Tensor:
    return x.reshape(-1, k)


@dataclass
class MxLinearLayerConfig:
    """The fields of vLLM's Mxfp8/MxFp6 LinearLayerConfig that the kernels read."""
    weight_quant_key: str = MXFP8_STATIC
    activation_quant_key: str = MXFP8_DYNAMIC
    weight_shape: Optional[tuple[int, int]] = None


class _Kernel:
    def __init__(self, config: Optional[MxLinearLayerConfig] = None):
        self.config = config or MxLinearLayerConfig()

    @classmethod
    def is_supported(cls, compute_capability=None) -> tuple[bool, Optional[str]]:
        return is_mi355x_available()


class Mxfp8LinearKernel(_Kernel):
    """W8A8 MXFP8: E4M3 weights [N, K] with E8M0 scales [N, K/32]; bf16 activations
    quantized on the fly (rule floor_carry175, the repo's quantizer); bf16 out.

    Mirrors ``Mxfp8Sm120LinearKernel`` (src/vllm_mach/mxfp6/dense_mxfp8.py:114-162).
    """

    act_rule = ops.FLOOR_CARRY175

    def __init__(self, config: Optional[MxLinearLayerConfig] = None, dual_m: tuple[int, ...] = ()):
        """``dual_m``: row counts served by two-limb activations (the reference's M32/M64
        dual dispatch, src/vllm_mach/mxfp8/dual.py:53-75); every other M uses one limb."""
        super().__init__(config)
        if any(m <= 0 or m > 64 for m in dual_m):
            raise ValueError("two-limb activations serve 1 <= M <= 64")
        self.dual_m = frozenset(dual_m)

    @classmethod
    def can_implement(cls, config: MxLinearLayerConfig) -> tuple[bool, Optional[str]]:
        return True, None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        weight = layer.weight.data
        if weight.ndim != 2 or any(d <= 0 or d % 128 for d in weight.shape):
            raise ValueError("MXFP8 requires positive N and K divisible by 128")
        if weight.dtype != torch.float8_e4m3fn:
            raise ValueError("MXFP8 requires E4M3 weights")
        if getattr(layer, "params_dtype", torch.bfloat16) != torch.bfloat16:
            raise ValueError("MXFP8 requires bfloat16 params")
        n, k = weight.shape
        scale = layer.weight_scale.data
        if scale.dtype != torch.uint8 or tuple(scale.shape) != (n, k // 32):
            raise ValueError("MXFP8 requires uint8 E8M0 scales shaped [N, K/32]")
        tiled, tiled_s = ops.pack_weight(weight.contiguous(), scale.contiguous(), ops.E4M3)
        _replace(layer, "weight", tiled)
        _replace(layer, "weight_scale", tiled_s)
        layer.mxl_shape = (n, k)
        layer.mxl_format = ops.E4M3
        layer.mxl_kernel = self

    def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        n, k = layer.mxl_shape
        if x.dtype != torch.bfloat16 or x.shape[-1] != k:
            raise ValueError("MXFP8 requires BF16 activations with matching K")
        if x.numel() == 0:
            return x.new_empty((*x.shape[:-1], n))
        x2 = _flatten(x, k).contiguous()
        gemm = ops.mx_gemm_from_float_dual if x2.shape[0] in self.dual_m else ops.mx_gemm_from_float
        y = gemm(x2, layer.weight, layer.weight_scale, n, layer.mxl_format, self.act_rule)
        y = y.reshape(*x.shape[:-1], n)
        return y if bias is None else y + bias


def logical_mxfp6_shape(weight: torch.Tensor) -> tuple[int, int]:
    """[N, 3K/4] packed -> (N, K) with the reference's admission rules
    (src/vllm_mach/mxfp6/dense.py:61-80): 4 values in 3 bytes, N % 8, K % 128."""
    if weight.ndim != 2:
        raise ValueError(f"MXFP6 requires a two-dimensional packed weight; got shape={tuple(weight.shape)}")
    n, packed = map(int, weight.shape)
    if packed % 3 != 0:
        raise ValueError(f"MXFP6 requires four FP6 values packed into three bytes; got packed K={packed}")
    k = packed * 4 // 3
    if n % 8 != 0 or k % 128 != 0:
        raise ValueError(f"MXFP6 requires N % 8 == 0 and K % 128 == 0; got N={n}, K={k}")
    return n, k


class Mxfp6LinearKernel(_Kernel):
    """W6A8: packed MXFP6 weights (E2M3 or E3M2) [N, 3K/4] + E8M0 [N, K/32];
    MXFP8 dynamic activations; bf16 out.

    Mirrors ``Mxfp6Sm120LinearKernel`` (src/vllm_mach/mxfp6/dense.py:160-214); E2M3 is
    admitted alongside the reference's E3M2.
    """

    act_rule = ops.FLOOR_CARRY175

    @classmethod
    def can_implement(cls, config: MxLinearLayerConfig) -> tuple[bool, Optional[str]]:
        if config.weight_quant_key not in _FP6_FORMAT:
            return False, "requires static MXFP6 (E3M2 or E2M3) weights"
        if config.activation_quant_key != MXFP8_DYNAMIC:
            return False, "requires dynamic MXFP8 E4M3 activations"
        return True, None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        n, k = logical_mxfp6_shape(layer.weight)
        fmt = _FP6_FORMAT[self.config.weight_quant_key]
        scale = layer.weight_scale.data
        if scale.dtype != torch.uint8 or tuple(scale.shape) != (n, k // 32):
            raise ValueError("MXFP6 requires uint8 E8M0 scales shaped [N, K/32]")
        tiled, tiled_s = ops.pack_weight(layer.weight.data.contiguous(), scale.contiguous(), fmt)
        _replace(layer, "weight", tiled)
        _replace(layer, "weight_scale", tiled_s)
        layer.mxl_shape = (n, k)
        layer.mxl_format = fmt
        layer.mxl_kernel = self

    def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        n, k = layer.mxl_shape
        if int(x.shape[-1]) != k:
            raise ValueError(f"MXFP6 activation and packed weight dimensions differ; got activation K="
                             f"{int(x.shape[-1])}, weight K={k}")
        if x.dtype != torch.bfloat16:
            raise ValueError("MXFP6 requires BF16 activations")
        if x.numel() == 0:
            return x.new_empty((*x.shape[:-1], n))
        y = ops.mx_gemm_from_float(_flatten(x, k).contiguous(), layer.weight, layer.weight_scale, n,
                                   layer.mxl_format, self.act_rule)
        y = y.reshape(*x.shape[:-1], n)
        return y if bias is None else y + bias


class BlockFp8LinearKernel(_Kernel):
    """Block-FP8: E4M3 weights [N, K] with fp32 ``weight_scale_inv`` [N/128, K/128];
    activations quantized per token per 128 (fp32 scales); bf16 out.

    Mirrors the patched ``CutlassFp8BlockScaledMMKernel`` (src/vllm_mach/fp8/linear.py:157-192).
    """

    @classmethod
    def can_implement(cls, config: MxLinearLayerConfig) -> tuple[bool, Optional[str]]:
        return (True, None) if config.weight_quant_key == FP8_BLOCK128 else (False, "requires block-128 FP8")

    @staticmethod
    def _scale(layer):
        scale = getattr(layer, "weight_scale_inv", None)
        return getattr(layer, "weight_scale", None) if scale is None else scale

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        weight = layer.weight.data
        scale = self._scale(layer)
        if weight.ndim != 2 or weight.dtype != torch.float8_e4m3fn or weight.shape[1] % 128:
            raise ValueError("block-FP8 requires E4M3 weights [N, K] with K % 128 == 0")
        n, k = weight.shape
        if scale is None or scale.dtype != torch.float32 or tuple(scale.shape) != ((n + 127) // 128, k // 128):
            raise ValueError("block-FP8 requires fp32 scales [ceil(N/128), K/128]")
        tiled, _ = ops.pack_weight(weight.contiguous(), None, ops.E4M3)
        _replace(layer, "weight", tiled)
        layer.mxl_block_scale = scale.data.contiguous()
        layer.mxl_shape = (n, k)
        layer.mxl_kernel = self

    def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        n, k = layer.mxl_shape
        if x.dtype != torch.bfloat16 or x.shape[-1] != k:
            raise ValueError("block-FP8 requires BF16 activations with matching K")
        if x.numel() == 0:
            return x.new_empty((*x.shape[:-1], n))
        y = ops.block_fp8_from_float(_flatten(x, k).contiguous(), layer.weight, layer.mxl_block_scale, n)
        y = y.reshape(*x.shape[:-1], n)
        return y if bias is None else y + bias


_KERNELS = {
    MXFP8_STATIC: Mxfp8LinearKernel,
    MXFP6_E3M2_STATIC: Mxfp6LinearKernel,
    MXFP6_E2M3_STATIC: Mxfp6LinearKernel,
    FP8_BLOCK128: BlockFp8LinearKernel,
}


class MxLinearMethod:
    """``LinearMethodBase``-shaped method for one of the quantized linear schemes.

    ``create_weights`` registers the checkpoint-format parameters (the layouts of
    compressed-tensors MXFP8, Quark OCP-MX packed FP6 and block-FP8 ``weight_scale_inv``);
    ``process_weights_after_loading`` repacks them to the MFMA-tiled layout;
    ``apply`` runs the layer.
    """

    def __init__(self, weight_quant_key: str = MXFP8_STATIC):
        if weight_quant_key not in _KERNELS:
            raise ValueError(f"unknown weight quant key {weight_quant_key!r}")
        act = FP8_BLOCK128 if weight_quant_key == FP8_BLOCK128 else MXFP8_DYNAMIC
        self.config = MxLinearLayerConfig(weight_quant_key, act)
        self.kernel = _KERNELS[weight_quant_key](self.config)

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: list[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        """Registers the checkpoint parameters.  Each carries ``output_dim``/``input_dim``
        and a ``weight_loader(param, loaded_weight, loaded_shard_id=None)``: the caller's
        (vLLM passes the layer's own in ``extra_weight_attrs``) or ``load_partition``,
        which places shard ``i`` of a merged layer at rows ``sum(widths[:i])``.  Other
        ``extra_weight_attrs`` are set on the parameters as vLLM's ``set_weight_attrs`` does;
        ``device`` picks where the empty parameters live."""
        n, k = sum(output_partition_sizes), input_size_per_partition
        if k % 128:
            raise ValueError("input size per partition must be a multiple of 128")
        if n <= 0 or any(w <= 0 for w in output_partition_sizes):
            raise ValueError("output partition sizes must be positive")
        key = self.config.weight_quant_key
        attrs = dict(extra_weight_attrs)
        device = attrs.pop("device", None)
        rows_per_scale = 1
        if key == MXFP8_STATIC:
            w = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=device)
            s = torch.empty((n, k // 32), dtype=torch.uint8, device=device)
            names = ("weight", "weight_scale")
        elif key in _FP6_FORMAT:
            w = torch.empty((n, k * 3 // 4), dtype=torch.uint8, device=device)
            s = torch.empty((n, k // 32), dtype=torch.uint8, device=device)
            names = ("weight", "weight_scale")
        else:
            # vLLM's block-shape validation: merged partitions start on a 128-row block
            if len(output_partition_sizes) > 1 and any(w % 128 for w in output_partition_sizes):
                raise ValueError("merged block-FP8 partitions must be multiples of 128 rows")
            w = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=device)
            s = torch.empty(((n + 127) // 128, k // 128), dtype=torch.float32, device=device)
            names = ("weight", "weight_scale_inv")
            rows_per_scale = 128
        for name, data, rows in ((names[0], w, 1), (names[1], s, rows_per_scale)):
            param = torch.nn.Parameter(data, requires_grad=False)
            param.output_dim, param.input_dim = 0, 1
            param.mxl_rows_per_entry = rows
            param.mxl_logical_widths = list(output_partition_sizes)
            param.weight_loader = load_partition
            for attr, value in attrs.items():
                setattr(param, attr, value)
            layer.register_parameter(name, param)
        layer.params_dtype = params_dtype
        layer.logical_widths = list(output_partition_sizes)
        layer.input_size_per_partition = k
        layer.output_size_per_partition = n

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        self.kernel.process_weights_after_loading(layer)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self.kernel.apply_weights(layer, x, bias)


def swiglu_mxfp8_down(gate_up: torch.Tensor, down: torch.nn.Module) -> torch.Tensor:
    """Fused SwiGLU -> MXFP8 -> down projection for a layer prepared by ``Mxfp8LinearKernel``
    (the ``mach_swiglu_mxfp8_down`` op, src/vllm_mach/mxfp6/mxfp8_mlp.py:15-22,71-76)."""
    n, k = down.mxl_shape
    if gate_up.shape[-1] != 2 * k:
        raise ValueError("gate_up width must be twice the down projection's K")
    return ops.swiglu_mx_down(gate_up, down.weight, down.weight_scale, n, down.mxl_format)


# registration: the reference prepends its kernels to vLLM's per-platform candidate
# lists (src/vllm_mach/mxfp6/dense.py:244-275, dense_mxfp8.py:165-174)
POSSIBLE_KERNELS: dict[str, list[type]] = {"mxfp8": [], "mxfp6": [], "fp8_block": []}


def register_kernels(registry: Optional[dict] = None) -> dict:
    registry = POSSIBLE_KERNELS if registry is None else registry
    for name, cls in (("mxfp8", Mxfp8LinearKernel), ("mxfp6", Mxfp6LinearKernel),
                      ("fp8_block", BlockFp8LinearKernel)):
        lst = registry.setdefault(name, [])
        while cls in lst:
            lst.remove(cls)
        lst.insert(0, cls)
    return registry
