"""vLLM quantization backends for the W4A8 linear on MI355X.

The reference plugs its kernel into vLLM as ``quant_method="midgroup_w4a8"``:
a ``QuantizationConfig`` read from config.json, a ``LinearMethodBase`` whose
``create_weights`` allocates int4-shaped parameters in the checkpoint layout,
whose ``process_weights_after_loading`` fixes the layout once, and whose
``apply`` runs quant + GEMM, plus a ``register()`` that adds the name to
vLLM's registry and the platform allow-list
(npu_ops/python/midgroup_quant.py:51-202).  This module provides the same
contract over this build's ops:

* ``midgroup_w4a8`` -- the reference's own checkpoint (``weight_packed
  [N, kpad/2]`` int8, ``weight_scale`` / ``weight_zero`` ``[N, G]`` bf16,
  ``weight_ksum [N, G]`` int32, asymmetric, group 1024 by default) on the
  compat pair ``midgroup_quant_a`` + ``midgroup_w4a8_gemm``.
* ``w4a8_pertoken`` -- the per-token symmetric format (``weight_packed
  [N, kpad/2]`` int8, ``weight_scale [N, G]`` fp16 or bf16), repacked once
  into MFMA tile order and served by ``w4a8_linear``.

vLLM is not part of this image.  The classes derive from vLLM's base classes
when vLLM imports and from ``object`` otherwise, so the contract (config
parsing, parameter shapes and attributes, the load-time transform, apply) is
usable and testable without it; ``register()`` needs vLLM.
"""
from __future__ import annotations

from typing import Any, List, Optional

import torch

from . import geometry as geo

try:  # pragma: no cover - vLLM is absent in this image
    from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    HAVE_VLLM = True
except ImportError:
    LinearBase = None
    UnquantizedLinearMethod = None
    LinearMethodBase = object
    QuantizationConfig = object
    HAVE_VLLM = False

_SCALE_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def _add_param(layer: torch.nn.Module, name: str, t: torch.Tensor, loader) -> None:
    """A frozen parameter with ``output_dim = 0``: vLLM's fused (qkv, gate_up) and
    column-parallel loaders then concatenate every tensor along N."""
    p = torch.nn.Parameter(t, requires_grad=False)
    p.output_dim = 0
    if loader is not None:
        p.weight_loader = loader
    layer.register_parameter(name, p)


def _check_k_shard(prefix: str, k: int, input_size: int, group: int) -> None:
    # A pre-quantised checkpoint fixes the group boundaries and the parameters
    # carry no input_dim, so a row-parallel K shard is refused rather than
    # loaded mis-scaled (midgroup_quant.py:20-32 and :112-117 do the same).
    if k != input_size:
        raise ValueError(f"{prefix}: row-parallel shard K={k} of {input_size} (group {group}): a "
                         f"pre-quantised checkpoint cannot be K-sharded; export one for this TP degree or run TP=1")


class _ConfigBase(QuantizationConfig):
    """Shared config surface (names as vLLM's QuantizationConfig defines them)."""

    NAME = ""

    def __init__(self, group_size: int, ignored_layers: Optional[List[str]] = None):
        if HAVE_VLLM:  # pragma: no cover
            super().__init__()
        self.group_size = int(group_size)
        self.ignored_layers = list(ignored_layers) if ignored_layers is not None else ["lm_head"]
        # vllm-ascend reads ``quant_description`` from unrelated layers (the
        # reference keeps it empty for the same reason)
        self.quant_description: dict = {}

    @classmethod
    def get_name(cls) -> str:
        return cls.NAME

    @classmethod
    def get_supported_act_dtypes(cls) -> List[torch.dtype]:
        return [torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 0

    @classmethod
    def get_config_filenames(cls) -> List[str]:
        return []

    def _method(self, prefix: str):
        raise NotImplementedError

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if LinearBase is not None and not isinstance(layer, LinearBase):  # pragma: no cover
            return None
        if any(ig in prefix for ig in self.ignored_layers):
            return UnquantizedLinearMethod() if UnquantizedLinearMethod is not None else None
        return self._method(prefix)


class MidGroupW4A8Config(_ConfigBase):
    """``quant_method = "midgroup_w4a8"`` (the reference's exporter writes it,
    export_w4a8_checkpoint.py:178-186)."""

    NAME = "midgroup_w4a8"

    def __init__(self, group_size: int = 1024, sym: bool = False, ignored_layers: Optional[List[str]] = None):
        super().__init__(group_size, ignored_layers)
        self.sym = bool(sym)

    def __repr__(self) -> str:
        return f"MidGroupW4A8Config(group_size={self.group_size}, sym={self.sym})"

    @classmethod
    def from_config(cls, config: dict) -> "MidGroupW4A8Config":
        return cls(group_size=config.get("group_size", 1024), sym=config.get("sym", False),
                   ignored_layers=config.get("ignored_layers", ["lm_head"]))

    def _method(self, prefix: str):
        return MidGroupW4A8LinearMethod(self, prefix)


class PerTokenW4A8Config(_ConfigBase):
    """``quant_method = "w4a8_pertoken"``: symmetric int4 weights with per-group
    scales (``scale_dtype`` "float16" or "bfloat16") and dynamic per-token int8
    activations."""

    NAME = "w4a8_pertoken"

    def __init__(self, group_size: int = 128, scale_dtype: str = "float16",
                 ignored_layers: Optional[List[str]] = None):
        super().__init__(group_size, ignored_layers)
        if scale_dtype not in _SCALE_DTYPES:
            raise ValueError(f"scale_dtype must be one of {sorted(_SCALE_DTYPES)}, got {scale_dtype!r}")
        self.scale_dtype = scale_dtype

    def __repr__(self) -> str:
        return f"PerTokenW4A8Config(group_size={self.group_size}, scale_dtype={self.scale_dtype})"

    @classmethod
    def from_config(cls, config: dict) -> "PerTokenW4A8Config":
        return cls(group_size=config.get("group_size", 128), scale_dtype=config.get("scale_dtype", "float16"),
                   ignored_layers=config.get("ignored_layers", ["lm_head"]))

    def _method(self, prefix: str):
        return PerTokenW4A8LinearMethod(self, prefix)


class MidGroupW4A8LinearMethod(LinearMethodBase):
    """The reference checkpoint's linear method on the compat pair."""

    def __init__(self, quant_config: MidGroupW4A8Config, prefix: str = ""):
        self.quant_config = quant_config
        self.prefix = prefix

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs: Any) -> None:
        group = self.quant_config.group_size
        k, n = input_size_per_partition, sum(output_partition_sizes)
        _check_k_shard(self.prefix, k, input_size, group)
        G = geo.num_groups(k, group)
        loader = extra_weight_attrs.get("weight_loader")
        _add_param(layer, "weight_packed", torch.empty(n, geo.kpad(k, group) // 2, dtype=torch.int8), loader)
        _add_param(layer, "weight_scale", torch.empty(n, G, dtype=torch.bfloat16), loader)
        _add_param(layer, "weight_zero", torch.empty(n, G, dtype=torch.bfloat16), loader)
        _add_param(layer, "weight_ksum", torch.empty(n, G, dtype=torch.int32), loader)
        layer.w4a8_k, layer.w4a8_n, layer.w4a8_group = k, n, group

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """The per-group tensors [N, G] -> [G, N], the layout the GEMM reads, and the packed
        weight -> midgroup_tile_weights' 1 KB tiles (the same bytes, read in whole tiles; the
        rows as stored are released), once."""
        for name in ("weight_scale", "weight_zero", "weight_ksum"):
            t = getattr(layer, name).data.t().contiguous()
            delattr(layer, name)
            layer.register_parameter(name, torch.nn.Parameter(t, requires_grad=False))
        if layer.weight_packed.is_cuda:
            w_tiles = torch.ops.npu.midgroup_tile_weights(layer.weight_packed.data, layer.w4a8_k, layer.w4a8_group)
            del layer.weight_packed
            layer.register_parameter("w_tiles", torch.nn.Parameter(w_tiles, requires_grad=False))

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        lead, k = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, k).to(torch.bfloat16).contiguous()
        rows = x2.shape[0]
        a_hi, a_lo, a_scale, a_ksum = torch.ops.npu.midgroup_quant_a(x2, layer.w4a8_group)
        if hasattr(layer, "w_tiles"):
            y = torch.ops.npu.midgroup_w4a8_gemm_tiled(a_hi, a_lo, a_scale, a_ksum, layer.w_tiles, layer.weight_scale,
                                                       layer.weight_ksum, layer.weight_zero, layer.w4a8_n, k,
                                                       layer.w4a8_group, rows)
        else:   # loaded off the GPU: the rows as stored (the same output bits)
            y = torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_scale, a_ksum, layer.weight_packed, layer.weight_scale,
                                                 layer.weight_ksum, layer.weight_zero, k, layer.w4a8_group, rows)
        if bias is not None:
            y = y + bias
        return y.reshape(*lead, layer.w4a8_n)


class PerTokenW4A8LinearMethod(LinearMethodBase):
    """Per-token W4A8: the checkpoint tensors are repacked into MFMA tile order at
    load time (the originals are released) and ``apply`` is one ``w4a8_linear``."""

    def __init__(self, quant_config: PerTokenW4A8Config, prefix: str = ""):
        self.quant_config = quant_config
        self.prefix = prefix

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs: Any) -> None:
        group = self.quant_config.group_size
        k, n = input_size_per_partition, sum(output_partition_sizes)
        _check_k_shard(self.prefix, k, input_size, group)
        loader = extra_weight_attrs.get("weight_loader")
        sdt = _SCALE_DTYPES[self.quant_config.scale_dtype]
        _add_param(layer, "weight_packed", torch.empty(n, geo.kpad(k, group) // 2, dtype=torch.int8), loader)
        _add_param(layer, "weight_scale", torch.empty(n, geo.num_groups(k, group), dtype=sdt), loader)
        layer.w4a8_k, layer.w4a8_n, layer.w4a8_group = k, n, group

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        k, group = layer.w4a8_k, layer.w4a8_group
        w_tiles, s_tiles = torch.ops.npu.w4a8_repack(layer.weight_packed.data,
                                                     layer.weight_scale.data.t().contiguous(), k, group)
        del layer.weight_packed, layer.weight_scale
        layer.register_parameter("w_tiles", torch.nn.Parameter(w_tiles, requires_grad=False))
        layer.register_parameter("s_tiles", torch.nn.Parameter(s_tiles, requires_grad=False))

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        lead, k = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, k).to(torch.bfloat16).contiguous()
        y = torch.ops.npu.w4a8_linear(x2, layer.w_tiles, layer.s_tiles, layer.w4a8_n, k, layer.w4a8_group)
        if bias is not None:
            y = y + bias
        return y.reshape(*lead, layer.w4a8_n)


CONFIGS = (MidGroupW4A8Config, PerTokenW4A8Config)


def register() -> None:
    """Make both ``quant_method`` names usable in vLLM: register the config
    classes and add the names to the current platform's allow-list (vLLM
    validates a method against it while building the model config), as the
    reference's ``register`` does (midgroup_quant.py:181-202).  Call it before
    constructing the engine."""
    if not HAVE_VLLM:
        raise ImportError("vllm_plugin.register() needs vLLM, which is not installed")
    from vllm.model_executor.layers.quantization import register_quantization_config  # pragma: no cover
    from vllm.platforms import current_platform  # pragma: no cover
    for cls in CONFIGS:  # pragma: no cover
        try:
            register_quantization_config(cls.get_name())(cls)
        except ValueError:
            pass  # already registered in this process
        allow = getattr(type(current_platform), "supported_quantization", None)
        if allow is not None and cls.get_name() not in allow:
            allow.append(cls.get_name())
