"""On-disk weight formats for the W4A8 linear: readers and the reference's exporter.

Two formats the reference deploys are read here (safetensors only: nothing is
unpickled):

* ``mg_kgeom_v1`` -- the reference's own mid-group export
  (npu_ops/python/export_w4a8_checkpoint.py:137-186): per quantised linear
  ``<base>.weight_packed [N, kpad/2]`` int8 (two int4 per byte along K, groups
  padded per mg_kgeom.h), ``<base>.weight_scale`` / ``weight_zero [N, G]`` bf16
  and ``<base>.weight_ksum [N, G]`` int32, with ``quantization_config`` =
  {"quant_method": "midgroup_w4a8", "packed_layout": "mg_kgeom_v1", ...}.
  ``export_midgroup`` writes it, ``load_midgroup_linear`` reads one linear into
  a :class:`MidGroupW4A8Linear`.

* the vendor ``W4A8_DYNAMIC`` layout (as the reference's random-checkpoint
  builder writes it, scripts/build_random_w4a8.py:102-147): ``<base>.weight
  [N/2, K]`` int8 holding two int4 codes per byte along the OUTPUT axis,
  ``weight_scale`` / ``weight_offset [N, 1]`` fp32, ``weight_scale_second`` /
  ``weight_offset_second [N, K/group]`` fp16 and ``scale_bias``.  The nibble
  order and the dequantisation rule belong to vllm-ascend / torch-npu, which
  the reference does not vendor; this reader assumes the low nibble holds the
  even output row and w[n, k] = code * weight_scale[n] * weight_scale_second[n, g]
  (symmetric), and rejects checkpoints with non-zero offsets or scale_bias.
  No reference file pins this conversion.  ``load_vendor_linear`` turns one
  linear into a :class:`W4A8Linear` on the per-token path.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from . import geometry as geo
from .linear import MidGroupW4A8Linear, W4A8Linear
from .packing import pack_grouped, quantize_weight_asym

MIDGROUP_SUFFIXES = ("weight_packed", "weight_scale", "weight_zero", "weight_ksum")


def load_safetensors(path: str, device: str = "cpu") -> Dict[str, torch.Tensor]:
    """All tensors of one safetensors file (no pickle is involved)."""
    from safetensors.torch import load_file
    return load_file(path, device=device)


# ---------------------------------------------------------------- mg_kgeom_v1
def quant_config(group: int = 1024) -> dict:
    """The ``quantization_config`` block of an mg_kgeom_v1 checkpoint
    (export_w4a8_checkpoint.py:178-186)."""
    return {"quant_method": "midgroup_w4a8", "group_size": group, "weight_bits": 4, "activation_bits": 8,
            "sym": False, "packed_layout": "mg_kgeom_v1", "ignored_layers": ["lm_head"]}


def _is_target(key: str) -> bool:
    # the reference quantises the decoder's projection weights and nothing else
    return key.endswith("_proj.weight") and ".layers." in key


def export_midgroup(tensors: Dict[str, torch.Tensor], group: int = 1024,
                    is_target: Callable[[str], bool] = _is_target) -> Dict[str, torch.Tensor]:
    """float checkpoint tensors -> mg_kgeom_v1 tensors (targets quantised, the rest passed
    through), as export_w4a8_checkpoint.py:137-157 does per shard."""
    out: Dict[str, torch.Tensor] = {}
    for key, t in tensors.items():
        if not is_target(key):
            out[key] = t.contiguous()
            continue
        wq, ws, wk, wz = quantize_weight_asym(t.to(torch.bfloat16), group)   # scales [G, N]
        base = key[: -len(".weight")]
        for suf, v in zip(MIDGROUP_SUFFIXES, (wq, ws.T.contiguous(), wz.T.contiguous(), wk.T.contiguous())):
            out[f"{base}.{suf}"] = v
    return out


def load_midgroup_linear(tensors: Dict[str, torch.Tensor], base: str, K: int, group: int = 1024,
                         bias: Optional[torch.Tensor] = None, device=None) -> MidGroupW4A8Linear:
    """One mg_kgeom_v1 linear of input size K -> MidGroupW4A8Linear (weights loaded,
    layout processed).  K comes from the model config, as in the reference's
    create_weights (midgroup_quant.py:104-120): a ragged last group's real length
    is not recoverable from the padded row."""
    missing = [s for s in MIDGROUP_SUFFIXES if f"{base}.{s}" not in tensors]
    if missing:
        raise KeyError(f"{base}: mg_kgeom_v1 tensors missing: {missing}")
    wq = tensors[f"{base}.weight_packed"]
    N, kb = wq.shape
    G = tensors[f"{base}.weight_scale"].shape[1]
    if kb != geo.kpad(K, group) // 2 or G != geo.num_groups(K, group):
        raise ValueError(f"{base}: packed row {kb} B / {G} groups do not match K={K}, group={group}")
    dev = device if device is not None else wq.device
    m = MidGroupW4A8Linear(K, N, group, bias is not None, device=dev)
    m.weight_packed.copy_(wq)
    m.weight_scale.copy_(tensors[f"{base}.weight_scale"])
    m.weight_zero.copy_(tensors[f"{base}.weight_zero"])
    m.weight_ksum.copy_(tensors[f"{base}.weight_ksum"])
    if bias is not None:
        m.bias.data.copy_(bias.to(torch.bfloat16))
    m.process_weights_after_loading()
    return m


# ---------------------------------------------------------------- vendor W4A8_DYNAMIC
def vendor_unpack_n(packed: torch.Tensor) -> torch.Tensor:
    """[N/2, K] int8, two int4 per byte along N (low nibble = even row) -> codes [N, K] int8."""
    p = packed.to(torch.int16) & 0xFF
    lo, hi = p & 0xF, (p >> 4) & 0xF
    codes = torch.stack([lo, hi], dim=1).reshape(packed.shape[0] * 2, packed.shape[1])
    return torch.where(codes >= 8, codes - 16, codes).to(torch.int8)


def vendor_to_grouped(tensors: Dict[str, torch.Tensor], base: str, group: int = 128,
                      scale_dtype: torch.dtype = torch.float16) -> Tuple[torch.Tensor, torch.Tensor, int, int]:
    """Vendor W4A8_DYNAMIC tensors of one linear -> (w_q [N, kpad/2] packed along K,
    w_scale [G, N], N, K), the inputs of ``torch.ops.npu.w4a8_repack``."""
    w = tensors[f"{base}.weight"]
    if w.dtype != torch.int8 or w.dim() != 2:
        raise ValueError(f"{base}.weight: expected int8 [N/2, K], got {w.dtype} {tuple(w.shape)}")
    N, K = 2 * w.shape[0], w.shape[1]
    s2 = tensors[f"{base}.weight_scale_second"].float()
    G = geo.num_groups(K, group)
    if tuple(s2.shape) != (N, G):
        raise ValueError(f"{base}.weight_scale_second: expected [{N}, {G}] for group {group}, got {tuple(s2.shape)}")
    s1 = tensors.get(f"{base}.weight_scale")
    s1 = torch.ones((N, 1)) if s1 is None else s1.float().reshape(N, -1)
    for name in ("weight_offset", "weight_offset_second", "scale_bias"):
        t = tensors.get(f"{base}.{name}")
        if t is not None and bool(torch.any(t != 0)):
            raise ValueError(f"{base}.{name} is non-zero: only the symmetric W4A8_DYNAMIC layout is read")
    codes = vendor_unpack_n(w)
    scale = (s1 * s2).to(scale_dtype)                                    # [N, G]
    return pack_grouped(codes, group), scale.T.contiguous(), N, K


def load_vendor_linear(tensors: Dict[str, torch.Tensor], base: str, group: int = 128,
                       bias: Optional[torch.Tensor] = None, device="cuda") -> W4A8Linear:
    """One vendor W4A8_DYNAMIC linear -> W4A8Linear on the per-token path."""
    w_q, w_scale, N, K = vendor_to_grouped(tensors, base, group)
    m = W4A8Linear(K, N, group, bias is not None, scale_dtype=w_scale.dtype, device=device)
    m.weight_packed.copy_(w_q)
    m.weight_scale.copy_(w_scale.T)
    if bias is not None:
        m.bias.data.copy_(bias.to(torch.bfloat16))
    m.process_weights_after_loading()
    return m
