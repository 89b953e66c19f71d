"""W4A8 linear layer: the caller side of the op surface.

``W4A8Linear`` reproduces the reference's vLLM linear method
(npu_ops/python/midgroup_quant.py:102-178): parameters are created in the
checkpoint layout (``weight_packed [N, kpad/2]`` int8, ``weight_scale [N, G]``,
output_dim 0 so fused q/k/v and gate/up loaders can concatenate along N),
``process_weights_after_loading`` converts them once into the kernel's layout
(here: the gfx950 MFMA repack, instead of the reference's [N,G]->[G,N]
transpose), and ``forward`` is the reference ``apply``: reshape to 2-D bf16,
quantise, GEMM, add bias, reshape -- straight-line, no shape-dependent Python,
so it can be captured in a HIP graph.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import geometry as geo
from . import ops  # noqa: F401  (registers torch.ops.npu.*)
from .packing import quantize_weight


def linear(x: torch.Tensor, w_tiles: torch.Tensor, s_tiles: torch.Tensor, N: int, group: int,
           bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x @ W.T with per-token int8 activations and per-group int4 weights.

    The reference's ``w4a8_ops.linear`` (npu_ops/python/w4a8_ops.py:243-252).
    """
    lead, K = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, K).to(torch.bfloat16).contiguous()
    y = torch.ops.npu.w4a8_linear(x2, w_tiles, s_tiles, N, K, group)
    if bias is not None:
        y = y + bias
    return y.reshape(*lead, N)


def linear_swiglu(x: torch.Tensor, w_tiles: torch.Tensor, s_tiles: torch.Tensor, N: int, group: int
                  ) -> torch.Tensor:
    """silu(g) * u of a merged gate/up projection (N = 2*I), fused into the GEMM.

    Equals ``g, u = linear(x, ...).split(N // 2, -1); F.silu(g) * u`` in bf16, the
    reference decoder layer's MLP activation (npu_ops/python/bench_decode_layer.py:78-81).
    """
    lead, K = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, K).to(torch.bfloat16).contiguous()
    a_q, a_scale = torch.ops.npu.w4a8_quant_pertoken(x2, group)
    y = torch.ops.npu.w4a8_gemm_swiglu(a_q, a_scale, w_tiles, s_tiles, N, K, group)
    return y.reshape(*lead, N // 2)


class W4A8Linear(nn.Module):
    """Drop-in W4A8 linear (symmetric int4 per-group weights, per-token int8 activations)."""

    def __init__(self, in_features: int, out_features: int, group: int = 128, bias: bool = False,
                 scale_dtype: torch.dtype = torch.bfloat16, device=None, act: Optional[str] = None):
        super().__init__()
        if act not in (None, "swiglu"):
            raise ValueError(f"W4A8Linear: unknown act {act!r}")
        if act == "swiglu" and (bias or out_features % 32):
            raise ValueError("W4A8Linear(act='swiglu'): merged gate/up without bias, out_features = 2*I, I % 16 == 0")
        self.act = act
        self.in_features = in_features
        self.out_features = out_features
        self.group = group
        K, N = in_features, out_features
        G = geo.num_groups(K, group)
        self.register_buffer("weight_packed", torch.zeros((N, geo.kpad(K, group) // 2), dtype=torch.int8,
                                                          device=device))
        self.register_buffer("weight_scale", torch.zeros((N, G), dtype=scale_dtype, device=device))
        self.bias = nn.Parameter(torch.zeros(N, dtype=torch.bfloat16, device=device),
                                 requires_grad=False) if bias else None
        self.w_tiles: Optional[torch.Tensor] = None
        self.s_tiles: Optional[torch.Tensor] = None

    @classmethod
    def from_float(cls, lin: nn.Linear, group: int = 128, scale_dtype: torch.dtype = torch.bfloat16,
                   act: Optional[str] = None) -> "W4A8Linear":
        """Quantise an nn.Linear's weight (symmetric RTN per group) and prepare it."""
        N, K = lin.weight.shape
        m = cls(K, N, group, lin.bias is not None, scale_dtype, device=lin.weight.device, act=act)
        w_q, w_scale = quantize_weight(lin.weight.data, group, scale_dtype)
        m.weight_packed.copy_(w_q)
        m.weight_scale.copy_(w_scale.T)
        if lin.bias is not None:
            m.bias.data.copy_(lin.bias.data.to(torch.bfloat16))
        m.process_weights_after_loading()
        return m

    def process_weights_after_loading(self) -> None:
        """One-time conversion to the kernel layout (the reference transposes
        scales to [G, N] here, npu_ops/python/midgroup_quant.py:148-161; this
        build repacks weight and scales into MFMA operand order)."""
        w_scale_gn = self.weight_scale.t().contiguous()
        self.w_tiles, self.s_tiles = torch.ops.npu.w4a8_repack(self.weight_packed, w_scale_gn,
                                                               self.in_features, self.group)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.w_tiles is None:
            raise RuntimeError("W4A8Linear: call process_weights_after_loading() after loading weights")
        if self.act == "swiglu":
            return linear_swiglu(x, self.w_tiles, self.s_tiles, self.out_features, self.group)
        return linear(x, self.w_tiles, self.s_tiles, self.out_features, self.group, self.bias)


# ---------------------------------------------------------------- mid-group compat pair
def midgroup_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wk: torch.Tensor, wz: torch.Tensor,
                    group: int = 1024) -> torch.Tensor:
    """y = x @ W.T with the reference's mid-group W4A8 tensors; x is bf16 [..., K].

    The reference's ``w4a8_ops.linear`` (npu_ops/python/w4a8_ops.py:243-252): quant_a pads the
    rows to TILE_M, so y has >= x's rows and is sliced before reshaping.
    """
    lead, K = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, K).to(torch.bfloat16).contiguous()
    a_hi, a_lo, a_scale, a_ksum = torch.ops.npu.midgroup_quant_a(x2, group)
    # only the real rows (the reference slices them from the padded product)
    y = torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_scale, a_ksum, wq, ws, wk, wz, K, group, x2.shape[0])
    return y.reshape(*lead, y.shape[-1])


class MidGroupW4A8Linear(nn.Module):
    """The reference's ``MidGroupW4A8LinearMethod`` as a module (npu_ops/python/midgroup_quant.py:102-178).

    Parameters in the checkpoint layout the reference exports (``weight_packed [N, kpad/2]`` int8,
    ``weight_scale``/``weight_zero`` ``[N, G]`` bf16, ``weight_ksum [N, G]`` int32, output_dim 0 so
    fused loaders concatenate along N); ``process_weights_after_loading`` transposes the three
    per-group tensors to ``[G, N]`` (midgroup_quant.py:148-161); ``forward`` is ``apply``
    (:163-178): quant_a, GEMM, slice to the real rows, bias, reshape.
    """

    def __init__(self, in_features: int, out_features: int, group: int = 1024, bias: bool = False, device=None):
        super().__init__()
        self.in_features, self.out_features, self.group = in_features, out_features, group
        K, N = in_features, out_features
        G = geo.num_groups(K, group)
        self.register_buffer("weight_packed", torch.zeros((N, geo.kpad(K, group) // 2), dtype=torch.int8,
                                                          device=device))
        self.register_buffer("weight_scale", torch.zeros((N, G), dtype=torch.bfloat16, device=device))
        self.register_buffer("weight_zero", torch.zeros((N, G), dtype=torch.bfloat16, device=device))
        self.register_buffer("weight_ksum", torch.zeros((N, G), dtype=torch.int32, device=device))
        self.bias = nn.Parameter(torch.zeros(N, dtype=torch.bfloat16, device=device),
                                 requires_grad=False) if bias else None
        self._gn = None
        self._tiles = None

    @classmethod
    def from_float(cls, lin: nn.Linear, group: int = 1024) -> "MidGroupW4A8Linear":
        """Export an nn.Linear the way the reference's quantize_weight does, then load it."""
        from .packing import quantize_weight_asym
        N, K = lin.weight.shape
        m = cls(K, N, group, lin.bias is not None, device=lin.weight.device)
        w_q, ws, wk, wz = quantize_weight_asym(lin.weight.data, group)
        m.weight_packed.copy_(w_q)
        m.weight_scale.copy_(ws.T)
        m.weight_zero.copy_(wz.T)
        m.weight_ksum.copy_(wk.T)
        if lin.bias is not None:
            m.bias.data.copy_(lin.bias.data.to(torch.bfloat16))
        m.process_weights_after_loading()
        return m

    def process_weights_after_loading(self) -> None:
        self._gn = tuple(getattr(self, n).t().contiguous() for n in ("weight_scale", "weight_ksum", "weight_zero"))
        # the packed weight as midgroup_tile_weights' 1 KB tiles (the same bytes, read in whole
        # tiles: 10-25% faster at decode); weights loaded off the GPU keep the rows as stored
        self._tiles = (torch.ops.npu.midgroup_tile_weights(self.weight_packed, self.in_features, self.group)
                       if self.weight_packed.is_cuda else None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._gn is None:
            raise RuntimeError("MidGroupW4A8Linear: call process_weights_after_loading() after loading weights")
        ws, wk, wz = self._gn
        lead, k = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, k).to(torch.bfloat16).contiguous()
        rows = x2.shape[0]
        a_hi, a_lo, a_scale, a_ksum = torch.ops.npu.midgroup_quant_a(x2, self.group)
        if self._tiles is not None and self._tiles.device == x2.device:
            y = torch.ops.npu.midgroup_w4a8_gemm_tiled(a_hi, a_lo, a_scale, a_ksum, self._tiles, ws, wk, wz,
                                                       self.out_features, k, self.group, rows)
        else:
            y = torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_scale, a_ksum, self.weight_packed, ws, wk, wz, k,
                                                 self.group, rows)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*lead, self.out_features)
