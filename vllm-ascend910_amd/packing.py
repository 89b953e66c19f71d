"""Offline weight preparation in the reference's packed layout (torch, any device).

These produce the tensors the op boundary accepts -- the same packed-int4
weight and group-major scales as the reference -- from a floating-point weight
or from int4 codes.  They are load-time helpers, not the hot path; the repack
into MFMA operand order happens on the GPU (``torch.ops.npu.w4a8_repack``).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import geometry as geo

BF16_TINY = torch.finfo(torch.bfloat16).tiny


def pack_int4(v: torch.Tensor) -> torch.Tensor:
    """[..., K] int8 codes in [-8, 7] -> [..., K/2] int8, even k in the LOW nibble.

    Same byte format as the reference's pack_int4 (npu_ops/python/w4a8_ops.py:142-148).
    """
    if v.shape[-1] % 2:
        raise ValueError("pack_int4: K must be even")
    lo = v[..., 0::2].to(torch.int16) & 0xF
    hi = v[..., 1::2].to(torch.int16) & 0xF
    return (lo | (hi << 4)).to(torch.uint8).view(torch.int8)


def unpack_int4(p: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_int4: [..., K/2] int8 -> [..., K] int8 codes in [-8, 7]."""
    b = p.view(torch.uint8).to(torch.int16)
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    out = torch.stack([lo, hi], dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return torch.where(out >= 8, out - 16, out).to(torch.int8)


def pack_grouped(codes: torch.Tensor, group: int) -> torch.Tensor:
    """[N, K] codes -> [N, kpad/2] packed with each group zero-padded to 64 elements.

    The reference's padded layout (npu_ops/python/w4a8_ops.py:231-239,
    npu_ops/kernel/mg_kgeom.h:23-33).  When kpad == K (e.g. K % group == 0 and
    group % 64 == 0) this is just pack_int4(codes).
    """
    N, K = codes.shape
    if geo.is_unpadded(K, group):
        return pack_int4(codes)
    G = geo.num_groups(K, group)
    stride = geo.group_stride(group)
    padded = codes.new_zeros((N, geo.kpad(K, group)))
    for g in range(G):
        real = geo.group_real(g, K, group)
        padded[:, g * stride:g * stride + real] = codes[:, g * group:g * group + real]
    return pack_int4(padded)


def quantize_weight(w: torch.Tensor, group: int, scale_dtype: torch.dtype = torch.bfloat16
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int4 per-group RTN: float [N, K] -> (w_q [N, kpad/2] int8, w_scale [G, N]).

    Per group (fakequant_lab/quant.py:102-105, :135-141 with QuantSpec(4, group, sym=True)):
    s = bf16(max|w| / 7) (bf16 tiny if zero), q = clamp(round_half_even(w / s), -8, 7).
    The last group of a ragged K is quantised on its real members
    (npu_ops/python/w4a8_ops.py:193-219).  ``scale_dtype`` float16 re-expresses the
    bf16 scale in fp16 (exact for the normal range).
    """
    N, K = w.shape
    G = geo.num_groups(K, group)
    codes = torch.empty((N, K), dtype=torch.int8, device=w.device)
    scales = torch.empty((N, G), dtype=torch.bfloat16, device=w.device)
    k_full = group * (K // group)
    # (start, width, group length): the full groups, then the ragged tail as one group.
    for g0, width, gl in ((0, k_full, group), (k_full, K - k_full, K - k_full)):
        if width == 0:
            continue
        ng = width // gl
        wg = w[:, g0:g0 + width].float().reshape(N, ng, gl)
        s = (wg.abs().amax(dim=-1, keepdim=True) / 7.0).to(torch.bfloat16)
        s = torch.where(s == 0, torch.full_like(s, BF16_TINY), s)
        q = torch.round(wg / s.float()).clamp_(-8, 7).to(torch.int8)
        codes[:, g0:g0 + width] = q.reshape(N, width)
        gi = g0 // group
        scales[:, gi:gi + ng] = s.squeeze(-1)
    return pack_grouped(codes, group), scales.to(scale_dtype).T.contiguous()


def quantize_weight_asym(w: torch.Tensor, group: int = 1024
                         ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric int4 per-group RTN, the reference's export for its mid-group pair
    (npu_ops/python/w4a8_ops.py:181-240): float [N, K] -> (w_q [N, kpad/2] int8,
    w_scale [G, N] bf16, w_ksum [G, N] int32 of the raw codes, w_zero [G, N] bf16).

    Per group (fakequant_lab/quant.py:106-141 with QuantSpec(4, group, sym=False)):
    s = bf16((max - min) / 15) (bf16 tiny if zero), z = bf16(-8 - round(min / s)),
    q = clamp(round(w / s) + z, -8, 7); a constant group takes s = bf16(|v| / 7),
    z = 0.  The ragged tail is quantised as its own group.
    """
    N, K = w.shape
    G = geo.num_groups(K, group)
    codes = torch.empty((N, K), dtype=torch.int8, device=w.device)
    scales = torch.empty((N, G), dtype=torch.bfloat16, device=w.device)
    zeros = torch.empty((N, G), dtype=torch.bfloat16, device=w.device)
    k_full = group * (K // group)
    tiny = lambda t: torch.where(t == 0, torch.full_like(t, BF16_TINY), t)  # noqa: E731
    for g0, width, gl in ((0, k_full, group), (k_full, K - k_full, K - k_full)):
        if width == 0:
            continue
        ng = width // gl
        wg = w[:, g0:g0 + width].float().reshape(N, ng, gl)
        mx, mn = wg.amax(dim=-1, keepdim=True), wg.amin(dim=-1, keepdim=True)
        rng = mx - mn
        s = tiny((rng / 15.0).to(torch.bfloat16))
        z = (-8.0 - torch.round(mn / s.float())).to(torch.bfloat16)
        const = rng == 0
        s = torch.where(const, tiny((mx.abs() / 7.0).to(torch.bfloat16)), s)
        z = torch.where(const, torch.zeros_like(z), z)
        q = (torch.round(wg / s.float()) + z.float()).clamp_(-8, 7).to(torch.int8)
        codes[:, g0:g0 + width] = q.reshape(N, width)
        gi = g0 // group
        scales[:, gi:gi + ng] = s.squeeze(-1)
        zeros[:, gi:gi + ng] = z.squeeze(-1)
    ksum = torch.stack([codes[:, g * group:g * group + geo.group_real(g, K, group)].to(torch.int32).sum(dim=1)
                        for g in range(G)], dim=0).to(torch.int32)
    return pack_grouped(codes, group), scales.T.contiguous(), ksum.contiguous(), zeros.T.contiguous()


def repacked_sizes(N: int, K: int, group: int) -> Tuple[int, tuple]:
    return geo.repacked_weight_bytes(N, K, group), geo.repacked_scale_shape(N, K, group)
