"""Seeded synthetic inputs at the benchmark's value distributions (numpy).

Distributions follow the benchmark configurations: activations bf16 N(0,1)
with 0.1% of channels scaled x20 (outliers); int4 weight codes uniform in
[-8, 7] (or round(clip(N(0, 2.5), -8, 7)) for the mid-group variants);
per-group scales uniform in [0.002, 0.02] stored as fp16 or bf16.  One seed
per tensor.  Used by the tests and the benchmark harness; the product path
takes these as ordinary inputs.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def activations(M: int, K: int, seed: int, outlier_frac: float = 0.001, outlier_scale: float = 20.0) -> np.ndarray:
    """bf16 bits [M, K]: N(0,1) with round(K*outlier_frac) (>= 1) channels scaled."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    n_out = max(1, int(round(K * outlier_frac)))
    ch = rng.choice(K, size=n_out, replace=False)
    x[:, ch] *= np.float32(outlier_scale)
    return f32_to_bf16_bits(x)


def activations_device(M: int, K: int, seed: int, device, outlier_frac: float = 0.001,
                       outlier_scale: float = 20.0):
    """The distribution of ``activations`` drawn on the device (for prefill-sized
    batches): a bf16 torch tensor [M, K], N(0,1) from a seeded device generator,
    the same number of outlier channels (chosen from the numpy seed) scaled."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn((M, K), dtype=torch.float32, device=device, generator=gen)
    n_out = max(1, int(round(K * outlier_frac)))
    ch = np.random.default_rng(seed).choice(K, size=n_out, replace=False)
    x[:, torch.from_numpy(ch).to(device)] *= outlier_scale
    return x.to(torch.bfloat16)


def weight_codes_uniform(N: int, K: int, seed: int) -> np.ndarray:
    """int8 [N, K] codes uniform in [-8, 7]."""
    return np.random.default_rng(seed).integers(-8, 8, size=(N, K), dtype=np.int8)


def weight_codes_clipped_normal(N: int, K: int, seed: int, std: float = 2.5) -> np.ndarray:
    """int8 [N, K] codes round(clip(N(0, std), -8, 7))."""
    w = np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(std)
    return np.round(np.clip(w, -8, 7)).astype(np.int8)


def group_scales(N: int, G: int, seed: int, dtype: str = "f16", lo: float = 0.002, hi: float = 0.02) -> np.ndarray:
    """uint16 bits [N, G] of fp16 ('f16') or bf16 ('bf16') scales uniform in [lo, hi]."""
    s = np.random.default_rng(seed).uniform(lo, hi, size=(N, G)).astype(np.float32)
    if dtype == "f16":
        return s.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        return f32_to_bf16_bits(s)
    raise ValueError(dtype)


def scale_bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f16":
        return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)
    return bf16_bits_to_f32(bits)


def pack_int4(v: np.ndarray) -> np.ndarray:
    """[..., K] codes -> [..., K/2] int8, even k in the low nibble (reference byte format)."""
    v = np.asarray(v, np.int16)
    return ((v[..., 0::2] & 0xF) | ((v[..., 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)


# QwQ-32B projection shapes (K -> N) of the benchmark.
QWQ_SHAPES = {
    "qkv_proj": (5120, 7168),
    "o_proj": (5120, 5120),
    "gate_up_proj": (5120, 55296),
    "down_proj": (27648, 5120),
}
