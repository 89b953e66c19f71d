"""Python mirror of the group geometry in csrc/kgeom.h.

Mirrors the reference's Python copy of its ragged-K geometry
(npu_ops/python/w4a8_ops.py:157-178, itself mirroring
npu_ops/kernel/mg_kgeom.h:47-129): G = ceil(K/group) groups, only the last
one short, group g at padded offset g * ceil_to(group, 64), each group padded
to a multiple of 64 elements.
"""
from __future__ import annotations

GROUP_ALIGN = 64    # packed-layout step, kgeom.h kGroupAlign
TILE_N = 16         # repacked tile: 16 output columns ...
TILE_K = 128        # ... by 128 padded-K = 1024 bytes
TILE_BYTES = TILE_N * TILE_K // 2


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def num_groups(K: int, group: int) -> int:
    return ceil_div(K, group)


def group_stride(group: int) -> int:
    return ceil_div(group, GROUP_ALIGN) * GROUP_ALIGN


def group_real(g: int, K: int, group: int) -> int:
    G = num_groups(K, group)
    return group if g + 1 < G else K - (G - 1) * group


def group_pad(g: int, K: int, group: int) -> int:
    return ceil_div(group_real(g, K, group), GROUP_ALIGN) * GROUP_ALIGN


def kpad(K: int, group: int) -> int:
    G = num_groups(K, group)
    return (G - 1) * group_stride(group) + group_pad(G - 1, K, group)


def col_blocks(N: int) -> int:
    return ceil_div(N, TILE_N)


def k_tiles(K: int, group: int) -> int:
    return ceil_div(kpad(K, group), TILE_K)


def repacked_weight_bytes(N: int, K: int, group: int) -> int:
    return col_blocks(N) * k_tiles(K, group) * TILE_BYTES


def repacked_scale_shape(N: int, K: int, group: int) -> tuple:
    return (col_blocks(N), num_groups(K, group), TILE_N)


def is_unpadded(K: int, group: int) -> bool:
    """True when the padded layout is the plain one (kpad == K), e.g. for
    group % 64 == 0 and K % group == 0."""
    return group > 0 and K > 0 and kpad(K, group) == K
