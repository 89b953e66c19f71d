"""numpy restatement of the reference's CPU W4A8 path (test infrastructure only).

Integer work is exact (int64 or fp32 matmuls of small integer codes whose sums
stay below 2^24); floating-point steps use IEEE fp32 in the order the
reference's torch code uses.  Citations are to files under the reference
repository GongCheng1919/vllm-ascend910.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

QMAX = {4: 7, 8: 127}     # fakequant_lab/quant.py:33
QMIN = {4: -8, 8: -128}   # fakequant_lab/quant.py:34
BF16_TINY_BITS = 0x0080   # torch.finfo(torch.bfloat16).tiny = 2^-126, quant.py:83-86
GROUP_ALIGN = 64          # npu_ops/kernel/mg_kgeom.h:52 (kCubeKElemsInt4)


# ------------------------------------------------------------------ bf16
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even, NaN kept quiet.

    int4_cube_lab/host/bf16.h:17-27 (FP32ToBF16); torch's .to(torch.bfloat16).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (exact).  int4_cube_lab/host/bf16.h:9-15."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (for normal x: 2^(floor(log2|x|) - 7))."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - 7)


# ------------------------------------------------------------------ geometry
def num_groups(K: int, group: int) -> int:
    """npu_ops/kernel/mg_kgeom.h:65-68."""
    return -(-K // group)


def group_real(g: int, K: int, group: int) -> int:
    """npu_ops/kernel/mg_kgeom.h:77-81."""
    G = num_groups(K, group)
    return group if g + 1 < G else K - (G - 1) * group


def group_stride(group: int) -> int:
    """npu_ops/kernel/mg_kgeom.h:71-74."""
    return -(-group // GROUP_ALIGN) * GROUP_ALIGN


def group_pad(g: int, K: int, group: int) -> int:
    """Padded width of group g (npu_ops/kernel/mg_kgeom.h:83-87)."""
    return -(-group_real(g, K, group) // GROUP_ALIGN) * GROUP_ALIGN


def group_offset(g: int, group: int) -> int:
    """Element offset of group g in a padded row (npu_ops/kernel/mg_kgeom.h:90-95)."""
    return g * group_stride(group)


def kpad(K: int, group: int) -> int:
    """npu_ops/kernel/mg_kgeom.h:98-102."""
    G = num_groups(K, group)
    return (G - 1) * group_stride(group) + -(-group_real(G - 1, K, group) // GROUP_ALIGN) * GROUP_ALIGN


# ------------------------------------------------------------------ quantiser
def group_params_sym(xg: np.ndarray, bits: int) -> np.ndarray:
    """Symmetric scale per group along the last axis, as bf16 bits.

    fakequant_lab/quant.py:102-105: scale = bf16(amax / qmax), tiny where zero.
    """
    amax = np.abs(xg.astype(np.float32)).max(axis=-1)
    s = f32_to_bf16_bits(amax / np.float32(QMAX[bits]))
    return np.where((s & 0x7FFF) == 0, np.uint16(BF16_TINY_BITS), s).astype(np.uint16)


def group_params_asym(xg: np.ndarray, bits: int) -> Tuple[np.ndarray, np.ndarray]:
    """Asymmetric (scale, zero) per group, as bf16 bits.  fakequant_lab/quant.py:106-132."""
    qmax, qmin = QMAX[bits], QMIN[bits]
    x = xg.astype(np.float32)
    mx, mn = x.max(axis=-1), x.min(axis=-1)
    rng = mx - mn
    s = f32_to_bf16_bits(rng / np.float32(qmax - qmin))
    s = np.where(s == 0, np.uint16(BF16_TINY_BITS), s)           # where(scale == 0, tiny)
    z = f32_to_bf16_bits(np.float32(qmin) - np.round(mn / bf16_bits_to_f32(s)))
    const = rng == 0
    sc = f32_to_bf16_bits(np.abs(mx) / np.float32(qmax))
    sc = np.where(sc == 0, np.uint16(BF16_TINY_BITS), sc)
    s = np.where(const, sc, s).astype(np.uint16)
    z = np.where(const, np.uint16(0), z).astype(np.uint16)
    return s, z


def quantize_with(x: np.ndarray, scale_bits: np.ndarray, zero_bits: Optional[np.ndarray], bits: int) -> np.ndarray:
    """fakequant_lab/quant.py:135-141: round_half_even(x / scale) (+ zero), clamp, int8.

    ``scale_bits``/``zero_bits`` broadcast against x's last axis.
    """
    q = np.round(x.astype(np.float32) / bf16_bits_to_f32(scale_bits))   # np.round = half to even
    if zero_bits is not None:
        q = q + bf16_bits_to_f32(zero_bits)
    return np.clip(q, QMIN[bits], QMAX[bits]).astype(np.int8)


def quant_act_per_token(x_bits: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-token int8 activation quant of a bf16 [M, K] (given as uint16 bits).

    fakequant_lab/quant.py:153-173 with QuantSpec(8, None) (one group spanning K):
    returns (a_q int8 [M, K], a_scale bf16 bits [M]).
    """
    x = bf16_bits_to_f32(x_bits)
    s = group_params_sym(x, 8)
    return quantize_with(x, s[:, None], None, 8), s


def quantize_weight_sym(w: np.ndarray, group: int, bits: int = 4) -> Tuple[np.ndarray, np.ndarray]:
    """Symmetric per-group weight quant of a float [N, K]: (codes int8 [N, K], scale bf16 bits [N, G]).

    fakequant_lab/quant.py:153-173 with QuantSpec(4, group, sym=True); a ragged last
    group is quantised on its real members (npu_ops/python/w4a8_ops.py:193-219).
    """
    N, K = w.shape
    G = num_groups(K, group)
    codes = np.empty((N, K), np.int8)
    scales = np.empty((N, G), np.uint16)
    for g in range(G):
        sl = slice(g * group, g * group + group_real(g, K, group))
        s = group_params_sym(w[:, sl], bits)
        scales[:, g] = s
        codes[:, sl] = quantize_with(w[:, sl], s[:, None], None, bits)
    return codes, scales


# ------------------------------------------------------------------ packing
def pack_int4(v: np.ndarray) -> np.ndarray:
    """[..., K] codes in [-8,7] -> [..., K/2] bytes, even k in the LOW nibble.

    npu_ops/python/w4a8_ops.py:142-148; int4_cube_lab/host/gemm_ref.cpp:9-24.
    """
    v = np.asarray(v, np.int16)
    lo = v[..., 0::2] & 0xF
    hi = v[..., 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8).view(np.int8)


def unpack_int4(p: np.ndarray) -> np.ndarray:
    b = np.asarray(p).view(np.uint8).astype(np.int16)
    out = np.stack([b & 0xF, b >> 4], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return np.where(out >= 8, out - 16, out).astype(np.int8)


def pad_groups(v: np.ndarray, group: int) -> np.ndarray:
    """[R, K] int8 -> [R, kpad] with group g's real members at g * group_stride
    and zeros in every padding slot: the padded K layout of both operands
    (weights: npu_ops/python/w4a8_ops.py:231-239; activations:
    int4_cube_lab/host/gemm_ref.cpp:62-90, whose padding decodes to 0)."""
    R, K = v.shape
    out = np.zeros((R, kpad(K, group)), np.int8)
    for g in range(num_groups(K, group)):
        r = group_real(g, K, group)
        out[:, g * group_stride(group):g * group_stride(group) + r] = v[:, g * group:g * group + r]
    return out


def pack_grouped(codes: np.ndarray, group: int) -> np.ndarray:
    """[N, K] codes -> [N, kpad/2] in the grouped zero-padded layout.

    npu_ops/python/w4a8_ops.py:231-239; int4_cube_lab/host/gemm_ref.cpp:42-60.
    """
    return pack_int4(pad_groups(codes, group))


# ------------------------------------------------------------------ GEMM
def group_partials(a_q: np.ndarray, w_codes: np.ndarray, group: int, exact_int64: bool = False) -> np.ndarray:
    """P[g, m, n] = sum_{k in g} a_q[m,k] * w[n,k] as int64 (exact).

    fakequant_lab/fake_linear.py:173-175 (``partial = F.linear(a_g, q_w[:, sl])``, an
    fp32 matmul of integer codes -- exact because |partial| <= 1024*group < 2^24);
    ``exact_int64`` computes the same with int64 arithmetic
    (fakequant_lab/run_selftest.py:115-116).
    """
    M, K = a_q.shape
    N = w_codes.shape[0]
    G = num_groups(K, group)
    # the fp32 route is exact only while every |partial| stays below 2^24
    # (|a| <= 128, |w| <= 8): longer groups (per-channel, group = K) take int64
    exact_int64 = exact_int64 or 1024 * min(group, K) >= (1 << 24)
    out = np.empty((G, M, N), np.int64)
    for g in range(G):
        sl = slice(g * group, g * group + group_real(g, K, group))
        if exact_int64:
            out[g] = a_q[:, sl].astype(np.int64) @ w_codes[:, sl].astype(np.int64).T
        else:
            out[g] = (a_q[:, sl].astype(np.float32) @ w_codes[:, sl].astype(np.float32).T).astype(np.int64)
    return out


def fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """fp32 fused multiply-add: a*b + c with one IEEE round-to-nearest-even.

    torch's CPU ``Tensor.addcmul_`` (the reference's accumulation,
    fakequant_lab/fake_linear.py:178) evaluates acc + t1*t2 this way.  The
    product of two fp32 values is exact in float64 (48 significant bits); the
    sum with c is rounded to float64 and its error recovered exactly (TwoSum);
    rounding the float64 sum to fp32 then equals rounding the exact value
    except when the sum sits exactly on an fp32 midpoint, where the sign of the
    error decides.  Finite inputs.
    """
    a64 = np.asarray(a, dtype=np.float32).astype(np.float64)
    b64 = np.asarray(b, dtype=np.float32).astype(np.float64)
    c64 = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a64 * b64
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    up = r.astype(np.float64) > s
    lo = np.where(up, np.nextafter(r, np.float32(-np.inf)), r)
    hi = np.where(up, r, np.nextafter(r, np.float32(np.inf)))
    mid = (lo.astype(np.float64) + hi.astype(np.float64)) * 0.5 == s
    r = np.where(mid & (e > 0), hi, np.where(mid & (e < 0), lo, r))
    return r.astype(np.float32)


def gemm_fp32(a_q: np.ndarray, a_scale_bits: np.ndarray, w_codes: np.ndarray, w_scale: np.ndarray,
              group: int, partials: Optional[np.ndarray] = None, return_abs: bool = False):
    """The reference's kernel-mode GEMM in fp32, per-token activation scale.

    fakequant_lab/fake_linear.py:166-179: for g in order,
        acc.addcmul_(partial_g, a_s[:, g] * w_s[:, g])    (fp32; a_s*w_s is exact;
                                                          addcmul_ rounds once, fma32)
    with the per-token a_s broadcast over groups (run_selftest.py:104-120 iterates
    the groups of the weight spec).  ``w_scale`` is [N, G] fp32 values (bf16 or
    fp16 scales, both exact in fp32).  Returns fp32 [M, N]; with ``return_abs``
    also the float64 sum of |partial_g * a_s * w_s| over groups, the magnitude
    that bounds any fp32 summation error (see ``fp32_sum_error_bound``).
    Partials are computed group by group unless given.
    """
    M, K = a_q.shape
    N = w_codes.shape[0]
    G = num_groups(K, group)
    a_s = bf16_bits_to_f32(a_scale_bits).astype(np.float32)
    acc = np.zeros((M, N), np.float32)
    mag = np.zeros((M, N), np.float64) if return_abs else None
    for g in range(G):
        if partials is not None:
            pg = partials[g]
        else:
            sl = slice(g * group, g * group + group_real(g, K, group))
            pg = a_q[:, sl].astype(np.float32) @ w_codes[:, sl].astype(np.float32).T
        s = (a_s[:, None] * w_scale[:, g].astype(np.float32)[None, :]).astype(np.float32)
        # acc.addcmul_(partial, s): one rounding of acc + partial * s (fma32)
        acc = fma32(pg.astype(np.float32), s, acc)
        if return_abs:
            mag += np.abs(pg.astype(np.float64) * s.astype(np.float64))
    return (acc, mag) if return_abs else acc


def fp32_sum_error_bound(mag: np.ndarray, n_groups: int) -> np.ndarray:
    """Worst-case |fp32 result - exact| for a sequential fp32 sum of n_groups
    rounded products plus a final scaling: (n_groups + 2) * 2^-24 * sum|terms|
    (the textbook recursive-summation bound, gamma_n = n*u)."""
    return (n_groups + 2) * 2.0 ** -24 * mag


def gemm_f64(a_q: np.ndarray, a_scale_bits: np.ndarray, w_codes: np.ndarray, w_scale: np.ndarray,
             group: int, partials: Optional[np.ndarray] = None) -> np.ndarray:
    """float64 restatement of fakequant_lab/run_selftest.py:104-120 (_exact_reference)."""
    G = num_groups(a_q.shape[1], group)
    a_s = bf16_bits_to_f32(a_scale_bits).astype(np.float64)
    if partials is None:
        partials = group_partials(a_q, w_codes, group, exact_int64=True)
    acc = np.zeros((a_q.shape[0], w_codes.shape[0]), np.float64)
    for g in range(G):
        acc += partials[g].astype(np.float64) * (a_s[:, None] * w_scale[:, g].astype(np.float64)[None, :])
    return acc


def gemm_midgroup_f64(a_q: np.ndarray, a_scale_bits: np.ndarray, w_codes: np.ndarray, w_scale_bits: np.ndarray,
                      w_zero_bits: Optional[np.ndarray], group: int,
                      partials: Optional[np.ndarray] = None) -> np.ndarray:
    """float64 value of ReferenceMidGroupGemm's definition (int4_cube_lab/host/gemm_ref.cpp:199-240):
    sum_g I_g[m,n] * ws[g,n] * as[g,m] with I_g = sum_{k in g} A*(W - wz), exact int64."""
    M = a_q.shape[0]
    G = num_groups(a_q.shape[1], group)
    if partials is None:
        partials = group_partials_asym(a_q, w_codes, w_zero_bits, group)
    acc = np.zeros((M, w_codes.shape[0]), np.float64)
    for g in range(G):
        acc += (partials[g].astype(np.float64) * bf16_bits_to_f32(w_scale_bits[g]).astype(np.float64)[None, :]
                * bf16_bits_to_f32(a_scale_bits[g, :M]).astype(np.float64)[:, None])
    return acc


def output_bar(y_bits: np.ndarray, y32: np.ndarray, exact) -> Tuple[np.ndarray, int]:
    """The bf16 output bar of the build's parity tests.

    An output passes when |y - y32| <= 1 bf16 ulp of y32, the oracle's fp32
    result (the north_star's max-abs bound).  One that does not -- where the
    groups cancel, two fp32 summation orders can differ by more than an ulp of
    the small result -- must lie within 1 bf16 ulp of the exact value instead:
    ``exact(rows, cols)`` returns the float64 restatement (``gemm_f64``,
    fakequant_lab/run_selftest.py:104-120) on the sorted unique rows x cols of
    those outputs.  Returns (mask of outputs failing both, number of outputs
    that needed the float64 value).
    """
    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    r = np.asarray(y32, np.float64)
    first = np.abs(y - r) > bf16_ulp(r)
    fail = np.zeros(y.shape, bool)
    n_fb = int(first.sum())
    if n_fb:
        ri, ci = np.nonzero(first)
        ur, uc = np.unique(ri), np.unique(ci)
        e = np.asarray(exact(ur, uc), np.float64)
        ev = e[np.searchsorted(ur, ri), np.searchsorted(uc, ci)]
        fail[ri, ci] = np.abs(y[ri, ci] - ev) > bf16_ulp(ev)
    return fail, n_fb


# ------------------------------------------------------------------ RMSNorm (decoder layer)
def add_bf16(x_bits: np.ndarray, r_bits: np.ndarray) -> np.ndarray:
    """bf16 + bf16 -> bf16 (the fp32 sum of two bf16 values, rounded once)."""
    return f32_to_bf16_bits((bf16_bits_to_f32(x_bits) + bf16_bits_to_f32(r_bits)).astype(np.float32))


def rms_norm_bf16(s_bits: np.ndarray, w_bits: np.ndarray, eps: float, return_h1: bool = False):
    """The reference decoder layer's rms_norm on a bf16 row (npu_ops/python/bench_decode_layer.py:36-38):
    v = float(s); h = bf16(v * rsqrt(mean(v^2) + eps)) * w in bf16.  The mean is taken exactly
    (float64) and rounded to fp32, rsqrt correctly rounded in fp32; torch's own fp32 summation
    order may move r by an fp32 ulp, so a bf16 result can differ by one ulp at a rounding tie."""
    v = bf16_bits_to_f32(s_bits)
    K = v.shape[-1]
    ms = ((v.astype(np.float64) ** 2).sum(axis=-1) / K).astype(np.float32)
    t = (ms + np.float32(eps)).astype(np.float32)
    r = (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)
    h1 = round_bf16((v * r[..., None]).astype(np.float32))
    h = f32_to_bf16_bits((h1 * bf16_bits_to_f32(w_bits)).astype(np.float32))
    return (h, h1) if return_h1 else h


# ------------------------------------------------------------------ mid-group compat path
def quant_act_midgroup(x_bits: np.ndarray, group: int) -> Tuple[np.ndarray, np.ndarray]:
    """Per (token, K-group) int8 quant of a bf16 [M, K]: (q int8 [M, K], scale bf16 bits [G, M]).

    fakequant_lab/quant.py:89-105, :135-141 applied to each group's real members
    (the activation side of npu_ops/kernel/midgroup_quant_a.inc:49-62; a short
    last group is quantised on what it holds).
    """
    M, K = x_bits.shape
    G = num_groups(K, group)
    x = bf16_bits_to_f32(x_bits)
    q = np.empty((M, K), np.int8)
    sc = np.empty((G, M), np.uint16)
    for g in range(G):
        sl = slice(g * group, g * group + group_real(g, K, group))
        s = group_params_sym(x[:, sl], 8)
        sc[g] = s
        q[:, sl] = quantize_with(x[:, sl], s[:, None], None, 8)
    return q, sc


def msd_planes(q: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """int8 codes -> (hi, lo) int4 values with q = 16*hi + lo + 8:
    hi = floor(q / 16), lo = q - 16*hi - 8 (npu_ops/kernel/midgroup_quant_a.inc:68-73)."""
    hi = np.floor_divide(q.astype(np.int16), 16)
    lo = q.astype(np.int16) - 16 * hi - 8
    return hi.astype(np.int8), lo.astype(np.int8)


def act_ksum_neg(q: np.ndarray, group: int) -> np.ndarray:
    """-sum_{k in g} q per (group, row): int32 [G, M] (midgroup_quant_a.inc:326-337)."""
    M, K = q.shape
    G = num_groups(K, group)
    out = np.empty((G, M), np.int32)
    for g in range(G):
        out[g] = -q[:, g * group:g * group + group_real(g, K, group)].astype(np.int64).sum(axis=1)
    return out


def tile_m_for(M: int) -> int:
    """The reference's row padding unit (npu_ops/host/midgroup_quant_a.cpp:37)."""
    return 16 if M <= 16 else (64 if M <= 64 else 128)


def midgroup_quant_a(x_bits: np.ndarray, group: int = 1024, Mp: Optional[int] = None):
    """The four tensors of the reference's midgroup_quant_a, as numpy arrays:
    a_hi, a_lo int8 [Mp, kpad/2] (packed int4 planes in the padded K layout),
    a_scale bf16 bits [G, Mp], a_ksum int32 [G, Mp]; rows [M, Mp) carry scale
    tiny, q = 0, ksum 0 (npu_ops/host/midgroup_quant_a.cpp:40-78,
    npu_ops/kernel/midgroup_quant_a.inc:7-28)."""
    M, K = x_bits.shape
    Mp = Mp if Mp is not None else -(-M // tile_m_for(M)) * tile_m_for(M)
    G = num_groups(K, group)
    q = np.zeros((Mp, K), np.int8)
    sc = np.full((G, Mp), BF16_TINY_BITS, np.uint16)
    qm, scm = quant_act_midgroup(x_bits, group)
    q[:M] = qm
    sc[:, :M] = scm
    hi, lo = msd_planes(pad_groups(q, group))
    # pad_groups leaves q = 0 in every padding slot, whose planes are hi 0, lo -8
    return pack_int4(hi), pack_int4(lo), sc, act_ksum_neg(q, group)


def quantize_weight_asym(w: np.ndarray, group: int, bits: int = 4):
    """Asymmetric per-group weight quant of a float [N, K], the reference's export
    (npu_ops/python/w4a8_ops.py:181-240 with QuantSpec(4, group, sym=False)):
    (codes int8 [N, K], scale bf16 bits [G, N], zero bf16 bits [G, N], ksum int32
    [G, N] of the raw codes).  A ragged last group is quantised as its own group."""
    N, K = w.shape
    G = num_groups(K, group)
    codes = np.empty((N, K), np.int8)
    sc = np.empty((G, N), np.uint16)
    zr = np.empty((G, N), np.uint16)
    ks = np.empty((G, N), np.int32)
    for g in range(G):
        sl = slice(g * group, g * group + group_real(g, K, group))
        s, z = group_params_asym(w[:, sl], bits)
        codes[:, sl] = quantize_with(w[:, sl], s[:, None], z[:, None], bits)
        sc[g], zr[g] = s, z
        ks[g] = codes[:, sl].astype(np.int64).sum(axis=1)
    return codes, sc, zr, ks


def group_partials_asym(a_q: np.ndarray, w_codes: np.ndarray, w_zero_bits: Optional[np.ndarray],
                        group: int) -> np.ndarray:
    """I[g, m, n] = sum_{k in g} A[m,k] * (W[n,k] - wz[g,n]) as int64, the definition the
    reference's C++ checks against (int4_cube_lab/host/gemm_ref.cpp:216-227,
    ragged_layout_test.cpp:128-135); wz is truncated to an integer as there."""
    M, K = a_q.shape
    N = w_codes.shape[0]
    G = num_groups(K, group)
    out = np.empty((G, M, N), np.int64)
    for g in range(G):
        sl = slice(g * group, g * group + group_real(g, K, group))
        w = w_codes[:, sl].astype(np.int64)
        if w_zero_bits is not None:
            w = w - np.trunc(bf16_bits_to_f32(w_zero_bits[g])).astype(np.int64)[:, None]
        a = a_q[:, sl].astype(np.int64)
        # float64 products and sums of these integers are exact in any order
        # while sum |a| * |w| stays below 2**53, which BLAS then computes fast
        if int(np.abs(a).max(initial=0)) * int(np.abs(w).max(initial=0)) * a.shape[1] < 2 ** 53:
            out[g] = (a.astype(np.float64) @ w.T.astype(np.float64)).astype(np.int64)
        else:
            out[g] = a @ w.T
    return out


def gemm_midgroup_fp32(a_q: np.ndarray, a_scale_bits: np.ndarray, w_codes: np.ndarray, w_scale_bits: np.ndarray,
                       w_zero_bits: Optional[np.ndarray], group: int, partials: Optional[np.ndarray] = None,
                       return_abs: bool = False):
    """ReferenceMidGroupGemm (int4_cube_lab/host/gemm_ref.cpp:199-240) in its fp32
    order: for g in order, acc += (float(I_g) * ws[g,n]) * as[g,m], each product and
    sum rounded to fp32.  a_scale_bits [G, >= M], w_scale/w_zero bits [G, N].
    With ``return_abs`` also sum_g |term_g| in float64 (for fp32_sum_error_bound)."""
    M, K = a_q.shape
    G = num_groups(K, group)
    if partials is None:
        partials = group_partials_asym(a_q, w_codes, w_zero_bits, group)
    acc = np.zeros((M, w_codes.shape[0]), np.float32)
    mag = np.zeros(acc.shape, np.float64) if return_abs else None
    for g in range(G):
        t1 = (partials[g].astype(np.float32) * bf16_bits_to_f32(w_scale_bits[g])[None, :]).astype(np.float32)
        t2 = (t1 * bf16_bits_to_f32(a_scale_bits[g, :M])[:, None]).astype(np.float32)
        acc = (acc + t2).astype(np.float32)
        if return_abs:
            mag += np.abs(t2.astype(np.float64))
    return (acc, mag) if return_abs else acc


def silu_mul_bf16(g_bits: np.ndarray, u_bits: np.ndarray) -> np.ndarray:
    """``F.silu(g) * u`` on bf16 tensors, as bf16 bits (npu_ops/python/bench_decode_layer.py:78-81).

    torch evaluates silu of a bf16 tensor in fp32 as g / (1 + exp(-g)) and
    rounds it to bf16, then multiplies two bf16 tensors in fp32 (exact: 8-bit
    significands) and rounds to bf16.  Each fp32 step is restated correctly
    rounded (exp taken in float64, then rounded to fp32, overflowing to inf
    for g < -88.7 as the fp32 formula does, which gives silu = -0 there); an
    fp32 exp may differ from it in the last bit, which moves the bf16 result
    only at a rounding tie.
    """
    g = bf16_bits_to_f32(g_bits).astype(np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
        s32 = (g / (np.float32(1.0) + e).astype(np.float32)).astype(np.float32)
    s = round_bf16(s32)
    return f32_to_bf16_bits((s * bf16_bits_to_f32(u_bits)).astype(np.float32))


def linear_bf16(x_bits: np.ndarray, w_codes: np.ndarray, w_scale: np.ndarray, group: int):
    """Whole path: per-token quant -> group GEMM -> bf16 (fakequant_lab/fake_linear.py:142-153).

    Returns (y bf16 bits [M,N], y fp32 [M,N], a_q, a_scale_bits, partials).
    """
    a_q, a_s = quant_act_per_token(x_bits)
    P = group_partials(a_q, w_codes, group)
    y32 = gemm_fp32(a_q, a_s, w_codes, w_scale, group, P)
    return f32_to_bf16_bits(y32), y32, a_q, a_s, P
