"""Pins the CPU oracle (oracle/w4a8.py) before it is trusted as the checker.

Each check is independent of the oracle's own formula: exact rational
arithmetic, brute-force integer sums, torch's conversions, and the reference's
own C++ CPU reference compiled from its sources (oracle/_ref, skipped when the
reference checkout was not available to build it).  Negative controls plant a
plausible mistake in a copy of the oracle's inputs or arithmetic and show
that the comparison catches it.
"""
from __future__ import annotations

import subprocess
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ref as oref
from oracle import w4a8 as ow

needs_ref = pytest.mark.skipif(not oref.available(), reason="oracle/_ref not built (reference checkout absent)")


# --------------------------------------------------------------- exact helpers
def round_to_float(fr: Fraction, mant_bits: int) -> Fraction:
    """Round a positive rational to the nearest value with `mant_bits` significant bits, ties to even
    (normal range only)."""
    if fr == 0:
        return Fraction(0)
    e = fr.numerator.bit_length() - fr.denominator.bit_length()
    while Fraction(2) ** e > fr:
        e -= 1
    while Fraction(2) ** (e + 1) <= fr:
        e += 1
    ulp = Fraction(2) ** (e - mant_bits + 1)
    q = fr / ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n * ulp


def round_half_even(fr: Fraction) -> int:
    n = fr.numerator // fr.denominator  # floor
    rem = fr - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n


def exact_quant_row(xbits: np.ndarray):
    """Per-token quant of one bf16 row in exact rational arithmetic."""
    xs = [Fraction(float(v)) for v in ow.bf16_bits_to_f32(xbits)]
    amax = max(abs(v) for v in xs)
    s = round_to_float(round_to_float(amax / 127, 24), 8)     # fp32 divide, then bf16
    if s == 0:
        s = Fraction(2) ** -126
    q = [max(-128, min(127, round_half_even(v / s))) for v in xs]
    return s, q


# --------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4e38, 1e-40, -1e-40, 1.1754944e-38], np.float32),
        # exact half-way points between bf16 neighbours (both parities)
        (np.arange(0x3F800000, 0x3F800000 + 64, dtype=np.uint32) * 0 + 0x3F808000).view(np.float32),
        np.array([0x3F818000, 0x3F828000, 0xBF818000], np.uint32).view(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ow.f32_to_bf16_bits(x), ref)


@needs_ref
def test_bf16_rounding_matches_reference_cpp():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 1e3,
                        np.array([0x3F808000, 0x3F818000, 0x7FC00001, 0x7F800001], np.uint32).view(np.float32)])
    assert np.array_equal(ow.f32_to_bf16_bits(x), oref.fp32_to_bf16(x))


# --------------------------------------------------------------- quantiser
def test_quant_per_token_matches_rational_arithmetic():
    rng = np.random.default_rng(3)
    M, K = 24, 96
    x = rng.standard_normal((M, K)).astype(np.float32) * rng.uniform(0.01, 50, size=(M, 1)).astype(np.float32)
    x[:, 7] *= 20  # an outlier channel
    xb = ow.f32_to_bf16_bits(x)
    q, s = ow.quant_act_per_token(xb)
    for m in range(M):
        s_exact, q_exact = exact_quant_row(xb[m])
        assert Fraction(float(ow.bf16_bits_to_f32(s[m]))) == s_exact
        assert q[m].tolist() == q_exact


def test_quant_ties_round_half_to_even():
    # amax = 127 -> scale exactly 1.0; every x/s below is an exact half-integer.
    vals = np.array([127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5], np.float32)
    q, s = ow.quant_act_per_token(ow.f32_to_bf16_bits(vals)[None, :])
    assert ow.bf16_bits_to_f32(s)[0] == 1.0
    assert q[0].tolist() == [127, 2, 4, -2, -4, 0, 0, 2, 126, -126]


def test_quant_zero_row_uses_bf16_tiny():
    q, s = ow.quant_act_per_token(np.zeros((2, 64), np.uint16))
    assert s.tolist() == [0x0080, 0x0080]
    assert not q.any()


def test_quant_tie_rows_match_rational_and_catch_reciprocal_multiply():
    """On rows built from exact half-way quotients the oracle agrees with exact
    rounding, while a reciprocal-multiply quantiser (the mistake the reference
    warns about, npu_ops/kernel/midgroup_quant_a.inc:55-62) does not."""
    from conftest import tie_rows
    xb = tie_rows(48, 128, seed=4)
    q, s = ow.quant_act_per_token(xb)
    for m in range(xb.shape[0]):
        s_exact, q_exact = exact_quant_row(xb[m])
        assert Fraction(float(ow.bf16_bits_to_f32(s[m]))) == s_exact
        assert q[m].tolist() == q_exact
    xf = ow.bf16_bits_to_f32(xb)
    recip = (np.float32(1.0) / ow.bf16_bits_to_f32(s)).astype(np.float32)
    q_bad = np.clip(np.round(xf * recip[:, None]), -128, 127).astype(np.int8)
    assert not np.array_equal(q_bad, q)


def reciprocal_quant(xf: np.ndarray, s: np.ndarray) -> np.ndarray:
    """numpy model of the GPU quantiser's arithmetic for a normal scale s:
    t = rint(fp32(x * fp32(1/s))), the exact residual d = x - t*s (an fma on the
    GPU, exact float64 here), and at |d| == s/2 the even neighbour."""
    s = s.astype(np.float32)
    r = (np.float32(1.0) / s).astype(np.float32)
    t = np.rint((xf * r).astype(np.float32)).astype(np.float64)
    d = xf.astype(np.float64) - t * s.astype(np.float64)
    tie = (np.abs(d) == 0.5 * s.astype(np.float64)) & (np.mod(t, 2) != 0)
    t = np.where(tie, t + np.sign(d), t)
    return np.clip(t, -128, 127).astype(np.int8)


def test_reciprocal_quant_equals_divide_exhaustively():
    """The reciprocal-plus-half-way-test quantiser gives the IEEE divide's codes for
    every bf16 x with |x| <= 127.25 s, every bf16 significand of s, at three scale
    exponents (large, mid, and near the 2^-125 lower limit of that path), and on the
    half-way tie rows where a bare reciprocal multiply fails."""
    allx = ow.bf16_bits_to_f32(np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16))
    allx = allx[np.isfinite(allx)]
    bare_misses = 0
    for e in (20, -40, -118):
        for m in range(128, 256):
            s = np.float32(m * 2.0 ** (e - 7))
            x = allx[np.abs(allx) <= np.float32(127.25) * s]
            div = np.clip(np.rint((x / s).astype(np.float32)), -128, 127).astype(np.int8)
            assert np.array_equal(reciprocal_quant(x, np.full_like(x, s)), div), (e, m)
            bare = np.clip(np.rint((x * (np.float32(1.0) / s)).astype(np.float32)), -128, 127).astype(np.int8)
            bare_misses += int(np.count_nonzero(bare != div))
    assert bare_misses > 0   # the half-way test is what makes the difference
    from conftest import tie_rows
    xb = tie_rows(48, 128, seed=4)
    q, sb = ow.quant_act_per_token(xb)
    sf = np.repeat(ow.bf16_bits_to_f32(sb)[:, None], 128, 1)
    assert np.array_equal(reciprocal_quant(ow.bf16_bits_to_f32(xb), sf), q)


# --------------------------------------------------------------- packing / geometry
RAGGED_CASES = [(5120, 128), (27648, 128), (1057, 128), (1279, 256), (1025, 1024), (33, 64), (1, 64), (65, 64),
                (63, 64), (2049, 512), (1023, 1024), (35, 32), (777, 96), (100, 33), (4096, 64)]


def test_pack_roundtrip_exhaustive():
    v = np.array([[a, b] for a in range(-8, 8) for b in range(-8, 8)], np.int8).reshape(1, -1)
    p = ow.pack_int4(v)
    assert np.array_equal(ow.unpack_int4(p), v)
    assert ow.pack_int4(np.array([[1, -1]], np.int8)).view(np.uint8)[0, 0] == 0xF1


@needs_ref
@pytest.mark.parametrize("K,gk", RAGGED_CASES)
def test_geometry_and_grouped_pack_match_reference(K, gk):
    lib = oref.lib()
    assert ow.num_groups(K, gk) == lib.ref_num_groups(K, gk)
    assert ow.kpad(K, gk) == lib.ref_kpad(K, gk)
    for g in range(ow.num_groups(K, gk)):
        assert ow.group_real(g, K, gk) == lib.ref_group_real(g, K, gk)
        assert g * ow.group_stride(gk) == lib.ref_group_offset(g, gk)
    codes = np.random.default_rng(K).integers(-8, 8, size=(3, K)).astype(np.int8)
    assert np.array_equal(ow.pack_grouped(codes, gk), oref.pack_int4_grouped(codes, gk))


@needs_ref
@pytest.mark.parametrize("K,gk", RAGGED_CASES)
def test_padded_activation_layout_matches_reference_planes(K, gk):
    """pad_groups places activations where the reference's grouped MSD plane
    split does (recombined a = 16*hi + lo + 8), with its padding decoding to 0."""
    a = np.random.default_rng(K + gk).integers(-128, 128, size=(3, K)).astype(np.int8)
    hi, lo = oref.split_planes_grouped(a, gk)
    recombined = 16 * ow.unpack_int4(hi).astype(np.int32) + ow.unpack_int4(lo).astype(np.int32) + 8
    assert np.array_equal(ow.pad_groups(a, gk).astype(np.int32), recombined)


def test_pad_groups_closed_form():
    """Brute force on the geometry's definition: element k of group k // group
    sits at (k // group) * ceil_to(group, 64) + k % group; everything else is 0."""
    for K, gk in ((100, 33), (1057, 96), (232, 192), (5000, 128), (1, 1024)):
        v = np.random.default_rng(K).integers(-128, 128, size=(2, K)).astype(np.int8)
        out = ow.pad_groups(v, gk)
        stride = -(-gk // 64) * 64
        dst = np.array([(k // gk) * stride + k % gk for k in range(K)])
        assert out.shape == (2, ow.kpad(K, gk))
        assert np.array_equal(out[:, dst], v)
        rest = np.ones(out.shape[1], bool)
        rest[dst] = False
        assert not out[:, rest].any()


@needs_ref
def test_reference_ragged_layout_binary_passes():
    out = subprocess.run([str(oref.RAGGED_TEST)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "ALL PASS" in out.stdout, out.stdout[-2000:]


# --------------------------------------------------------------- GEMM
def test_group_partials_fp32_path_is_exact():
    rng = np.random.default_rng(5)
    for M, N, K, G in ((5, 48, 1024, 1024), (17, 33, 640, 128), (3, 16, 192, 64)):
        a = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
        w = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
        a[0, :] = -128
        w[0, :] = -8   # extreme products: |P| reaches 1024*G
        assert np.array_equal(ow.group_partials(a, w, G), ow.group_partials(a, w, G, exact_int64=True))
        # brute force one entry
        g = K // G - 1
        assert ow.group_partials(a, w, G)[g, 1, 2] == sum(int(a[1, k]) * int(w[2, k]) for k in range(g * G, (g + 1) * G))


def _gemm_case(seed, M=8, N=64, K=512, G=128):
    rng = np.random.default_rng(seed)
    xb = ow.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    wsb = ow.f32_to_bf16_bits(rng.uniform(0.002, 0.02, size=(N, K // G)).astype(np.float32))
    return xb, w, wsb


def test_gemm_fp32_close_to_float64_definition():
    xb, w, wsb = _gemm_case(6)
    a_q, a_s = ow.quant_act_per_token(xb)
    ws = ow.bf16_bits_to_f32(wsb)
    y32 = ow.gemm_fp32(a_q, a_s, w, ws, 128)
    y64 = ow.gemm_f64(a_q, a_s, w, ws, 128)
    assert np.max(np.abs(y32 - y64)) <= 1e-6 * np.max(np.abs(y64))     # run_selftest.py:137-141 bar


@needs_ref
def _round_f32_exact(v: Fraction) -> np.float32:
    """Round an exact rational to fp32, ties to even (normal range)."""
    f = np.float32(float(v))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    dist = [abs(Fraction(float(c)) - v) for c in cands]
    best = min(dist)
    ties = [c for c, d in zip(cands, dist) if d == best]
    if len(ties) == 1:
        return ties[0]
    return [c for c in ties if (np.array(c, np.float32).view(np.uint32) & 1) == 0][0]


def test_fma32_matches_torch_addcmul():
    """fake_linear.py:178 accumulates with acc.addcmul_(partial, a_s*w_s): on torch's
    CPU path that is one rounding of acc + partial*s.  fma32 equals it on every element,
    in the reference's broadcast form too; the two-rounding evaluation does not."""
    rng = np.random.default_rng(11)
    n = 1 << 18
    acc = (rng.standard_normal(n) * 1000).astype(np.float32)
    p = rng.integers(-130000, 130000, n).astype(np.float32)
    sc = (rng.uniform(0.002, 0.02, n) * rng.uniform(0.001, 0.05, n)).astype(np.float32)
    t = torch.from_numpy(acc.copy())
    t.addcmul_(torch.from_numpy(p), torch.from_numpy(sc))
    assert np.array_equal(ow.fma32(p, sc, acc), t.numpy())
    two = (acc + (p * sc).astype(np.float32)).astype(np.float32)
    assert np.mean(two != t.numpy()) > 0.01, "negative control: unfused evaluation must differ"
    M, N = 32, 2048
    acc2 = (rng.standard_normal((M, N)) * 100).astype(np.float32)
    P = rng.integers(-130000, 130000, (M, N)).astype(np.float32)
    a_s = rng.uniform(0.001, 0.05, (M, 1)).astype(np.float32)
    w_s = rng.uniform(0.002, 0.02, (1, N)).astype(np.float32)
    t2 = torch.from_numpy(acc2.copy())
    t2.addcmul_(torch.from_numpy(P), torch.from_numpy(a_s) * torch.from_numpy(w_s))
    assert np.array_equal(ow.fma32(P, (a_s * w_s).astype(np.float32), acc2), t2.numpy())


def test_fma32_matches_rational_rounding():
    """Exact rational a*b + c rounded once to fp32, on random operands and on sums built
    to land exactly on an fp32 midpoint (where a float64 sum alone would round twice)."""
    rng = np.random.default_rng(12)
    a = rng.integers(-130000, 130000, 600).astype(np.float32)
    b = rng.uniform(1e-5, 1e-3, 600).astype(np.float32)
    c = (rng.standard_normal(600) * 50).astype(np.float32)
    # a*b an exact fp32 midpoint (3 * (1 + odd * 2^-23) has 25 significant bits); c = +-2^-100
    # leaves the float64 sum on the midpoint while the exact value is off it, c = 0 is a tie
    for i in range(300):
        a[i] = np.float32(3.0)
        b[i] = np.float32(1.0 + 2.0 ** -23 * (2 * int(rng.integers(0, 1 << 20)) + 1))
        c[i] = np.float32((0.0, 2.0 ** -100, -(2.0 ** -100))[i % 3])
    got = ow.fma32(a, b, c)
    for i in range(600):
        want = _round_f32_exact(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)
    # the constructed cases do need the midpoint rule: rounding the float64 sum alone
    # gets the nonzero-c ones wrong whenever ties-to-even points the other way (about half)
    naive = (a[:300].astype(np.float64) * b[:300] + c[:300]).astype(np.float32)
    assert np.sum(naive != got[:300]) >= 50


def test_gemm_fp32_equals_reference_torch_loop():
    """gemm_fp32 is the reference's kernel-mode loop run on torch's CPU path (the
    fake_linear.py:166-179 statement sequence on int8 codes and fp32 scales), bit for bit."""
    rng = np.random.default_rng(13)
    M, N, K, G = 6, 40, 512, 128
    q = rng.integers(-128, 128, (M, K)).astype(np.int8)
    w = rng.integers(-8, 8, (N, K)).astype(np.int8)
    sb = ow.f32_to_bf16_bits((rng.uniform(0.001, 0.05, M)).astype(np.float32))
    ws = rng.uniform(0.002, 0.02, (N, K // G)).astype(np.float16).astype(np.float32)
    a_s = torch.from_numpy(ow.bf16_bits_to_f32(sb))
    acc = torch.zeros((M, N), dtype=torch.float32)
    for g in range(K // G):
        sl = slice(g * G, (g + 1) * G)
        partial = torch.from_numpy(q[:, sl].astype(np.float32)) @ torch.from_numpy(w[:, sl].astype(np.float32)).T
        acc.addcmul_(partial, a_s[:, None] * torch.from_numpy(ws[:, g])[None, :])
    assert np.array_equal(ow.gemm_fp32(q, sb, w, ws, G), acc.numpy())


def test_gemm_bf16_matches_reference_cpp():
    for seed, (M, N, K, G) in enumerate(((8, 64, 512, 128), (16, 128, 5120 // 4, 256), (4, 32, 1024, 64))):
        xb, w, wsb = _gemm_case(seed + 10, M, N, K, G)
        a_q, a_s = ow.quant_act_per_token(xb)
        y = ow.f32_to_bf16_bits(ow.gemm_fp32(a_q, a_s, w, ow.bf16_bits_to_f32(wsb), G))
        Gn = K // G
        yr = oref.midgroup_gemm(a_q, np.repeat(a_s[None, :], Gn, axis=0), w, wsb.T.copy(), G)
        d = np.abs(ow.bf16_bits_to_f32(y).astype(np.float64) - ow.bf16_bits_to_f32(yr))
        assert np.all(d <= ow.bf16_ulp(ow.bf16_bits_to_f32(yr)))
        assert np.mean(y == yr) > 0.99


@needs_ref
def test_gemm_negative_control_transposed_scales():
    xb, w, wsb = _gemm_case(20, 8, 64, 512, 128)
    a_q, a_s = ow.quant_act_per_token(xb)
    G = 4
    yr = oref.midgroup_gemm(a_q, np.repeat(a_s[None, :], G, axis=0), w, wsb.T.copy(), 128)
    ws_bad = ow.bf16_bits_to_f32(wsb)[:, ::-1].copy()   # groups in the wrong order
    y_bad = ow.f32_to_bf16_bits(ow.gemm_fp32(a_q, a_s, w, ws_bad, 128))
    assert np.mean(y_bad == yr) < 0.5


# --------------------------------------------------------------- SwiGLU
def test_silu_mul_matches_torch_bf16():
    """The oracle's SwiGLU against torch's own `F.silu(g) * u` on bf16 CPU
    tensors (an independent fp32 silu): equal except where torch's fp32 silu
    lands on the other side of a bf16 rounding tie, and never more than one
    bf16 ulp apart."""
    rng = np.random.default_rng(7)
    g = ow.f32_to_bf16_bits((rng.standard_normal(200000) * 6).astype(np.float32))
    u = ow.f32_to_bf16_bits((rng.standard_normal(200000) * 3).astype(np.float32))
    g[:6] = ow.f32_to_bf16_bits(np.array([0.0, -0.0, 100.0, -100.0, 1e-30, -89.0], np.float32))
    ours = ow.bf16_bits_to_f32(ow.silu_mul_bf16(g, u)).astype(np.float64)
    tg = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    tu = torch.from_numpy(u.view(np.int16)).view(torch.bfloat16)
    ref = (torch.nn.functional.silu(tg) * tu).float().numpy().astype(np.float64)
    assert np.mean(ours == ref) > 0.999
    assert np.all(np.abs(ours - ref) <= ow.bf16_ulp(ref))
    assert ours[3] == 0.0 and ours[5] == 0.0     # silu(-100), silu(-89): exp(-g) overflows fp32
    # a plausible slip -- gate and up swapped -- is caught
    wrong = ow.bf16_bits_to_f32(ow.silu_mul_bf16(u, g)).astype(np.float64)
    assert np.mean(wrong == ref) < 0.5


# --------------------------------------------------------------- mid-group compat path
MID_CASES = [(5120, 1024), (1057, 1024), (3456, 1024), (300, 128), (2049, 512)]


def test_midgroup_quant_matches_rational_arithmetic():
    """Per (token, group) quant == exact rational restatement of quant.py on each
    group's real members, including a zero group and exact half-way quotients."""
    rng = np.random.default_rng(3)
    for K, gk in ((1057, 1024), (300, 128)):
        x = ow.f32_to_bf16_bits((rng.standard_normal((3, K)) * 2).astype(np.float32))
        x[1, :gk] = 0                                      # an all-zero group
        x[2, :256] = tie_rows_bits(1, 256)[0]              # exact .5 quotients
        q, sc = ow.quant_act_midgroup(x, gk)
        for m in range(3):
            for g in range(ow.num_groups(K, gk)):
                sl = slice(g * gk, g * gk + ow.group_real(g, K, gk))
                s, qe = exact_quant_row(x[m, sl])
                assert Fraction(float(ow.bf16_bits_to_f32(sc[g:g + 1, m])[0])) == s
                assert list(q[m, sl]) == qe


def tie_rows_bits(n, K):
    from conftest import tie_rows
    return tie_rows(n, K, seed=9)


@needs_ref
@pytest.mark.parametrize("K,gk", MID_CASES)
def test_midgroup_quant_a_layout_matches_reference(K, gk):
    """The four compat tensors: planes == the reference's grouped MSD split of the
    same codes, ksums == its ActKSumNegPerGroup, padded rows hold q = 0 / tiny."""
    x = ow.f32_to_bf16_bits(np.random.default_rng(K).standard_normal((5, K)).astype(np.float32))
    q, sc = ow.quant_act_midgroup(x, gk)
    a_hi, a_lo, a_scale, a_ksum = ow.midgroup_quant_a(x, gk)        # Mp = 16
    assert a_hi.shape == (16, ow.kpad(K, gk) // 2) and a_scale.shape == (ow.num_groups(K, gk), 16)
    hi_ref, lo_ref = oref.split_planes_grouped(q, gk)
    assert np.array_equal(a_hi[:5], hi_ref) and np.array_equal(a_lo[:5], lo_ref)
    assert np.array_equal(a_ksum[:, :5], oref.act_ksum_neg(q, gk))
    assert np.array_equal(a_scale[:, :5], sc)
    assert not a_hi[5:].any() and np.all(a_lo[5:].view(np.uint8) == 0x88)
    assert np.all(a_scale[:, 5:] == ow.BF16_TINY_BITS) and not a_ksum[:, 5:].any()


def test_msd_planes_exhaustive():
    q = np.arange(-128, 128, dtype=np.int8)
    hi, lo = ow.msd_planes(q)
    assert np.array_equal(16 * hi.astype(np.int32) + lo + 8, q.astype(np.int32))
    assert hi.min() == -8 and hi.max() == 7 and lo.min() == -8 and lo.max() == 7


def _exact_asym(xs, bits=4):
    """quant.py:106-132 for one group in rational arithmetic with fp32/bf16 roundings."""
    qmax, qmin = 7, -8
    mx, mn = max(xs), min(xs)
    rng_ = mx - mn
    if rng_ == 0:
        s = round_to_float(round_to_float(abs(mx) / qmax, 24), 8) if mx != 0 else Fraction(0)
        return (s if s != 0 else Fraction(2) ** -126), Fraction(0)
    rf = round_to_float(rng_, 24)                       # fp32 subtraction
    s = round_to_float(round_to_float(rf / (qmax - qmin), 24), 8)
    s = s if s != 0 else Fraction(2) ** -126
    z = Fraction(qmin) - round_half_even(round_to_float(mn / s, 24) if mn >= 0 else -round_to_float(-mn / s, 24))
    return s, round_to_float(z, 8) if z > 0 else (-round_to_float(-z, 8) if z < 0 else Fraction(0))


def test_group_params_asym_matches_rational_arithmetic():
    rng = np.random.default_rng(11)
    w = ow.round_bf16((rng.standard_normal((40, 64)) * 0.05 + rng.uniform(-0.02, 0.02, (40, 1))).astype(np.float32))
    w[3] = np.float32(0.25)                              # constant group: scale |v|/7, zero 0
    w[4] = 0.0                                           # all-zero group
    s_bits, z_bits = ow.group_params_asym(w, 4)
    for r in range(w.shape[0]):
        s, z = _exact_asym([Fraction(float(v)) for v in w[r]])
        assert Fraction(float(ow.bf16_bits_to_f32(s_bits[r:r + 1])[0])) == s, r
        assert Fraction(float(ow.bf16_bits_to_f32(z_bits[r:r + 1])[0])) == z, r


@needs_ref
def test_quantize_weight_asym_ksum_matches_reference():
    w = np.random.default_rng(2).standard_normal((48, 1057)).astype(np.float32)
    codes, sc, zr, ks = ow.quantize_weight_asym(w, 1024)
    assert codes.min() >= -8 and codes.max() <= 7 and sc.shape == (2, 48)
    assert np.array_equal(ks, oref.weight_ksum(codes, 1024))


@needs_ref
@pytest.mark.parametrize("K,gk", MID_CASES)
def test_midgroup_partials_identity_and_definition(K, gk):
    """I = sum A*(W - wz) by brute force, and the rank-1 identity the GPU kernel uses,
    16*S_hi + S_lo + 8*w_ksum + wz*a_ksum (planes and ksums from the reference's C++)."""
    rng = np.random.default_rng(K + gk)
    M, N = 3, 20
    a = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    w = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    wz = ow.f32_to_bf16_bits(rng.integers(-8, 8, size=(ow.num_groups(K, gk), N)).astype(np.float32))
    I = ow.group_partials_asym(a, w, wz, gk)
    hi_p, lo_p = oref.split_planes_grouped(a, gk)
    hi = ow.unpack_int4(hi_p).astype(np.int64)
    lo = ow.unpack_int4(lo_p).astype(np.int64)
    wp = ow.unpack_int4(ow.pack_grouped(w, gk)).astype(np.int64)
    aks, wks = oref.act_ksum_neg(a, gk), oref.weight_ksum(w, gk)
    st = ow.group_stride(gk)
    for g in range(ow.num_groups(K, gk)):
        sl = slice(g * st, g * st + ow.group_pad(g, K, gk))
        s_hi, s_lo = hi[:, sl] @ wp[:, sl].T, lo[:, sl] @ wp[:, sl].T
        zi = ow.bf16_bits_to_f32(wz[g]).astype(np.int64)
        ident = 16 * s_hi + s_lo + 8 * wks[g][None, :] + zi[None, :] * aks[g][:, None]
        assert np.array_equal(ident, I[g])
        brute = np.array([[sum(int(a[m, k]) * (int(w[n, k]) - int(zi[n]))
                               for k in range(g * gk, g * gk + ow.group_real(g, K, gk)))
                           for n in range(2)] for m in range(2)])
        assert np.array_equal(brute, I[g][:2, :2])


@needs_ref
@pytest.mark.parametrize("K,gk", MID_CASES)
@pytest.mark.parametrize("asym", [True, False])
def test_midgroup_gemm_matches_reference_cpp_bitwise(K, gk, asym):
    """gemm_midgroup_fp32 restates ReferenceMidGroupGemm's fp32 order exactly: the
    bf16 outputs are identical; scales taken from the wrong groups (a plausible
    indexing slip) are caught."""
    rng = np.random.default_rng(K * 3 + asym)
    M, N = 7, 40
    xb = ow.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    q, sc = ow.quant_act_midgroup(xb, gk)
    codes, ws, wz, _ = ow.quantize_weight_asym(rng.standard_normal((N, K)).astype(np.float32), gk)
    wz = wz if asym else None
    ours = ow.f32_to_bf16_bits(ow.gemm_midgroup_fp32(q, sc, codes, ws, wz, gk))
    ref = oref.midgroup_gemm(q, sc, codes, ws, gk, wz)
    assert np.array_equal(ours, ref)
    if ow.num_groups(K, gk) > 1:
        wrong = ow.f32_to_bf16_bits(ow.gemm_midgroup_fp32(q, sc, codes, ws[::-1].copy(), wz, gk))
        assert not np.array_equal(wrong, ref)



# --------------------------------------------------------------- RMSNorm
def test_rms_norm_matches_torch_formula():
    """The oracle against the reference's own torch expression on CPU
    (bench_decode_layer.py:36-38), with its fp32 summation order."""
    rng = np.random.default_rng(8)
    x = ow.f32_to_bf16_bits((rng.standard_normal((64, 5120)) * rng.uniform(0.1, 20, (64, 1))).astype(np.float32))
    w = ow.f32_to_bf16_bits(rng.uniform(0.5, 1.5, 5120).astype(np.float32))
    ours = ow.bf16_bits_to_f32(ow.rms_norm_bf16(x, w, 1e-6)).astype(np.float64)
    tx = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    tw = torch.from_numpy(w.view(np.int16)).view(torch.bfloat16)
    v = tx.float()
    ref = ((v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * tw).float().numpy()
    assert np.mean(ours == ref) > 0.999
    assert np.all(np.abs(ours - ref) <= ow.bf16_ulp(ref))


def test_rms_norm_matches_high_precision():
    """Small rows against exact rational mean and a 40-digit square root, each fp32
    step rounded as the formula prescribes; and the residual add exactly."""
    from decimal import Decimal, getcontext
    getcontext().prec = 40
    rng = np.random.default_rng(1)
    for _ in range(20):
        s = ow.f32_to_bf16_bits((rng.standard_normal(16) * 3).astype(np.float32))
        w = ow.f32_to_bf16_bits(rng.uniform(0.5, 1.5, 16).astype(np.float32))
        vs = [Fraction(float(v)) for v in ow.bf16_bits_to_f32(s)]
        ms = round_to_float(sum(v * v for v in vs) / 16, 24)
        t = round_to_float(ms + round_to_float(Fraction(1e-6), 24), 24)
        rd = Decimal(1) / (Decimal(t.numerator) / Decimal(t.denominator)).sqrt()
        r = round_to_float(Fraction(rd), 24)
        exp = []
        for v, wv in zip(vs, ow.bf16_bits_to_f32(w)):
            p = v * r
            h1 = (round_to_float(round_to_float(abs(p), 24), 8) if p else Fraction(0)) * (1 if p >= 0 else -1)
            q = h1 * Fraction(float(wv))
            exp.append(float((round_to_float(abs(q), 8) if q else Fraction(0)) * (1 if q >= 0 else -1)))
        got = ow.bf16_bits_to_f32(ow.rms_norm_bf16(s[None, :], w, 1e-6))[0]
        assert list(got) == exp
    # a half-ulp tie rounds to even, just above half rounds up, exact cancellation
    a = ow.f32_to_bf16_bits(np.array([1.0, 1.0, -2.5], np.float32))
    b = ow.f32_to_bf16_bits(np.array([2.0 ** -8, 3 * 2.0 ** -9, 2.5], np.float32))
    assert list(ow.bf16_bits_to_f32(ow.add_bf16(a, b))) == [1.0, 1.0078125, 0.0]
