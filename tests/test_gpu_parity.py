"""GPU parity: the HIP path against the CPU oracle, through torch.ops.npu.* (C ABI).

Bars (stated per test):
  * activation quant: int8 codes and bf16 scales byte-exact
  * per-group int32 partials (dumped by the production kernel): bit-exact
  * bf16 output: |y - y32| <= 1 bf16 ulp of the oracle's fp32 result y32 for every
    element, or, where the groups cancel, <= 1 bf16 ulp of the exact float64 value
    (see check_output); rel-L2 against the oracle's bf16 output <= 1e-3, and >= 99%
    of outputs equal
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from conftest import OUTPUT_CHECKS, bf16_bits_tensor, tensor_bf16_bits, tie_rows
from oracle import w4a8 as ow

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def make_problem(pkg, M, N, K, G, seed=0, scale_dtype="f16", codes="uniform"):
    synth = pkg.synth
    xb = synth.activations(M, K, seed)
    w = synth.weight_codes_uniform(N, K, seed + 1) if codes == "uniform" else \
        synth.weight_codes_clipped_normal(N, K, seed + 1)
    sb = synth.group_scales(N, ow.num_groups(K, G), seed + 2, scale_dtype)
    ws32 = synth.scale_bits_to_f32(sb, scale_dtype)
    tdt = torch.float16 if scale_dtype == "f16" else torch.bfloat16
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(tdt)
    return xb, w, ws32, w_scale


def run_hip(dev, xb, w, w_scale, N, K, G, partials=True):
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev), G)
    if partials:
        y, P = torch.ops.npu.w4a8_gemm_partials(a_q, a_s, w_tiles, s_tiles, N, K, G)
    else:
        y, P = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G), None
    torch.cuda.synchronize()
    return y, P, a_q, a_s


def assert_production_equals_dump(pkg, dev, a_q, a_s, w, w_scale, y_dump, N, K, G):
    """The plain GEMM (the production kernel variant, whose plan may differ from
    the partial dump's, e.g. 64-row prefill tiles) returns the dump call's output
    bit for bit."""
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev),
                                                 w_scale.to(dev), K, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_dump.view(torch.int16)), "production output differs from the dump's"


def check_output(y_bits: np.ndarray, y32: np.ndarray, tag: str, exact) -> None:
    """Output bars.

    max-abs (the north_star's): every |y - y32| <= 1 bf16 ulp of the oracle's fp32
    result y32; an output outside it (where the groups cancel, two fp32
    summation orders differ by more than an ulp of the small result) must lie
    within 1 bf16 ulp of the exact float64 value instead (``exact(rows, cols)``,
    the restatement of fakequant_lab/run_selftest.py:104-120).  How many outputs
    needed the float64 value is printed.
    rel-L2: between the bf16 outputs (ours vs the oracle's bf16(y32), which is
    what the reference's path returns, fakequant_lab/fake_linear.py:149) <= 1e-3,
    and >= 99% of them bit-equal.
    """
    fail, n_fb = ow.output_bar(y_bits, y32, exact)
    OUTPUT_CHECKS.append((tag, int(y32.size), n_fb))
    assert not fail.any(), f"{tag}: {int(fail.sum())} outputs outside 1 bf16 ulp of both the fp32 and float64 oracle"
    y = ow.bf16_bits_to_f32(y_bits).astype(np.float64)
    rb = ow.round_bf16(y32).astype(np.float64)
    rel = np.linalg.norm(y - rb) / max(np.linalg.norm(rb), 1e-30)
    assert rel <= 1e-3, f"{tag}: rel-L2 {rel}"
    assert np.mean(y == rb) > 0.99, f"{tag}: only {np.mean(y == rb):.4f} of outputs equal bf16(oracle)"
    assert np.linalg.norm(y32.astype(np.float64)) > 0, f"{tag}: vacuous reference"


def exact_sym(q_ref, s_ref, w, ws32, G):
    """float64 outputs (rows, cols) of the per-token symmetric path."""
    return lambda r, c: ow.gemm_f64(q_ref[r], s_ref[r], w[c], ws32[c], G)


def exact_mid(qp, a_scale_bits, codes, sc, zr, G):
    """float64 outputs (rows, cols) of the mid-group path (scale/zero bits [G, N], a_scale [G, >= M])."""
    return lambda r, c: ow.gemm_midgroup_f64(qp[r], a_scale_bits[:, r], codes[c], sc[:, c],
                                             None if zr is None else zr[:, c], G)


# ------------------------------------------------------------------ quant
@pytest.mark.parametrize("M", [1, 4, 7, 9, 16, 64, 128, 512, 1024])
@pytest.mark.parametrize("K", [5120, 27648])
def test_quant_byte_exact(pkg, dev, M, K):
    say(f"quant M={M} K={K}")
    xb = pkg.synth.activations(M, K, seed=M * 7 + K)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    assert np.array_equal(a_q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("K", [8, 1001, 4096, 40000])
def test_quant_byte_exact_odd_and_large_rows(pkg, dev, K):
    say(f"quant odd K={K}")
    xb = pkg.synth.activations(5, K, seed=K)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    assert np.array_equal(a_q.cpu().numpy(), q_ref)


def test_quant_ties_zero_rows_and_strided_input(dev):
    say("quant ties/zero/strided")
    xb = tie_rows(64, 512, seed=11)
    xb[5] = 0
    x = bf16_bits_tensor(xb).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    assert np.array_equal(a_q.cpu().numpy(), q_ref)
    # A row-strided view (ldx > K) goes through the same kernels.
    wide = torch.zeros((64, 640), dtype=torch.bfloat16, device=dev)
    wide[:, :512] = x
    a_q2, a_s2 = torch.ops.npu.w4a8_quant_pertoken(wide[:, :512])
    assert torch.equal(a_q2, a_q) and torch.equal(a_s2, a_s)


@pytest.mark.parametrize("K", [512, 27648])
def test_quant_tiny_and_boundary_scales(pkg, dev, K):
    """Rows whose scale is subnormal, at the 2^-125 edge of the reciprocal path,
    or whose elements are subnormal: byte-exact against the oracle's divide."""
    say(f"quant tiny scales K={K}")
    rng = np.random.default_rng(K)
    amaxes = [1e-30, 2.0 ** -118, 2.0 ** -118 * 0.99, 127 * 2.0 ** -125, 1e-37, 3e-39, 1.0, 3e4]
    rows = []
    for a in amaxes:
        v = rng.standard_normal(K).astype(np.float32)
        v *= np.float32(a) / np.abs(v).max()
        rows.append(ow.f32_to_bf16_bits(v))
    xb = np.stack(rows)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    assert np.array_equal(a_q.cpu().numpy(), q_ref)


def test_quant_empty(dev):
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(torch.empty((0, 256), dtype=torch.bfloat16, device=dev))
    assert a_q.shape == (0, 256) and a_s.shape == (0,)


# ------------------------------------------------------------------ repack layout
def repack_model(w_q_packed: np.ndarray, N: int, K: int, G: int) -> np.ndarray:
    """numpy model of the MFMA tile layout documented in csrc/repack.hip."""
    codes = ow.unpack_int4(w_q_packed)              # [N, kpad]
    kp = codes.shape[1]
    NB, KT = -(-N // 16), -(-kp // 128)
    full = np.zeros((NB * 16, KT * 128), np.int8)
    full[:N, :kp] = codes
    out = np.zeros((NB, KT, 64, 4, 4), np.uint8)   # [nb][kt][lane][dword][byte]
    for lane in range(64):
        col = np.arange(NB) * 16 + lane % 16
        for d in range(4):
            k0 = (d // 2) * 64 + (lane // 16) * 16 + (d % 2) * 8
            for j in range(4):
                lo = full[col][:, k0 + j::128][:, :KT] & 0xF
                hi = full[col][:, k0 + 4 + j::128][:, :KT] & 0xF
                out[:, :, lane, d, j] = (lo | (hi << 4)).astype(np.uint8)
    return out.reshape(-1)


@pytest.mark.parametrize("N,K,G", [(16, 128, 128), (100, 512, 64), (48, 1024, 256)])
def test_repack_layout(pkg, dev, N, K, G):
    say(f"repack N={N} K={K} G={G}")
    w = pkg.synth.weight_codes_uniform(N, K, 3)
    sb = pkg.synth.group_scales(N, K // G, 4, "bf16")
    w_q = ow.pack_grouped(w, G)
    ws = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.bfloat16)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(w_q).to(dev), ws.to(dev), K, G)
    assert np.array_equal(w_tiles.cpu().numpy(), repack_model(w_q, N, K, G))
    st = tensor_bf16_bits(s_tiles)
    NB = -(-N // 16)
    exp = np.zeros((NB * 16, K // G), np.uint16)
    exp[:N] = sb
    assert np.array_equal(st, exp.reshape(NB, 16, K // G).transpose(0, 2, 1))


# ------------------------------------------------------------------ GEMM
GEMM_CASES = [
    # (M, N, K, G, scale dtype)
    (1, 256, 1024, 128, "f16"),
    (4, 512, 2048, 64, "bf16"),
    (7, 100, 512, 256, "f16"),       # N not a multiple of 16
    (16, 5120, 5120, 128, "f16"),    # o_proj decode, C1
    (33, 1024, 4096, 512, "bf16"),
    (3, 200, 1536, 192, "bf16"),     # decode, groups ending on a tile's lower slab
    (9, 300, 1920, 320, "f16"),      # decode, 5 slabs per group: ends on either slab
    (2, 160, 2560, 640, "bf16"),     # decode, 10 slabs per group (not a power-of-two multiple of 128)
    (5, 96, 3072, 256, "f16"),       # decode, two tiles per group
    (64, 7168, 5120, 128, "f16"),    # qkv decode, M=64
    (12, 32768, 1024, 128, "bf16"),  # wide N past 8 rows: four column blocks per workgroup
    (40, 32768, 1024, 128, "f16"),   # wide N past 16 rows: activations shared through LDS
    (48, 32768, 1024, 64, "bf16"),   # the same, group stride 64
    (20, 33000, 1920, 320, "f16"),   # the same, groups ending on either slab, ragged column groups
    (64, 32768, 3072, 512, "bf16"),  # the same, groups of four tiles
    (20, 1000, 16384, 128, "f16"),   # narrow N, long K past 8 rows: K split over 16 workgroups, ragged N
    (40, 512, 16384, 320, "bf16"),   # the same, split on 5-tile group-aligned units
    (64, 256, 16384, 256, "f16"),    # the same, 64 rows, two tiles per group
    (9, 2048, 16384, 64, "bf16"),    # the same, one row tile, group stride 64
    (20, 16, 16400, 128, "bf16"),    # the same, one column block over 16 splits, a 16-element last group
    (11, 300, 20000, 1024, "f16"),   # the same, group 1024: 8-tile split units, a short last group
    (17, 336, 1536, 192, "f16"),     # two 16-row groups, the second with one row; 11 column groups
    (40, 1000, 2048, 64, "bf16"),    # three row groups, ragged N
    (50, 200, 3072, 320, "f16"),     # row groups with groups ending on either slab
    (65, 384, 1024, 128, "bf16"),    # first prefill-path M
    (128, 256, 1024, 1024, "f16"),
    (300, 1000, 2048, 128, "bf16"),  # ragged M and N tiles
    (130, 512, 1024, 64, "f16"),     # prefill, two groups per 128-K step
    (200, 300, 768, 192, "bf16"),    # prefill, groups ending mid-step, K % 128 == 64
    (96, 520, 2048, 256, "f16"),     # prefill, a group spans two steps
    (257, 264, 1024, 512, "bf16"),
    (3200, 2000, 384, 128, "bf16"),  # four-wave 128-row prefill tiles (400 of them), ragged N
    (6200, 1000, 448, 96, "f16"),    # the same, group 96 (stride 128, every group padded), ragged K
]


@pytest.mark.parametrize("M,N,K,G,sd", GEMM_CASES)
def test_gemm_partials_bit_exact_and_output(pkg, dev, M, N, K, G, sd):
    say(f"gemm M={M} N={N} K={K} G={G} scales={sd}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + N, scale_dtype=sd)
    y, P, a_q, a_s = run_hip(dev, xb, w, w_scale, N, K, G)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(a_q.cpu().numpy(), ow.pad_groups(q_ref, G))
    P_ref = ow.group_partials(q_ref, w, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G, P_ref)
    check_output(tensor_bf16_bits(y), y32, f"M{M} N{N} K{K} G{G}", exact_sym(q_ref, s_ref, w, ws32, G))
    assert_production_equals_dump(pkg, dev, a_q, a_s, w, w_scale, y, N, K, G)


# The reference's ragged-K cases (int4_cube_lab/host/ragged_layout_test.cpp:195-223:
# TP shards of K at group 1024, short last groups down to one element, odd K,
# groups that are not multiples of 64) plus one ragged case per group mode of
# each kernel, at decode and prefill M.
RAGGED_CASES = [
    # (M, N, K, G, scale dtype)
    (3, 128, 640, 1024, "bf16"),      # 5120 / 8: one short group
    (3, 128, 3456, 1024, "bf16"),     # 27648 / 8: a short last group of 384
    (1, 256, 13824, 1024, "f16"),     # 27648 / 2
    (3, 128, 1057, 1024, "bf16"),
    (3, 128, 1279, 1024, "f16"),
    (3, 128, 1025, 1024, "bf16"),
    (3, 128, 33, 1024, "bf16"),
    (3, 128, 1, 1024, "bf16"),
    (3, 128, 65, 1024, "f16"),
    (3, 128, 63, 1024, "bf16"),
    (3, 128, 2049, 1024, "bf16"),
    (2, 128, 1023, 1024, "f16"),
    (2, 128, 35, 1024, "bf16"),
    (3, 128, 100, 33, "bf16"),        # group stride 64, every group padded
    (3, 128, 1057, 96, "f16"),        # group stride 128
    (17, 256, 777, 1024, "bf16"),     # ragged M and a single short group
    (4, 200, 5000, 128, "f16"),       # stride 128, last group of 8 in a padding tile
    (5, 96, 900, 256, "bf16"),        # stride 256: last group ends on a lower slab
    (3, 200, 232, 192, "bf16"),       # stride 192: two groups end in one tile
    (1, 64, 2000, 320, "f16"),        # stride 320 with a K split across waves
    (100, 300, 1057, 1024, "bf16"),   # prefill
    (130, 256, 100, 33, "f16"),       # prefill, stride 64
    (96, 200, 5000, 128, "bf16"),     # prefill, stride 128, last group on a lower half
    (200, 136, 232, 192, "f16"),      # prefill, stride 192
    (80, 128, 3456, 1024, "bf16"),    # prefill, TP shard
]


@pytest.mark.parametrize("M,N,K,G,sd", RAGGED_CASES)
def test_gemm_ragged_k(pkg, dev, M, N, K, G, sd):
    say(f"gemm ragged M={M} N={N} K={K} G={G} scales={sd}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=K + G, scale_dtype=sd)
    y, P, a_q, a_s = run_hip(dev, xb, w, w_scale, N, K, G)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(a_q.cpu().numpy(), ow.pad_groups(q_ref, G)), "padded activation layout"
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    P_ref = ow.group_partials(q_ref, w, G, exact_int64=True)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G, P_ref)
    check_output(tensor_bf16_bits(y), y32, f"ragged M{M} N{N} K{K} G{G}", exact_sym(q_ref, s_ref, w, ws32, G))
    assert_production_equals_dump(pkg, dev, a_q, a_s, w, w_scale, y, N, K, G)


@pytest.mark.parametrize("K,G", [(1057, 1024), (100, 33), (1057, 96), (3456, 1024), (5000, 128), (35, 1024),
                                 (1, 1024), (1001, 100), (20000, 1000)])
def test_quant_padded_layout_byte_exact(pkg, dev, K, G):
    """Vector path (K % 8 == 0 and group % 8 == 0) and scalar path alike write
    the padded group layout with zeroed padding."""
    say(f"quant padded K={K} G={G}")
    xb = pkg.synth.activations(6, K, seed=K * 3 + G)
    x = bf16_bits_tensor(xb).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert a_q.shape == (6, ow.kpad(K, G))
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    assert np.array_equal(a_q.cpu().numpy(), ow.pad_groups(q_ref, G))


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_gemm_qwq_decode_shapes(pkg, dev, proj, M):
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"qwq decode {proj} M={M}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, 128, seed=M)
    y, _, _, _ = run_hip(dev, xb, w, w_scale, N, K, 128, partials=False)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, 128)
    check_output(tensor_bf16_bits(y), y32, f"{proj} M{M}", exact_sym(q_ref, s_ref, w, ws32, 128))


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
def test_gemm_qwq_prefill_column_sample(pkg, dev, proj):
    """M=1024 at full shape; the oracle is evaluated on 192 sampled columns
    (output columns are independent, so a column sample is exact for them)."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    M = 1024
    say(f"qwq prefill {proj} M={M}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, 128, seed=3)
    y, _, _, _ = run_hip(dev, xb, w, w_scale, N, K, 128, partials=False)
    cols = np.sort(np.random.default_rng(0).choice(N, 192, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], 128)
    check_output(tensor_bf16_bits(y)[:, cols], y32, f"{proj} M{M}", exact_sym(q_ref, s_ref, w[cols], ws32[cols], 128))


@pytest.mark.parametrize("M", [4096, 16384, 65536])
@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
def test_gemm_qwq_prefill_large_sample(pkg, dev, proj, M):
    """configs[2]'s larger batches, M=4096 and 16384, and configs[4]'s prefill at
    concurrency 64 (64 prompts of 1024 tokens: M=65536 through every linear), at full
    shape and group 128; the
    oracle runs on 96 sampled rows x 160 sampled columns (per-token rows and output
    columns are independent), first and last row and column included."""
    synth = pkg.synth
    K, N = synth.QWQ_SHAPES[proj]
    G = 128
    say(f"qwq prefill {proj} M={M} (sampled check)")
    x = synth.activations_device(M, K, seed=11 + M, device=dev)
    w = synth.weight_codes_uniform(N, K, 12)
    sb = synth.group_scales(N, ow.num_groups(K, G), 13, "f16")
    ws32 = synth.scale_bits_to_f32(sb, "f16")
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.float16)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev),
                                                 w_scale.to(dev), K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    rows = np.sort(np.concatenate([rng.choice(M, 94, replace=False), [0, M - 1]]))
    cols = np.sort(np.concatenate([rng.choice(N, 158, replace=False), [0, N - 1]]))
    rt = torch.from_numpy(rows).to(dev)
    xb = tensor_bf16_bits(x.index_select(0, rt))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(tensor_bf16_bits(a_s.index_select(0, rt)), s_ref)
    assert np.array_equal(a_q.index_select(0, rt).cpu().numpy(), q_ref)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
    got = tensor_bf16_bits(y.index_select(0, rt))[:, cols]
    check_output(got, y32, f"{proj} M{M} sample", exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


def test_gemm_row_chunks_large_m(pkg, dev):
    """A call whose activations exceed 32-bit offsets (K=27648 at 80000 rows) runs as
    balanced row chunks; rows on both sides of every chunk boundary, the first and
    the last match the oracle."""
    synth = pkg.synth
    M, N, K, G = 80000, 256, 27648, 128
    lib = pkg._abi.lib()
    chunk = lib.w4a8_gemm_row_chunk(M, K)
    assert 0 < chunk < M
    n = -(-M // chunk)
    bounds = [(M * i) // n for i in range(n + 1)]
    say(f"row chunks M={M} K={K}: {n} launches, boundaries {bounds}")
    x = synth.activations_device(M, K, seed=21, device=dev)
    w = synth.weight_codes_uniform(N, K, 22)
    sb = synth.group_scales(N, ow.num_groups(K, G), 23, "bf16")
    ws32 = synth.scale_bits_to_f32(sb, "bf16")
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.bfloat16)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev),
                                                 w_scale.to(dev), K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    rows = sorted({0, M - 1, *[b + d for b in bounds[1:-1] for d in (-2, -1, 0, 1)]})
    rt = torch.tensor(rows, device=dev)
    xb = tensor_bf16_bits(x.index_select(0, rt))
    del x
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(a_q.index_select(0, rt).cpu().numpy(), q_ref)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    check_output(tensor_bf16_bits(y.index_select(0, rt)), y32, "row chunks", exact_sym(q_ref, s_ref, w, ws32, G))


# Per-channel weights (one group spanning K, the reference's per-channel variant,
# int4_cube_lab/kernels/perchannel_w4a8_gemm.inc): the K split falls on any tile and
# the waves' / workgroups' int32 sums are added before the one fold.
PERCHANNEL_CASES = [
    # (M, N, K, scale dtype)
    (1, 512, 5120, "f16"),        # fused single-row path's kernel plan, ten waves
    (4, 320, 27648, "bf16"),      # eight waves over 216 tiles
    (16, 256, 27648, "f16"),      # K split over workgroups, int32 sums reduced by the second kernel
    (40, 1000, 16384, "bf16"),    # the 32-row split layout
    (64, 200, 27648, "f16"),      # the 64-row split layout
    (24, 640, 5120, "bf16"),      # row groups
    (12, 33024, 1024, "f16"),     # wide N, one split
    (3, 136, 5000, "bf16"),       # K % 128 != 0: a padding slab in the last tile
    (300, 512, 5120, "f16"),      # prefill
    (130, 264, 27648, "bf16"),    # prefill, long K (|16P| may exceed 2^24: fp32 rounding of the one fold)
]


@pytest.mark.parametrize("M,N,K,sd", PERCHANNEL_CASES)
def test_gemm_perchannel_partials_and_output(pkg, dev, M, N, K, sd):
    G = K
    say(f"per-channel M={M} N={N} K={K}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + N + 1, scale_dtype=sd)
    y, P, a_q, a_s = run_hip(dev, xb, w, w_scale, N, K, G)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    P_ref = ow.group_partials(q_ref, w, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    y2, _, _, _ = run_hip(dev, xb, w, w_scale, N, K, G, partials=False)
    assert torch.equal(y, y2), "the partial dump changed the output"
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G, P_ref)
    check_output(tensor_bf16_bits(y), y32, f"per-channel M{M} N{N} K{K}", exact_sym(q_ref, s_ref, w, ws32, G))


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
@pytest.mark.parametrize("M", [1, 16, 64, 1024])
def test_gemm_qwq_perchannel(pkg, dev, proj, M):
    """The QwQ-32B projections with per-channel scales (G = K), decode and prefill
    rows, through w4a8_linear (the fused single-row launch at M=1); sampled columns."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"qwq per-channel {proj} M={M}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, K, seed=M + 3)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, K)).to(dev),
                                                 w_scale.to(dev), K, K)
    y = torch.ops.npu.w4a8_linear(bf16_bits_tensor(xb).to(dev), w_tiles, s_tiles, N, K, K)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(M).choice(N, 256, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], K)
    check_output(tensor_bf16_bits(y)[:, cols], y32, f"per-channel {proj} M{M}",
                 exact_sym(q_ref, s_ref, w[cols], ws32[cols], K))


# One GPU's TP=4 slice of each QwQ-32B projection: column-parallel qkv/gate_up split N,
# row-parallel o/down split K ((K, N) per projection; MGCKPT/P7_LOWDIM_KERNEL.md:13-21).
TP4_SHAPES = {"qkv_proj": (5120, 1792), "o_proj": (1280, 5120), "gate_up_proj": (5120, 13824),
              "down_proj": (6912, 5120)}


@pytest.mark.parametrize("proj", sorted(TP4_SHAPES))
@pytest.mark.parametrize("M", [1, 16, 64, 1024])
def test_linear_tp4_shard_shapes(pkg, dev, proj, M):
    """The TP=4 shard shapes at group 128 through w4a8_linear (quant + GEMM; one fused
    launch at M=1), sampled columns against the oracle; the plain GEMM on the same
    quantised rows returns the same bits."""
    K, N = TP4_SHAPES[proj]
    G = 128
    say(f"tp4 shard {proj} M={M} N={N} K={K}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + K + N)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev),
                                                 w_scale.to(dev), K, G)
    x = bf16_bits_tensor(xb).to(dev)
    y = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y2 = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "linear differs from quant + gemm"
    cols = np.sort(np.random.default_rng(M + 5).choice(N, 128, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(a_q.cpu().numpy(), q_ref) and np.array_equal(tensor_bf16_bits(a_s), s_ref)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
    check_output(tensor_bf16_bits(y)[:, cols], y32, f"tp4 {proj} M{M}", exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


def test_gemm_perchannel_every_decode_row_count(pkg, dev):
    """Every M from 1 to 64 with per-channel scales on a narrow N with long K (the K
    split over workgroups with int32 sums from 9 rows on) and a narrow N with short K."""
    cols_rng = np.random.default_rng(19)
    for N, K in ((1000, 16384), (640, 5120)):
        xb_all, w, ws32, w_scale = make_problem(pkg, 64, N, K, K, seed=N + 7)
        w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, K)).to(dev),
                                                     w_scale.to(dev), K, K)
        cols = np.sort(cols_rng.choice(N, 48, replace=False))
        for M in range(1, 65):
            say(f"per-channel rows M={M} N={N} K={K}")
            xb = xb_all[:M]
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev), K)
            y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, K)
            torch.cuda.synchronize()
            q_ref, s_ref = ow.quant_act_per_token(xb)
            y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], K)
            check_output(tensor_bf16_bits(y)[:, cols], y32, f"per-channel M{M} N{N} K{K}",
                         exact_sym(q_ref, s_ref, w[cols], ws32[cols], K))


def test_gemm_every_decode_row_count(pkg, dev):
    """Every M from 1 to 64 on a wide (2048 column groups) and a narrow N, and on a
    narrow N with long K: each picks a built kernel variant (a missing one is a launch
    error) and matches the oracle on a column sample."""
    G = 128
    cols_rng = np.random.default_rng(9)
    for N, K in ((32768, 512), (1000, 512), (1000, 16384)):
        xb_all, w, ws32, w_scale = make_problem(pkg, 64, N, K, G, seed=N)
        w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
        w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
        cols = np.sort(cols_rng.choice(N, 48, replace=False))
        for M in range(1, 65):
            say(f"decode rows M={M} N={N} K={K}")
            xb = xb_all[:M]
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev), G)
            y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
            torch.cuda.synchronize()
            q_ref, s_ref = ow.quant_act_per_token(xb)
            y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
            check_output(tensor_bf16_bits(y)[:, cols], y32, f"M{M} N{N} K{K}", exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


@pytest.mark.parametrize("M,N,K", [(16, 5120, 5120), (16, 5120, 27648), (48, 5120, 27648), (64, 5120, 27648),
                                   (4, 5120, 27648), (16, 55296, 5120), (64, 55296, 5120), (1024, 7168, 5120)])
def test_gemm_deterministic_and_stress(pkg, dev, M, N, K):
    """Repeated launches give identical bits (the reference's --stress relaunch check,
    int4_cube_lab/host/mg_harness.h:307-334): the decode kernel's in-workgroup K split,
    the K split over workgroups with its reduce kernel and workspace (down_proj M=16),
    the 64-row prefill tile split along K with the same reduce (down_proj M=48 and 64),
    the staged activations (M=4), the wide kernel's LDS-shared activations (gate_up
    M=16 and 64), and a prefill shape; every relaunch is compared, and the first against
    the oracle."""
    G = 128
    say(f"gemm stress M={M} N={N} K={K}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=5)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev))
    first = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    for i in range(30):
        y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
        junk = torch.full((1 << 20,), i, dtype=torch.int32, device=dev)   # other work between relaunches
        assert torch.equal(y, first), f"relaunch {i} differs"
        del junk
    cols = np.sort(np.random.default_rng(1).choice(N, 128, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
    check_output(tensor_bf16_bits(first)[:, cols], y32, f"stress M{M} N{N} K{K}",
                 exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
def test_decode_plans_relaunch_deterministic(pkg, dev, proj):
    """Every decode plan of a QwQ-32B projection (1 to 64 rows: fused single-row linear,
    staged activations, per-tile rings, row groups, the wide kernel with and without its K
    split, the split 64-row prefill tile, the SwiGLU epilogue on gate_up) relaunched 20
    times with other work between: identical bits every time (the reference's --stress
    check, int4_cube_lab/host/mg_harness.h:307-334, over all plans)."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    G = 128
    xb_all, w, ws32, w_scale = make_problem(pkg, 64, N, K, G, seed=11)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    x_all = bf16_bits_tensor(xb_all).to(dev)
    for M in (1, 2, 4, 8, 12, 16, 24, 32, 48, 64):
        say(f"relaunch {proj} M={M}")
        x = x_all[:M].contiguous()
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
        runs = [lambda: torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G),
                lambda: torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)]
        if proj == "gate_up_proj":
            runs.append(lambda: torch.ops.npu.w4a8_gemm_swiglu(a_q, a_s, w_tiles, s_tiles, N, K, G))
        for fn in runs:
            first = fn()
            for i in range(20):
                y = fn()
                junk = torch.full((1 << 18,), i, dtype=torch.int32, device=dev)
                assert torch.equal(y, first), f"{proj} M={M}: relaunch {i} differs"
                del junk
        torch.cuda.synchronize()


@pytest.mark.parametrize("N,K", [(7168, 5120), (5120, 27648)])
def test_linear_fused_deterministic_and_stress(pkg, dev, N, K):
    """The fused single-row linear (quant prologue in every workgroup: every wave reading the
    whole row at K=5120, the waves' absmax meeting in LDS behind a barrier at K=27648)
    relaunched 30 times with other work between: identical output, a_q and a_scale bits,
    the first equal to quant + GEMM and within the oracle bar."""
    G = 128
    say(f"fused linear stress N={N} K={K}")
    xb, w, ws32, w_scale = make_problem(pkg, 1, N, K, G, seed=6)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    x = bf16_bits_tensor(xb).to(dev)
    lib = pkg._abi.lib()
    assert lib.w4a8_linear_fused(x.data_ptr(), K, 1, N, K, G) == 1, "this shape should take the fused launch"
    first = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
    for i in range(30):
        y = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
        junk = torch.full((1 << 20,), i, dtype=torch.int32, device=dev)
        assert torch.equal(y, first), f"relaunch {i} differs"
        del junk
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
    pair = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    assert torch.equal(first, pair), "fused linear differs from quant + GEMM"
    cols = np.sort(np.random.default_rng(2).choice(N, 128, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
    check_output(tensor_bf16_bits(first)[:, cols], y32, f"fused stress N{N} K{K}",
                 exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


@pytest.mark.parametrize("M,N,K", [(64, 5120, 27648), (48, 5120, 27648), (40, 1000, 16384)])
def test_gemm_split_prefill_tile_equals_fallback_plan(pkg, dev, M, N, K):
    """Narrow N with long K past 32 rows runs one 64-row tile of the prefill kernel
    split along K (gemm_prefill_cols_kernel + wide_reduce_kernel).  The partial dump
    runs that shape on the fallback wide plan instead, whose K split has the same
    boundaries and the same per-group fold order: the two outputs must be equal bit
    for bit, the dumped int32 partials must equal the oracle's exactly, and the
    output meets the bars."""
    G = 128
    say(f"split prefill tile vs fallback M={M} N={N} K={K}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + 31)
    y_fb, P, a_q, a_s = run_hip(dev, xb, w, w_scale, N, K, G, partials=True)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev),
                                                 w_scale.to(dev), K, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_fb.view(torch.int16)), "split prefill tile differs from the wide plan"
    cols = np.sort(np.random.default_rng(M).choice(N, 96, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    Pn = P.cpu().numpy()
    assert np.array_equal(Pn[:, :, cols], ow.group_partials(q_ref, w[cols], G)), "dumped partials differ"
    y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
    check_output(tensor_bf16_bits(y)[:, cols], y32, f"split prefill tile M{M} N{N} K{K}",
                 exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


def test_gemm_m0_and_errors(dev):
    say("gemm edge/errors")
    N, K, G = 64, 256, 128
    w_q = torch.zeros((N, K // 2), dtype=torch.int8, device=dev)
    ws = torch.ones((K // G, N), dtype=torch.float16, device=dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, ws, K, G)
    a_q = torch.zeros((0, K), dtype=torch.int8, device=dev)
    a_s = torch.zeros((0,), dtype=torch.bfloat16, device=dev)
    assert torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G).shape == (0, N)
    with pytest.raises(RuntimeError, match="a_q"):
        torch.ops.npu.w4a8_gemm(a_q.float(), a_s, w_tiles, s_tiles, N, K, G)
    with pytest.raises(RuntimeError, match="kpad"):
        torch.ops.npu.w4a8_repack(w_q[:, :64], ws, K, G)
    with pytest.raises(RuntimeError, match="padded group layout"):
        torch.ops.npu.w4a8_gemm(torch.zeros((2, 300), dtype=torch.int8, device=dev), a_s[:0].new_zeros(2),
                                *torch.ops.npu.w4a8_repack(torch.zeros((N, 160), dtype=torch.int8, device=dev),
                                                           torch.ones((3, N), dtype=torch.float16, device=dev),
                                                           300, 128), N, 300, 128)


def test_w4a8_linear_module(pkg, dev):
    """The caller layer (apply semantics: reshape, quant, gemm, bias, reshape)."""
    say("W4A8Linear")
    K, N, G = 1024, 384, 128
    torch.manual_seed(0)
    lin = torch.nn.Linear(K, N, bias=True, dtype=torch.bfloat16)
    m = pkg.W4A8Linear.from_float(lin.to(dev), group=G)
    x = torch.randn(2, 3, K, dtype=torch.bfloat16)
    y = m(x.to(dev))
    torch.cuda.synchronize()
    assert y.shape == (2, 3, N) and y.dtype == torch.bfloat16
    codes, sc = ow.quantize_weight_sym(lin.weight.detach().float().cpu().numpy(), G)
    xb = tensor_bf16_bits(x.reshape(-1, K))
    _, y32, _, _, _ = ow.linear_bf16(xb, codes, ow.bf16_bits_to_f32(sc), G)
    # bias added in bf16 after the GEMM (npu_ops/python/midgroup_quant.py:175-176)
    y_ref = (torch.from_numpy(ow.bf16_bits_to_f32(ow.f32_to_bf16_bits(y32))).to(torch.bfloat16)
             + lin.bias.detach().cpu()).float().numpy()
    got = y.reshape(-1, N).float().cpu().numpy()
    assert np.max(np.abs(got - y_ref) - 2 * ow.bf16_ulp(y_ref)) <= 0


# w4a8_linear: quant + GEMM, fused into one kernel for small batches on narrow N.
LINEAR_CASES = [
    # (M, N, K, G, scale dtype, note)
    (1, 7168, 5120, 128, "f16", "fused: qkv"),
    (4, 5120, 5120, 128, "bf16", "two-kernel: o, four rows"),
    (1, 5120, 5120, 128, "bf16", "fused: o"),
    (2, 1024, 4096, 128, "bf16", "two-kernel: two rows"),
    (1, 5120, 27648, 128, "f16", "fused: down, one row (long K, eight waves of 27 tiles)"),
    (1, 5120, 13824, 128, "f16", "fused: half of down's K (twelve waves)"),
    (2, 5120, 27648, 128, "f16", "two-kernel: down, two rows"),
    (1, 640, 4096, 64, "bf16", "fused: group stride 64"),
    (1, 320, 6144, 512, "f16", "fused: groups of 4 tiles"),
    (1, 480, 3200, 320, "bf16", "fused: groups ending on either slab"),
    (1, 96, 1024, 1024, "f16", "fused: one group, one column group"),
    (5, 512, 2048, 128, "f16", "two-kernel: five rows"),
    (1, 55296, 1024, 128, "bf16", "fused: wide N (two waves per column group)"),
    (1, 55296, 5120, 128, "f16", "fused: gate_up"),
    (3, 256, 1057, 1024, "f16", "two-kernel: ragged K"),
]


def run_linear_abi(pkg, dev, x, w_tiles, s_tiles, N, K, G):
    """w4a8_linear through the C ABI: (y, a_q, a_scale)."""
    M = x.shape[0]
    width = ow.kpad(K, G)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    a_q = torch.full((M, width), 99, dtype=torch.int8, device=dev)
    a_s = torch.empty((M,), dtype=torch.bfloat16, device=dev)
    lib = pkg._abi.lib()
    st = lib.w4a8_linear(x.data_ptr(), x.stride(0), w_tiles.data_ptr(), s_tiles.data_ptr(),
                         1 if s_tiles.dtype == torch.bfloat16 else 0, y.data_ptr(), N, a_q.data_ptr(), width,
                         a_s.data_ptr(), M, N, K, G, None, 0, torch.cuda.current_stream(dev).cuda_stream)
    pkg._abi.check(st, "w4a8_linear")
    torch.cuda.synchronize()
    return y, a_q, a_s


@pytest.mark.parametrize("M,N,K,G,sd,note", LINEAR_CASES)
def test_linear_equals_quant_then_gemm(pkg, dev, M, N, K, G, sd, note):
    """w4a8_linear == w4a8_quant_act + w4a8_gemm bit for bit (y, a_q, a_scale), and y
    within the output bar of the oracle."""
    say(f"linear M={M} N={N} K={K} G={G} ({note})")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M * 31 + K, scale_dtype=sd)
    x = bf16_bits_tensor(xb).to(dev)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    fused = pkg._abi.lib().w4a8_linear_fused(x.data_ptr(), x.stride(0), M, N, K, G)
    assert fused == (1 if note.startswith("fused") else 0), f"path {fused} for '{note}'"
    y, a_q, a_s = run_linear_abi(pkg, dev, x, w_tiles, s_tiles, N, K, G)
    a_q2, a_s2 = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y2 = torch.ops.npu.w4a8_gemm(a_q2, a_s2, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert torch.equal(a_q, a_q2), "quantised activations differ"
    assert np.array_equal(tensor_bf16_bits(a_s), tensor_bf16_bits(a_s2))
    assert np.array_equal(tensor_bf16_bits(y), tensor_bf16_bits(y2)), "y differs from quant + gemm"
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    check_output(tensor_bf16_bits(y), y32, f"linear {note}", exact_sym(q_ref, s_ref, w, ws32, G))
    # the torch op: same result
    y3 = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert np.array_equal(tensor_bf16_bits(y3), tensor_bf16_bits(y))


def random_shapes(seed: int, n: int, max_mnk: float = 3e8, max_gmn: float = 1.2e7):
    """n seeded random (M, N, K, group, scale dtype) draws spread over the plans:
    M mostly decode-sized with a tail into the prefill tiles, N and K anywhere
    from 1 up (N not a multiple of 16, K not a multiple of the group), the group
    half the time a common stride and otherwise any value up to past K (one short
    group).  N and K are drawn under caps that keep the oracle to a few seconds
    (M*N*K <= max_mnk, groups*M*N <= max_gmn)."""
    rng = np.random.default_rng(seed)
    strides = [32, 64, 96, 128, 192, 256, 320, 512, 640, 1024]
    out = []
    while len(out) < n:
        u = rng.random()
        M = int(rng.integers(1, 17)) if u < 0.5 else int(rng.integers(17, 97)) if u < 0.8 else \
            int(rng.integers(97, 700))
        N = int(rng.integers(1, min(4096, int(max_mnk / (M * 64))) + 1))
        K = int(rng.integers(1, min(6000, int(max_mnk / (M * N))) + 1))
        G = int(rng.choice(strides)) if rng.random() < 0.5 else int(rng.integers(1, K + 300))
        if ow.num_groups(K, G) * M * N > max_gmn:
            continue
        out.append((M, N, K, G, "f16" if rng.random() < 0.5 else "bf16"))
    return out


# W4A8_RANDOM_SCALE multiplies the number of random draws (a longer campaign than the
# default suite runs; the draws of the default count are its first ones)
RANDOM_SCALE = max(1, int(os.environ.get("W4A8_RANDOM_SCALE", "1")))


@pytest.mark.parametrize("M,N,K,G,sd", random_shapes(20261202, 64 * RANDOM_SCALE))
def test_gemm_random_shapes(pkg, dev, M, N, K, G, sd):
    """Seeded random shapes through the GEMM: partials bit-exact, padded a_q and a_scale
    byte-exact, output within the bars, the production launch equal to the dump."""
    say(f"gemm random M={M} N={N} K={K} G={G} scales={sd}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M * 7 + N + K, scale_dtype=sd)
    y, P, a_q, a_s = run_hip(dev, xb, w, w_scale, N, K, G)
    q_ref, s_ref = ow.quant_act_per_token(xb)
    assert np.array_equal(a_q.cpu().numpy(), ow.pad_groups(q_ref, G)), "padded activation layout"
    assert np.array_equal(tensor_bf16_bits(a_s), s_ref)
    P_ref = ow.group_partials(q_ref, w, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G, P_ref)
    check_output(tensor_bf16_bits(y), y32, f"random M{M} N{N} K{K} G{G}", exact_sym(q_ref, s_ref, w, ws32, G))
    assert_production_equals_dump(pkg, dev, a_q, a_s, w, w_scale, y, N, K, G)


@pytest.mark.parametrize("M,N,K,G,sd", [(int(m) % 4 + 1, n, k, g, sd)
                                        for m, n, k, g, sd in random_shapes(77, 24 * RANDOM_SCALE)])
def test_linear_random_shapes(pkg, dev, M, N, K, G, sd):
    """Seeded random shapes through w4a8_linear at one to four rows (the fused launch
    where it applies): equal to quant + GEMM bit for bit, and within the bars."""
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + 3 * K, scale_dtype=sd)
    x = bf16_bits_tensor(xb).to(dev)
    fused = pkg._abi.lib().w4a8_linear_fused(x.data_ptr(), x.stride(0), M, N, K, G)
    say(f"linear random M={M} N={N} K={K} G={G} scales={sd} fused={fused}")
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    y, a_q, a_s = run_linear_abi(pkg, dev, x, w_tiles, s_tiles, N, K, G)
    a_q2, a_s2 = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y2 = torch.ops.npu.w4a8_gemm(a_q2, a_s2, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    assert torch.equal(a_q, a_q2), "quantised activations differ"
    assert np.array_equal(tensor_bf16_bits(a_s), tensor_bf16_bits(a_s2))
    assert np.array_equal(tensor_bf16_bits(y), tensor_bf16_bits(y2)), "y differs from quant + gemm"
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    check_output(tensor_bf16_bits(y), y32, f"linear random M{M} N{N} K{K} G{G}",
                 exact_sym(q_ref, s_ref, w, ws32, G))


def test_linear_unaligned_and_strided_input(pkg, dev):
    """x rows not 16-byte aligned or ldx % 8 != 0 take the two-kernel path; a row-strided
    aligned x takes the fused one; the results are the same."""
    say("linear strided / unaligned x")
    M, N, K, G = 1, 1024, 2048, 128
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=5)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    x = bf16_bits_tensor(xb).to(dev)
    y_ref, _, _ = run_linear_abi(pkg, dev, x, w_tiles, s_tiles, N, K, G)
    for off, ld, fused in ((0, K + 64, 1), (1, K + 64, 0), (0, K + 4, 0)):
        big = torch.zeros((M, ld + 8), dtype=torch.bfloat16, device=dev)
        big[:, off:off + K] = x
        xv = big[:, off:off + K]
        assert pkg._abi.lib().w4a8_linear_fused(xv.data_ptr(), xv.stride(0), M, N, K, G) == fused
        y, _, _ = run_linear_abi(pkg, dev, xv, w_tiles, s_tiles, N, K, G)
        assert np.array_equal(tensor_bf16_bits(y), tensor_bf16_bits(y_ref)), (off, ld)


def test_vllm_plugin_methods_apply(pkg, dev):
    """Both quant methods end to end -- create_weights, load the checkpoint tensors,
    process_weights_after_loading, apply -- bit-equal to the modules they mirror."""
    say("vllm plugin methods")
    vp = pkg.vllm_plugin
    K, N = 1600, 384
    torch.manual_seed(3)
    w = (torch.randn(N, K) * 0.05).to(torch.bfloat16)
    x = torch.randn(2, 3, K, dtype=torch.bfloat16).to(dev)
    bias = (torch.randn(N) * 0.1).to(torch.bfloat16).to(dev)

    # per-token, group 64 (an unpadded layout), fp16 scales
    G = 64
    w_q, w_scale = pkg.packing.quantize_weight(w, G, torch.float16)
    layer = torch.nn.Module()
    m = vp.PerTokenW4A8Config(group_size=G, scale_dtype="float16").get_quant_method(layer, "l.0.o_proj")
    m.create_weights(layer, K, [N], K, N, torch.bfloat16)
    with torch.no_grad():
        layer.weight_packed.copy_(w_q)
        layer.weight_scale.copy_(w_scale.t())
    layer.to(dev)
    m.process_weights_after_loading(layer)
    y = m.apply(layer, x, bias)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q.to(dev), w_scale.to(dev), K, G)
    y_ref = pkg.linear(x, w_tiles, s_tiles, N, G, bias)
    torch.cuda.synchronize()
    assert y.shape == (2, 3, N)
    assert np.array_equal(tensor_bf16_bits(y.reshape(-1, N)), tensor_bf16_bits(y_ref.reshape(-1, N)))

    # mid-group, the reference's group 1024 with a short last group (1600 = 1024 + 576)
    G = 1024
    wq, ws, wk, wz = pkg.packing.quantize_weight_asym(w, G)     # scales [G, N]
    layer = torch.nn.Module()
    m = vp.MidGroupW4A8Config(group_size=G).get_quant_method(layer, "l.0.down_proj")
    m.create_weights(layer, K, [N], K, N, torch.bfloat16)
    with torch.no_grad():
        layer.weight_packed.copy_(wq)
        layer.weight_scale.copy_(ws.t())
        layer.weight_zero.copy_(wz.t())
        layer.weight_ksum.copy_(wk.t())
    layer.to(dev)
    m.process_weights_after_loading(layer)
    y = m.apply(layer, x, bias)
    y_ref = pkg.midgroup_linear(x, wq.to(dev), ws.to(dev), wk.to(dev), wz.to(dev), G) + bias
    torch.cuda.synchronize()
    assert np.array_equal(tensor_bf16_bits(y.reshape(-1, N)), tensor_bf16_bits(y_ref.reshape(-1, N)))


def test_workspace_reuse_across_shapes(pkg, dev):
    """Consecutive calls of different shapes, some splitting K over workgroups
    (fp32 sums in the stream's one workspace, which grows between them), each
    match the oracle: no call reads what an earlier one left there."""
    cases = [(16, 256, 4096, 128), (1, 32768, 1024, 128), (8, 1024, 8192, 256), (1, 32768, 1024, 128),
             (24, 1000, 16384, 128), (12, 512, 16384, 128), (24, 1000, 16384, 128)]
    for i, (M, N, K, G) in enumerate(cases):
        say(f"workspace reuse step {i}: M={M} N={N} K={K} G={G}")
        xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=40 + i)
        y, _, _, _ = run_hip(dev, xb, w, w_scale, N, K, G, partials=False)
        q_ref, s_ref = ow.quant_act_per_token(xb)
        y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
        check_output(tensor_bf16_bits(y), y32, f"reuse step {i}", exact_sym(q_ref, s_ref, w, ws32, G))


def test_split_k_gemm_in_a_graph(pkg, dev):
    """A call that splits K over workgroups (two kernels and a workspace) captured in a
    HIP graph: every replay, with eager GEMMs of other shapes on the same stream in
    between, equals the eager result bit for bit; so does a graph of w4a8_linear."""
    M, N, K, G = 24, 1000, 16384, 128
    say(f"split-K graph M={M} N={N} K={K} G={G}")
    assert pkg._abi.lib().w4a8_gemm_workspace_bytes(M, N, K, G) > 0
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=77)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    x = bf16_bits_tensor(xb).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        eager = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
        eager_lin = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
        y_lin = torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, G)
    # a shape between the replays that splits K with a larger workspace: the stream's
    # workspace grows, and the one the graph captured must stay allocated
    lib = pkg._abi.lib()
    assert lib.w4a8_gemm_workspace_bytes(64, 2048, 16384, 256) > lib.w4a8_gemm_workspace_bytes(M, N, K, G)
    xo, wo, _, wso = make_problem(pkg, 64, 2048, 16384, 256, seed=78)
    wt2, st2 = torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(wo, 256)).to(dev), wso.to(dev), 16384, 256)
    aq2, as2 = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xo).to(dev), 256)
    for r in range(4):
        with torch.cuda.stream(s):
            y.zero_()
            y_lin.zero_()
            g.replay()
            other = torch.ops.npu.w4a8_gemm(aq2, as2, wt2, st2, 2048, 16384, 256)
            junk = torch.full((1 << 22,), 7, dtype=torch.int32, device=dev)   # reuses freed memory, if any
        torch.cuda.synchronize()
        del other, junk
        assert torch.equal(y, eager), f"replay {r}: split-K GEMM differs from eager"
        assert torch.equal(y_lin, eager_lin), f"replay {r}: linear differs from eager"
    # the graph owns its workspace: replayed on another stream while eager calls of
    # the same shape run on the capture stream, neither reads the other's sums
    ops = pkg.ops
    eager_ws = ops._WORKSPACES[(dev.index or 0, s.cuda_stream)].data_ptr()
    assert all(t.data_ptr() != eager_ws for t in ops._CAPTURE_WS.values())
    t = torch.cuda.Stream(device=dev)
    xb2, _, _, _ = make_problem(pkg, M, N, K, G, seed=79)
    aq3, as3 = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb2).to(dev), G)
    with torch.cuda.stream(s):
        eager3 = torch.ops.npu.w4a8_gemm(aq3, as3, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    for r in range(3):
        with torch.cuda.stream(t):
            y.zero_()
            g.replay()
        with torch.cuda.stream(s):
            y3 = torch.ops.npu.w4a8_gemm(aq3, as3, w_tiles, s_tiles, N, K, G)
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {r} on another stream differs from eager"
        assert torch.equal(y3, eager3), f"eager call {r} beside a replay differs"
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    check_output(tensor_bf16_bits(eager), y32, "split-K eager", exact_sym(q_ref, s_ref, w, ws32, G))


# ------------------------------------------------------------------ SwiGLU epilogue
def check_swiglu(got_bits: np.ndarray, exp_bits: np.ndarray, min_equal: float, tag: str) -> None:
    """Every output within one bf16 ulp of the expected SwiGLU value and at least
    `min_equal` of them bit-equal (the fp32 exp of the kernel and the correctly
    rounded one of the oracle can straddle a bf16 rounding tie)."""
    got = ow.bf16_bits_to_f32(got_bits).astype(np.float64)
    exp = ow.bf16_bits_to_f32(exp_bits).astype(np.float64)
    assert np.all(np.abs(got - exp) <= ow.bf16_ulp(exp)), f"{tag}: SwiGLU output off by more than 1 bf16 ulp"
    eq = np.mean(got == exp)
    assert eq >= min_equal, f"{tag}: only {eq:.5f} of SwiGLU outputs bit-equal"
    assert np.any(exp != 0), f"{tag}: vacuous"


def run_swiglu_pair(dev, xb, w, w_scale, N, K, G):
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    w_tiles, s_tiles = torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(bf16_bits_tensor(xb).to(dev), G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, w_tiles, s_tiles, N, K, G)
    yf = torch.ops.npu.w4a8_gemm_swiglu(a_q, a_s, w_tiles, s_tiles, N, K, G)
    torch.cuda.synchronize()
    return tensor_bf16_bits(y), tensor_bf16_bits(yf)


SWIGLU_CASES = [
    # (M, I, K, G, scale dtype): merged gate/up weight of N = 2*I rows
    (16, 16384, 512, 128, "f16"),     # wide N past 8 rows: four column blocks per workgroup
    (33, 16384, 1024, 128, "bf16"),   # wide N past 16 rows: activations shared through LDS
    (24, 16384, 512, 128, "bf16"),    # the same, two row tiles
    (24, 1024, 16384, 128, "f16"),    # narrow N, long K: no SwiGLU pairs in the K-split layout
    (1, 512, 1024, 128, "f16"),
    (4, 1024, 2048, 64, "bf16"),
    (5, 16384, 512, 128, "bf16"),     # wide N up to 8 rows: staged activations, one wave per workgroup
    (2, 16384, 1024, 64, "f16"),      # the same, two waves, group stride 64
    (33, 256, 1024, 256, "bf16"),
    (64, 512, 5120, 512, "bf16"),
    (3, 128, 1057, 1024, "bf16"),    # ragged K
    (100, 272, 1024, 128, "bf16"),   # prefill, I not a multiple of the 64-column tile
    (300, 512, 2048, 256, "f16"),
    (130, 256, 1000, 192, "bf16"),   # prefill, ragged K at stride 192
]


@pytest.mark.parametrize("M,I,K,G,sd", SWIGLU_CASES)
def test_gemm_swiglu(pkg, dev, M, I, K, G, sd):
    """Fused epilogue == torch's F.silu(g) * u on the unfused GPU output (each
    gate/up column accumulates as in the plain GEMM), and the whole chain
    against the oracle."""
    N = 2 * I
    say(f"gemm swiglu M={M} I={I} K={K} G={G} scales={sd}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + I + K, scale_dtype=sd)
    y, yf = run_swiglu_pair(dev, xb, w, w_scale, N, K, G)
    assert yf.shape == (M, I)
    check_swiglu(yf, ow.silu_mul_bf16(y[:, :I], y[:, I:]), 0.999, f"fused vs unfused M{M} I{I}")
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    full = ow.silu_mul_bf16(ow.f32_to_bf16_bits(y32[:, :I]), ow.f32_to_bf16_bits(y32[:, I:]))
    got, exp = ow.bf16_bits_to_f32(yf).astype(np.float64), ow.bf16_bits_to_f32(full).astype(np.float64)
    assert np.linalg.norm(got - exp) / np.linalg.norm(exp) <= 1e-3
    assert np.mean(got == exp) > 0.99


@pytest.mark.parametrize("M,I,K,G,sd", [(m, max(16, n // 32 * 16), k, g, sd)
                                        for m, n, k, g, sd in random_shapes(4242, 16 * RANDOM_SCALE)])
def test_gemm_swiglu_random_shapes(pkg, dev, M, I, K, G, sd):
    """Seeded random shapes (I a multiple of 16) through the fused SwiGLU epilogue:
    within the bar of the unfused GPU output and of the oracle."""
    N = 2 * I
    say(f"gemm swiglu random M={M} I={I} K={K} G={G} scales={sd}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + I + 5 * K, scale_dtype=sd)
    y, yf = run_swiglu_pair(dev, xb, w, w_scale, N, K, G)
    check_swiglu(yf, ow.silu_mul_bf16(y[:, :I], y[:, I:]), 0.99, f"fused vs unfused M{M} I{I}")
    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, G)
    full = ow.silu_mul_bf16(ow.f32_to_bf16_bits(y32[:, :I]), ow.f32_to_bf16_bits(y32[:, I:]))
    got, exp = ow.bf16_bits_to_f32(yf).astype(np.float64), ow.bf16_bits_to_f32(full).astype(np.float64)
    assert np.linalg.norm(got - exp) / np.linalg.norm(exp) <= 1e-3
    assert np.mean(got == exp) > 0.99


# Config 4 of the benchmark matrix: the four QwQ-32B projections at M in {16, 4096}
# with groups 64/256/512, bf16 scales, codes round(clip(N(0, 2.5), -8, 7)); gate_up
# with the fused SwiGLU (output 27648).  Oracle on a column sample (columns are
# independent); the fused output against the unfused GPU output in full.
@pytest.mark.parametrize("G", [64, 256, 512])
@pytest.mark.parametrize("M", [16, 4096])
@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
def test_config4_midgroup_variants(pkg, dev, proj, M, G):
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"config4 {proj} M={M} G={G}")
    xb, w, ws32, w_scale = make_problem(pkg, M, N, K, G, seed=M + G, scale_dtype="bf16", codes="clipped_normal")
    cols = np.sort(np.random.default_rng(G).choice(N // 2 if proj == "gate_up_proj" else N, 96, replace=False))
    q_ref, s_ref = ow.quant_act_per_token(xb)
    if proj == "gate_up_proj":
        I = N // 2
        y, yf = run_swiglu_pair(dev, xb, w, w_scale, N, K, G)
        check_swiglu(yf, ow.silu_mul_bf16(y[:, :I], y[:, I:]), 0.999, f"config4 gate_up M{M} G{G}")
        both = np.concatenate([cols, cols + I])
        y32 = ow.gemm_fp32(q_ref, s_ref, w[both], ws32[both], G)
        check_output(y[:, both], y32, f"config4 gate_up M{M} G{G}", exact_sym(q_ref, s_ref, w[both], ws32[both], G))
        full = ow.silu_mul_bf16(ow.f32_to_bf16_bits(y32[:, :len(cols)]), ow.f32_to_bf16_bits(y32[:, len(cols):]))
        got = ow.bf16_bits_to_f32(yf[:, cols]).astype(np.float64)
        exp = ow.bf16_bits_to_f32(full).astype(np.float64)
        assert np.linalg.norm(got - exp) / np.linalg.norm(exp) <= 1e-3
    else:
        y, _, _, _ = run_hip(dev, xb, w, w_scale, N, K, G, partials=False)
        y32 = ow.gemm_fp32(q_ref, s_ref, w[cols], ws32[cols], G)
        check_output(tensor_bf16_bits(y)[:, cols], y32, f"config4 {proj} M{M} G{G}", exact_sym(q_ref, s_ref, w[cols], ws32[cols], G))


# ------------------------------------------------------------------ mid-group compat pair
def bits_tensor(a: np.ndarray, dtype):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


@pytest.mark.parametrize("M", [1, 5, 16, 17, 64, 65, 130])
@pytest.mark.parametrize("K,G", [(5120, 1024), (1057, 1024), (3456, 1024), (27648, 1024), (300, 128)])
def test_midgroup_quant_a_byte_exact(pkg, dev, M, K, G):
    """All four tensors of midgroup_quant_a byte-exact, padded rows and slots included."""
    say(f"midgroup quant_a M={M} K={K} G={G}")
    xb = pkg.synth.activations(M, K, seed=M * 3 + K)
    got = torch.ops.npu.midgroup_quant_a(bf16_bits_tensor(xb).to(dev), G)
    torch.cuda.synchronize()
    exp = ow.midgroup_quant_a(xb, G)
    names = ("a_hi", "a_lo", "a_scale", "a_ksum")
    for name, g, e in zip(names, got, exp):
        gn = tensor_bf16_bits(g) if g.dtype == torch.bfloat16 else g.cpu().numpy()
        assert gn.shape == e.shape, f"{name} shape {gn.shape} vs {e.shape}"
        assert np.array_equal(gn.view(e.dtype) if gn.dtype != e.dtype else gn, e), f"{name} differs"


@pytest.mark.parametrize("M,K,G", [(2500, 27648, 1024), (2300, 30000, 1000)])
def test_midgroup_quant_a_large_calls(pkg, dev, M, K, G):
    """Past 64k (row, group) workgroups the quant takes four rows per workgroup (the last
    one holding padded rows past M): all four tensors byte-exact, ragged groups included."""
    say(f"midgroup quant_a large M={M} K={K} G={G}")
    xb = pkg.synth.activations(M, K, seed=M + K)
    got = torch.ops.npu.midgroup_quant_a(bf16_bits_tensor(xb).to(dev), G)
    torch.cuda.synchronize()
    assert got[0].shape[0] * ow.num_groups(K, G) > 65536
    exp = ow.midgroup_quant_a(xb, G)
    for name, g, e in zip(("a_hi", "a_lo", "a_scale", "a_ksum"), got, exp):
        gn = tensor_bf16_bits(g) if g.dtype == torch.bfloat16 else g.cpu().numpy()
        assert gn.shape == e.shape, f"{name} shape {gn.shape} vs {e.shape}"
        assert np.array_equal(gn.view(e.dtype) if gn.dtype != e.dtype else gn, e), f"{name} differs"


@pytest.mark.parametrize("G", [1000, 250])
@pytest.mark.parametrize("offset", [0, 1])
def test_midgroup_quant_a_ties_zero_and_tiny_groups(pkg, dev, G, offset):
    """midgroup_quant_a on a group whose quotients x/s are all exact half-integers (s = 0.5,
    round half to even), an all-zero row (tiny scale), a row of subnormal-range scales (the
    divide path) and random rows; group 250 and a source shifted by one element put the
    16-byte chunks off alignment: all four tensors byte-exact."""
    say(f"midgroup quant_a ties G={G} offset={offset}")
    M, K = 6, 3000
    rng = np.random.default_rng(17)
    x = rng.standard_normal((M, K + 1)).astype(np.float32)
    odd = rng.choice(np.arange(-253, 254, 2), size=K + 1).astype(np.float32)
    x[0] = odd * 0.25                      # x / s = odd / 2 with s = bf16(63.5 / 127) = 0.5
    x[0, ::97] = 63.5                      # every group's absmax
    x[1] = 0.0
    x[2] = rng.standard_normal(K + 1).astype(np.float32) * 1e-38
    xb_all = ow.f32_to_bf16_bits(x)
    src = bf16_bits_tensor(xb_all).to(dev)[:, offset:offset + K]
    got = torch.ops.npu.midgroup_quant_a(src, G)
    torch.cuda.synchronize()
    exp = ow.midgroup_quant_a(np.ascontiguousarray(xb_all[:, offset:offset + K]), G)
    names = ("a_hi", "a_lo", "a_scale", "a_ksum")
    for name, g, e in zip(names, got, exp):
        gn = tensor_bf16_bits(g) if g.dtype == torch.bfloat16 else g.cpu().numpy()
        assert gn.shape == e.shape, f"{name} shape {gn.shape} vs {e.shape}"
        assert np.array_equal(gn.view(e.dtype) if gn.dtype != e.dtype else gn, e), f"{name} differs"
    s_row0 = ow.bf16_bits_to_f32(exp[2][:, 0])
    assert np.all(s_row0 == 0.5), "row 0 is not on the half-integer scale"


MIDGROUP_CASES = [
    # (M, N, K, G, asym)
    (1, 512, 5120, 1024, True),
    (5, 384, 1057, 1024, True),       # ragged K, single short group + full group
    (16, 256, 3456, 1024, True),      # a K shard at group 1024
    (33, 640, 2049, 1024, False),     # symmetric: zero point all 0
    (64, 1024, 5120, 1024, True),
    (100, 256, 1057, 1024, True),     # rows padded to 128 by quant_a
    (300, 384, 5120, 1024, True),
    (16, 200, 2048, 256, True),       # stride 256 (two tiles per group), N not a multiple of 16
    (70, 160, 1000, 128, True),       # stride 128, ragged tail of 104
    (512, 1040, 3072, 1024, True),    # prefill 64x64 tiles, K over 3 waves, last column tile one block wide
    (1536, 1296, 2048, 1024, False),  # prefill tiles, K over 2 waves
    (2048, 2064, 2048, 1024, True),   # prefill tiles, 1056 workgroups: one wave walks all of K
    (200, 200, 6400, 128, True),      # 50 groups: scales too many for the 64x64 tile, 64x32 instead
    (16, 16400, 2048, 1024, True),    # wide N: four column waves share staged activations, last workgroup 1 block
    (1, 16384, 1057, 1024, True),     # the same kernel at one row, ragged K
    (5, 16400, 1152, 128, False),     # the same at stride 128 with an odd tile count (last step one tile)
]


def run_midgroup(pkg, dev, M, N, K, G, asym, seed):
    xb = pkg.synth.activations(M, K, seed=seed)
    w = np.random.default_rng(seed).standard_normal((N, K)).astype(np.float32) * 0.05
    codes, sc, zr, ks = ow.quantize_weight_asym(w, G)
    if not asym:
        zr = np.zeros_like(zr)
    a = torch.ops.npu.midgroup_quant_a(bf16_bits_tensor(xb).to(dev), G)
    args = (torch.from_numpy(ow.pack_grouped(codes, G)).to(dev), bits_tensor(sc, torch.bfloat16).to(dev),
            torch.from_numpy(ks).to(dev), bits_tensor(zr, torch.bfloat16).to(dev))
    y, P = torch.ops.npu.midgroup_w4a8_gemm_partials(*a, *args, K, G)
    torch.cuda.synchronize()
    return xb, codes, sc, zr, a, args, y, P


@pytest.mark.parametrize("M,N,K,G,asym", MIDGROUP_CASES)
def test_midgroup_gemm_partials_bit_exact_and_output(pkg, dev, M, N, K, G, asym):
    """int32 I_g = sum A*(W - wz) bit-exact; bf16 output equal to bf16 of ReferenceMidGroupGemm's
    fp32 result (the oracle restates its order bit for bit), and within the main path's bars."""
    say(f"midgroup gemm M={M} N={N} K={K} G={G} asym={asym}")
    xb, codes, sc, zr, a, args, y, P = run_midgroup(pkg, dev, M, N, K, G, asym, seed=M + N + K)
    Mp = a[0].shape[0]
    q, s = ow.quant_act_midgroup(xb, G)
    qp = np.zeros((Mp, K), np.int8)
    qp[:M] = q
    P_ref = ow.group_partials_asym(qp, codes, zr, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    a_scale = tensor_bf16_bits(a[2])
    y32 = ow.gemm_midgroup_fp32(qp, a_scale, codes, sc, zr, G, partials=P_ref)
    assert y.shape == (Mp, N)
    check_output(tensor_bf16_bits(y)[:M], y32[:M], f"midgroup M{M} N{N} K{K}", exact_mid(qp, a_scale, codes, sc, zr, G))
    assert np.array_equal(tensor_bf16_bits(y)[:M], ow.f32_to_bf16_bits(y32[:M])), "not bf16 of the oracle's fp32 result"
    assert not tensor_bf16_bits(y)[M:].any() or np.all(ow.bf16_bits_to_f32(tensor_bf16_bits(y)[M:]) == 0)


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
@pytest.mark.parametrize("M", [1, 16])
def test_midgroup_qwq_decode_shapes(pkg, dev, proj, M):
    """The reference's own decode configuration: group 1024 at QwQ-32B shapes (partial dump
    on: int32 partials and bf16 of the oracle's fp32 result, bit for bit)."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"midgroup qwq {proj} M={M}")
    xb, codes, sc, zr, a, args, y, P = run_midgroup(pkg, dev, M, N, K, 1024, True, seed=M)
    Mp = a[0].shape[0]
    q, _ = ow.quant_act_midgroup(xb, 1024)
    qp = np.zeros((Mp, K), np.int8)
    qp[:M] = q
    y32 = ow.gemm_midgroup_fp32(qp, tensor_bf16_bits(a[2]), codes, sc, zr, 1024)
    check_output(tensor_bf16_bits(y)[:M], y32[:M], f"midgroup {proj} M{M}", exact_mid(qp, tensor_bf16_bits(a[2]), codes, sc, zr, 1024))
    assert np.array_equal(tensor_bf16_bits(y)[:M], ow.f32_to_bf16_bits(y32[:M])), "not bf16 of the oracle's fp32 result"


MIDGROUP_PREFILL_CASES = [
    # (M, N, K, G, asym): past 16 rows with 64-row output tiles for at least half
    # of 256 CUs (no partial dump), the compat GEMM runs the LDS-tiled prefill
    # waves on the activation rows rebuilt into a workspace; from 1024 rows on
    # weight tiles repacked there too
    (17, 16400, 1057, 1024, False),    # the first row count on it (wide N), ragged K
    (40, 16400, 2048, 1024, True),     # one partial row tile
    (65, 8200, 5120, 1024, True),      # last column tile partial
    (100, 8192, 1057, 1024, True),     # ragged K: the last step's upper half is padding
    (300, 3000, 5120, 1024, False),    # symmetric: zero point all 0
    (512, 2100, 3072, 1024, True),     # N not a multiple of 16
    (200, 4200, 3456, 256, True),      # stride 256 (two steps per group)
    (129, 4000, 1152, 384, True),      # stride 384 (three steps per group)
    (700, 2064, 2048, 1024, True),     # 64-row tiles
    (2048, 2064, 2048, 1024, True),    # repacked weight tiles, 128-row tiles
    (2048, 1000, 1057, 1024, False),   # repacked tiles, ragged K, N not a multiple of 16
]


def _midgroup_inputs(pkg, dev, M, N, K, G, asym, seed):
    xb = pkg.synth.activations(M, K, seed=seed)
    w = np.random.default_rng(seed).standard_normal((N, K)).astype(np.float32) * 0.05
    codes, sc, zr, ks = ow.quantize_weight_asym(w, G)
    if not asym:
        zr = np.zeros_like(zr)
    a = torch.ops.npu.midgroup_quant_a(bf16_bits_tensor(xb).to(dev), G)
    args = (torch.from_numpy(ow.pack_grouped(codes, G)).to(dev), bits_tensor(sc, torch.bfloat16).to(dev),
            torch.from_numpy(ks).to(dev), bits_tensor(zr, torch.bfloat16).to(dev))
    return xb, codes, sc, zr, a, args


@pytest.mark.parametrize("M,N,K,G,asym", MIDGROUP_PREFILL_CASES)
def test_midgroup_prefill_path_equals_reference_order(pkg, dev, M, N, K, G, asym):
    """One wave walks each output's groups in order, with the reference's roundings, so
    the bf16 output equals bf16(ReferenceMidGroupGemm's fp32 result) bit for bit
    (int4_cube_lab/host/gemm_ref.cpp:199-240, restated by the oracle)."""
    say(f"midgroup prefill path M={M} N={N} K={K} G={G} asym={asym}")
    xb, codes, sc, zr, a, args = _midgroup_inputs(pkg, dev, M, N, K, G, asym, seed=3 * M + N + K)
    Mp = a[0].shape[0]
    assert pkg._abi.lib().w4a8_midgroup_gemm_workspace_bytes(Mp, N, K, G) > 0, "case not on the prefill path"
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G)
    torch.cuda.synchronize()
    q, _ = ow.quant_act_midgroup(xb, G)
    qp = np.zeros((Mp, K), np.int8)
    qp[:M] = q
    y32 = ow.gemm_midgroup_fp32(qp, tensor_bf16_bits(a[2]), codes, sc, zr, G)
    got = tensor_bf16_bits(y)
    want = ow.f32_to_bf16_bits(y32)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} outputs differ from bf16(oracle fp32)"
    assert np.abs(y32).max() > 0


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
@pytest.mark.parametrize("M", [512, 4096])
def test_midgroup_prefill_qwq_shapes(pkg, dev, proj, M):
    """The reference's group 1024 at QwQ-32B shapes (stored weights at 512 rows, repacked
    tiles at 4096), on 40 sampled rows (every column) against the oracle's fp32 order, bit
    for bit."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"midgroup prefill qwq {proj} M={M}")
    xb, codes, sc, zr, a, args = _midgroup_inputs(pkg, dev, M, N, K, 1024, True, seed=11)
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, 1024)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(5).choice(M, 40, replace=False))
    q, _ = ow.quant_act_midgroup(xb[rows], 1024)
    y32 = ow.gemm_midgroup_fp32(q, tensor_bf16_bits(a[2])[:, rows], codes, sc, zr, 1024)
    got = tensor_bf16_bits(y)[rows]
    want = ow.f32_to_bf16_bits(y32)
    assert np.array_equal(got, want), f"{proj}: {int((got != want).sum())} of {got.size} sampled outputs differ"


@pytest.mark.parametrize("proj", ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"])
@pytest.mark.parametrize("M", [1, 16, 64])
def test_midgroup_decode_reference_order(pkg, dev, proj, M):
    """Decode rows at group 1024: the K split over waves adds exact int32 group sums and folds
    once in group order (or one wave walks every group), so the output is bf16 of the
    reference's fp32 result bit for bit -- down_proj past 16 rows included, whose 27 groups
    of 64-row sums exceed the LDS and which takes 32-row tiles."""
    K, N = pkg.synth.QWQ_SHAPES[proj]
    say(f"midgroup decode order {proj} M={M}")
    xb, codes, sc, zr, a, args = _midgroup_inputs(pkg, dev, M, N, K, 1024, True, seed=31 + M)
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, 1024, M)
    torch.cuda.synchronize()
    q, _ = ow.quant_act_midgroup(xb, 1024)
    y32 = ow.gemm_midgroup_fp32(q, tensor_bf16_bits(a[2])[:, :M], codes, sc, zr, 1024)
    got = tensor_bf16_bits(y)
    want = ow.f32_to_bf16_bits(y32)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} outputs differ"


def _tiles_ref(w_q: np.ndarray, KT: int) -> np.ndarray:
    """midgroup_tile_weights' layout built on the CPU: tiles[nb][kt][q][c][16 bytes] =
    w_q[16 nb + c][64 kt + 16 q .. +15], zero past N and past the row."""
    N, kb = w_q.shape
    NB = -(-N // 16)
    pad = np.zeros((NB * 16, KT * 64), np.int8)
    pad[:N, :kb] = w_q
    return pad.reshape(NB, 16, KT, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


@pytest.mark.parametrize("M,N,K,G", [
    (1, 7168, 5120, 1024),      # per-wave kernel, int32 group sums
    (16, 1000, 1057, 1024),     # ragged K (a half-padding last tile), N not a multiple of 16
    (1, 16400, 1057, 1024),     # shared-activation kernel on wide N
    (64, 5120, 27648, 1024),    # 32-row tiles (27 groups of sums)
    (48, 2064, 3456, 256),      # 64-row tiles, stride 256
    (300, 8200, 5120, 1024),    # prefill path on the tiles
    (2048, 1000, 1057, 1024),   # prefill path (the stored rows would be repacked per call)
])
def test_midgroup_tiled_weights_equal_stored_rows(pkg, dev, M, N, K, G):
    """midgroup_tile_weights equals its CPU construction byte for byte, and the GEMM on the
    tiles returns the bits of the GEMM on the rows as stored, on every compat path."""
    say(f"midgroup tiles M={M} N={N} K={K} G={G}")
    _, _, _, _, a, args = _midgroup_inputs(pkg, dev, M, N, K, G, True, seed=41 + M)
    w_q = args[0]
    tiles = torch.ops.npu.midgroup_tile_weights(w_q, K, G)
    KT = -(-pkg.geometry.kpad(K, G) // 128)
    assert np.array_equal(tiles.cpu().numpy(), _tiles_ref(w_q.cpu().numpy(), KT))
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G, M)
    yt = torch.ops.npu.midgroup_w4a8_gemm_tiled(*a, tiles, *args[1:], N, K, G, M)
    torch.cuda.synchronize()
    assert torch.equal(yt.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_midgroup_gemm_real_rows_equal_padded_rows(pkg, dev, M):
    """rows=M computes only the real rows of quant_a's padded planes: the same bits as the
    padded product's first M rows (the plan does not depend on the row count up to 64)."""
    say(f"midgroup rows={M}")
    K, N, G = 5120, 7168, 1024
    _, _, _, _, a, args = _midgroup_inputs(pkg, dev, M, N, K, G, True, seed=21 + M)
    y_pad = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G)
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G, M)
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y_pad.shape[0] >= M
    assert torch.equal(y.view(torch.int16), y_pad[:M].view(torch.int16))
    with pytest.raises(RuntimeError, match="exceeds"):
        torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G, y_pad.shape[0] + 1)


@pytest.mark.parametrize("M,N,K,G", [
    (1, 5120, 27648, 128),     # 216 groups: one 16-row tile's staged values past 64 KiB
    (16, 2048, 27648, 128),
    (40, 1296, 12730, 128),    # 100 groups: 64-row tiles within 128 KiB
    (64, 2048, 27648, 128),    # 216 groups: 16-row tiles (64 rows' values past 128 KiB)
    (100, 700, 27648, 128),    # past 64 rows, off the prefill path: 16-row tiles
    (33, 2000, 40000, 256),    # 157 groups
])
def test_midgroup_many_groups(pkg, dev, M, N, K, G):
    """More groups than 64 KiB of staged row and column values hold (group 128 on down_proj's
    K): int32 partials bit-exact, the output bf16 of the oracle's fp32 result bit for bit, and
    the call without the dump returns the dump call's bits."""
    say(f"midgroup many groups M={M} N={N} K={K} G={G}")
    xb, codes, sc, zr, a, args, y, P = run_midgroup(pkg, dev, M, N, K, G, True, seed=M + N + K + G)
    Mp = a[0].shape[0]
    q, _ = ow.quant_act_midgroup(xb, G)
    qp = np.zeros((Mp, K), np.int8)
    qp[:M] = q
    P_ref = ow.group_partials_asym(qp, codes, zr, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), P_ref), "int32 partials differ"
    a_scale = tensor_bf16_bits(a[2])
    y32 = ow.gemm_midgroup_fp32(qp, a_scale, codes, sc, zr, G, partials=P_ref)
    got, want = tensor_bf16_bits(y)[:M], ow.f32_to_bf16_bits(y32[:M])
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} outputs differ"
    y_plain = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G)
    torch.cuda.synchronize()
    assert torch.equal(y_plain.view(torch.int16), y.view(torch.int16))


def random_midgroup_shapes(seed: int, n: int, max_mnk: float = 2e9, max_gmn: float = 3e7):
    """n seeded random (M, N, K, group, asym) draws for the compat GEMM: any N, K not a
    multiple of the group, groups whose padded stride is a multiple of 128 (the path's
    contract, 250 and 1000 among them), rows from one token to past the prefill path's
    tile rule (the last third of the draws sized for it), up to 125 groups at decode rows
    (past what the exact LDS group sums hold).  Capped so the oracle takes seconds."""
    rng = np.random.default_rng(seed)
    groups = [128, 250, 256, 384, 512, 640, 1000, 1024, 2048]
    out = []
    while len(out) < n:
        G = int(rng.choice(groups))
        u = rng.random()
        if u < 0.4:
            M, N, K = int(rng.integers(1, 65)), int(rng.integers(1, 9001)), int(rng.integers(1, 16001))
        elif u < 0.67:
            M, N, K = int(rng.integers(65, 700)), int(rng.integers(1, 3001)), int(rng.integers(1, 4001))
        else:
            M = int(rng.integers(256, 2600))
            N = int(rng.integers((1 << 20) // M + 1, 5001))
            K = int(rng.integers(1, 2001))
        if M * N * K > max_mnk or ow.num_groups(K, G) * M * N > max_gmn or N * K > 4e7:
            continue
        out.append((M, N, K, G, bool(rng.random() < 0.75)))
    return out


@pytest.mark.parametrize("M,N,K,G,asym", random_midgroup_shapes(20261203, 12 * RANDOM_SCALE))
def test_midgroup_random_shapes(pkg, dev, M, N, K, G, asym):
    """Seeded random compat shapes through every plan the row count, width and group count
    select.  On each: bf16 of the oracle's ReferenceMidGroupGemm fp32 result
    (int4_cube_lab/host/gemm_ref.cpp:199-240) bit for bit -- every plan folds each output's
    groups in order (one wave, or exact int32 group sums met in LDS, in chunks past what LDS
    holds at once) -- and the GEMM on weight tiles equal to the GEMM on the stored rows."""
    say(f"midgroup random M={M} N={N} K={K} G={G} asym={asym}")
    xb, codes, sc, zr, a, args = _midgroup_inputs(pkg, dev, M, N, K, G, asym, seed=7 * M + N + K + G)
    y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G, M)
    tiles = torch.ops.npu.midgroup_tile_weights(args[0], K, G)
    yt = torch.ops.npu.midgroup_w4a8_gemm_tiled(*a, tiles, *args[1:], N, K, G, M)
    torch.cuda.synchronize()
    assert y.shape == (M, N)
    assert torch.equal(yt.view(torch.int16), y.view(torch.int16)), "tiled weights differ from stored rows"
    q, _ = ow.quant_act_midgroup(xb, G)
    as_bits = tensor_bf16_bits(a[2])[:, :M]
    y32 = ow.gemm_midgroup_fp32(q, as_bits, codes, sc, zr, G)
    got = tensor_bf16_bits(y)
    want = ow.f32_to_bf16_bits(y32)
    path = "prefill" if pkg._abi.lib().w4a8_midgroup_gemm_workspace_bytes(M, N, K, G) > 0 else "mid-group"
    assert np.array_equal(got, want), f"{path} path: {int((got != want).sum())} of {got.size} outputs differ"
    assert np.abs(y32).max() > 0


def test_midgroup_prefill_path_without_zero_points(pkg, dev):
    """The C ABI's symmetric call (w_zero NULL: the variant without the zero-point term)
    equals the call with an all-zero w_zero, through w4a8_midgroup_gemm_ws."""
    say("midgroup prefill path, w_zero NULL")
    M, N, K, G = 300, 3000, 3072, 1024
    _, _, _, _, a, args = _midgroup_inputs(pkg, dev, M, N, K, G, False, seed=9)
    y0 = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G)
    a_hi, a_lo, a_scale, a_ksum = a
    w_q, w_scale = args[0], args[1]
    Mp = a_hi.shape[0]
    lib = pkg._abi.lib()
    need = lib.w4a8_midgroup_gemm_workspace_bytes(Mp, N, K, G)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    y1 = torch.empty((Mp, N), dtype=torch.bfloat16, device=dev)
    rc = lib.w4a8_midgroup_gemm_ws(a_hi.data_ptr(), a_lo.data_ptr(), a_scale.data_ptr(), a_ksum.data_ptr(), Mp,
                                   a_scale.stride(0), w_q.data_ptr(), w_scale.data_ptr(), None, y1.data_ptr(), N,
                                   None, N, K, G, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.w4a8_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_midgroup_prefill_path_relaunch_deterministic(pkg, dev):
    """Repeated calls of the prefill path (pre-pass, then the GEMM on a fresh workspace)
    return the same bytes (the reference's --stress relaunch check, mg_harness.h:307-334)."""
    for M in (600, 2048):   # stored weights, then weight tiles repacked per call
        say(f"midgroup prefill relaunch M={M}")
        _, _, _, _, a, args = _midgroup_inputs(pkg, dev, M, 3000, 5120, 1024, True, seed=7)
        ys = [torch.ops.npu.midgroup_w4a8_gemm(*a, *args, 5120, 1024) for _ in range(6)]
        torch.cuda.synchronize()
        for y in ys[1:]:
            assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))


def test_midgroup_linear_module(pkg, dev):
    """The reference's MidGroupW4A8LinearMethod.apply semantics: [N, G] checkpoint tensors,
    quant_a, GEMM, slice to the real rows, bias, reshape."""
    say("MidGroupW4A8Linear")
    K, N = 2049, 384
    torch.manual_seed(1)
    lin = torch.nn.Linear(K, N, bias=True, dtype=torch.float32)
    m = pkg.MidGroupW4A8Linear.from_float(lin.to(dev))
    x = torch.randn(2, 3, K, dtype=torch.bfloat16)
    y = m(x.to(dev))
    torch.cuda.synchronize()
    assert y.shape == (2, 3, N) and y.dtype == torch.bfloat16
    codes, sc, zr, _ = ow.quantize_weight_asym(lin.weight.detach().cpu().numpy(), 1024)
    xb = tensor_bf16_bits(x.reshape(-1, K))
    q, s = ow.quant_act_midgroup(xb, 1024)
    y32 = ow.gemm_midgroup_fp32(q, s, codes, sc, zr, 1024)
    y_ref = (torch.from_numpy(ow.round_bf16(y32)).to(torch.bfloat16) + lin.bias.detach().cpu().to(torch.bfloat16)
             ).float().numpy()
    got = y.reshape(-1, N).float().cpu().numpy()
    assert np.max(np.abs(got - y_ref) - 2 * ow.bf16_ulp(y_ref)) <= 0


# ------------------------------------------------------------------ RMSNorm + quant
@pytest.mark.parametrize("M", [1, 4, 16, 64, 300])
@pytest.mark.parametrize("K,G", [(5120, 0), (5120, 128), (27648, 128), (3456, 1024), (1024, 0)])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm_quant(pkg, dev, M, K, G, with_res):
    """Two-stage bar: the emitted normalised row within one bf16 ulp of the oracle's
    rms_norm (>= 99.9% equal: the fp32 sum order is not fixed by any reference file), and
    the int8 codes and scales byte-exact against the per-token quant of that emitted row;
    the residual sum exactly."""
    say(f"rmsnorm_quant M={M} K={K} G={G} res={with_res}")
    rng = np.random.default_rng(M + K + G)
    xb = pkg.synth.activations(M, K, seed=M + K)
    rb = ow.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32)) if with_res else None
    wb = ow.f32_to_bf16_bits(rng.uniform(0.5, 1.5, K).astype(np.float32))
    x = bf16_bits_tensor(xb).to(dev)
    w = bf16_bits_tensor(wb).to(dev)
    r = bf16_bits_tensor(rb).to(dev) if with_res else None
    a_q, a_s, s, h = torch.ops.npu.w4a8_rmsnorm_quant(x, w, 1e-6, r, G, True)
    torch.cuda.synchronize()
    sb = ow.add_bf16(xb, rb) if with_res else xb
    if with_res:
        assert np.array_equal(tensor_bf16_bits(s), sb), "residual sum"
    hg = tensor_bf16_bits(h)
    he, h1 = ow.rms_norm_bf16(sb, wb, 1e-6, return_h1=True)
    # the GPU's intermediate bf16(s * r) may sit one bf16 ulp from the oracle's (r differs
    # in its last fp32 bit); the final product must then be one of the three outcomes
    wf = ow.bf16_bits_to_f32(wb)
    ok = hg == he
    for k in (-1, 1):
        h1k = (h1.astype(np.float64) + k * ow.bf16_ulp(h1)).astype(np.float32)
        ok |= hg == ow.f32_to_bf16_bits((h1k * wf).astype(np.float32))
    bad = np.argwhere(~ok)
    assert ok.all(), f"{len(bad)} normed values outside one intermediate ulp, first at {bad[:3].tolist()}"
    assert np.mean(hg == he) >= 0.999
    q, sc = ow.quant_act_per_token(hg)
    assert np.array_equal(tensor_bf16_bits(a_s), sc)
    assert np.array_equal(a_q.cpu().numpy(), ow.pad_groups(q, G) if G else q)


@pytest.mark.parametrize("K", [5120, 4096, 3072])
def test_rmsnorm_quant_rows_do_not_depend_on_batch(pkg, dev, K):
    """A row's outputs are the same bytes whatever the batch: up to 64 rows the launch
    gives each thread one 8-element unit (512 or 1024 threads at these K), past 64 rows
    256 threads with two to four units each, and the sum of squares is one tree over the
    unit index either way.  Rows 0..63 of a 65-row call equal those of a 64-row call
    (and of one-row calls), with and without the residual add."""
    say(f"rmsnorm_quant batch independence K={K}")
    rng = np.random.default_rng(K)
    xb = pkg.synth.activations(65, K, seed=K + 1)
    rb = ow.f32_to_bf16_bits(rng.standard_normal((65, K)).astype(np.float32))
    wb = ow.f32_to_bf16_bits(rng.uniform(0.5, 1.5, K).astype(np.float32))
    x, w, r = bf16_bits_tensor(xb).to(dev), bf16_bits_tensor(wb).to(dev), bf16_bits_tensor(rb).to(dev)
    for res in (None, r):
        outs = {}
        for M in (65, 64, 1):
            outs[M] = torch.ops.npu.w4a8_rmsnorm_quant(x[:M], w, 1e-6, None if res is None else res[:M], 128, True)
        torch.cuda.synchronize()
        for t65, t64, t1 in zip(outs[65], outs[64], outs[1]):
            assert torch.equal(t65[:64].view(torch.int8).cpu(), t64.view(torch.int8).cpu()), "rows differ, M=64 vs 65"
            assert torch.equal(t65[:1].view(torch.int8).cpu(), t1.view(torch.int8).cpu()), "row 0 differs, M=1 vs 65"


# ------------------------------------------------------------------ checkpoint formats
def test_vendor_checkpoint_linear(pkg, dev):
    """A vendor W4A8_DYNAMIC linear (packed along N, per-channel x per-group scales) loaded
    onto the per-token path, against the oracle with the same codes and scales."""
    say("vendor W4A8_DYNAMIC linear")
    g = torch.Generator().manual_seed(9)
    N, K, G = 256, 1024, 128
    codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, generator=g)
    s2 = (torch.rand((N, K // G), generator=g) * 0.01 + 0.002).to(torch.float16)
    c = codes.to(torch.int16) & 0xF
    base = "model.layers.0.self_attn.o_proj"
    t = {f"{base}.weight": (c[0::2] | (c[1::2] << 4)).to(torch.uint8).view(torch.int8),
         f"{base}.weight_scale": torch.ones((N, 1)), f"{base}.weight_offset": torch.zeros((N, 1)),
         f"{base}.weight_scale_second": s2}
    m = pkg.checkpoint.load_vendor_linear(t, base, G, device=dev)
    xb = pkg.synth.activations(5, K, seed=3)
    y = m(bf16_bits_tensor(xb).to(dev))
    torch.cuda.synchronize()
    q, s = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q, s, codes.numpy(), s2.float().numpy(), G)
    check_output(tensor_bf16_bits(y), y32, "vendor linear", exact_sym(q, s, codes.numpy(), s2.float().numpy(), G))


def test_midgroup_checkpoint_linear(pkg, dev):
    """An mg_kgeom_v1 export loaded into MidGroupW4A8Linear, against the oracle."""
    say("mg_kgeom_v1 linear")
    w = torch.randn((320, 2049), generator=torch.Generator().manual_seed(10)) * 0.04
    base = "model.layers.3.mlp.down_proj"
    out = pkg.checkpoint.export_midgroup({f"{base}.weight": w}, 1024)
    m = pkg.checkpoint.load_midgroup_linear(out, base, K=2049, device=dev)
    xb = pkg.synth.activations(7, 2049, seed=4)
    y = m(bf16_bits_tensor(xb).to(dev))
    torch.cuda.synchronize()
    codes, sc, zr, _ = ow.quantize_weight_asym(w.to(torch.bfloat16).float().numpy(), 1024)
    q, s = ow.quant_act_midgroup(xb, 1024)
    y32 = ow.gemm_midgroup_fp32(q, s, codes, sc, zr, 1024)
    check_output(tensor_bf16_bits(y), y32, "mg_kgeom_v1 linear", exact_mid(q, s, codes, sc, zr, 1024))
