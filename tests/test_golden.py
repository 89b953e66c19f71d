"""Golden vectors of the reference's own C++ CPU reference (tests/golden/reference_vectors.npz,
written by tests/golden/make_golden.py from int4_cube_lab/host/gemm_ref.cpp and
mg_kgeom.h compiled in place).

CPU: the oracle restatement reproduces them (packing, plane split, ksums and
geometry byte-exact; ReferenceMidGroupGemm's fp32 order bit-exact; the per-token
torch order and the per-channel order to the output bar).  GPU: the HIP kernels
on the same inputs against the reference's outputs.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import w4a8 as ow

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "reference_vectors.npz")


def gv(name):
    return GOLDEN[name]


def unpacked(wq: np.ndarray, K: int, G: int) -> np.ndarray:
    """codes [N, K] from the reference's packed grouped layout (padding slots dropped)."""
    full = ow.unpack_int4(wq)
    cols = np.concatenate([np.arange(ow.group_offset(g, G), ow.group_offset(g, G) + ow.group_real(g, K, G))
                           for g in range(ow.num_groups(K, G))])
    return full[:, cols]


def bar_and_equal(y_bits, ref_bits, y32, exact, min_equal=0.99):
    fail, _ = ow.output_bar(y_bits, y32, exact)
    assert not fail.any()
    assert np.mean(y_bits == ref_bits) >= min_equal, np.mean(y_bits == ref_bits)


def test_golden_geometry():
    for K, G, ng, kp, off, real in gv("geometry"):
        assert ow.num_groups(K, G) == ng and ow.kpad(K, G) == kp
        assert ow.group_offset(ng - 1, G) == off and ow.group_real(ng - 1, K, G) == real


def test_golden_per_token_path():
    M, K, N, G = (int(v) for v in gv("pt_shape"))
    aq, as_ = ow.quant_act_per_token(gv("pt_x"))
    assert np.array_equal(aq, gv("pt_aq")) and np.array_equal(as_, gv("pt_as"))
    codes = unpacked(gv("pt_wq"), K, G)
    assert np.array_equal(ow.pack_grouped(codes, G), gv("pt_wq"))
    ws32 = ow.bf16_bits_to_f32(gv("pt_ws")).T.copy()
    y32 = ow.gemm_fp32(aq, as_, codes, ws32, G)
    # the reference C++ associates (float(P) * ws) * as, the torch path P * (as * ws)
    bar_and_equal(gv("pt_y"), ow.f32_to_bf16_bits(y32), y32,
                  lambda r, c: ow.gemm_f64(aq[r], as_[r], codes[c], ws32[c], G))


def test_golden_midgroup_path():
    M, K, N, G = (int(v) for v in gv("mg_shape"))
    aq, as_g = ow.quant_act_midgroup(gv("mg_x"), G)
    assert np.array_equal(aq, gv("mg_aq")) and np.array_equal(as_g, gv("mg_as"))
    hi, lo = ow.msd_planes(ow.pad_groups(aq, G))
    assert np.array_equal(ow.pack_int4(hi), gv("mg_hi")) and np.array_equal(ow.pack_int4(lo), gv("mg_lo"))
    assert np.array_equal(ow.act_ksum_neg(aq, G), gv("mg_aksum"))
    codes = unpacked(gv("mg_wq"), K, G)
    assert np.array_equal(ow.pack_grouped(codes, G), gv("mg_wq"))
    wsum = np.stack([codes[:, g * G:g * G + ow.group_real(g, K, G)].astype(np.int64).sum(1)
                     for g in range(ow.num_groups(K, G))])
    assert np.array_equal(wsum, gv("mg_wksum"))
    y32 = ow.gemm_midgroup_fp32(aq, as_g, codes, gv("mg_ws"), gv("mg_wz"), G)
    assert np.array_equal(ow.f32_to_bf16_bits(y32), gv("mg_y")), "ReferenceMidGroupGemm's order is restated bitwise"


def test_golden_perchannel_path():
    M, K, N = (int(v) for v in gv("pc_shape"))
    aq, as_ = ow.quant_act_per_token(gv("pc_x"))
    assert np.array_equal(aq, gv("pc_aq")) and np.array_equal(as_, gv("pc_as"))
    codes = unpacked(gv("pc_wq"), K, K)
    ws32 = ow.bf16_bits_to_f32(gv("pc_ws"))[:, None].astype(np.float32)
    y32 = ow.gemm_fp32(aq, as_, codes, ws32, K)
    bar_and_equal(gv("pc_y"), ow.f32_to_bf16_bits(y32), y32,
                  lambda r, c: ow.gemm_f64(aq[r], as_[r], codes[c], ws32[c], K))


def test_golden_negative_control():
    """A dropped group (a plausible indexing slip) fails the per-token golden comparison."""
    M, K, N, G = (int(v) for v in gv("pt_shape"))
    codes = unpacked(gv("pt_wq"), K, G)
    ws32 = ow.bf16_bits_to_f32(gv("pt_ws")).T.copy()
    ws_bad = ws32.copy()
    ws_bad[:, 3] = 0
    y_bad = ow.f32_to_bf16_bits(ow.gemm_fp32(gv("pt_aq"), gv("pt_as"), codes, ws_bad, G))
    assert np.mean(y_bad == gv("pt_y")) < 0.5


# ------------------------------------------------------------------ GPU against the reference's outputs
@pytest.mark.gpu
def test_gpu_golden_per_token(pkg, dev):
    import torch
    from conftest import tensor_bf16_bits
    M, K, N, G = (int(v) for v in gv("pt_shape"))
    print(f"golden per-token M={M} K={K} N={N} G={G}", flush=True)
    ws = torch.from_numpy(gv("pt_ws").view(np.int16)).view(torch.bfloat16).to(dev)
    wt, st = torch.ops.npu.w4a8_repack(torch.from_numpy(gv("pt_wq")).to(dev), ws, K, G)
    x = torch.from_numpy(gv("pt_x").view(np.int16)).view(torch.bfloat16).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)
    yl = torch.ops.npu.w4a8_linear(x, wt, st, N, K, G)
    torch.cuda.synchronize()
    assert np.array_equal(a_q.cpu().numpy(), gv("pt_aq")) and np.array_equal(tensor_bf16_bits(a_s), gv("pt_as"))
    codes = unpacked(gv("pt_wq"), K, G)
    ws32 = ow.bf16_bits_to_f32(gv("pt_ws")).T.copy()
    y32 = ow.gemm_fp32(gv("pt_aq"), gv("pt_as"), codes, ws32, G)
    for got in (tensor_bf16_bits(y), tensor_bf16_bits(yl)):
        bar_and_equal(got, gv("pt_y"), y32, lambda r, c: ow.gemm_f64(gv("pt_aq")[r], gv("pt_as")[r], codes[c],
                                                                     ws32[c], G))


@pytest.mark.gpu
def test_gpu_golden_midgroup(pkg, dev):
    import torch
    from conftest import tensor_bf16_bits
    M, K, N, G = (int(v) for v in gv("mg_shape"))
    print(f"golden midgroup M={M} K={K} N={N} G={G}", flush=True)
    x = torch.from_numpy(gv("mg_x").view(np.int16)).view(torch.bfloat16).to(dev)
    a_hi, a_lo, a_scale, a_ksum = torch.ops.npu.midgroup_quant_a(x, G)
    assert np.array_equal(a_hi[:M].cpu().numpy(), gv("mg_hi")) and np.array_equal(a_lo[:M].cpu().numpy(), gv("mg_lo"))
    assert np.array_equal(tensor_bf16_bits(a_scale)[:, :M], gv("mg_as"))
    assert np.array_equal(a_ksum[:, :M].cpu().numpy(), gv("mg_aksum"))
    t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    y = torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_scale, a_ksum, torch.from_numpy(gv("mg_wq")).to(dev),
                                         t(gv("mg_ws")), torch.from_numpy(gv("mg_wksum")).to(dev), t(gv("mg_wz")),
                                         K, G)
    torch.cuda.synchronize()
    # the compat GEMM evaluates the reference's own fp32 order
    assert np.array_equal(tensor_bf16_bits(y)[:M], gv("mg_y"))


@pytest.mark.gpu
def test_gpu_golden_perchannel(pkg, dev):
    """The reference's ReferencePerchannelGemm output on the same per-channel inputs
    (its association float(P) * as * ws differs from the kernel's by fp32 rounding only)."""
    import torch
    from conftest import tensor_bf16_bits
    M, K, N = (int(v) for v in gv("pc_shape"))
    print(f"golden per-channel M={M} K={K} N={N}", flush=True)
    ws = torch.from_numpy(gv("pc_ws").reshape(1, N).view(np.int16)).view(torch.bfloat16).to(dev)
    wt, st = torch.ops.npu.w4a8_repack(torch.from_numpy(gv("pc_wq")).to(dev), ws, K, K)
    x = torch.from_numpy(gv("pc_x").view(np.int16)).view(torch.bfloat16).to(dev)
    y = torch.ops.npu.w4a8_linear(x, wt, st, N, K, K)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, K)
    y2, P = torch.ops.npu.w4a8_gemm_partials(a_q, a_s, wt, st, N, K, K)
    torch.cuda.synchronize()
    codes = unpacked(gv("pc_wq"), K, K)
    assert np.array_equal(P[0].cpu().numpy().astype(np.int64),
                          gv("pc_aq").astype(np.int64) @ codes.astype(np.int64).T)
    ws32 = ow.bf16_bits_to_f32(gv("pc_ws"))[:, None].astype(np.float32)
    y32 = ow.gemm_fp32(gv("pc_aq"), gv("pc_as"), codes, ws32, K)
    for got in (tensor_bf16_bits(y), tensor_bf16_bits(y2)):
        bar_and_equal(got, gv("pc_y"), y32, lambda r, c: ow.gemm_f64(gv("pc_aq")[r], gv("pc_as")[r], codes[c],
                                                                     ws32[c], K))


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 2, 4, 8])
def test_gpu_golden_row_prefixes(pkg, dev, rows):
    """The first rows of the per-token and per-channel golden cases through the
    GEMM and the linear (outputs are row-independent, so each prefix must match
    the reference's rows): up to 8 rows run the staged decode variants, one row
    the fused single-row linear."""
    import torch
    from conftest import tensor_bf16_bits
    M, K, N, G = (int(v) for v in gv("pt_shape"))
    print(f"golden per-token prefix rows={rows} K={K} N={N} G={G}", flush=True)
    ws = torch.from_numpy(gv("pt_ws").view(np.int16)).view(torch.bfloat16).to(dev)
    wt, st = torch.ops.npu.w4a8_repack(torch.from_numpy(gv("pt_wq")).to(dev), ws, K, G)
    x = torch.from_numpy(gv("pt_x")[:rows].view(np.int16)).view(torch.bfloat16).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    y = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)
    yl = torch.ops.npu.w4a8_linear(x, wt, st, N, K, G)
    y2, P = torch.ops.npu.w4a8_gemm_partials(a_q, a_s, wt, st, N, K, G)
    torch.cuda.synchronize()
    aq, as_ = gv("pt_aq")[:rows], gv("pt_as")[:rows]
    assert np.array_equal(a_q.cpu().numpy(), aq) and np.array_equal(tensor_bf16_bits(a_s), as_)
    codes = unpacked(gv("pt_wq"), K, G)
    assert np.array_equal(P.cpu().numpy().astype(np.int64), ow.group_partials(aq, codes, G))
    ws32 = ow.bf16_bits_to_f32(gv("pt_ws")).T.copy()
    y32 = ow.gemm_fp32(aq, as_, codes, ws32, G)
    for got in (tensor_bf16_bits(y), tensor_bf16_bits(yl), tensor_bf16_bits(y2)):
        bar_and_equal(got, gv("pt_y")[:rows], y32, lambda r, c: ow.gemm_f64(aq[r], as_[r], codes[c], ws32[c], G))

    Mc, Kc, Nc = (int(v) for v in gv("pc_shape"))
    wsc = torch.from_numpy(gv("pc_ws").reshape(1, Nc).view(np.int16)).view(torch.bfloat16).to(dev)
    wtc, stc = torch.ops.npu.w4a8_repack(torch.from_numpy(gv("pc_wq")).to(dev), wsc, Kc, Kc)
    xc = torch.from_numpy(gv("pc_x")[:rows].view(np.int16)).view(torch.bfloat16).to(dev)
    yc = torch.ops.npu.w4a8_linear(xc, wtc, stc, Nc, Kc, Kc)
    torch.cuda.synchronize()
    aqc, asc = gv("pc_aq")[:rows], gv("pc_as")[:rows]
    codes_c = unpacked(gv("pc_wq"), Kc, Kc)
    ws32c = ow.bf16_bits_to_f32(gv("pc_ws"))[:, None].astype(np.float32)
    y32c = ow.gemm_fp32(aqc, asc, codes_c, ws32c, Kc)
    bar_and_equal(tensor_bf16_bits(yc), gv("pc_y")[:rows], y32c,
                  lambda r, c: ow.gemm_f64(aqc[r], asc[r], codes_c[c], ws32c[c], Kc))
