"""Writes tests/golden/reference_vectors.npz: input/output vectors of the reference's
own C++ CPU reference -- TEST INFRASTRUCTURE.

The outputs come from the reference's code compiled where it lies
(int4_cube_lab/host/gemm_ref.cpp, bf16.h, int4_cube_lab/kernels/mg_kgeom.h, built
into oracle/_ref by oracle/Makefile); the inputs are seeded synthetic data made
here.  The reference's activation quantiser (int4_cube_lab/host/quant_harness.h)
needs ACL and is not built, so the activation codes stored as GEMM inputs come
from the oracle's per-token / per-group quantiser (pinned separately by exact
rational arithmetic).  Run in the build container, where /root/reference exists:

    make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref as oref  # noqa: E402
from oracle import w4a8 as ow  # noqa: E402

OUT = Path(__file__).resolve().parent / "reference_vectors.npz"
GEOM_CASES = [(5120, 128), (27648, 128), (1057, 1024), (3456, 1024), (100, 33), (1057, 96), (232, 192),
              (5000, 128), (1, 1024), (2049, 1024), (640, 1024), (900, 256)]


def activations(M, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, max(1, K // 1000), replace=False)] *= 20.0
    return ow.f32_to_bf16_bits(x)


def main() -> None:
    if not oref.available():
        raise SystemExit("oracle/_ref is not built: run `make -C oracle` where /root/reference exists")
    rng = np.random.default_rng(2026)
    out = {}

    # 1. per-token activations, symmetric group-128 weight (configs[0]'s path at
    #    a fixture size): ReferenceMidGroupGemm with the token scale in every group
    M, K, N, G = 16, 1024, 256, 128
    xb = activations(M, K, 1)
    aq, as_ = ow.quant_act_per_token(xb)
    codes = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    ws = ow.f32_to_bf16_bits(rng.uniform(0.002, 0.02, size=(ow.num_groups(K, G), N)).astype(np.float32))
    out.update(pt_x=xb, pt_aq=aq, pt_as=as_, pt_wq=oref.pack_int4_grouped(codes, G), pt_ws=ws,
               pt_y=oref.midgroup_gemm(aq, np.repeat(as_[None, :], ws.shape[0], axis=0), codes, ws, G),
               pt_shape=np.array([M, K, N, G]))

    # 2. the reference's own mid-group path: ragged K at group 1024, asymmetric
    #    weight with zero points, per-group activation scales; its plane
    #    splitter and ksums as well
    M, K, N, G = 5, 2049, 128, 1024
    xb = activations(M, K, 2)
    aq, as_g = ow.quant_act_midgroup(xb, G)
    w = rng.standard_normal((N, K)).astype(np.float32) * 0.04
    wcodes, wsc, wzr, _ = ow.quantize_weight_asym(ow.bf16_bits_to_f32(ow.f32_to_bf16_bits(w)), G)
    hi, lo = oref.split_planes_grouped(aq, G)
    out.update(mg_x=xb, mg_aq=aq, mg_as=as_g, mg_wq=oref.pack_int4_grouped(wcodes, G), mg_ws=wsc, mg_wz=wzr,
               mg_hi=hi, mg_lo=lo, mg_aksum=oref.act_ksum_neg(aq, G), mg_wksum=oref.weight_ksum(wcodes, G),
               mg_y=oref.midgroup_gemm(aq, as_g, wcodes, wsc, G, wzr), mg_shape=np.array([M, K, N, G]))

    # 3. per-channel (one group spanning K): ReferencePerchannelGemm
    M, K, N = 8, 5120, 128
    xb = activations(M, K, 3)
    aq, as_ = ow.quant_act_per_token(xb)
    codes = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    wsn = ow.f32_to_bf16_bits(rng.uniform(0.002, 0.02, size=(N,)).astype(np.float32))
    out.update(pc_x=xb, pc_aq=aq, pc_as=as_, pc_wq=oref.pack_int4_grouped(codes, K), pc_ws=wsn,
               pc_y=oref.perchannel_gemm(aq, as_, codes, wsn), pc_shape=np.array([M, K, N]))

    # 4. group geometry of mg_kgeom.h: (K, group, G, kpad, offset of the last group)
    geo = []
    for K, G in GEOM_CASES:
        ng = oref.num_groups(K, G)
        geo.append([K, G, ng, oref.kpad(K, G), oref.group_offset(ng - 1, G), oref.group_real(ng - 1, K, G)])
    out["geometry"] = np.array(geo, np.int64)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
