"""Bitwise regression digests of the HIP path's outputs (GPU only).

The reference pins kernel changes old-against-new bit for bit
(npu_ops/python/test_pad_regress.py:1-18): a kernel rewrite must reproduce the
previous build's output bytes, not only stay inside a tolerance.  This script
runs one seeded case per kernel path of this build (activation quant, the
staged, per-tile and row-group decode plans, the wide and K-split decode
kernels, the fused single-row linear, the SwiGLU epilogue, per-channel scales,
both prefill tile shapes at group 128 and the prefill at group 256, the
reference-compat pair at decode sizes, on wide N and at prefill sizes, with
and without the partial dump) and
records the SHA-256 of each output's bytes.
tests/test_gpu_regress.py recomputes them and fails on any changed bit.

Every input is drawn by numpy from fixed seeds (the same bytes on every host),
and the plans depend on the GPU's compute-unit count, which is recorded with
the digests.  A change that alters output bits on purpose (a new fold order, a
new plan) must pass the parity suite first; then regenerate:

    python tests/golden/make_regress.py tests/golden/output_digests.json
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def _bf16(bits: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _digest(*tensors) -> str:
    import torch
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().cpu().contiguous().view(-1).view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def _weights(pkg, dev, N, K, G, seed):
    import torch
    from oracle import w4a8 as ow
    synth = pkg.synth
    w = synth.weight_codes_uniform(N, K, seed)
    sb = synth.group_scales(N, ow.num_groups(K, G), seed + 1, "f16")
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.float16)
    w_q = torch.from_numpy(ow.pack_grouped(w, G)).to(dev)
    return torch.ops.npu.w4a8_repack(w_q, w_scale.to(dev), K, G)


def _gemm_case(M, N, K, G, seed, op="gemm"):
    def run(pkg, dev):
        import torch
        xb = pkg.synth.activations(M, K, seed)
        wt, st = _weights(pkg, dev, N, K, G, seed + 7)
        x = _bf16(xb).to(dev)
        if op == "linear":
            y = torch.ops.npu.w4a8_linear(x, wt, st, N, K, G)
            return _digest(y)
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
        if op == "swiglu":
            y = torch.ops.npu.w4a8_gemm_swiglu(a_q, a_s, wt, st, N, K, G)
        else:
            y = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)
        return _digest(y)
    return run


def _quant_case(M, K, seed):
    def run(pkg, dev):
        import torch
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(_bf16(pkg.synth.activations(M, K, seed)).to(dev))
        return _digest(a_q, a_s)
    return run


def _midgroup_case(M, N, K, G, seed, partials=False):
    def run(pkg, dev):
        import torch
        from oracle import w4a8 as ow
        xb = pkg.synth.activations(M, K, seed)
        w = np.random.default_rng(seed + 1).standard_normal((N, K)).astype(np.float32) * np.float32(0.05)
        codes, sc, zr, ks = ow.quantize_weight_asym(w, G)
        a = torch.ops.npu.midgroup_quant_a(_bf16(xb).to(dev), G)
        args = (torch.from_numpy(ow.pack_grouped(codes, G)).to(dev), _bf16(sc).to(dev),
                torch.from_numpy(ks).to(dev), _bf16(zr).to(dev))
        if partials:
            return _digest(*a, *torch.ops.npu.midgroup_w4a8_gemm_partials(*a, *args, K, G))
        y = torch.ops.npu.midgroup_w4a8_gemm(*a, *args, K, G)
        return _digest(*a, y)
    return run


# name -> (kernel path it pins, runner)
CASES = {
    "quant_m64_k5120": ("quant_act_vec_kernel", _quant_case(64, 5120, 1)),
    "gemm_m4_o_proj": ("gemm_decode_kernel, staged activations", _gemm_case(4, 5120, 5120, 128, 2)),
    "gemm_m16_qkv_proj": ("gemm_decode_kernel, per-tile activations", _gemm_case(16, 7168, 5120, 128, 3)),
    "gemm_m64_o_proj": ("gemm_decode_kernel, 32-row groups", _gemm_case(64, 5120, 5120, 128, 4)),
    "gemm_m16_wide_n": ("gemm_wide_kernel, 16 rows", _gemm_case(16, 32768, 1024, 128, 5)),
    "gemm_m64_wide_n": ("gemm_wide_kernel, 64 rows", _gemm_case(64, 32768, 1024, 128, 6)),
    "gemm_m16_long_k": ("gemm_wide_kernel K split + wide_reduce_kernel", _gemm_case(16, 1024, 16384, 128, 7)),
    "gemm_m48_long_k_psplit": ("gemm_prefill_cols_kernel 64-row tile K split + wide_reduce_kernel",
                               _gemm_case(48, 1000, 16384, 128, 17)),
    "linear_m1_qkv_proj": ("linear_decode_kernel (fused quant)", _gemm_case(1, 7168, 5120, 128, 8, op="linear")),
    "swiglu_m16": ("SwiGLU epilogue", _gemm_case(16, 2048, 1024, 128, 9, op="swiglu")),
    "gemm_m4_perchannel": ("one group over K", _gemm_case(4, 5120, 5120, 5120, 10)),
    "gemm_m2048_prefill_g128": ("gemm_prefill_cols_kernel (128-row tiles)", _gemm_case(2048, 2048, 1024, 128, 11)),
    "gemm_m512_prefill_g128": ("gemm_prefill_kernel, 64-row tiles", _gemm_case(512, 1024, 1024, 128, 12)),
    "gemm_m2048_prefill_g256": ("gemm_prefill_kernel, group 256", _gemm_case(2048, 2048, 1024, 256, 13)),
    "midgroup_m16_g1024": ("compat quant_a + mid-group GEMM", _midgroup_case(16, 2048, 4096, 1024, 14)),
    "midgroup_m512_g1024": ("compat GEMM prefill path: compat_act_kernel + gemm_prefill_kernel (CM = 2)",
                            _midgroup_case(512, 2048, 4096, 1024, 15)),
    "midgroup_m512_g1024_partials": ("compat mid-group GEMM, 64x64 tiles with the partial dump",
                                     _midgroup_case(512, 2048, 4096, 1024, 15, partials=True)),
    "midgroup_m16_wide_n": ("compat mid-group GEMM, shared-activation decode", _midgroup_case(16, 16384, 2048, 1024, 16)),
}


def cu_count() -> int:
    import torch
    return int(torch.cuda.get_device_properties(0).multi_processor_count)


def compute(pkg, dev) -> dict:
    import torch
    out = {}
    for name, (_, run) in CASES.items():
        print(f"regress case {name}", flush=True)
        out[name] = run(pkg, dev)
        torch.cuda.synchronize()
    return out


def main(path: str) -> None:
    import torch
    import __graft_entry__ as ge
    pkg = ge.package()
    dev = torch.device("cuda:0")
    doc = {"cu_count": cu_count(), "paths": {k: v[0] for k, v in CASES.items()}, "digests": compute(pkg, dev)}
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {len(doc['digests'])} digests to {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else str(Path(__file__).with_name("output_digests.json")))
