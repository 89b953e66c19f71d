"""The allocation-free GEMM (w4a8_gemm_noalloc) against w4a8_gemm, through the C ABI.

Bar: bit-identical outputs (the same kernels on the same K split; only the
memory holding the fp32 split sums differs), on two calls in a row that use
the static scratch, the second with fewer rows, then on a shape that needs no
scratch; a shape whose split sums exceed the scratch is refused before any
launch.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits_tensor
from oracle import w4a8 as ow

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _weights(pkg, dev, N, K, G, seed):
    synth = pkg.synth
    w = synth.weight_codes_uniform(N, K, seed)
    sb = synth.group_scales(N, ow.num_groups(K, G), seed + 1, "bf16")
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.ops.npu.w4a8_repack(torch.from_numpy(ow.pack_grouped(w, G)).to(dev), w_scale, K, G)


def _noalloc(lib, dev, a_q, a_s, wt, st, N, K, G):
    M = a_q.shape[0]
    y = torch.full((M, N), -1.0, dtype=torch.bfloat16, device=dev)   # every output must be written
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = lib.w4a8_gemm_noalloc(a_q.data_ptr(), a_q.stride(0), a_s.data_ptr(), wt.data_ptr(), st.data_ptr(),
                               1, y.data_ptr(), N, M, N, K, G, stream)
    assert rc == 0, lib.w4a8_last_error()
    return y


def test_gemm_noalloc_matches_gemm(pkg, dev):
    lib = pkg._abi.lib()
    K, N, G = 27648, 5120, 128          # down_proj: K split over workgroups past 8 rows
    wt, st = _weights(pkg, dev, N, K, G, seed=31)
    for M in (64, 16):                  # the second call is smaller and reuses the scratch
        need = lib.w4a8_gemm_workspace_bytes(M, N, K, G)
        assert 0 < need <= pkg._abi.NOALLOC_SCRATCH_BYTES
        say(f"noalloc down_proj M={M} (split sums {need} B in the static scratch)")
        x = bf16_bits_tensor(pkg.synth.activations(M, K, seed=32 + M)).to(dev)
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
        ref = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)
        got = _noalloc(lib, dev, a_q, a_s, wt, st, N, K, G)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"M={M}: differs from w4a8_gemm"
    # a shape without a K split takes no scratch
    K2, N2 = 5120, 7168
    wt2, st2 = _weights(pkg, dev, N2, K2, G, seed=33)
    assert lib.w4a8_gemm_workspace_bytes(4, N2, K2, G) == 0
    say("noalloc qkv_proj M=4 (no scratch)")
    x = bf16_bits_tensor(pkg.synth.activations(4, K2, seed=34)).to(dev)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
    ref = torch.ops.npu.w4a8_gemm(a_q, a_s, wt2, st2, N2, K2, G)
    got = _noalloc(lib, dev, a_q, a_s, wt2, st2, N2, K2, G)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_gemm_noalloc_refuses_shapes_beyond_the_scratch(pkg, dev):
    lib = pkg._abi.lib()
    M, N, K, G = 64, 8320, 16384, 128
    need = lib.w4a8_gemm_workspace_bytes(M, N, K, G)
    assert need > pkg._abi.NOALLOC_SCRATCH_BYTES, need
    say(f"noalloc refusal: M={M} N={N} K={K} needs {need} B")
    y = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    # nothing is launched: the operand pointers are never read
    rc = lib.w4a8_gemm_noalloc(16, K, 16, 16, 16, 1, y.data_ptr(), N, M, N, K, G, None)
    assert rc == 6 and b"static scratch" in lib.w4a8_last_error()
    torch.cuda.synchronize()
    assert not y.view(torch.int16).any()
