"""w4a8_rope_kv: the decoder's rotary embedding + KV-cache append in one kernel.

Bar: bit-identical to the torch evaluation it replaces -- the projection bias
added as a bf16 add, q and k rotated with fp32 products and sums on float
tensors (rotate-half form), rounded to bf16, then k written at [b, h, :, p] of
the transposed K cache and v at [b, h, p, :]
-- for decode (one token at a device-held position), prefill (many tokens from
position 0 and from an offset), a token range crossing the cache end (q zero,
nothing written past it), a K cache given as a strided view, and replays of a
captured step that advances the position on the device.
"""
from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, T, heads, D] bf16, cos/sin [T, D/2] fp32 -> bf16 (torch's float-tensor evaluation)."""
    h = x.shape[-1] // 2
    xf = x.float()
    x1, x2 = xf[..., :h], xf[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).to(torch.bfloat16)


def tables(L, D, dev, theta=1.0e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = torch.arange(L, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang), torch.sin(ang)


def reference(qkv, cos, sin, p0, kc, vc, H, KVH, bias=None):
    """The torch path: (q, k_cache', v_cache') for tokens at p0 .. p0+T-1 (all inside the cache),
    the projection bias added first as a bf16 add."""
    if bias is not None:
        qkv = qkv + bias
    B, T, W = qkv.shape
    D = W // (H + 2 * KVH)
    x = qkv.view(B, T, H + 2 * KVH, D)
    c, s = cos[p0:p0 + T], sin[p0:p0 + T]
    q = rope_ref(x[:, :, :H], c, s)
    k = rope_ref(x[:, :, H:H + KVH], c, s)
    v = x[:, :, H + KVH:]
    kc, vc = kc.clone(), vc.clone()
    kc[:, :, :, p0:p0 + T] = k.permute(0, 2, 3, 1)
    vc[:, :, p0:p0 + T, :] = v.permute(0, 2, 1, 3)
    return q, kc, vc


def bits_equal(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def make(B, T, H, KVH, D, L, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = (torch.randn((B, T, (H + 2 * KVH) * D), device=dev, generator=g) * 3).to(torch.bfloat16)
    kc = torch.randn((B, KVH, D, L), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((B, KVH, L, D), device=dev, generator=g).to(torch.bfloat16)
    return qkv, kc, vc


@pytest.mark.parametrize("B,T,H,KVH,D,L,p0,with_bias", [
    (2, 1, 40, 8, 128, 64, 17, True),      # QwQ-32B heads (qkv bias), one decode token
    (1, 1, 40, 8, 128, 1280, 1279, True),  # the last slot of a 1024 + 256 cache
    (3, 37, 40, 8, 128, 48, 0, True),      # prefill from position 0
    (2, 23, 4, 2, 64, 40, 5, False),       # small heads, no bias, prefill after 5 cached tokens
    (2, 1, 4, 2, 64, 40, 9, False),
])
def test_rope_kv_matches_torch(pkg, dev, B, T, H, KVH, D, L, p0, with_bias):
    say(f"rope_kv B={B} T={T} H={H} KVH={KVH} D={D} L={L} p0={p0} bias={with_bias}")
    qkv, kc, vc = make(B, T, H, KVH, D, L, dev, seed=B * 1000 + T)
    cos, sin = tables(L, D, dev)
    bias = None
    if with_bias:
        g = torch.Generator(device=dev).manual_seed(99)
        bias = ((torch.rand(((H + 2 * KVH) * D,), device=dev, generator=g) - 0.5) * 0.2).to(torch.bfloat16)
    q_ref, kc_ref, vc_ref = reference(qkv, cos, sin, p0, kc, vc, H, KVH, bias)
    pos = torch.tensor([p0], dtype=torch.int64, device=dev)
    q = torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, pos, kc, vc, H, KVH, bias)
    torch.cuda.synchronize()
    assert q.shape == (B, T, H, D)
    assert bits_equal(q, q_ref)
    assert bits_equal(kc, kc_ref)
    assert bits_equal(vc, vc_ref)


def test_rope_kv_stops_at_the_cache_end(pkg, dev):
    B, T, H, KVH, D, L = 2, 5, 4, 2, 64, 20
    say("rope_kv tokens crossing the cache end")
    qkv, kc, vc = make(B, T, H, KVH, D, L, dev, seed=7)
    cos, sin = tables(L, D, dev)
    p0 = L - 2                                        # tokens 0, 1 fit; 2, 3, 4 fall past L
    q_ref, kc_ref, vc_ref = reference(qkv[:, :2], cos, sin, p0, kc, vc, H, KVH)
    q = torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, torch.tensor([p0], device=dev), kc, vc, H, KVH)
    torch.cuda.synchronize()
    assert bits_equal(q[:, :2], q_ref)
    assert torch.count_nonzero(q[:, 2:].view(torch.int16)) == 0
    assert bits_equal(kc, kc_ref) and bits_equal(vc, vc_ref)


def test_rope_kv_strided_k_cache(pkg, dev):
    """A K cache handed over as a transposed view of a [B, KVH, L, D] buffer."""
    B, T, H, KVH, D, L, p0 = 2, 3, 8, 2, 128, 16, 4
    say("rope_kv strided K cache view")
    qkv, kc, vc = make(B, T, H, KVH, D, L, dev, seed=11)
    cos, sin = tables(L, D, dev)
    q_ref, kc_ref, vc_ref = reference(qkv, cos, sin, p0, kc, vc, H, KVH)
    k_store = kc.permute(0, 1, 3, 2).contiguous()     # [B, KVH, L, D]
    k_view = k_store.permute(0, 1, 3, 2)              # [B, KVH, D, L], non-contiguous
    q = torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, torch.tensor([p0], device=dev), k_view, vc, H, KVH)
    torch.cuda.synchronize()
    assert bits_equal(q, q_ref)
    assert bits_equal(k_view, kc_ref) and bits_equal(vc, vc_ref)


def test_rope_kv_graph_replays_follow_the_position(pkg, dev):
    """Captured once; each replay reads the position from the device and the step advances it."""
    B, H, KVH, D, L = 2, 40, 8, 128, 32
    say("rope_kv graph replays")
    qkv, kc, vc = make(B, 1, H, KVH, D, L, dev, seed=13)
    cos, sin = tables(L, D, dev)
    pos = torch.tensor([3], dtype=torch.int64, device=dev)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_out = torch.empty((B, 1, H, D), dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        q_out.copy_(torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, pos, kc, vc, H, KVH))   # warm-up at position 3
        pos.add_(1)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    q_ref, kc_ref, vc_ref = reference(qkv, cos, sin, 3, kc_ref, vc_ref, H, KVH)
    assert bits_equal(q_out, q_ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        q_out.copy_(torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, pos, kc, vc, H, KVH))
        pos.add_(1)
    # capture does not run the step: the position is still 4
    for p in range(4, 9):
        g.replay()
        torch.cuda.synchronize()
        _ = torch.ones(100, device=dev).sum().item()      # eager work between replays
        q_ref, kc_ref, vc_ref = reference(qkv, cos, sin, p, kc_ref, vc_ref, H, KVH)
        assert bits_equal(q_out, q_ref), f"replay at position {p}"
        assert bits_equal(kc, kc_ref) and bits_equal(vc, vc_ref), f"caches after position {p}"
    assert int(pos.item()) == 9
