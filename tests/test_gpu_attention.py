"""w4a8_attention (csrc/attention.hip) against a float64 CPU reference.

Bars:
  * every output within 2^-8 * sum_t w_t |v_t| + 1 bf16 ulp of the float64 value
    (w = the exact softmax weights): the kernel rounds the probabilities to bf16
    (2^-9 relative) for the product with V and the output to bf16, every other
    step is fp32; rel-L2 over a call <= 4e-3;
  * the decode launch (one workgroup per split + combine) and the prefill launch
    (one workgroup walks every split) return the same bits for the same rows;
  * a captured decode launch replayed with the position advanced on the device
    equals the eager launch at that position.
"""
from __future__ import annotations

import math
import os
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_inputs(dev, B, T, H, KVH, D, L, seed, q_scale=1.0):
    Lc = -(-L // 64) * 64
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn((B, T, H, D), generator=g, device=dev) * q_scale).to(torch.bfloat16)
    k = torch.randn((B, KVH, Lc, D), generator=g, device=dev).to(torch.bfloat16)
    vt = torch.randn((B, KVH, D, Lc), generator=g, device=dev).to(torch.bfloat16)
    # positions past L hold what an unused cache slot holds: zeros
    k[:, :, L:] = 0
    vt[:, :, :, L:] = 0
    return q, k, vt, Lc


def reference(q, k, vt, pos0, L, scale=None):
    """float64 outputs [B, T, H, D] and the magnitudes sum_t w_t |v_t|."""
    B, T, H, D = q.shape
    KVH = k.shape[1]
    G = H // KVH
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    qd, kd, vd = q.double().cpu(), k.double().cpu(), vt.double().cpu().transpose(2, 3)   # v [B, KVH, Lc, D]
    out = torch.empty((B, T, H, D), dtype=torch.float64)
    mag = torch.empty_like(out)
    for t in range(T):
        p = min(max(pos0 + t, 0), L - 1)
        for h in range(KVH):
            qs = qd[:, t, h * G:(h + 1) * G]                                  # [B, G, D]
            s = torch.einsum("bgd,bld->bgl", qs, kd[:, h, :p + 1]) * sc
            w = torch.softmax(s, dim=-1)
            out[:, t, h * G:(h + 1) * G] = torch.einsum("bgl,bld->bgd", w, vd[:, h, :p + 1])
            mag[:, t, h * G:(h + 1) * G] = torch.einsum("bgl,bld->bgd", w, vd[:, h, :p + 1].abs())
    return out, mag


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def check(got, ref, mag, tag):
    g = got.double().cpu()
    err = (g - ref).abs()
    bound = 2.0 ** -8 * mag + bf16_ulp(ref)
    worst = (err / bound).max().item()
    rel = ((g - ref).norm() / ref.norm()).item()
    say(f"  {tag}: max err/bound {worst:.3f}, rel-L2 {rel:.2e}")
    assert torch.all(err <= bound), f"{tag}: {int((err > bound).sum())} outputs outside the bound"
    assert rel <= 4e-3, f"{tag}: rel-L2 {rel}"


def attn(q, k, vt, pos, L, cps, split, scale=None):
    return torch.ops.npu.w4a8_attention(q, k, vt, pos, L, cps, split, scale)


CASES = [
    # (B, T, H, KVH, D, L, note)
    (2, 12, 4, 2, 64, 40, "tiny decoder shape, one chunk"),
    (2, 150, 40, 8, 128, 300, "QwQ heads, prompt of 150 in a 300-position cache"),
    (1, 70, 48, 2, 128, 128, "24 query heads per KV head: rows straddle 16-row tiles"),
    (3, 33, 16, 1, 64, 200, "16 query heads per KV head: one tile per token"),
]


@pytest.mark.parametrize("B,T,H,KVH,D,L,note", CASES)
def test_prefill_matches_reference_and_decode_bits(pkg, dev, B, T, H, KVH, D, L, note):
    say(f"attention prefill B={B} T={T} H={H} KVH={KVH} D={D} L={L} ({note})")
    q, k, vt, Lc = make_inputs(dev, B, T, H, KVH, D, L, seed=B + T + H)
    pos0 = torch.zeros((1,), dtype=torch.int64, device=dev)
    for cps in sorted({1, pkg.ops.attention_chunks_per_split(B, H, KVH, Lc), Lc // 64}):
        pre = attn(q, k, vt, pos0, L, cps, split=False)
        ref, mag = reference(q, k, vt, 0, L)
        check(pre, ref, mag, f"prefill cps={cps}")
        # the split launch over the same T rows: same bits
        spl = attn(q, k, vt, pos0, L, cps, split=True)
        assert torch.equal(pre, spl), f"split launch differs from the prefill launch (cps={cps})"
        # token by token, as decode steps at position t: same bits as the prefill's row t
        for t in sorted({0, 1, T // 2, T - 1}):
            pt = torch.full((1,), t, dtype=torch.int64, device=dev)
            dec = attn(q[:, t:t + 1].contiguous(), k, vt, pt, L, cps, split=True)
            assert torch.equal(dec[:, 0], pre[:, t]), f"decode at position {t} differs from prefill row {t}"
    torch.cuda.synchronize()


@pytest.mark.parametrize("B", [1, 8, 64])
def test_decode_qwq_cache(pkg, dev, B):
    """QwQ-32B heads over a 1280-position cache at the decoder bench's batch sizes, at
    positions on and off chunk and split boundaries."""
    H, KVH, D, L = 40, 8, 128, 1280
    say(f"attention decode B={B} over {L} positions")
    q, k, vt, Lc = make_inputs(dev, B, 1, H, KVH, D, L, seed=B)
    cps = pkg.ops.attention_chunks_per_split(B, H, KVH, Lc)
    for p in (0, 63, 64, 319, 320, 700, 1279):
        pt = torch.full((1,), p, dtype=torch.int64, device=dev)
        dec = attn(q, k, vt, pt, L, cps, split=True)
        nb = min(B, 4)     # the reference on a few sequences (the CPU loop is the cost)
        ref, mag = reference(q[:nb], k[:nb], vt[:nb], p, L)
        check(dec[:nb], ref, mag, f"B={B} pos={p} cps={cps}")
        pre = attn(q, k, vt, pt, L, cps, split=False)
        assert torch.equal(dec, pre), f"pos {p}: split and loop launches differ"


def test_large_scores_and_scale(pkg, dev):
    """Scores of magnitude ~100 (the running maximum moves between chunks and most
    probabilities underflow), and an explicit softmax scale."""
    B, T, H, KVH, D, L = 2, 100, 8, 2, 128, 260
    q, k, vt, Lc = make_inputs(dev, B, T, H, KVH, D, L, seed=11, q_scale=8.0)
    pos0 = torch.zeros((1,), dtype=torch.int64, device=dev)
    for scale in (None, 0.3):
        say(f"attention large scores, scale={scale}")
        ref, mag = reference(q, k, vt, 0, L, scale)
        for cps in (1, 2):
            pre = attn(q, k, vt, pos0, L, cps, False, scale)
            check(pre, ref, mag, f"scale={scale} cps={cps}")
            assert torch.equal(pre, attn(q, k, vt, pos0, L, cps, True, scale))


def test_positions_clamp_to_cache(pkg, dev):
    """pos[0] + t past L - 1 attends to the whole cache, a negative position to position 0."""
    B, H, KVH, D, L = 2, 8, 2, 64, 100
    q, k, vt, Lc = make_inputs(dev, B, 3, H, KVH, D, L, seed=5)
    say("attention position clamp")
    for p, eff in ((L + 5, L - 1), (-3, 0)):
        pt = torch.full((1,), p, dtype=torch.int64, device=dev)
        got = attn(q, k, vt, pt, L, 1, split=True)
        ref, mag = reference(q, k, vt, p, L)
        check(got, ref, mag, f"pos {p}")
        same = attn(q, k, vt, torch.full((1,), eff, dtype=torch.int64, device=dev), L, 1, split=True)
        if p > 0:   # every token clamps to L - 1
            assert torch.equal(got[:, 0], same[:, 0])


def test_decode_launch_in_a_graph(pkg, dev):
    """The split launch (workspace + combine) captured once and replayed at advancing
    positions, with eager work between replays: every replay equals the eager launch."""
    B, H, KVH, D, L = 4, 40, 8, 128, 512
    q, k, vt, Lc = make_inputs(dev, B, 1, H, KVH, D, L, seed=21)
    cps = pkg.ops.attention_chunks_per_split(B, H, KVH, Lc)
    pos = torch.zeros((1,), dtype=torch.int64, device=dev)
    say(f"attention decode in a graph, cps={cps}")
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        out = attn(q, k, vt, pos, L, cps, split=True)           # warm-up (workspace for this stream)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        out = attn(q, k, vt, pos, L, cps, split=True)
    torch.cuda.synchronize()
    for p in (3, 64, 200, 511, 130):
        pos.fill_(p)
        gr.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1000, device=dev).sum().item()
        eager = attn(q, k, vt, torch.full((1,), p, dtype=torch.int64, device=dev), L, cps, split=True)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay at position {p} differs"


@pytest.mark.parametrize("B,H,KVH,D,L,bias", [
    (1, 40, 8, 128, 1280, True),     # QwQ decode, one sequence
    (8, 40, 8, 128, 1280, True),
    (64, 40, 8, 128, 1280, True),    # one split
    (2, 4, 2, 64, 40, False),        # tiny decoder shape
    (3, 48, 2, 128, 300, True),      # 24 query heads per KV head: two row tiles per pair
])
def test_attention_rope_equals_rope_kv_then_attention(pkg, dev, B, H, KVH, D, L, bias):
    """The fused decode launch (rotary embedding of q and of the step's k, KV append, attention)
    returns the bits of w4a8_rope_kv followed by w4a8_attention(split=True), and leaves the
    caches as w4a8_rope_kv leaves them, at positions on and off chunk and split boundaries,
    the last one, and one past the cache (nothing written, zero query)."""
    say(f"attention + rope B={B} H={H} KVH={KVH} D={D} L={L} bias={bias}")
    g = torch.Generator(device=dev).manual_seed(B + H + L)
    W = (H + 2 * KVH) * D
    Lc = -(-L // 64) * 64
    k0 = torch.randn((B, KVH, Lc, D), generator=g, device=dev).to(torch.bfloat16)
    v0 = torch.randn((B, KVH, D, Lc), generator=g, device=dev).to(torch.bfloat16)
    inv = 1.0 / (1.0e4 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = torch.arange(L, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    bvec = ((torch.rand((W,), generator=g, device=dev) - 0.5) * 0.2).to(torch.bfloat16) if bias else None
    cps = pkg.ops.attention_chunks_per_split(B, H, KVH, Lc)
    for p in sorted({0, 63, 64, L // 2, L - 1, L}):
        qkv = torch.randn((B, W), generator=g, device=dev).to(torch.bfloat16)
        pos = torch.full((1,), p, dtype=torch.int64, device=dev)
        # reference: rope_kv into copies of the caches, then the split attention
        k1, v1 = k0.clone(), v0.clone()
        q = torch.ops.npu.w4a8_rope_kv(qkv.view(B, 1, W), cos, sin, pos, k1[:, :, :L].transpose(2, 3),
                                       v1[..., :L].transpose(2, 3), H, KVH, bvec)
        ref = torch.ops.npu.w4a8_attention(q, k1, v1, pos, L, cps, True)
        k2, v2 = k0.clone(), v0.clone()
        got = torch.ops.npu.w4a8_attention_rope(qkv, cos, sin, pos, k2, v2, H, KVH, L, cps, bvec)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"position {p}: output differs from rope_kv + attention"
        assert torch.equal(k2, k1) and torch.equal(v2, v1), f"position {p}: caches differ from rope_kv's"


@pytest.mark.parametrize("B", [1, 8, 64])
def test_attention_relaunch_deterministic(pkg, dev, B):
    """The decode launches (split + combine, split alone, the fused rotary form) and the
    prefill launch relaunched 20 times with other work between: identical bits."""
    H, KVH, D, L = 40, 8, 128, 1280
    say(f"attention relaunch B={B}")
    q, k, vt, Lc = make_inputs(dev, B, 1, H, KVH, D, L, seed=B + 3)
    pos = torch.full((1,), 1000, dtype=torch.int64, device=dev)
    cps = pkg.ops.attention_chunks_per_split(B, H, KVH, Lc)
    qp, kp, vp, _ = make_inputs(dev, 1 if B == 64 else B, 200, H, KVH, D, 256, seed=B + 4)
    pos0 = torch.zeros((1,), dtype=torch.int64, device=dev)
    g = torch.Generator(device=dev).manual_seed(B)
    qkv = torch.randn((B, (H + 2 * KVH) * D), generator=g, device=dev).to(torch.bfloat16)
    inv = 1.0 / (1.0e4 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = torch.arange(L, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    runs = [lambda: attn(q, k, vt, pos, L, cps, True), lambda: attn(qp, kp, vp, pos0, 256, 1, False),
            lambda: torch.ops.npu.w4a8_attention_rope(qkv, cos, sin, pos, k, vt, H, KVH, L, cps)]
    for fn in runs:
        first = fn()
        for i in range(20):
            y = fn()
            junk = torch.full((1 << 18,), i, dtype=torch.int32, device=dev)
            assert torch.equal(y, first), f"B={B}: relaunch {i} differs"
            del junk
    torch.cuda.synchronize()


def random_attention_shapes(seed: int, n: int):
    """n seeded (B, T, H, KVH, D, L, pos0) draws: 1-6 sequences, 1-40 tokens, 1-20 query
    heads per KV head (tiles of 16 rows straddled or not), head_dim 64 or 128, caches of
    1-700 positions (one chunk to eleven), the first token anywhere in the cache."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        KVH = int(rng.integers(1, 5))
        G = int(rng.integers(1, 21))
        D = int(rng.choice([64, 128]))
        L = int(rng.integers(1, 701))
        T = int(rng.integers(1, min(40, L) + 1))
        pos0 = int(rng.integers(0, L - T + 1))
        out.append((int(rng.integers(1, 7)), T, KVH * G, KVH, D, L, pos0))
    return out


@pytest.mark.parametrize("B,T,H,KVH,D,L,pos0",
                         random_attention_shapes(5, 16 * max(1, int(os.environ.get("W4A8_RANDOM_SCALE", "1")))))
def test_attention_random_shapes(pkg, dev, B, T, H, KVH, D, L, pos0):
    """Seeded random shapes: both launches within the bound of the float64 attention and
    equal to each other bit for bit, at the library's split size and at one chunk per split."""
    say(f"attention random B={B} T={T} H={H} KVH={KVH} D={D} L={L} pos0={pos0}")
    q, k, vt, Lc = make_inputs(dev, B, T, H, KVH, D, L, seed=B * 31 + T + L)
    pos = torch.full((1,), pos0, dtype=torch.int64, device=dev)
    ref, mag = reference(q, k, vt, pos0, L)
    for cps in sorted({1, pkg.ops.attention_chunks_per_split(B, H, KVH, Lc)}):
        pre = attn(q, k, vt, pos, L, cps, split=False)
        check(pre, ref, mag, f"cps={cps}")
        assert torch.equal(pre, attn(q, k, vt, pos, L, cps, split=True)), f"split launch differs (cps={cps})"


def test_attention_rejects_bad_arguments(pkg, dev):
    q, k, vt, Lc = make_inputs(dev, 1, 1, 4, 2, 64, 64, seed=1)
    pos = torch.zeros((1,), dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError, match="chunks_per_split"):
        attn(q, k, vt, pos, 64, 2, split=True)
    with pytest.raises(RuntimeError, match="cache"):
        attn(q, k, vt, pos, 65, 1, split=True)
    with pytest.raises(RuntimeError, match="caches must be"):
        attn(q, k, vt[:, :, :32].contiguous(), pos, 64, 1, split=False)
