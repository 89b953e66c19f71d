"""torch.ops.npu.* -- the W4A8 op surface on PyTorch-ROCm.

Keeps the reference's registration namespace ``npu`` (the reference defines
its ops with TORCH_LIBRARY_FRAGMENT(npu, ...), npu_ops/host/midgroup_quant_a.cpp:87-91
and npu_ops/host/midgroup_w4a8_gemm.cpp:149-153) and adds the per-token /
group-size-parameterised ops of this build:

    torch.ops.npu.w4a8_quant_pertoken(x, group=0) -> (a_q, a_scale)
    torch.ops.npu.w4a8_repack(w_q, w_scale, K, group) -> (w_tiles, s_tiles)
    torch.ops.npu.w4a8_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group) -> y
    torch.ops.npu.w4a8_gemm_partials(a_q, a_scale, w_tiles, s_tiles, N, K, group) -> (y, partials)
    torch.ops.npu.w4a8_gemm_swiglu(a_q, a_scale, w_tiles, s_tiles, N, K, group) -> y [M, N/2]
    torch.ops.npu.w4a8_linear(x, w_tiles, s_tiles, N, K, group) -> y   (quant + GEMM)

and two producer-side helpers of the decoder forward that drives them:

    torch.ops.npu.w4a8_rmsnorm_quant(x, weight, eps, residual=None, group=0, want_normed=False)
        -> (a_q, a_scale, s, h)
    torch.ops.npu.w4a8_rope_kv(qkv, cos, sin, pos, k_cache, v_cache, heads, kv_heads, bias=None) -> q
    torch.ops.npu.w4a8_attention(q, k_cache, vt_cache, pos, L, chunks_per_split, split=False, scale=None) -> out
    torch.ops.npu.w4a8_attention_rope(qkv, cos, sin, pos, k_cache, vt_cache, heads, kv_heads, L,
                                      chunks_per_split, bias=None, scale=None) -> out   (decode step: rope_kv fused in)

and, with the reference's own names and schemas (group appended with the
reference's fixed value as default), its mid-group compat pair:

    torch.ops.npu.midgroup_quant_a(x, group=1024) -> [a_hi, a_lo, a_scale, a_ksum]
    torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero,
                                     K, group=1024, rows=-1) -> y   (rows >= 0: only the first rows)
    torch.ops.npu.midgroup_w4a8_gemm_partials(...) -> (y, partials)   (parity hook)

and the same GEMM on a weight reordered once at load time (1 KB tiles, the
same bytes; what the compat linear module and vLLM method keep):

    torch.ops.npu.midgroup_tile_weights(w_q, K, group=1024) -> w_tiles
    torch.ops.npu.midgroup_w4a8_gemm_tiled(a_hi, a_lo, a_scale, a_ksum, w_tiles, w_scale, w_ksum, w_zero,
                                           N, K, group=1024, rows=-1) -> y

Only the CUDA (= HIP on ROCm) dispatch key and fake (meta) kernels are
registered: CPU tensors raise, there is no fallback path.  Each impl checks
dtypes and shapes like the reference's host impls (TORCH_CHECK ->
RuntimeError, npu_ops/host/midgroup_w4a8_gemm.cpp:51-85), allocates outputs
with torch, and calls the C ABI on the current stream without synchronising.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Tuple

import torch

from . import _abi
from . import geometry as geo

_LIB = torch.library.Library("npu", "FRAGMENT")
_LIB.define("w4a8_quant_pertoken(Tensor x, int group=0) -> (Tensor, Tensor)")
_LIB.define("w4a8_repack(Tensor w_q, Tensor w_scale, int K, int group) -> (Tensor, Tensor)")
_LIB.define("w4a8_gemm(Tensor a_q, Tensor a_scale, Tensor w_tiles, Tensor s_tiles, "
            "int N, int K, int group) -> Tensor")
_LIB.define("w4a8_gemm_partials(Tensor a_q, Tensor a_scale, Tensor w_tiles, Tensor s_tiles, "
            "int N, int K, int group) -> (Tensor, Tensor)")
_LIB.define("w4a8_gemm_swiglu(Tensor a_q, Tensor a_scale, Tensor w_tiles, Tensor s_tiles, "
            "int N, int K, int group) -> Tensor")
_LIB.define("w4a8_linear(Tensor x, Tensor w_tiles, Tensor s_tiles, int N, int K, int group) -> Tensor")
_LIB.define("w4a8_rmsnorm_quant(Tensor x, Tensor weight, float eps, Tensor? residual=None, int group=0, "
            "bool want_normed=False) -> (Tensor, Tensor, Tensor, Tensor)")
_LIB.define("w4a8_rope_kv(Tensor qkv, Tensor cos, Tensor sin, Tensor pos, Tensor(a!) k_cache, Tensor(b!) v_cache, "
            "int heads, int kv_heads, Tensor? bias=None) -> Tensor")
_LIB.define("w4a8_attention(Tensor q, Tensor k_cache, Tensor vt_cache, Tensor pos, int L, int chunks_per_split, "
            "bool split=False, float? scale=None) -> Tensor")
_LIB.define("w4a8_attention_rope(Tensor qkv, Tensor cos, Tensor sin, Tensor pos, Tensor(a!) k_cache, "
            "Tensor(b!) vt_cache, int heads, int kv_heads, int L, int chunks_per_split, Tensor? bias=None, "
            "float? scale=None) -> Tensor")
_LIB.define("midgroup_quant_a(Tensor x, int group=1024) -> Tensor[]")
_LIB.define("midgroup_w4a8_gemm(Tensor a_hi, Tensor a_lo, Tensor a_scale, Tensor a_ksum, Tensor w_q, "
            "Tensor w_scale, Tensor w_ksum, Tensor w_zero, int K, int group=1024, int rows=-1) -> Tensor")
_LIB.define("midgroup_w4a8_gemm_partials(Tensor a_hi, Tensor a_lo, Tensor a_scale, Tensor a_ksum, Tensor w_q, "
            "Tensor w_scale, Tensor w_ksum, Tensor w_zero, int K, int group=1024) -> (Tensor, Tensor)")
_LIB.define("midgroup_tile_weights(Tensor w_q, int K, int group=1024) -> Tensor")
_LIB.define("midgroup_w4a8_gemm_tiled(Tensor a_hi, Tensor a_lo, Tensor a_scale, Tensor a_ksum, Tensor w_tiles, "
            "Tensor w_scale, Tensor w_ksum, Tensor w_zero, int N, int K, int group=1024, int rows=-1) -> Tensor")

_SCALE_DT = {torch.float16: _abi.W4A8_DT_F16, torch.bfloat16: _abi.W4A8_DT_BF16}


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


# One workspace per (device, stream), allocated only when the library asks
# for one (decode shapes that split K over workgroups); it only grows.  Eager
# calls on one stream are stream-ordered, so sharing per stream is safe.
_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}
# Calls captured into a HIP graph get a workspace of that capture instead:
# the graph may be replayed on any stream, while eager calls keep using the
# stream's own, so the two never share memory.  Calls inside one graph run in
# its captured order and share the capture's workspace.
_CAPTURE_WS: Dict[Tuple[int, int], torch.Tensor] = {}
# Workspaces replaced by a larger one stay allocated: a captured HIP graph
# keeps the address it was captured with, so that memory must never return
# to the caching allocator (nor may a capture's own workspace).
_RETIRED: list = []

def _capture_id(stream_handle: int) -> int:
    """The HIP capture sequence id of a stream that is being captured, asked
    through the W4A8 library (bound to the HIP runtime the process loaded)."""
    cid = ctypes.c_ulonglong(0)
    rc = _abi.lib().w4a8_stream_capture_id(ctypes.c_void_p(stream_handle), ctypes.byref(cid))
    if rc != 0:
        raise RuntimeError(f"w4a8: could not read the capture id of stream {stream_handle:#x}: "
                           f"{_abi.lib().w4a8_last_error().decode('utf-8', 'replace')}")
    return int(cid.value)


def _workspace(dev: torch.device, need: int) -> torch.Tensor:
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(dev).cuda_stream
    if torch.cuda.is_current_stream_capturing():
        table, key = _CAPTURE_WS, (index, _capture_id(stream))
    else:
        table, key = _WORKSPACES, (index, stream)
    ws = table.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _RETIRED.append(ws)
        # no clearing needed: the split GEMM writes every sum the reduce reads
        ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=dev)
        table[key] = ws
    return ws


# ---------------------------------------------------------------- quant
def _quant_width(K: int, group: int) -> int:
    # group > 0: the GEMM's padded group layout (kpad == K when nothing is padded)
    return geo.kpad(K, group) if group > 0 else K


@torch.library.impl(_LIB, "w4a8_quant_pertoken", "CUDA")
def _quant_pertoken_cuda(x: torch.Tensor, group: int = 0):
    """a_q [M, K] (group 0) or [M, kpad(K, group)] in the padded group layout
    the GEMM reads (padding slots zero), and a_scale bf16 [M]."""
    _require(x.dim() == 2, "w4a8_quant_pertoken: x must be [M, K]")
    _require(x.dtype == torch.bfloat16, "w4a8_quant_pertoken: x must be bfloat16")
    _require(group >= 0, "w4a8_quant_pertoken: group must be >= 0")
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    width = _quant_width(K, group)
    a_q = torch.empty((M, width), dtype=torch.int8, device=x.device)
    a_scale = torch.empty((M,), dtype=torch.bfloat16, device=x.device)
    if M:
        _abi.check(_abi.lib().w4a8_quant_act(x.data_ptr(), x.stride(0), a_q.data_ptr(), width,
                                             a_scale.data_ptr(), M, K, group, _stream(x.device)),
                   "w4a8_quant_pertoken")
    return a_q, a_scale


@torch.library.register_fake("npu::w4a8_quant_pertoken")
def _quant_pertoken_fake(x, group=0):
    M, K = x.shape
    return (x.new_empty((M, _quant_width(K, group)), dtype=torch.int8),
            x.new_empty((M,), dtype=torch.bfloat16))


# ---------------------------------------------------------------- repack
def _check_ref_weight(w_q, w_scale, K, group):
    _require(w_q.dim() == 2 and w_q.dtype in (torch.int8, torch.uint8),
             "w4a8_repack: w_q must be a 2-D int8 [N, kpad/2] packed-int4 tensor")
    _require(w_scale.dtype in _SCALE_DT, "w4a8_repack: w_scale must be float16 or bfloat16")
    N = w_q.shape[0]
    G = geo.num_groups(K, group)
    _require(w_q.shape[1] == geo.kpad(K, group) // 2,
             f"w4a8_repack: packed row length must be kpad/2 = {geo.kpad(K, group) // 2} "
             f"for K={K}, group={group}; got {w_q.shape[1]}")
    _require(tuple(w_scale.shape) == (G, N), f"w4a8_repack: w_scale must be group-major [{G}, {N}]")
    return N, G


@torch.library.impl(_LIB, "w4a8_repack", "CUDA")
def _repack_cuda(w_q: torch.Tensor, w_scale: torch.Tensor, K: int, group: int):
    N, G = _check_ref_weight(w_q, w_scale, K, group)
    w_q = w_q.contiguous()
    w_scale = w_scale.contiguous()
    w_tiles = torch.empty((geo.repacked_weight_bytes(N, K, group),), dtype=torch.uint8, device=w_q.device)
    s_tiles = torch.empty(geo.repacked_scale_shape(N, K, group), dtype=w_scale.dtype, device=w_q.device)
    _abi.check(_abi.lib().w4a8_repack(w_q.data_ptr(), w_scale.data_ptr(), _SCALE_DT[w_scale.dtype],
                                      w_tiles.data_ptr(), s_tiles.data_ptr(), N, K, group,
                                      _stream(w_q.device)), "w4a8_repack")
    return w_tiles, s_tiles


@torch.library.register_fake("npu::w4a8_repack")
def _repack_fake(w_q, w_scale, K, group):
    N = w_q.shape[0]
    return (w_q.new_empty((geo.repacked_weight_bytes(N, K, group),), dtype=torch.uint8),
            w_scale.new_empty(geo.repacked_scale_shape(N, K, group)))


# ---------------------------------------------------------------- gemm
def _check_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group):
    _require(a_q.dim() == 2 and a_q.dtype == torch.int8, "w4a8_gemm: a_q must be int8 [M, kpad]")
    _require(a_q.shape[1] == geo.kpad(K, group),
             f"w4a8_gemm: a_q has {a_q.shape[1]} columns; the padded group layout of K={K}, "
             f"group={group} has {geo.kpad(K, group)} (w4a8_quant_pertoken(x, group))")
    _require(a_scale.dtype == torch.bfloat16 and a_scale.dim() == 1 and a_scale.shape[0] == a_q.shape[0],
             "w4a8_gemm: a_scale must be bfloat16 [M]")
    _require(w_tiles.dtype == torch.uint8 and w_tiles.numel() == geo.repacked_weight_bytes(N, K, group),
             "w4a8_gemm: w_tiles must be the uint8 output of w4a8_repack for (N, K, group)")
    _require(s_tiles.dtype in _SCALE_DT and tuple(s_tiles.shape) == geo.repacked_scale_shape(N, K, group),
             "w4a8_gemm: s_tiles must be the scale output of w4a8_repack for (N, K, group)")


def _run_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group, partials, swiglu=False):
    _check_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group)
    if swiglu:
        _require(N % 32 == 0, f"w4a8_gemm_swiglu: N={N} must be 2*I with I a multiple of 16")
    if a_q.stride(1) != 1 or a_q.stride(0) % 16:
        a_q = a_q.contiguous()
    a_scale = a_scale.contiguous()
    M = a_q.shape[0]
    dev = a_q.device
    ncols = N // 2 if swiglu else N
    y = torch.empty((M, ncols), dtype=torch.bfloat16, device=dev)
    if M == 0:
        return y
    lib = _abi.lib()
    need = lib.w4a8_gemm_workspace_bytes(M, N, K, group)
    ws = _workspace(dev, need) if need > 0 else None
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    args_head = (a_q.data_ptr(), a_q.stride(0), a_scale.data_ptr(), w_tiles.data_ptr(), s_tiles.data_ptr(),
                 _SCALE_DT[s_tiles.dtype], y.data_ptr(), ncols)
    if swiglu:
        st = lib.w4a8_gemm_swiglu(*args_head, M, N, K, group, ws_ptr, ws_bytes, _stream(dev))
    elif partials is None:
        st = lib.w4a8_gemm(*args_head, M, N, K, group, ws_ptr, ws_bytes, _stream(dev))
    else:
        st = lib.w4a8_gemm_debug_partials(*args_head, partials.data_ptr(), M, N, K, group, ws_ptr, ws_bytes,
                                          _stream(dev))
    _abi.check(st, "w4a8_gemm")
    return y


@torch.library.impl(_LIB, "w4a8_gemm", "CUDA")
def _gemm_cuda(a_q, a_scale, w_tiles, s_tiles, N: int, K: int, group: int):
    return _run_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group, None)


@torch.library.register_fake("npu::w4a8_gemm")
def _gemm_fake(a_q, a_scale, w_tiles, s_tiles, N, K, group):
    return a_q.new_empty((a_q.shape[0], N), dtype=torch.bfloat16)


@torch.library.impl(_LIB, "w4a8_gemm_swiglu", "CUDA")
def _gemm_swiglu_cuda(a_q, a_scale, w_tiles, s_tiles, N: int, K: int, group: int):
    """silu(y[:, :N/2]) * y[:, N/2:] of the merged gate/up GEMM, fused."""
    return _run_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group, None, swiglu=True)


@torch.library.register_fake("npu::w4a8_gemm_swiglu")
def _gemm_swiglu_fake(a_q, a_scale, w_tiles, s_tiles, N, K, group):
    return a_q.new_empty((a_q.shape[0], N // 2), dtype=torch.bfloat16)


@torch.library.impl(_LIB, "w4a8_gemm_partials", "CUDA")
def _gemm_partials_cuda(a_q, a_scale, w_tiles, s_tiles, N: int, K: int, group: int):
    M = a_q.shape[0]
    partials = torch.empty((geo.num_groups(K, group), M, N), dtype=torch.int32, device=a_q.device)
    y = _run_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group, partials)
    return y, partials


@torch.library.register_fake("npu::w4a8_gemm_partials")
def _gemm_partials_fake(a_q, a_scale, w_tiles, s_tiles, N, K, group):
    M = a_q.shape[0]
    return (a_q.new_empty((M, N), dtype=torch.bfloat16),
            a_q.new_empty((geo.num_groups(K, group), M, N), dtype=torch.int32))


# ---------------------------------------------------------------- quant + GEMM
@torch.library.impl(_LIB, "w4a8_linear", "CUDA")
def _linear_cuda(x: torch.Tensor, w_tiles, s_tiles, N: int, K: int, group: int):
    """The W4A8 dynamic linear of bf16 x [M, K]: w4a8_quant_pertoken(x, group) then
    w4a8_gemm, bit for bit, with the quant fused into the GEMM kernel for a
    single row (midgroup_quant.py:163-177 is the reference's pair of calls)."""
    _require(x.dim() == 2 and x.dtype == torch.bfloat16, "w4a8_linear: x must be bfloat16 [M, K]")
    _require(x.shape[1] == K, f"w4a8_linear: x has {x.shape[1]} columns, K={K}")
    if x.stride(1) != 1:
        x = x.contiguous()
    M = x.shape[0]
    dev = x.device
    width = geo.kpad(K, group)
    a_q = torch.empty((M, width), dtype=torch.int8, device=dev)
    a_scale = torch.empty((M,), dtype=torch.bfloat16, device=dev)
    _check_gemm(a_q, a_scale, w_tiles, s_tiles, N, K, group)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if M == 0:
        return y
    lib = _abi.lib()
    need = lib.w4a8_gemm_workspace_bytes(M, N, K, group)
    ws = _workspace(dev, need) if need > 0 else None
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    _abi.check(lib.w4a8_linear(x.data_ptr(), x.stride(0), w_tiles.data_ptr(), s_tiles.data_ptr(),
                               _SCALE_DT[s_tiles.dtype], y.data_ptr(), N, a_q.data_ptr(), width,
                               a_scale.data_ptr(), M, N, K, group, ws_ptr, ws_bytes, _stream(dev)),
               "w4a8_linear")
    return y


@torch.library.register_fake("npu::w4a8_linear")
def _linear_fake(x, w_tiles, s_tiles, N, K, group):
    return x.new_empty((x.shape[0], N), dtype=torch.bfloat16)


# ---------------------------------------------------------------- RMSNorm + quant
@torch.library.impl(_LIB, "w4a8_rmsnorm_quant", "CUDA")
def _rmsnorm_quant_cuda(x: torch.Tensor, weight: torch.Tensor, eps: float, residual=None, group: int = 0,
                        want_normed: bool = False):
    """(a_q, a_scale, s, h): the per-token quant of h = rms_norm(s) * weight, s = x + residual
    (s is empty without a residual -- the stream is x itself; h is empty unless want_normed)."""
    _require(x.dim() == 2 and x.dtype == torch.bfloat16, "w4a8_rmsnorm_quant: x must be bfloat16 [M, K]")
    M, K = x.shape
    _require(weight.dtype == torch.bfloat16 and tuple(weight.shape) == (K,),
             "w4a8_rmsnorm_quant: weight must be bfloat16 [K]")
    if x.stride(1) != 1 or x.stride(0) % 8:
        x = x.contiguous()
    weight = weight.contiguous()
    dev = x.device
    if residual is not None:
        _require(residual.dtype == torch.bfloat16 and residual.shape == x.shape,
                 "w4a8_rmsnorm_quant: residual must match x")
        if residual.stride(1) != 1 or residual.stride(0) % 8:
            residual = residual.contiguous()
        s = torch.empty_like(x)
    else:
        s = x.new_empty((0, K))
    width = _quant_width(K, group)
    a_q = torch.empty((M, width), dtype=torch.int8, device=dev)
    a_scale = torch.empty((M,), dtype=torch.bfloat16, device=dev)
    h = torch.empty((M, K) if want_normed else (0, K), dtype=torch.bfloat16, device=dev)
    if M:
        _abi.check(_abi.lib().w4a8_rmsnorm_quant(
            x.data_ptr(), x.stride(0), residual.data_ptr() if residual is not None else None,
            residual.stride(0) if residual is not None else 0, weight.data_ptr(), float(eps),
            s.data_ptr() if residual is not None else None, K, h.data_ptr() if want_normed else None, K,
            a_q.data_ptr(), width, a_scale.data_ptr(), M, K, group, _stream(dev)), "w4a8_rmsnorm_quant")
    return a_q, a_scale, s, h


@torch.library.register_fake("npu::w4a8_rmsnorm_quant")
def _rmsnorm_quant_fake(x, weight, eps, residual=None, group=0, want_normed=False):
    M, K = x.shape
    return (x.new_empty((M, _quant_width(K, group)), dtype=torch.int8), x.new_empty((M,), dtype=torch.bfloat16),
            x.new_empty((M, K) if residual is not None else (0, K)), x.new_empty((M, K) if want_normed else (0, K)))


# ---------------------------------------------------------------- RoPE + KV-cache append
@torch.library.impl(_LIB, "w4a8_rope_kv", "CUDA")
def _rope_kv_cuda(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
                  k_cache: torch.Tensor, v_cache: torch.Tensor, heads: int, kv_heads: int,
                  bias=None) -> torch.Tensor:
    """q [B, T, heads, D]: the rotated q heads of qkv [B, T, (heads + 2 kv_heads) * D] (+ bias, a bf16
    add); the rotated k heads go to k_cache [B, kv_heads, D, L] and the v heads to v_cache
    [B, kv_heads, L, D] at positions pos[0] + t (any strides; cos/sin fp32 [>= L, >= D/2] angle tables)."""
    _require(qkv.dim() == 3 and qkv.dtype == torch.bfloat16, "w4a8_rope_kv: qkv must be bfloat16 [B, T, W]")
    B, T, W = qkv.shape
    _require(heads > 0 and kv_heads > 0 and W % (heads + 2 * kv_heads) == 0,
             "w4a8_rope_kv: qkv width must be (heads + 2 kv_heads) * head_dim")
    D = W // (heads + 2 * kv_heads)
    _require(D % 2 == 0, "w4a8_rope_kv: head_dim must be even")
    _require(k_cache.dim() == 4 and v_cache.dim() == 4 and k_cache.dtype == torch.bfloat16
             and v_cache.dtype == torch.bfloat16, "w4a8_rope_kv: caches must be 4-D bfloat16")
    L = k_cache.shape[3]
    _require(tuple(k_cache.shape) == (B, kv_heads, D, L) and tuple(v_cache.shape) == (B, kv_heads, L, D),
             "w4a8_rope_kv: caches must be k [B, kv_heads, D, L] and v [B, kv_heads, L, D]")
    for t, name in ((cos, "cos"), (sin, "sin")):
        _require(t.dim() == 2 and t.dtype == torch.float32 and t.shape[0] >= L and t.shape[1] >= D // 2
                 and t.stride(1) == 1, f"w4a8_rope_kv: {name} must be float32 [>= L, >= head_dim / 2]")
    _require(cos.stride(0) == sin.stride(0), "w4a8_rope_kv: cos and sin must share a row stride")
    _require(pos.dtype == torch.int64 and pos.numel() == 1 and pos.device == qkv.device,
             "w4a8_rope_kv: pos must be one int64 on the device (the position of token 0, shared by every "
             "sequence; per-sequence positions are not supported)")
    if qkv.stride(2) != 1 or qkv.stride(0) != T * qkv.stride(1):
        qkv = qkv.contiguous()
    if bias is not None:
        _require(bias.dtype == torch.bfloat16 and bias.numel() == W and bias.device == qkv.device,
                 "w4a8_rope_kv: bias must be bfloat16 [(heads + 2 kv_heads) * head_dim] on the device")
        bias = bias.contiguous()
    q = torch.empty((B, T, heads, D), dtype=torch.bfloat16, device=qkv.device)
    if B * T:
        ks = (ctypes.c_int64 * 4)(*k_cache.stride())
        vs = (ctypes.c_int64 * 4)(*v_cache.stride())
        _abi.check(_abi.lib().w4a8_rope_kv(
            qkv.data_ptr(), qkv.stride(1), bias.data_ptr() if bias is not None else None, cos.data_ptr(),
            sin.data_ptr(), cos.stride(0), L, pos.data_ptr(),
            q.data_ptr(), k_cache.data_ptr(), ks, v_cache.data_ptr(), vs, B, T, heads, kv_heads, D,
            _stream(qkv.device)), "w4a8_rope_kv")
    return q


@torch.library.register_fake("npu::w4a8_rope_kv")
def _rope_kv_fake(qkv, cos, sin, pos, k_cache, v_cache, heads, kv_heads, bias=None):
    B, T, W = qkv.shape
    return qkv.new_empty((B, T, heads, W // (heads + 2 * kv_heads)))


# ---------------------------------------------------------------- attention over the KV cache
def attention_chunks_per_split(batch: int, heads: int, kv_heads: int, cache_len: int) -> int:
    """The split size (in chunks of 64 positions) the library picks for a decode step of
    `batch` sequences over a cache axis of cache_len positions (a multiple of 64)."""
    cps = _abi.lib().w4a8_attention_chunks_per_split(batch, heads, kv_heads, cache_len)
    _require(cps > 0, f"w4a8_attention: bad shape for the split size (B={batch}, H={heads}, KVH={kv_heads}, "
             f"Lc={cache_len})")
    return int(cps)


@torch.library.impl(_LIB, "w4a8_attention", "CUDA")
def _attention_cuda(q: torch.Tensor, k_cache: torch.Tensor, vt_cache: torch.Tensor, pos: torch.Tensor, L: int,
                    chunks_per_split: int, split: bool = False, scale=None) -> torch.Tensor:
    """out [B, T, H, D]: query rows q [B, T, H, D] over k_cache [B, KVH, Lc, D] and the
    transposed values vt_cache [B, KVH, D, Lc]; token t attends to positions 0 .. pos[0] + t
    (clamped to [0, L)).  split=True runs one workgroup per split plus a combine kernel
    (decode), split=False one workgroup per row tile (prefill): the same bits either way."""
    _require(q.dim() == 4 and q.dtype == torch.bfloat16, "w4a8_attention: q must be bfloat16 [B, T, H, D]")
    B, T, H, D = q.shape
    _require(k_cache.dim() == 4 and vt_cache.dim() == 4 and k_cache.dtype == torch.bfloat16
             and vt_cache.dtype == torch.bfloat16, "w4a8_attention: caches must be 4-D bfloat16")
    KVH, Lc = k_cache.shape[1], k_cache.shape[2]
    _require(tuple(k_cache.shape) == (B, KVH, Lc, D) and tuple(vt_cache.shape) == (B, KVH, D, Lc),
             "w4a8_attention: caches must be k [B, kv_heads, Lc, D] and vt [B, kv_heads, D, Lc]")
    _require(k_cache.is_contiguous() and vt_cache.is_contiguous(), "w4a8_attention: caches must be contiguous")
    _require(pos.dtype == torch.int64 and pos.numel() == 1 and pos.device == q.device,
             "w4a8_attention: pos must be one int64 on the device")
    q = q.contiguous()
    out = torch.empty_like(q)
    if B * T == 0:
        return out
    sc = float(scale) if scale is not None else 1.0 / float(D) ** 0.5
    lib = _abi.lib()
    ws_ptr, ws_bytes = None, 0
    if split:
        need = lib.w4a8_attention_workspace_bytes(B, T, H, D, Lc, chunks_per_split)
        _require(need >= 0, "w4a8_attention: bad shape for the workspace size")
        ws = _workspace(q.device, max(need, 16))
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    _abi.check(lib.w4a8_attention(q.data_ptr(), k_cache.data_ptr(), vt_cache.data_ptr(), out.data_ptr(),
                                  pos.data_ptr(), B, T, H, KVH, D, L, Lc, chunks_per_split, sc, ws_ptr, ws_bytes,
                                  _stream(q.device)), "w4a8_attention")
    return out


@torch.library.register_fake("npu::w4a8_attention")
def _attention_fake(q, k_cache, vt_cache, pos, L, chunks_per_split, split=False, scale=None):
    return torch.empty_like(q)


@torch.library.impl(_LIB, "w4a8_attention_rope", "CUDA")
def _attention_rope_cuda(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
                         k_cache: torch.Tensor, vt_cache: torch.Tensor, heads: int, kv_heads: int, L: int,
                         chunks_per_split: int, bias=None, scale=None) -> torch.Tensor:
    """A decode step's attention with w4a8_rope_kv fused in: qkv [B, (heads + 2 kv_heads) * D]
    (one token per sequence), the q heads rotated in the kernel, the step's rotated k and raw
    v (+ bias) used at position pos[0] and appended to k_cache [B, KVH, Lc, D] / vt_cache
    [B, KVH, D, Lc] there; returns out [B, 1, heads, D] -- the bits of w4a8_rope_kv followed
    by w4a8_attention(split=True)."""
    _require(qkv.dim() == 2 and qkv.dtype == torch.bfloat16, "w4a8_attention_rope: qkv must be bfloat16 [B, W]")
    B, W = qkv.shape
    _require(heads > 0 and kv_heads > 0 and W % (heads + 2 * kv_heads) == 0,
             "w4a8_attention_rope: qkv width must be (heads + 2 kv_heads) * head_dim")
    D = W // (heads + 2 * kv_heads)
    _require(k_cache.dim() == 4 and vt_cache.dim() == 4 and k_cache.dtype == torch.bfloat16
             and vt_cache.dtype == torch.bfloat16, "w4a8_attention_rope: caches must be 4-D bfloat16")
    Lc = k_cache.shape[2]
    _require(tuple(k_cache.shape) == (B, kv_heads, Lc, D) and tuple(vt_cache.shape) == (B, kv_heads, D, Lc)
             and k_cache.is_contiguous() and vt_cache.is_contiguous(),
             "w4a8_attention_rope: caches must be contiguous k [B, kv_heads, Lc, D] and vt [B, kv_heads, D, Lc]")
    for t, name in ((cos, "cos"), (sin, "sin")):
        _require(t.dim() == 2 and t.dtype == torch.float32 and t.shape[0] >= L and t.shape[1] >= D // 2
                 and t.stride(1) == 1, f"w4a8_attention_rope: {name} must be float32 [>= L, >= head_dim / 2]")
    _require(cos.stride(0) == sin.stride(0), "w4a8_attention_rope: cos and sin must share a row stride")
    _require(pos.dtype == torch.int64 and pos.numel() == 1 and pos.device == qkv.device,
             "w4a8_attention_rope: pos must be one int64 on the device")
    if qkv.stride(1) != 1 or qkv.stride(0) % 8:
        qkv = qkv.contiguous()
    if bias is not None:
        _require(bias.dtype == torch.bfloat16 and bias.numel() == W and bias.device == qkv.device,
                 "w4a8_attention_rope: bias must be bfloat16 [(heads + 2 kv_heads) * head_dim] on the device")
        bias = bias.contiguous()
    out = torch.empty((B, 1, heads, D), dtype=torch.bfloat16, device=qkv.device)
    if B == 0:
        return out
    sc = float(scale) if scale is not None else 1.0 / float(D) ** 0.5
    lib = _abi.lib()
    need = lib.w4a8_attention_workspace_bytes(B, 1, heads, D, Lc, chunks_per_split)
    _require(need >= 0, "w4a8_attention_rope: bad shape for the workspace size")
    ws = _workspace(qkv.device, max(need, 16))
    _abi.check(lib.w4a8_attention_rope(qkv.data_ptr(), qkv.stride(0), bias.data_ptr() if bias is not None else None,
                                       cos.data_ptr(), sin.data_ptr(), cos.stride(0), k_cache.data_ptr(),
                                       vt_cache.data_ptr(), out.data_ptr(), pos.data_ptr(), B, heads, kv_heads, D, L,
                                       Lc, chunks_per_split, sc, ws.data_ptr(), ws.numel(), _stream(qkv.device)),
               "w4a8_attention_rope")
    return out


@torch.library.register_fake("npu::w4a8_attention_rope")
def _attention_rope_fake(qkv, cos, sin, pos, k_cache, vt_cache, heads, kv_heads, L, chunks_per_split, bias=None,
                         scale=None):
    B, W = qkv.shape
    return qkv.new_empty((B, 1, heads, W // (heads + 2 * kv_heads)))


# ---------------------------------------------------------------- mid-group compat pair
def tile_m_for(M: int) -> int:
    """Row padding unit of the reference's compat pair (npu_ops/host/midgroup_quant_a.cpp:37)."""
    return 16 if M <= 16 else (64 if M <= 64 else 128)


def _padded_rows(M: int) -> int:
    t = tile_m_for(M)
    return -(-M // t) * t


@torch.library.impl(_LIB, "midgroup_quant_a", "CUDA")
def _midgroup_quant_a_cuda(x: torch.Tensor, group: int = 1024):
    """The reference's run_midgroup_quant_a (npu_ops/host/midgroup_quant_a.cpp:40-78):
    a_hi/a_lo int8 [Mp, kpad/2], a_scale bf16 [G, Mp], a_ksum int32 [G, Mp]."""
    _require(x.dim() == 2, "midgroup_quant_a: x must be [M, K]")
    _require(x.dtype == torch.bfloat16, "midgroup_quant_a: x must be bfloat16")
    _require(group > 0, "midgroup_quant_a: group must be > 0")
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    G, kb = geo.num_groups(K, group), geo.kpad(K, group) // 2
    Mp = _padded_rows(M) if M else 0
    dev = x.device
    a_hi = torch.empty((Mp, kb), dtype=torch.int8, device=dev)
    a_lo = torch.empty((Mp, kb), dtype=torch.int8, device=dev)
    a_scale = torch.empty((G, Mp), dtype=torch.bfloat16, device=dev)
    a_ksum = torch.empty((G, Mp), dtype=torch.int32, device=dev)
    if Mp:
        _abi.check(_abi.lib().w4a8_midgroup_quant_a(x.data_ptr(), x.stride(0), a_hi.data_ptr(), a_lo.data_ptr(),
                                                    a_scale.data_ptr(), a_ksum.data_ptr(), M, Mp, K, group,
                                                    _stream(dev)), "midgroup_quant_a")
    return [a_hi, a_lo, a_scale, a_ksum]


@torch.library.register_fake("npu::midgroup_quant_a")
def _midgroup_quant_a_fake(x, group=1024):
    M, K = x.shape
    G, kb = geo.num_groups(K, group), geo.kpad(K, group) // 2
    Mp = _padded_rows(M) if M else 0
    return [x.new_empty((Mp, kb), dtype=torch.int8), x.new_empty((Mp, kb), dtype=torch.int8),
            x.new_empty((G, Mp), dtype=torch.bfloat16), x.new_empty((G, Mp), dtype=torch.int32)]


def _check_midgroup(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group):
    # the reference's checks (npu_ops/host/midgroup_w4a8_gemm.cpp:51-85); N % 128 is not required here
    _require(a_hi.dim() == 2 and a_lo.dim() == 2 and w_q.dim() == 2,
             "midgroup_w4a8_gemm: a_hi/a_lo [M,K/2] and w_q [N,K/2] must be 2-D")
    _require(a_hi.dtype == torch.int8 and a_lo.dtype == torch.int8 and w_q.dtype == torch.int8,
             "midgroup_w4a8_gemm: packed int4 planes must be int8 tensors")
    _require(a_scale.dtype == torch.bfloat16 and w_scale.dtype == torch.bfloat16 and w_zero.dtype == torch.bfloat16,
             "midgroup_w4a8_gemm: a_scale/w_scale/w_zero must be bfloat16")
    _require(a_ksum.dtype == torch.int32 and w_ksum.dtype == torch.int32,
             "midgroup_w4a8_gemm: a_ksum/w_ksum must be int32")
    kb = geo.kpad(K, group) // 2
    _require(a_hi.shape[1] == kb and a_lo.shape == a_hi.shape and w_q.shape[1] == kb,
             f"midgroup_w4a8_gemm: packed row length must be Kpad/2 = {kb} for K={K} (group-padded layout); "
             f"got a_hi {a_hi.shape[1]} w_q {w_q.shape[1]}")
    M, N, G = a_hi.shape[0], w_q.shape[0], geo.num_groups(K, group)
    _require(a_scale.dim() == 2 and a_scale.shape[0] == G and a_scale.shape[1] >= M and a_ksum.shape == a_scale.shape,
             "midgroup_w4a8_gemm: a_scale/a_ksum must be group-major [K/group, M]")
    _require(tuple(w_scale.shape) == (G, N) and tuple(w_zero.shape) == (G, N) and tuple(w_ksum.shape) == (G, N),
             "midgroup_w4a8_gemm: w_scale/w_zero/w_ksum must be group-major [K/group, N]")
    return M, N, G


def _run_midgroup(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group, partials: bool,
                  rows: int = -1, tiles_n: int = -1):
    if tiles_n >= 0:
        # w_q holds midgroup_tile_weights' tiles of an [N, kpad/2] weight
        nbytes = _abi.lib().w4a8_midgroup_tiles_bytes(tiles_n, K, group)
        _require(w_q.dtype == torch.int8 and w_q.numel() == nbytes and w_q.is_contiguous(),
                 f"midgroup_w4a8_gemm_tiled: w_tiles must be the {nbytes} int8 bytes of midgroup_tile_weights")
        shape_ref = torch.empty((tiles_n, geo.kpad(K, group) // 2), dtype=torch.int8, device="meta")
        M, N, G = _check_midgroup(a_hi, a_lo, a_scale, a_ksum, shape_ref, w_scale, w_ksum, w_zero, K, group)
    else:
        M, N, G = _check_midgroup(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group)
    if rows >= 0:
        # the first `rows` rows only (the real rows before quant_a's padding):
        # the padding rows' activation planes are then never read
        _require(rows <= M, f"midgroup_w4a8_gemm: rows={rows} exceeds the {M} activation rows")
        M = rows
    a_hi, a_lo, w_q = a_hi.contiguous(), a_lo.contiguous(), w_q.contiguous()
    a_scale, a_ksum = a_scale.contiguous(), a_ksum.contiguous()
    w_scale, w_zero = w_scale.contiguous(), w_zero.contiguous()
    dev = a_hi.device
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    P = torch.empty((G, M, N), dtype=torch.int32, device=dev) if partials else None
    if M:
        # w_ksum is validated but not read: the activation bytes are rebuilt
        # exactly from the two planes, so the kernel needs no +8 correction.
        # Prefill sizes get a workspace for the rebuilt rows, allocated per
        # call as the reference host allocates its GEMM workspace
        # (npu_ops/host/midgroup_w4a8_gemm.cpp:116-118).
        need = 0 if partials else _abi.lib().w4a8_midgroup_gemm_workspace_bytes(M, N, K, group)
        ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
        entry = _abi.lib().w4a8_midgroup_gemm_tiled if tiles_n >= 0 else _abi.lib().w4a8_midgroup_gemm_ws
        _abi.check(entry(a_hi.data_ptr(), a_lo.data_ptr(), a_scale.data_ptr(),
                                                    a_ksum.data_ptr(), M, a_scale.stride(0), w_q.data_ptr(),
                                                    w_scale.data_ptr(), w_zero.data_ptr(), y.data_ptr(), N,
                                                    P.data_ptr() if P is not None else None, N, K, group,
                                                    ws.data_ptr() if ws is not None else None, need,
                                                    _stream(dev)), "midgroup_w4a8_gemm")
    return (y, P) if partials else y


@torch.library.impl(_LIB, "midgroup_w4a8_gemm", "CUDA")
def _midgroup_gemm_cuda(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K: int, group: int = 1024,
                        rows: int = -1):
    """The reference's run_midgroup_w4a8_gemm (npu_ops/host/midgroup_w4a8_gemm.cpp:45-140): y bf16
    [a_hi rows, N]; callers slice back to their real rows, as with the reference.  ``rows`` >= 0
    computes and returns only the first ``rows`` rows (the same values): callers that know their
    real row count (``midgroup_linear``, ``MidGroupW4A8Linear``, the vLLM method) skip the padding."""
    return _run_midgroup(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group, False, rows)


@torch.library.register_fake("npu::midgroup_w4a8_gemm")
def _midgroup_gemm_fake(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group=1024, rows=-1):
    return a_scale.new_empty((a_hi.shape[0] if rows < 0 else rows, w_q.shape[0]), dtype=torch.bfloat16)


@torch.library.impl(_LIB, "midgroup_w4a8_gemm_partials", "CUDA")
def _midgroup_gemm_partials_cuda(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K: int,
                                 group: int = 1024):
    return _run_midgroup(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group, True)


@torch.library.impl(_LIB, "midgroup_tile_weights", "CUDA")
def _midgroup_tile_weights_cuda(w_q, K: int, group: int = 1024):
    """w_q [N, kpad/2] -> the 1 KB tiles midgroup_w4a8_gemm_tiled reads (the same bytes)."""
    _require(w_q.dim() == 2 and w_q.dtype == torch.int8, "midgroup_tile_weights: w_q must be int8 [N, kpad/2]")
    _require(w_q.shape[1] == geo.kpad(K, group) // 2,
             f"midgroup_tile_weights: packed row length must be Kpad/2 = {geo.kpad(K, group) // 2} for K={K}")
    w_q = w_q.contiguous()
    N = w_q.shape[0]
    out = torch.empty(max(0, _abi.lib().w4a8_midgroup_tiles_bytes(N, K, group)), dtype=torch.int8, device=w_q.device)
    if N:
        _abi.check(_abi.lib().w4a8_midgroup_tile_weights(w_q.data_ptr(), out.data_ptr(), N, K, group,
                                                         _stream(w_q.device)), "midgroup_tile_weights")
    return out


@torch.library.register_fake("npu::midgroup_tile_weights")
def _midgroup_tile_weights_fake(w_q, K, group=1024):
    N, KT = w_q.shape[0], -(-geo.kpad(K, group) // 128)
    return w_q.new_empty(((N + 15) // 16 * KT * 1024,), dtype=torch.int8)


@torch.library.impl(_LIB, "midgroup_w4a8_gemm_tiled", "CUDA")
def _midgroup_gemm_tiled_cuda(a_hi, a_lo, a_scale, a_ksum, w_tiles, w_scale, w_ksum, w_zero, N: int, K: int,
                              group: int = 1024, rows: int = -1):
    """midgroup_w4a8_gemm on midgroup_tile_weights' tiles of the [N, kpad/2] weight: the same output bits."""
    return _run_midgroup(a_hi, a_lo, a_scale, a_ksum, w_tiles, w_scale, w_ksum, w_zero, K, group, False, rows, N)


@torch.library.register_fake("npu::midgroup_w4a8_gemm_tiled")
def _midgroup_gemm_tiled_fake(a_hi, a_lo, a_scale, a_ksum, w_tiles, w_scale, w_ksum, w_zero, N, K, group=1024,
                              rows=-1):
    return a_scale.new_empty((a_hi.shape[0] if rows < 0 else rows, N), dtype=torch.bfloat16)


@torch.library.register_fake("npu::midgroup_w4a8_gemm_partials")
def _midgroup_gemm_partials_fake(a_hi, a_lo, a_scale, a_ksum, w_q, w_scale, w_ksum, w_zero, K, group=1024):
    M, N, G = a_hi.shape[0], w_q.shape[0], geo.num_groups(K, group)
    return (a_scale.new_empty((M, N), dtype=torch.bfloat16), a_scale.new_empty((G, M, N), dtype=torch.int32))
