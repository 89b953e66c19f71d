"""QwQ-32B-shaped decoder forward with every linear on the W4A8 kernels.

The reference measures its W4A8 linear inside whole decoder layers
(npu_ops/python/bench_decode_layer.py:40-82, bench_decode_graph.py:44-65):
RMSNorm -> qkv -> attention over a KV cache -> o -> residual -> RMSNorm ->
gate_up -> SwiGLU -> down -> residual.  This module builds that model
(Qwen2 architecture: grouped-query attention with q/k/v bias, rotary
embeddings, RMSNorm) on this build's ops:

* RMSNorm, the residual add and the activation quant run as one kernel
  (``torch.ops.npu.w4a8_rmsnorm_quant``) in front of qkv and gate_up;
* gate_up runs with the fused SwiGLU epilogue (``w4a8_gemm_swiglu``);
* o and down run ``w4a8_linear`` (quant + GEMM, one launch for a single row);
* the rotary embedding of q and k and the KV-cache append run as one kernel
  (``torch.ops.npu.w4a8_rope_kv``, fp32 products and sums rounded to bf16 as
  torch rounds them on float tensors);
* attention runs on this build's grouped-query attention kernel
  (``torch.ops.npu.w4a8_attention``, bf16 MFMA, csrc/attention.hip; a decode
  step calls ``w4a8_attention_rope``, which also rotates q and appends the
  step's k and v, in place of ``w4a8_rope_kv`` + ``w4a8_attention``): the
  query heads of one KV head form the rows of one problem (no head repeat),
  the causal limit of every row and the cache length of a captured decode
  step are read on the device, so a decode step reads only the positions
  written so far.  Decode launches one workgroup per split of the cache plus a
  combine kernel; prefill walks all splits per workgroup; both return the
  same bits for the same row, so a prefill of t + 1 tokens and a prefill of t
  tokens followed by a decode step agree exactly.  The K cache is stored
  ``[B, KVH, Lc, D]`` and V transposed ``[B, KVH, D, Lc]`` (Lc = max_len
  rounded up to 64).  The PyTorch paths stay selectable --
  ``attention="torch"`` is configs[4]'s own setting (bf16 attention left on
  PyTorch-ROCm: batched products below ``SDPA_MIN_BATCH`` sequences, SDPA from
  it on): ``attention="sdpa"`` calls
  ``torch.nn.functional.scaled_dot_product_attention`` on its efficient
  backend only (the reference's own call,
  npu_ops/python/bench_decode_layer.py:73; the math backend, whose batched
  products take a transposed bf16 operand, is never used) over a K cache
  stored ``[B, KVH, L, D]``; ``attention="matmul"`` two contiguous batched
  products over a K cache stored transposed ``[B, KVH, D, L]``, the scores
  returned in fp32.  Measured on MI355X (graph replays, one layer's decode
  attention at position 1100 of a 1280-position cache, us): kernel / products
  / SDPA 10.6 / 25 / 60 at 1 sequence, 14.8 / 28 / 65 at 8, 53.9 / 120 / 93 at
  64; prefill of one 1024-token sequence 34.7 / 233 / 94.5;
* the decode step is shape-static -- position, RoPE row, KV write index and
  mask are device tensors -- so it is captured once per batch size in a HIP
  graph and replayed, the greedy token feeding the next step inside the graph.

Weights are random (seeded), as in the reference's latency benches: codes
uniform in [-8, 7], group scales U[0.002, 0.02] at group 128.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from . import geometry as geo
from . import ops  # noqa: F401  (registers torch.ops.npu.*)


@dataclass
class DecoderConfig:
    """QwQ-32B (Qwen2) shapes by default."""
    layers: int = 64
    hidden: int = 5120
    heads: int = 40
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 27648
    vocab: int = 152064
    group: int = 128
    rms_eps: float = 1e-5
    rope_theta: float = 1.0e6
    qkv_bias: bool = True

    @property
    def qkv_out(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


class _Linear:
    """Repacked W4A8 weight of one projection (random codes, seeded)."""

    def __init__(self, N: int, K: int, group: int, gen: torch.Generator, device, bias: bool = False,
                 keep: bool = False):
        codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, device=device, generator=gen)
        from .packing import pack_grouped
        w_q = pack_grouped(codes, group)
        G = geo.num_groups(K, group)
        ws = (torch.rand((G, N), device=device, generator=gen) * 0.018 + 0.002).to(torch.bfloat16)
        self.w_tiles, self.s_tiles = torch.ops.npu.w4a8_repack(w_q, ws, K, group)
        # codes and scales kept only for reference checks of small models
        self.codes, self.scales = (codes, ws) if keep else (None, None)
        del codes
        self.N, self.K, self.group = N, K, group
        self.bias = ((torch.rand((N,), device=device, generator=gen) - 0.5) * 0.2).to(torch.bfloat16) if bias \
            else None

    def gemm(self, a_q: torch.Tensor, a_s: torch.Tensor) -> torch.Tensor:
        """The GEMM alone (the bias left to the consumer)."""
        return torch.ops.npu.w4a8_gemm(a_q, a_s, self.w_tiles, self.s_tiles, self.N, self.K, self.group)

    def __call__(self, a_q: torch.Tensor, a_s: torch.Tensor) -> torch.Tensor:
        y = self.gemm(a_q, a_s)
        return y + self.bias if self.bias is not None else y

    def linear(self, x: torch.Tensor) -> torch.Tensor:
        """quant + GEMM of bf16 x (one launch for a single row)."""
        y = torch.ops.npu.w4a8_linear(x, self.w_tiles, self.s_tiles, self.N, self.K, self.group)
        return y + self.bias if self.bias is not None else y

    def swiglu(self, a_q: torch.Tensor, a_s: torch.Tensor) -> torch.Tensor:
        return torch.ops.npu.w4a8_gemm_swiglu(a_q, a_s, self.w_tiles, self.s_tiles, self.N, self.K, self.group)


# attention="torch": batches from this size on attend through scaled_dot_product_attention,
# smaller ones through the two batched products (the faster PyTorch path on either side).
SDPA_MIN_BATCH = 48


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) + mask) v on the efficient backend (an error, not a fallback,
    where it cannot run).  q [B, KVH, R, D], k and v [B, KVH, L, D], mask bf16 broadcastable
    to [B, KVH, R, L] with 0 and -inf."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
        return torch.nn.functional.scaled_dot_product_attention(
            q, k, v, attn_mask=mask.expand(q.shape[0], q.shape[1], q.shape[2], k.shape[2]))


class W4A8Decoder:
    """The decoder with a static KV cache for ``batch`` sequences of up to ``max_len`` tokens."""

    def __init__(self, cfg: DecoderConfig, batch: int, max_len: int, device="cuda", seed: int = 0,
                 keep_weights=False, attention: str = "auto"):
        """keep_weights: True keeps every linear's int8 codes and scales (reference
        checks of small models), a collection of layer indices keeps those layers' only.
        attention: "hip" (this build's attention kernel; "auto" is the same), "sdpa",
        "matmul", or "torch" (PyTorch-ROCm as configs[4] states it: "matmul" below
        SDPA_MIN_BATCH sequences, "sdpa" from it on, chosen again by resize()), for prefill
        and decode alike (the paths round differently, so a prefill and the decode after it
        share one).  self.attention is the path in use."""
        if attention not in ("auto", "hip", "torch", "sdpa", "matmul"):
            raise ValueError(f"attention must be 'auto', 'hip', 'torch', 'sdpa' or 'matmul', not {attention!r}")
        self.attention_mode = "hip" if attention == "auto" else attention
        self.cfg, self.batch, self.max_len = cfg, batch, max_len
        dev = torch.device(device)
        self.device = dev
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        c = cfg
        self.embed = (torch.randn((c.vocab, c.hidden), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        self.lm_head = (torch.randn((c.vocab, c.hidden), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        self.final_norm = (1.0 + 0.1 * torch.randn((c.hidden,), device=dev, generator=gen)).to(torch.bfloat16)
        self.layers = []
        for li in range(c.layers):
            keep = keep_weights if isinstance(keep_weights, bool) else li in keep_weights
            self.layers.append({
                "ln1": (1.0 + 0.1 * torch.randn((c.hidden,), device=dev, generator=gen)).to(torch.bfloat16),
                "ln2": (1.0 + 0.1 * torch.randn((c.hidden,), device=dev, generator=gen)).to(torch.bfloat16),
                "qkv": _Linear(c.qkv_out, c.hidden, c.group, gen, dev, bias=c.qkv_bias, keep=keep),
                "o": _Linear(c.hidden, c.heads * c.head_dim, c.group, gen, dev, keep=keep),
                "gate_up": _Linear(2 * c.ffn, c.hidden, c.group, gen, dev, keep=keep),
                "down": _Linear(c.hidden, c.ffn, c.group, gen, dev, keep=keep),
            })
        d = c.head_dim
        self._alloc_cache(batch, max_len)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, d, 2, device=dev, dtype=torch.float32) / d))
        ang = torch.arange(max_len, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)          # [L, d/2] fp32
        self.positions = torch.arange(max_len, device=dev)
        # decode-step state (device tensors, so a captured step is position-independent)
        self.pos = torch.zeros((1,), dtype=torch.long, device=dev)
        self._pos0 = torch.zeros((1,), dtype=torch.long, device=dev)   # prefill writes from position 0
        self.tokens = torch.zeros((batch,), dtype=torch.long, device=dev)
        self._graph: Optional[torch.cuda.CUDAGraph] = None

    def resize(self, batch: int, max_len: int) -> None:
        """New KV cache and decode state for another batch size (weights are kept)."""
        c, dev = self.cfg, self.device
        self.batch, self.max_len = batch, max_len
        self._graph = None
        self.k_cache = self.v_cache = self._k_ld = self._k_store = self._vt_store = None
        torch.cuda.empty_cache()
        self._alloc_cache(batch, max_len)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=dev, dtype=torch.float32) / c.head_dim))
        ang = torch.arange(max_len, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)
        self.positions = torch.arange(max_len, device=dev)
        self.tokens = torch.zeros((batch,), dtype=torch.long, device=dev)
        self.pos.zero_()

    def _alloc_cache(self, batch: int, max_len: int) -> None:
        """KV caches in the layout of the attention path.  k_cache[li] is always a
        [B, KVH, D, L] tensor and v_cache[li] a [B, KVH, L, D] tensor (what w4a8_rope_kv
        writes through):
          hip     views of _k_store[li] [B, KVH, Lc, D] and _vt_store[li] [B, KVH, D, Lc]
                  (Lc = max_len rounded up to 64; positions past max_len stay zero);
          sdpa    a transposed view of _k_ld[li] [B, KVH, L, D]; v_cache itself;
          matmul  both caches themselves."""
        c, dev = self.cfg, self.device
        kvh, d = c.kv_heads, c.head_dim
        mode = self.attention_mode
        self.attention = mode if mode in ("hip", "sdpa", "matmul") else (
            "sdpa" if batch >= SDPA_MIN_BATCH else "matmul")
        self.sdpa = self.attention == "sdpa"
        self._k_ld = self._k_store = self._vt_store = None
        if self.attention == "hip":
            lc = -(-max_len // 64) * 64
            self._k_store = [torch.zeros((batch, kvh, lc, d), dtype=torch.bfloat16, device=dev) for _ in self.layers]
            self._vt_store = [torch.zeros((batch, kvh, d, lc), dtype=torch.bfloat16, device=dev)
                              for _ in self.layers]
            self.k_cache = [k[:, :, :max_len].transpose(2, 3) for k in self._k_store]
            self.v_cache = [v[..., :max_len].transpose(2, 3) for v in self._vt_store]
            self.cps = ops.attention_chunks_per_split(batch, c.heads, kvh, lc)
            return
        if self.sdpa:
            self._k_ld = [torch.zeros((batch, kvh, max_len, d), dtype=torch.bfloat16, device=dev) for _ in self.layers]
            self.k_cache = [k.transpose(2, 3) for k in self._k_ld]
        else:
            self.k_cache = [torch.zeros((batch, kvh, d, max_len), dtype=torch.bfloat16, device=dev)
                            for _ in self.layers]
        self.v_cache = [torch.zeros((batch, kvh, max_len, d), dtype=torch.bfloat16, device=dev) for _ in self.layers]

    # ------------------------------------------------------------ pieces
    def _rope_kv(self, li: int, L: dict, aq: torch.Tensor, as_: torch.Tensor, T: int,
                 pos: torch.Tensor) -> torch.Tensor:
        """qkv projection of layer li, then its bias (a bf16 add), the rotary embedding (rotate-half
        form, fp32 products and sums, bf16 result) of the q and k heads, and k and v appended to
        the layer's caches at positions pos[0] + t; returns q [B, T, heads, head_dim].  The bias,
        rotation and append are one kernel (w4a8_rope_kv)."""
        c = self.cfg
        qkv = L["qkv"].gemm(aq, as_).view(self.batch, T, -1)
        return torch.ops.npu.w4a8_rope_kv(qkv, self.cos, self.sin, pos, self.k_cache[li], self.v_cache[li],
                                          c.heads, c.kv_heads, L["qkv"].bias)

    def _attend(self, q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
        """q [B, KVH, R, D] (R = query heads per KV head x query tokens), kc [B, KVH, D, L],
        vc [B, KVH, L, D], additive bias broadcast to [B, KVH, R, L] -> [B, KVH, R, D].

        The scores q.k leave the batched product in fp32 (``out_dtype``: the precision
        scaled_dot_product_attention keeps them in, which prefill uses), then 1/sqrt(D) and
        the bias apply as one torch.add with alpha: the bias holds only 0 and -inf, so the one
        rounding of the product is that of a separate multiply and add, fused multiply-add or
        not.  The probabilities are rounded to bf16 for the second product."""
        B, H, R, D = q.shape
        L = kc.shape[-1]
        s = torch.bmm(q.reshape(B * H, R, D), kc.reshape(B * H, D, L), out_dtype=torch.float32).view(B, H, R, L)
        scores = torch.add(bias, s, alpha=1.0 / math.sqrt(self.cfg.head_dim))
        p = torch.softmax(scores, dim=-1).to(torch.bfloat16)
        return torch.matmul(p, vc)

    def _mlp_and_next(self, L: dict, s: torch.Tensor, a_attn: torch.Tensor):
        """o projection, residual, RMSNorm+quant, gate_up+SwiGLU, down; returns (stream, delta)."""
        c = self.cfg
        o = L["o"].linear(a_attn)
        aq2, as2, s2, _ = torch.ops.npu.w4a8_rmsnorm_quant(o, L["ln2"], c.rms_eps, s, c.group)
        h = L["gate_up"].swiglu(aq2, as2)
        return s2, L["down"].linear(h)

    # ------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor) -> torch.Tensor:
        """tokens [B, S] -> greedy next tokens [B]; fills the KV cache for positions [0, S)."""
        c, B = self.cfg, self.batch
        S = tokens.shape[1]
        assert tokens.shape[0] == B and S <= self.max_len
        G = c.heads // c.kv_heads
        if self.attention != "hip":
            # rows of one KV head's problem are (query head g, token s) = g * S + s
            bias = torch.full((S, S), float("-inf"), device=self.device).triu_(1).repeat(G, 1)
            mask = bias.to(torch.bfloat16).view(1, 1, G * S, S)
        x = self.embed[tokens.reshape(-1)]                               # [B*S, hidden]
        delta = None
        for li, L in enumerate(self.layers):
            aq, as_, s, _ = torch.ops.npu.w4a8_rmsnorm_quant(x, L["ln1"], c.rms_eps, delta, c.group)
            x = s if delta is not None else x
            q = self._rope_kv(li, L, aq, as_, S, self._pos0)        # [B, S, H, D]; caches filled for [0, S)
            if self.attention == "hip":
                out = torch.ops.npu.w4a8_attention(q, self._k_store[li], self._vt_store[li], self._pos0,
                                                   self.max_len, self.cps, False).view(B * S, -1)
                x, delta = self._mlp_and_next(L, x, out)
                continue
            qg = q.view(B, S, c.kv_heads, G, c.head_dim).permute(0, 2, 3, 1, 4).reshape(B, c.kv_heads, G * S,
                                                                                       c.head_dim)
            if self.sdpa:
                o = _sdpa(qg, self._k_ld[li][:, :, :S, :], self.v_cache[li][:, :, :S, :], mask)   # [B, KVH, G*S, D]
            else:
                kc = self.k_cache[li][:, :, :, :S].contiguous()
                vc = self.v_cache[li][:, :, :S, :].contiguous()
                o = torch.empty((B, c.kv_heads, G * S, c.head_dim), dtype=torch.bfloat16, device=self.device)
                for b in range(B):                                    # one sequence at a time bounds the scores
                    o[b:b + 1] = self._attend(qg[b:b + 1].contiguous(), kc[b:b + 1], vc[b:b + 1], bias)
            out = o.view(B, c.kv_heads, G, S, c.head_dim).permute(0, 3, 1, 2, 4).reshape(B * S, c.heads * c.head_dim)
            x, delta = self._mlp_and_next(L, x, out)
        last = (x + delta).view(B, S, c.hidden)[:, -1]
        return self._logits_argmax(last)

    def _logits(self, x_last: torch.Tensor) -> torch.Tensor:
        c = self.cfg
        v = x_last.float()
        h = (v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + c.rms_eps)).to(torch.bfloat16) * self.final_norm
        return torch.nn.functional.linear(h, self.lm_head)

    def _logits_argmax(self, x_last: torch.Tensor) -> torch.Tensor:
        logits = self._logits(x_last)
        self.last_logits = logits
        return logits.argmax(dim=-1)

    # ------------------------------------------------------------ decode
    def _decode_step(self) -> None:
        """One greedy step at self.pos for self.tokens, updating both in place (capturable)."""
        c, B = self.cfg, self.batch
        G = c.heads // c.kv_heads
        if self.attention != "hip":
            bias = torch.where(self.positions > self.pos, float("-inf"), 0.0).view(1, 1, 1, self.max_len)
            if self.sdpa:
                bias = bias.to(torch.bfloat16)
        x = self.embed.index_select(0, self.tokens)                      # [B, hidden]
        delta = None
        for li, L in enumerate(self.layers):
            aq, as_, s, _ = torch.ops.npu.w4a8_rmsnorm_quant(x, L["ln1"], c.rms_eps, delta, c.group)
            x = s if delta is not None else x
            if self.attention == "hip":
                # qkv projection, then one launch for the rotary embedding, the KV append and attention
                qkv = L["qkv"].gemm(aq, as_)
                o = torch.ops.npu.w4a8_attention_rope(qkv, self.cos, self.sin, self.pos, self._k_store[li],
                                                      self._vt_store[li], c.heads, c.kv_heads, self.max_len,
                                                      self.cps, L["qkv"].bias)
                x, delta = self._mlp_and_next(L, x, o.view(B, c.heads * c.head_dim))
                continue
            q = self._rope_kv(li, L, aq, as_, 1, self.pos)               # [B, 1, H, D]
            qg = q.view(B, c.kv_heads, G, c.head_dim)
            if self.sdpa:
                o = _sdpa(qg, self._k_ld[li], self.v_cache[li], bias)              # [B, KVH, G, D]
            else:
                o = self._attend(qg, self.k_cache[li], self.v_cache[li], bias)      # [B, KVH, G, D]
            x, delta = self._mlp_and_next(L, x, o.reshape(B, c.heads * c.head_dim))
        self.tokens.copy_(self._logits_argmax(x + delta))
        self.pos.add_(1)

    @torch.no_grad()
    def decode(self, first_tokens: torch.Tensor, start_pos: int, steps: int, graph: bool = True) -> List[torch.Tensor]:
        """Greedy decode ``steps`` tokens after a prefill of ``start_pos`` tokens; returns them."""
        assert start_pos + steps <= self.max_len
        self.tokens.copy_(first_tokens)
        self.pos.fill_(start_pos)
        out = []
        if not graph:
            for _ in range(steps):
                self._decode_step()
                out.append(self.tokens.clone())
            return out
        g = self.capture()
        self.tokens.copy_(first_tokens)
        self.pos.fill_(start_pos)
        for _ in range(steps):
            g.replay()
            out.append(self.tokens.clone())
        return out

    def capture(self) -> torch.cuda.CUDAGraph:
        """Capture one decode step (once); the step advances its own position.

        The warm-up step before capture runs at the last cache slot, whatever the
        current position (a position left at max_len by an earlier decode would
        index past the cache), and that slot's K/V are restored afterwards, so
        capturing leaves the cache and the decode state as they were.  The graph
        may only be replayed while the position is below max_len (decode()
        checks this).
        """
        if self._graph is None:
            slot = self.max_len - 1
            saved_t, saved_p = self.tokens.clone(), self.pos.clone()
            saved_k = [k[..., slot].clone() for k in self.k_cache]
            saved_v = [v[:, :, slot].clone() for v in self.v_cache]
            s = torch.cuda.Stream(device=self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                self.pos.fill_(slot)
                self._decode_step()               # warm-up outside capture (allocator, lazy init)
            torch.cuda.current_stream(self.device).wait_stream(s)
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._decode_step()
            torch.cuda.synchronize(self.device)
            self.tokens.copy_(saved_t)
            self.pos.copy_(saved_p)
            for k, sk in zip(self.k_cache, saved_k):
                k[..., slot] = sk
            for v, sv in zip(self.v_cache, saved_v):
                v[:, :, slot] = sv
            self._graph = g
        return self._graph
