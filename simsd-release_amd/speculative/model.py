"""Random-init SDAR-shape decoders on the MI355X kernels.

The draft (SDAR-1.7B shape) and the target (SDAR-8B shape) are the
reference's dense block-diffusion decoders (sdar/modeling_sdar.py: RMSNorm,
q/k-normed GQA attention with RoPE, SiLU-gated MLP), here with random weights
of the real shapes (no checkpoint is available offline).  Each layer runs as

    qkv = rmsnorm + merged q/k/v projection       (thin_rmsnorm_linear)
    q   = q/k norm + RoPE + K/V cache write        (qkv_rope_cache)
    a   = attention over the static cache          (block_attention)
          (the two in one launch, qkv_rope_attention, for the runner's
          forwards of up to 16 rows at the end of the valid range)
    h  += o_proj(a)                                (thin_linear_residual)
    g   = rmsnorm + gate/up projection + SiLU.mul  (thin_rmsnorm_linear_silu_mul)
    h  += down_proj(g)                             (thin_linear_residual)

and the head is rmsnorm + lm_head (thin_rmsnorm_linear).  Above 8 rows, where
each norm would be a launch of its own, the projections hand their split-K
partials to the launch that consumes them instead of reducing them first:

    xn      = rmsnorm(h)                               (first layer only)
    q       = qkv partials -> reduce + q/k norm + RoPE + cache write
                                                       (reduce_qkv_rope_cache)
    a       = attention                                (block_attention)
    h, xn   = o partials -> reduce + residual + rmsnorm (reduce_residual_rmsnorm)
    g       = gate/up + SiLU.mul                       (thin_linear_silu_mul)
    h, xn   = down partials -> reduce + residual + the next layer's (or the
              final) rmsnorm                           (reduce_residual_rmsnorm)

in 8 launches a layer instead of 11.  Each consuming launch sums the partials
as the reduce launch would, so with the same splits the values are those of
the form above; the partials' own geometry table (PARTIALS_RANGES) splits some
projections differently, which changes only the k-chunking of their sums.  A forward takes its
rows' token ids, RoPE positions, cache slots and mask rows, all as device
tensors, so one captured graph serves every step of a growing context.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from kernels.attention_fused import (BlockKVCache, block_attention, default_inv_freq, fused_attention_ok,
                                     gather_rope_rows, qkv_rope_attention, qkv_rope_cache, reduce_qkv_rope_cache,
                                     rope_table_pair, rope_tables)
from kernels.thin_linear_fused import (reduce_residual_rmsnorm, thin_linear, thin_linear_partials,
                                       thin_linear_residual, thin_linear_silu_mul, thin_rmsnorm,
                                       thin_rmsnorm_linear, thin_rmsnorm_linear_silu_mul)


@dataclass(frozen=True)
class ModelShape:
    hidden: int
    n_layers: int
    n_q_heads: int
    n_kv_heads: int
    intermediate: int
    vocab: int
    head_dim: int = 128
    eps: float = 1e-6
    rope_theta: float = 1000000.0


# SDAR-1.7B / SDAR-8B (Qwen3-1.7B / Qwen3-8B layouts)
DRAFT_1P7B = ModelShape(hidden=2048, n_layers=28, n_q_heads=16, n_kv_heads=8, intermediate=6144, vocab=151936)
TARGET_8B = ModelShape(hidden=4096, n_layers=36, n_q_heads=32, n_kv_heads=8, intermediate=12288, vocab=151936)


class _Layer:
    __slots__ = ("ln1", "wqkv", "qn", "kn", "wo", "ln2", "wgu", "wd")


class SynthModel:
    """Random-init decoder of ``shape`` (weights ~N(0, 0.02), norm weights ~1)
    with a BlockKVCache of ``max_ctx`` committed slots and ``max_rows`` rows
    per forward."""

    def __init__(self, shape: ModelShape, device, seed: int, max_ctx: int, max_rows: int,
                 dtype=torch.bfloat16):
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        g = torch.Generator(device=self.device).manual_seed(seed)
        H, D, I = shape.hidden, shape.head_dim, shape.intermediate
        qkv_rows = (shape.n_q_heads + 2 * shape.n_kv_heads) * D

        def w(*sh, s=0.02):
            t = torch.empty(*sh, device=self.device, dtype=dtype)
            for i in range(0, sh[0], 8192):      # bounded fp32 temporaries
                n = min(8192, sh[0] - i)
                t[i:i + n] = (torch.randn(n, *sh[1:], device=self.device, generator=g) * s).to(dtype)
            return t

        def norm(n):
            return (1.0 + 0.05 * torch.randn(n, device=self.device, generator=g)).to(dtype)

        self.embed = w(shape.vocab, H, s=1.0)
        self.layers = []
        for _ in range(shape.n_layers):
            L = _Layer()
            L.ln1, L.wqkv, L.qn, L.kn = norm(H), w(qkv_rows, H), norm(D), norm(D)
            L.wo, L.ln2 = w(H, shape.n_q_heads * D), norm(H)
            L.wgu, L.wd = w(2 * I, H), w(H, I)
            self.layers.append(L)
        self.lnf = norm(H)
        self.lm_head = w(shape.vocab, H)
        self.cache = BlockKVCache(shape.n_layers, shape.n_kv_heads, max_ctx, max_rows, self.device, dtype)
        # interleaved, so a forward gathers its rows' cos / sin in one launch
        self.cos, self.sin = rope_table_pair(*rope_tables(default_inv_freq(D, shape.rope_theta, self.device),
                                                          self.cache.full_len + 64, dtype))

    @torch.inference_mode()
    def forward(self, ids, pos, slots, mask, valid_len=None, valid_len_dev=None, head_rows=None, head=True,
                rows_at_end=False):
        """ids/pos/slots: int64 [M]; mask [M, >= valid] (bool); returns the
        logits of ``head_rows`` (a slice or an index tensor; all rows when
        None) or, with ``head=False``, nothing (the forward only writes the
        cache).  ``rows_at_end``: the caller guarantees slots[r] = valid - M + r
        (valid: the device-side valid length when ``valid_len_dev`` is given,
        else valid_len), which lets small forwards take the fused attention
        launch."""
        s = self.shape
        I = s.intermediate
        M = int(ids.shape[0])
        L_attn = self.cache.full_len if valid_len is None else int(valid_len)
        fused = rows_at_end and fused_attention_ok(M, s.n_q_heads, s.n_kv_heads, L_attn)
        h = F.embedding(ids, self.embed)
        # the one-launch attention takes the rows' cos / sin gathered once for
        # every layer, not positions it would have to load before them
        rope = gather_rope_rows(self.cos, self.sin, pos) if fused else None
        if self.partials_path(M):
            return self._forward_partials(h, pos, slots, mask, valid_len, valid_len_dev, head_rows, head, rope)
        for li, L in enumerate(self.layers):
            qkv = thin_rmsnorm_linear(h, L.ln1, s.eps, L.wqkv)
            if fused:
                a = qkv_rope_attention(qkv, s.n_q_heads, L.qn, L.kn, s.eps, *rope, None, self.cache, li,
                                       mask, valid_len=valid_len, valid_len_dev=valid_len_dev)
            else:
                q = qkv_rope_cache(qkv, s.n_q_heads, L.qn, L.kn, s.eps, self.cos, self.sin, pos, slots, self.cache,
                                   li)
                a = block_attention(q, self.cache, li, mask, valid_len=valid_len, valid_len_dev=valid_len_dev)
            h = thin_linear_residual(a, L.wo, h)
            g = thin_rmsnorm_linear_silu_mul(h, L.ln2, s.eps, L.wgu[:I], L.wgu[I:])
            h = thin_linear_residual(g, L.wd, h)
        if not head:
            return None
        if head_rows is not None:
            h = h[head_rows]
        return thin_rmsnorm_linear(h, self.lnf, s.eps, self.lm_head)

    def partials_path(self, M: int) -> bool:
        """Above 8 rows (the norms are launches of their own there) and for
        16-bit rows the consuming launches can take (hidden % 8 == 0, <= 8192)."""
        H = self.shape.hidden
        return M > 8 and self.dtype != torch.float32 and H % 8 == 0 and H <= 8192 and not self.reduce_first

    reduce_first = False   # True: each projection reduced before its consumer at every row count

    def _forward_partials(self, h, pos, slots, mask, valid_len, valid_len_dev, head_rows, head, rope):
        s = self.shape
        I = s.intermediate
        n = len(self.layers)
        xn = thin_rmsnorm(h, self.layers[0].ln1, s.eps)
        for li, L in enumerate(self.layers):
            if rope is not None:
                a = qkv_rope_attention(thin_linear(xn, L.wqkv), s.n_q_heads, L.qn, L.kn, s.eps, *rope, None,
                                       self.cache, li, mask, valid_len=valid_len, valid_len_dev=valid_len_dev)
            else:
                q = reduce_qkv_rope_cache(thin_linear_partials(xn, L.wqkv), s.n_q_heads, L.qn, L.kn, s.eps,
                                          self.cos, self.sin, pos, slots, self.cache, li)
                a = block_attention(q, self.cache, li, mask, valid_len=valid_len, valid_len_dev=valid_len_dev)
            h, xn = reduce_residual_rmsnorm(thin_linear_partials(a, L.wo), h, L.ln2, s.eps, out=h)
            g = thin_linear_silu_mul(xn, L.wgu[:I], L.wgu[I:])
            nxt = self.layers[li + 1].ln1 if li + 1 < n else self.lnf
            h, xn = reduce_residual_rmsnorm(thin_linear_partials(g, L.wd), h, nxt, s.eps, out=h)
        if not head:
            return None
        return thin_linear(xn if head_rows is None else xn[head_rows], self.lm_head)
