"""Attention of the speculative step on MI355X: q/k norm, RoPE and the KV
cache write in one launch, then attention of the block's few query rows over
the static cache.

Reference path, per attention layer (speculative_decoding/adapters/base.py:
161-265 with SDAR's qkv, sdar/modeling_sdar.py:250-262, and the cache class
StaticBlockCache, speculative_decoding/cache_aware.py:195-298)::

    q = q_norm(q_proj(x)); k = k_norm(k_proj(x)); v = v_proj(x)
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    for i in range(n_rep):                       # GQA "expand" cache
        key_cache[:, i::n_rep].index_copy_(2, cur_scratch_pos, k)   # (+ values,
        ...                                                         #  + cache_position)
    out = F.scaled_dot_product_attention(q, key_cache, value_cache, attn_mask=mask_bool)

Here: ``qkv_rope_cache`` (one launch) and ``block_attention``.  For up to 32
query rows per KV head the attention is one launch up to ``ONE_LAUNCH_SLOTS``
slots: one workgroup per KV head over a short valid length, over a longer one
several, the last of which merges their partials; two launches past it
(chunked partials, then their merge).  The form and the chunking follow the
host's ``valid_len`` bound, so a caller replaying graphs over a growing
context captures one graph per bound; ``valid_len_dev`` then lowers the
length at run time, and the kernels trim their work to it.  The cache
(``BlockKVCache``) keeps one copy of each KV head (no per-query-head replicas)
in tiles laid out in the order the attention kernels read them, so every
wave-wide load covers 1 KB of contiguous memory; ``keys`` / ``values`` /
``store`` convert to and from the reference's [Hkv, L, D] orientation.  The
slot space is the reference's: [0, max_cache_len) the permanent cache,
[max_cache_len, full_len) the scratch of the current forward.
``rope_tables`` computes cos/sin exactly as the rotary embedding does
(modeling_sdar.py:418-435).  Head dim 128; bf16 or fp16.
"""
from __future__ import annotations

import torch

from . import _native

HEAD_DIM = 128
ONE_LAUNCH_SLOTS = 4096   # block_attention's one-launch form up to this valid_len


def rope_tables(inv_freq: torch.Tensor, n_pos: int, dtype: torch.dtype, attention_scaling: float = 1.0):
    """(cos, sin) [n_pos, D] in ``dtype`` for positions 0..n_pos-1, computed as
    SDARRotaryEmbedding.forward does (fp32 outer product, duplicated halves,
    cos/sin, scaled, cast)."""
    pos = torch.arange(n_pos, device=inv_freq.device, dtype=torch.float32)
    freqs = (inv_freq.float()[None, :, None] @ pos[None, None, :]).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return ((emb.cos() * attention_scaling).to(dtype).contiguous(),
            (emb.sin() * attention_scaling).to(dtype).contiguous())


def default_inv_freq(head_dim: int = HEAD_DIM, theta: float = 1000000.0, device=None) -> torch.Tensor:
    """The default RoPE frequencies, 1 / theta^(2i / D)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=device).float() / head_dim))


class BlockKVCache:
    """Static per-layer K and V tiles (zeroed), L = max_cache_len + max_cur_len
    rounded up to a multiple of 32.  Slots [0, max_cache_len) hold the
    committed context, [max_cache_len, L) the scratch of the current forward,
    as in the reference's StaticBlockCache.

    Per layer and KV head, (slot s, dim d) lives at
      K: ((s/16 * 16 + d/8) * 16 + s%16) * 8 + d%8           ``k_tiles[l]`` [Hkv, L/16, 16, 16, 8]
      V: ((((s/32 * 8 + d/16) * 16 + d%16) * 4 + s/4%4) * 2 + s/16%2) * 4 + s%4
                                                              ``v_tiles[l]`` [Hkv, L/32, 8, 16, 4, 2, 4]
    (the order of the attention kernels' MFMA operand loads)."""

    def __init__(self, n_layers: int, n_kv_heads: int, max_cache_len: int, max_cur_len: int,
                 device, dtype=torch.bfloat16, head_dim: int = HEAD_DIM):
        if head_dim != HEAD_DIM:
            raise ValueError(f"head_dim must be {HEAD_DIM}")
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.max_cache_len, self.max_cur_len = max_cache_len, max_cur_len
        self.full_len = (max_cache_len + max_cur_len + 31) // 32 * 32
        self.dtype = dtype
        L, H = self.full_len, n_kv_heads
        self.k_tiles = [torch.zeros(H, L // 16, 16, 16, 8, device=device, dtype=dtype) for _ in range(n_layers)]
        self.v_tiles = [torch.zeros(H, L // 32, 8, 16, 4, 2, 4, device=device, dtype=dtype)
                        for _ in range(n_layers)]
        # the attention's workspace: zeroed once, its arrival counters left at
        # zero by every call; outgrown ones stay referenced (captured graphs
        # may still use them)
        self._attn_ws = None
        self._attn_ws_held = []

    def attention_workspace(self, nbytes: int, device) -> torch.Tensor:
        """The zero-initialised workspace the attention calls on this cache
        share (grown outside graph capture only)."""
        ws = self._attn_ws
        if ws is None or ws.numel() < nbytes or ws.device != torch.device(device):
            if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("block_attention: the cache's workspace must be sized before graph capture "
                                   "(run the same call once outside the capture)")
            ws = torch.zeros(max(int(nbytes), 4096), device=device, dtype=torch.uint8)
            self._attn_ws_held.append(ws)
            self._attn_ws = ws
        return ws

    def __len__(self) -> int:
        return self.n_layers

    @property
    def head_stride(self) -> int:
        """Elements per KV head in either tile array."""
        return self.full_len * self.head_dim

    def reset(self) -> None:
        for t in self.k_tiles + self.v_tiles:
            t.zero_()

    def keys(self, layer: int) -> torch.Tensor:
        """K of a layer in the reference's [Hkv, L, D] orientation (a copy)."""
        H, L, D = self.n_kv_heads, self.full_len, self.head_dim
        return self.k_tiles[layer].permute(0, 1, 3, 2, 4).reshape(H, L, D)

    def values(self, layer: int) -> torch.Tensor:
        """V of a layer in the reference's [Hkv, L, D] orientation (a copy)."""
        H, L, D = self.n_kv_heads, self.full_len, self.head_dim
        return self.v_tiles[layer].permute(0, 1, 5, 4, 6, 2, 3).reshape(H, L, D)

    def store(self, layer: int, k: torch.Tensor, v: torch.Tensor, start: int = 0) -> None:
        """Write K and V [Hkv, n, D] (the reference's orientation) at slots
        [start, start + n) of a layer."""
        H, L, D = self.n_kv_heads, self.full_len, self.head_dim
        n = k.shape[1]
        if k.shape != (H, n, D) or v.shape != (H, n, D) or not 0 <= start <= L - n:
            raise ValueError(f"store: K/V must be [{H}, n, {D}] within {L} slots")
        kf, vf = self.keys(layer), self.values(layer)
        kf[:, start:start + n] = k.to(self.dtype)
        vf[:, start:start + n] = v.to(self.dtype)
        self.k_tiles[layer].copy_(kf.view(H, L // 16, 16, 16, 8).permute(0, 1, 3, 2, 4))
        self.v_tiles[layer].copy_(vf.view(H, L // 32, 2, 4, 4, 8, 16).permute(0, 1, 5, 6, 3, 2, 4))


def qkv_rope_cache(qkv: torch.Tensor, n_q_heads: int, q_norm_weight, k_norm_weight, eps: float,
                   cos: torch.Tensor, sin: torch.Tensor, position_ids: torch.Tensor,
                   slots: torch.Tensor, cache: BlockKVCache, layer: int,
                   slots2: torch.Tensor | None = None) -> torch.Tensor:
    """q/k norm + RoPE of the merged projection output and the K/V cache write.

    qkv:          [M, (Hq + 2 Hkv) * 128] (q heads, k heads, v heads)
    position_ids: int64 [M] rows of cos/sin
    slots:        int64 [M] cache slots (the scratch positions); ``slots2``:
                  int64 [M] permanent positions written too (store_kv)
    -> q [M, Hq, 128] after norm and RoPE.
    """
    code = _native.DTYPE_CODES.get(qkv.dtype)
    if code is None or qkv.dtype == torch.float32:
        raise TypeError(f"qkv_rope_cache: dtype must be bf16 or fp16, got {qkv.dtype}")
    if qkv.ndim != 2:
        raise ValueError("qkv_rope_cache: qkv must be [M, (Hq + 2 Hkv) * D]")
    M = qkv.shape[0]
    Hkv, D = cache.n_kv_heads, cache.head_dim
    if qkv.shape[1] != (n_q_heads + 2 * Hkv) * D or n_q_heads % Hkv != 0:
        raise ValueError(f"qkv_rope_cache: width {qkv.shape[1]} != ({n_q_heads} + 2*{Hkv}) * {D}")
    if qkv.stride(1) != 1:
        qkv = qkv.contiguous()
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != qkv.dtype or t.ndim != 2 or t.shape[1] != D or t.stride(1) != 1:
            raise ValueError(f"qkv_rope_cache: {name} must be [n_pos, {D}] in {qkv.dtype}")
    if cos.shape != sin.shape or cos.stride(0) != sin.stride(0):
        raise ValueError("qkv_rope_cache: cos and sin differ in shape or stride")
    for name, t in (("position_ids", position_ids), ("slots", slots), ("slots2", slots2)):
        if t is not None and (t.dtype != torch.int64 or t.shape != (M,) or (M > 1 and t.stride(0) != 1)):
            raise ValueError(f"qkv_rope_cache: {name} must be int64 [M] with unit stride")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if t is not None and (t.dtype != qkv.dtype or t.shape != (D,) or t.stride(0) != 1):
            raise ValueError(f"qkv_rope_cache: {name} must be [{D}] in {qkv.dtype}")
    kc, vc = cache.k_tiles[layer], cache.v_tiles[layer]
    if kc.dtype != qkv.dtype:
        raise TypeError("qkv_rope_cache: cache dtype differs from qkv")
    dev = _native.require_device(qkv, cos, sin, position_ids, slots, slots2, kc, q_norm_weight, k_norm_weight)
    q = torch.empty((M, n_q_heads, D), device=dev, dtype=qkv.dtype)
    if M == 0:
        return q
    with _native.device_guard(dev):
        status = _native.lib().simsd_qkv_rope_cache(
            qkv.data_ptr(), qkv.stride(0),
            q_norm_weight.data_ptr() if q_norm_weight is not None else None,
            k_norm_weight.data_ptr() if k_norm_weight is not None else None, float(eps),
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], position_ids.data_ptr(),
            slots.data_ptr(), slots2.data_ptr() if slots2 is not None else None,
            kc.data_ptr(), vc.data_ptr(), cache.head_stride, cache.full_len,
            q.data_ptr(), q.stride(0), q.stride(1), M, n_q_heads, Hkv, D, code, _native.stream_of(dev))
    _native.check(status, "qkv_rope_cache")
    return q


REDUCE_MAX_SPLIT = 8   # partials the cache-write launch sums


def reduce_qkv_rope_cache(part: torch.Tensor, n_q_heads: int, q_norm_weight, k_norm_weight, eps: float,
                          cos: torch.Tensor, sin: torch.Tensor, position_ids: torch.Tensor,
                          slots: torch.Tensor, cache: BlockKVCache, layer: int,
                          slots2: torch.Tensor | None = None) -> torch.Tensor:
    """``qkv_rope_cache`` on the merged projection given as its split-K
    partials (``thin_linear_fused.thin_linear_partials``: fp32
    [split, M, (Hq + 2 Hkv) * 128]), summed and rounded in the same launch:
    the reduce of the projection and the prologue's norm, RoPE and cache
    write in one.  Bit-identical to ``qkv_rope_cache`` of the reduced
    projection.  The dtype is the cache's.  -> q [M, Hq, 128]."""
    kc, vc = cache.k_tiles[layer], cache.v_tiles[layer]
    code = _native.DTYPE_CODES.get(kc.dtype)
    if code is None or kc.dtype == torch.float32:
        raise TypeError(f"reduce_qkv_rope_cache: cache dtype must be bf16 or fp16, got {kc.dtype}")
    Hkv, D = cache.n_kv_heads, cache.head_dim
    if part.dtype != torch.float32 or part.ndim != 3 or not part.is_contiguous():
        raise ValueError("reduce_qkv_rope_cache: partials must be contiguous fp32 [split, M, N]")
    split, M, N = part.shape
    if not 1 <= split <= REDUCE_MAX_SPLIT:
        raise ValueError(f"reduce_qkv_rope_cache: split {split} outside 1..{REDUCE_MAX_SPLIT}")
    if N != (n_q_heads + 2 * Hkv) * D or n_q_heads % Hkv != 0:
        raise ValueError(f"reduce_qkv_rope_cache: width {N} != ({n_q_heads} + 2*{Hkv}) * {D}")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != kc.dtype or t.ndim != 2 or t.shape[1] != D or t.stride(1) != 1:
            raise ValueError(f"reduce_qkv_rope_cache: {name} must be [n_pos, {D}] in {kc.dtype}")
    if cos.shape != sin.shape or cos.stride(0) != sin.stride(0):
        raise ValueError("reduce_qkv_rope_cache: cos and sin differ in shape or stride")
    for name, t in (("position_ids", position_ids), ("slots", slots), ("slots2", slots2)):
        if t is not None and (t.dtype != torch.int64 or t.shape != (M,) or (M > 1 and t.stride(0) != 1)):
            raise ValueError(f"reduce_qkv_rope_cache: {name} must be int64 [M] with unit stride")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if t is not None and (t.dtype != kc.dtype or t.shape != (D,) or t.stride(0) != 1):
            raise ValueError(f"reduce_qkv_rope_cache: {name} must be [{D}] in {kc.dtype}")
    dev = _native.require_device(part, cos, sin, position_ids, slots, slots2, kc, q_norm_weight, k_norm_weight)
    q = torch.empty((M, n_q_heads, D), device=dev, dtype=kc.dtype)
    if M == 0:
        return q
    with _native.device_guard(dev):
        status = _native.lib().simsd_reduce_qkv_rope_cache(
            part.data_ptr(), split, part.numel() * 4,
            q_norm_weight.data_ptr() if q_norm_weight is not None else None,
            k_norm_weight.data_ptr() if k_norm_weight is not None else None, float(eps),
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], position_ids.data_ptr(),
            slots.data_ptr(), slots2.data_ptr() if slots2 is not None else None,
            kc.data_ptr(), vc.data_ptr(), cache.head_stride, cache.full_len,
            q.data_ptr(), q.stride(0), q.stride(1), M, n_q_heads, Hkv, D, code, _native.stream_of(dev))
    _native.check(status, "reduce_qkv_rope_cache")
    return q


def _mask_u8(mask, M: int, L: int, what: str):
    """The mask as uint8 rows the kernels read 4 bytes at a time (padded copy
    when the view's layout does not allow it), or None."""
    if mask is None:
        return None
    if mask.ndim != 2 or mask.shape[0] != M or mask.shape[1] < L:
        raise ValueError(f"{what}: mask must be [{M}, >= {L}]")
    m8 = mask.view(torch.uint8) if mask.dtype == torch.bool else mask
    if m8.dtype != torch.uint8:
        raise TypeError(f"{what}: mask must be bool or uint8")
    need = (L + 3) // 4 * 4
    if m8.stride(1) != 1 or m8.stride(0) % 4 or m8.data_ptr() % 4 or m8.shape[1] < need:
        pad = torch.zeros((M, max(need, (m8.shape[1] + 3) // 4 * 4)), device=m8.device, dtype=torch.uint8)
        pad[:, :m8.shape[1]].copy_(m8)
        m8 = pad
    return m8


# rows of a forward that qkv_rope_attention takes in one launch
FUSED_MAX_ROWS = 16


def fused_attention_ok(M: int, n_q_heads: int, n_kv_heads: int, valid_len: int) -> bool:
    """Whether qkv_rope_attention runs a forward of these sizes (the head form
    of the attention: at most 32 query rows per KV head over at most
    ONE_LAUNCH_SLOTS slots, and at most FUSED_MAX_ROWS rows)."""
    return (0 < M <= FUSED_MAX_ROWS and n_q_heads % n_kv_heads == 0
            and (n_q_heads // n_kv_heads) * M <= 32 and valid_len <= ONE_LAUNCH_SLOTS)


def qkv_rope_attention(qkv: torch.Tensor, n_q_heads: int, q_norm_weight, k_norm_weight, eps: float,
                       cos: torch.Tensor, sin: torch.Tensor, position_ids: torch.Tensor, cache: BlockKVCache,
                       layer: int, mask: torch.Tensor | None = None, valid_len: int | None = None,
                       valid_len_dev: torch.Tensor | None = None, scale: float | None = None) -> torch.Tensor:
    """``block_attention(qkv_rope_cache(...))`` in one launch, for a forward
    whose M rows occupy the last M slots of the valid range: row r writes its
    K/V at slot valid - M + r (valid = the device-side valid length when
    ``valid_len_dev`` is given, else ``valid_len``), as every forward of the
    speculative runner does.  Sizes must pass ``fused_attention_ok``.

    qkv: [M, (Hq + 2 Hkv) * 128] merged projection output; the rest as in
    qkv_rope_cache and block_attention.  ``position_ids=None``: cos / sin are
    the rows' own tables (row m at row m, ``gather_rope_rows``), gathered once
    for all layers of a forward so that no launch waits for the positions
    before its cos / sin loads.  -> [M, Hq * 128].
    """
    code = _native.DTYPE_CODES.get(qkv.dtype)
    if code is None or qkv.dtype == torch.float32:
        raise TypeError(f"qkv_rope_attention: dtype must be bf16 or fp16, got {qkv.dtype}")
    M = qkv.shape[0]
    Hkv, D = cache.n_kv_heads, cache.head_dim
    if qkv.ndim != 2 or qkv.shape[1] != (n_q_heads + 2 * Hkv) * D or n_q_heads % Hkv != 0:
        raise ValueError(f"qkv_rope_attention: qkv must be [M, ({n_q_heads} + 2*{Hkv}) * {D}]")
    L = cache.full_len if valid_len is None else int(valid_len)
    if not 0 <= L <= cache.full_len:
        raise ValueError(f"qkv_rope_attention: valid_len {L} outside [0, {cache.full_len}]")
    if not fused_attention_ok(M, n_q_heads, Hkv, L):
        raise ValueError(f"qkv_rope_attention: {M} rows x {n_q_heads // Hkv} heads per KV head over {L} slots "
                         "need the two-launch form (qkv_rope_cache, then block_attention)")
    if qkv.stride(1) != 1 or qkv.stride(0) % 8 or qkv.data_ptr() % 16:
        qkv = qkv.contiguous()
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != qkv.dtype or t.ndim != 2 or t.shape[1] != D or t.stride(1) != 1:
            raise ValueError(f"qkv_rope_attention: {name} must be [n_pos, {D}] in {qkv.dtype}")
    if cos.shape != sin.shape or cos.stride(0) != sin.stride(0):
        raise ValueError("qkv_rope_attention: cos and sin differ in shape or stride")
    if position_ids is None:
        if cos.shape[0] < M:
            raise ValueError(f"qkv_rope_attention: without position_ids, cos / sin must hold the {M} rows' tables")
    elif position_ids.dtype != torch.int64 or position_ids.shape != (M,) or (M > 1 and position_ids.stride(0) != 1):
        raise ValueError("qkv_rope_attention: position_ids must be int64 [M] with unit stride")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if t is not None and (t.dtype != qkv.dtype or t.shape != (D,) or t.stride(0) != 1 or t.data_ptr() % 16):
            raise ValueError(f"qkv_rope_attention: {name} must be a 16-byte aligned [{D}] vector in {qkv.dtype}")
    m8 = _mask_u8(mask, M, L, "qkv_rope_attention")
    if valid_len_dev is not None and (valid_len_dev.dtype != torch.int64 or valid_len_dev.numel() != 1):
        raise ValueError("qkv_rope_attention: valid_len_dev must be one int64 on the device")
    kc, vc = cache.k_tiles[layer], cache.v_tiles[layer]
    dev = _native.require_device(qkv, cos, sin, position_ids, kc, m8, valid_len_dev, q_norm_weight, k_norm_weight)
    out = torch.empty((M, n_q_heads * D), device=dev, dtype=qkv.dtype)
    lib = _native.lib()
    need = lib.simsd_block_attention_workspace_bytes(M, n_q_heads, Hkv, L)
    if need < 0:
        _native.check(-1, "qkv_rope_attention")
    ws = cache.attention_workspace(need, dev)
    with _native.device_guard(dev):
        status = lib.simsd_qkv_rope_attention(
            qkv.data_ptr(), qkv.stride(0),
            q_norm_weight.data_ptr() if q_norm_weight is not None else None,
            k_norm_weight.data_ptr() if k_norm_weight is not None else None, float(eps),
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0],
            position_ids.data_ptr() if position_ids is not None else None,
            kc.data_ptr(), vc.data_ptr(), cache.head_stride, cache.full_len,
            m8.data_ptr() if m8 is not None else None, m8.stride(0) if m8 is not None else 0,
            out.data_ptr(), out.stride(0), D, M, n_q_heads, Hkv, L,
            valid_len_dev.data_ptr() if valid_len_dev is not None else None, D,
            float(D ** -0.5 if scale is None else scale), code, ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    _native.check(status, "qkv_rope_attention")
    return out


def gather_rope_rows(cos: torch.Tensor, sin: torch.Tensor, position_ids: torch.Tensor):
    """The rows' own cos / sin tables, [M, D] each, for
    ``qkv_rope_attention(..., position_ids=None)``: one gather when ``cos``
    and ``sin`` are the two halves of an interleaved [n_pos, 2, D] table
    (``rope_table_pair``), else two.  Positions must lie in [0, n_pos)."""
    D, es = cos.shape[1], cos.element_size()
    if cos.stride(0) == sin.stride(0) == 2 * D and sin.data_ptr() == cos.data_ptr() + D * es:
        pair = torch.as_strided(cos, (cos.shape[0], 2, D), (2 * D, D, 1))
        g = pair.index_select(0, position_ids)
        return g[:, 0], g[:, 1]
    return cos.index_select(0, position_ids), sin.index_select(0, position_ids)


def rope_table_pair(cos: torch.Tensor, sin: torch.Tensor):
    """cos / sin [n_pos, D] stored interleaved ([n_pos, 2, D]) and returned as
    the two [n_pos, D] views (row stride 2 D), which every call here takes
    and ``gather_rope_rows`` gathers in one launch."""
    pair = torch.stack((cos, sin), dim=1)
    return pair[:, 0], pair[:, 1]


def block_attention(q: torch.Tensor, cache: BlockKVCache, layer: int, mask: torch.Tensor | None = None,
                    valid_len: int | None = None, scale: float | None = None,
                    valid_len_dev: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(scale * q K^T, masked) V over the cache's slots [0, valid_len).

    q:    [M, Hq, 128] (query head hq reads KV head hq // (Hq / Hkv))
    mask: bool/uint8 [M, >= valid_len], True = visible (the reference's SDPA
          mask rows), or None (all visible)
    valid_len_dev: optional int64 scalar tensor on the device that lowers
          valid_len when the kernels run (for graphs replayed over a growing
          context)
    -> [M, Hq * 128] (the layout o_proj takes).
    """
    code = _native.DTYPE_CODES.get(q.dtype)
    if code is None or q.dtype == torch.float32:
        raise TypeError(f"block_attention: dtype must be bf16 or fp16, got {q.dtype}")
    if q.ndim != 3 or q.shape[2] != cache.head_dim:
        raise ValueError("block_attention: q must be [M, Hq, 128]")
    M, Hq, D = q.shape
    Hkv = cache.n_kv_heads
    if Hq % Hkv != 0:
        raise ValueError(f"block_attention: {Hq} query heads not a multiple of {Hkv} KV heads")
    L = cache.full_len if valid_len is None else int(valid_len)
    if not 0 <= L <= cache.full_len:
        raise ValueError(f"block_attention: valid_len {L} outside [0, {cache.full_len}]")
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    m8 = _mask_u8(mask, M, L, "block_attention")
    kc, vc = cache.k_tiles[layer], cache.v_tiles[layer]
    if valid_len_dev is not None and (valid_len_dev.dtype != torch.int64 or valid_len_dev.numel() != 1):
        raise ValueError("block_attention: valid_len_dev must be one int64 on the device")
    dev = _native.require_device(q, kc, m8, valid_len_dev)
    out = torch.empty((M, Hq, D), device=dev, dtype=q.dtype)
    if M == 0:
        return out.view(M, Hq * D)
    lib = _native.lib()
    need = lib.simsd_block_attention_workspace_bytes(M, Hq, Hkv, L)
    if need < 0:
        _native.check(-1, "block_attention")
    ws = cache.attention_workspace(need, dev)
    with _native.device_guard(dev):
        status = lib.simsd_block_attention(
            q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), cache.head_stride,
            cache.full_len,
            m8.data_ptr() if m8 is not None else None, m8.stride(0) if m8 is not None else 0,
            out.data_ptr(), out.stride(0), out.stride(1), M, Hq, Hkv, L,
            valid_len_dev.data_ptr() if valid_len_dev is not None else None, D,
            float(D ** -0.5 if scale is None else scale), code, ws.data_ptr(), ws.numel(),
            _native.stream_of(dev))
    _native.check(status, "block_attention")
    return out.view(M, Hq * D)


def block_mask(n_cols: int, ctx_len: int, s0: int, n_prefix: int = 0, n_free: int = 0,
               step_maps: torch.Tensor | None = None, block_length: int = 4, block_size: int = 4,
               out: torch.Tensor | None = None, device=None) -> torch.Tensor:
    """Mask rows [n_prefix committed | n_free denoising | K verify blocks] of
    a cached forward over ``n_cols`` slots (context [0, ctx_len), the rows'
    scratch slots from ``s0``); ``step_maps`` int64 [K, block_length] on the
    device (-1 = never drafted).  -> bool [rows, n_cols] (written into ``out``
    when given: bool or uint8 with unit column stride and a row stride that is
    a multiple of 4)."""
    K = 0 if step_maps is None else int(step_maps.shape[0])
    if step_maps is not None:
        if step_maps.dtype != torch.int64 or step_maps.ndim != 2 or step_maps.shape[1] != block_length:
            raise ValueError("block_mask: step_maps must be int64 [K, block_length]")
        step_maps = step_maps.contiguous()
        device = step_maps.device
    rows = n_prefix + n_free + 2 * K * block_length
    if out is None:
        out = torch.empty((rows, (n_cols + 3) // 4 * 4), device=device, dtype=torch.bool)
    if out.shape[0] != rows or out.shape[1] < n_cols or out.stride(1) != 1:
        raise ValueError(f"block_mask: out must be [{rows}, >= {n_cols}] with unit column stride")
    if rows == 0:
        return out[:, :n_cols]
    dev = _native.require_device(out, step_maps)
    with _native.device_guard(dev):
        status = _native.lib().simsd_block_mask(
            out.data_ptr(), out.stride(0), n_cols, ctx_len, s0, n_prefix, n_free, K, block_length, block_size,
            step_maps.data_ptr() if step_maps is not None else None, _native.stream_of(dev))
    _native.check(status, "block_mask")
    return out[:, :n_cols]
