"""Oracle of the attention prologue and the block attention (test
infrastructure only).

qk_norm_rope   the SDAR q/k path, sdar/modeling_sdar.py:250-262: the stock
               RMSNorm over each head (fp64 statistics, x * r rounded to the
               dtype, times the weight, rounded), then apply_rotary_pos_emb
               (modeling_sdar.py:122-153) with the reference's bf16 rounding
               points: dtype(dtype(x * cos) + dtype(rotate_half(x) * sin)), the
               sum formed in fp32 as torch's bf16 add does.
attention      softmax(scale * q k^T + mask) v in fp64 with grouped KV heads
               (query head hq reads KV head hq // n_rep, modeling_sdar.py:
               156-166 repeat_kv) -- F.scaled_dot_product_attention with a bool
               mask, adapters/base.py:245-262.  Rows with no visible key give 0.

Pinned in tests against torch's CPU composition of the reference's own ops
(bit-exact for qk_norm_rope) and torch's CPU scaled_dot_product_attention in
fp32, plus closed forms: position 0 leaves the normed head unchanged, one
visible key returns that key's value row, equal keys average the visible
values.
"""
from __future__ import annotations

import numpy as np

from .numerics import ROUNDERS


def qk_norm_rope(x: np.ndarray, weight: np.ndarray | None, eps: float, cos: np.ndarray, sin: np.ndarray,
                 dtype: str = "bf16") -> np.ndarray:
    """x [M, H, D] (dtype values), cos/sin [M, D] (dtype values) -> [M, H, D]."""
    rnd = ROUNDERS[dtype]
    x = np.asarray(x, dtype=np.float64)
    if weight is not None:
        var = (x * x).mean(axis=-1, keepdims=True)
        r = 1.0 / np.sqrt(var + eps)
        x = rnd(np.asarray(weight, dtype=np.float64) * rnd(x * r))
    D = x.shape[-1]
    rot = np.concatenate([-x[..., D // 2:], x[..., :D // 2]], axis=-1)
    c = np.asarray(cos, dtype=np.float64)[:, None, :]
    s = np.asarray(sin, dtype=np.float64)[:, None, :]
    # the sum of the two rounded terms is formed in fp32, as the dtype's add does
    return rnd((rnd(x * c) + rnd(rot * s)).astype(np.float32).astype(np.float64))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray | None, scale: float) -> np.ndarray:
    """q [M, Hq, D], k/v [Hkv, L, D], mask [M, L] bool or None -> [M, Hq, D] fp64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    M, Hq, D = q.shape
    Hkv, L, _ = k.shape
    n_rep = Hq // Hkv
    vis = np.ones((M, L), dtype=bool) if mask is None else np.asarray(mask, dtype=bool)[:, :L]
    out = np.zeros((M, Hq, D), dtype=np.float64)
    for hq in range(Hq):
        h = hq // n_rep
        s = (q[:, hq, :] @ k[h].T) * scale           # [M, L]
        s = np.where(vis, s, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        ok = np.isfinite(mx[:, 0])
        e = np.where(vis & ok[:, None], np.exp(s - np.where(ok[:, None], mx, 0.0)), 0.0)
        den = e.sum(axis=1, keepdims=True)
        out[:, hq, :] = np.where(ok[:, None], (e @ v[h]) / np.where(den > 0, den, 1.0), 0.0)
    return out
