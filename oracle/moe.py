"""Oracle of the fused MoE step (test infrastructure only).

route_topk      top-k routing; ids by a stable sort of -logits (ties -> lower
                index), scores softmax/sigmoid, renormalised when k > 1,
                scaled -- the rule of _routing,
                kernels/workspace/moe_dispatch/build_oracle.py:71-90, with the
                softmax option the 256-expert, top-8 MoE step uses.
align           the integer tables of _align, kernels/moe_dispatch_fused.py:93-132
                (counts, offsets, stable permutation, 16-padded slot table,
                per-tile experts), plus the padded offsets.
dispatch_grouped  the stock per-expert loop, reference_moe_dispatch,
                kernels/workspace/moe_dispatch/build_oracle.py:34-67, with the
                dtype discipline of kernels/workspace/moe_dispatch/CONTRACT.md:26-40
                (g, u, silu(g), h, y rounded to the dtype; weighting and the
                k-sum in fp32; cast back last), evaluated in fp64.
dispatch_direct per-token evaluation of the same formula, no sorting -- pins
                the grouping/gather/scatter of dispatch_grouped.
"""
from __future__ import annotations

import numpy as np

from .numerics import ROUNDERS

BLOCK_M = 16


def _identity(a):
    return np.asarray(a, dtype=np.float64)


def _rounder(dtype: str):
    return _identity if dtype == "fp64" else ROUNDERS[dtype]


# ───────────────────────────────────────────────────────────── routing ───
def route_topk(logits, k: int, scoring: str = "softmax", renorm: bool = True,
               scale: float = 1.0):
    """logits (T, E) -> (ids int64 (T, k), weights float64 (T, k))."""
    lg = np.asarray(logits, dtype=np.float64)
    ids = np.argsort(-lg, axis=1, kind="stable")[:, :k].astype(np.int64)
    picked = np.take_along_axis(lg, ids, axis=1)
    if scoring == "softmax":
        mx = lg.max(axis=1, keepdims=True)
        z = np.exp(lg - mx).sum(axis=1, keepdims=True)
        s = np.exp(picked - mx) / z
    elif scoring == "sigmoid":
        s = 1.0 / (1.0 + np.exp(-picked))
    else:
        raise ValueError(scoring)
    if renorm and k > 1:
        s = s / (s.sum(axis=1, keepdims=True) + 1e-20)
    return ids, s * scale


# ─────────────────────────────────────────────────────────────── align ───
def num_tiles(M: int, E: int) -> int:
    """_num_tiles, kernels/moe_dispatch_fused.py:135-137."""
    return min(E, M) + (M + BLOCK_M - 1) // BLOCK_M


def align(ids, E: int, n_tiles: int | None = None) -> dict:
    """Integer tables for flat slot ids (any shape, flattened).

    Slot ids outside [0, E) belong to no group: they sort after every valid
    slot (in slot order) and never appear in ``slots``.
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    M = flat.size
    if n_tiles is None:
        n_tiles = num_tiles(M, E)
    valid = (flat >= 0) & (flat < E)
    key = np.where(valid, flat, E)
    counts = np.bincount(key, minlength=E + 1)[:E]
    padded = (counts + BLOCK_M - 1) // BLOCK_M * BLOCK_M
    pad_end = np.cumsum(padded)
    pad_start = pad_end - padded
    grp_start = np.cumsum(counts) - counts
    offsets = np.concatenate([grp_start, [counts.sum()]])
    pad_offsets = np.concatenate([pad_start, [padded.sum()]])
    perm = np.argsort(key, kind="stable")
    slots = np.full(n_tiles * BLOCK_M, -1, dtype=np.int64)
    sorted_keys = key[perm]
    start_ext = np.concatenate([grp_start, [counts.sum()]])
    rank = np.arange(M) - start_ext[sorted_keys]
    ok = sorted_keys < E
    dest = pad_start[sorted_keys[ok]] + rank[ok]
    inside = dest < slots.size
    slots[dest[inside]] = perm[ok][inside]
    tile_expert = np.searchsorted(pad_end, np.arange(n_tiles) * BLOCK_M, side="right")
    i32 = lambda a: np.asarray(a, dtype=np.int32)
    return {"counts": i32(counts), "offsets": i32(offsets), "pad_offsets": i32(pad_offsets),
            "perm": i32(perm), "slots": i32(slots), "tile_expert": i32(tile_expert)}


# ──────────────────────────────────────────────────────────── dispatch ───
def _silu(v):
    return v / (1.0 + np.exp(-v))


def _mlp(tok, wg, wu, wd, rnd):
    g = rnd(tok @ wg.T)
    u = rnd(tok @ wu.T)
    h = rnd(rnd(_silu(g)) * u)
    return rnd(h @ wd.T)


def dispatch_grouped(x, ids, w, w_gate, w_up, w_down, dtype: str = "bf16", shared=None):
    """The stock loop over experts (sorted slots, one matmul per expert).

    x (T, H), ids (T, k), w (T, k) fp32, w_gate/w_up (E, I, H), w_down (E, H, I);
    inputs are values representable in `dtype`; dtype "fp64" disables every
    intermediate rounding (the fp64 ground truth).  Returns float64 (T, H).
    """
    rnd = _rounder(dtype)
    x = np.asarray(x, dtype=np.float64)
    ids = np.asarray(ids, dtype=np.int64)
    w = np.asarray(w, dtype=np.float64)
    wg, wu, wd = (np.asarray(a, dtype=np.float64) for a in (w_gate, w_up, w_down))
    T, k = ids.shape
    E = wg.shape[0]
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    y = np.zeros((T * k, x.shape[1]))
    start = 0
    counts = np.bincount(flat[(flat >= 0) & (flat < E)], minlength=E)
    sorted_ids = flat[order]
    for e in range(E):
        n = int(counts[e])
        if n == 0:
            continue
        idx = order[np.searchsorted(sorted_ids, e):][:n]
        y[idx] = _mlp(x[idx // k], wg[e], wu[e], wd[e], rnd)
        start += n
    ok = ((ids >= 0) & (ids < E)).astype(np.float64)
    f32 = _identity if dtype == "fp64" else ROUNDERS["fp32"]
    acc = np.zeros((T, x.shape[1]))
    for j in range(k):   # fp32 weighting and k-ordered fp32 sum
        acc = f32(acc + f32(y.reshape(T, k, -1)[:, j, :] * (w[:, j] * ok[:, j])[:, None]))
    out = rnd(acc)
    if shared is not None:
        sg, su, sd = (np.asarray(a, dtype=np.float64) for a in shared)
        out = rnd(out + _mlp(x, sg, su, sd, rnd))
    return out


def dispatch_direct(x, ids, w, w_gate, w_up, w_down, dtype: str = "bf16", shared=None):
    """Same formula token by token (no sort, no grouping)."""
    rnd = _rounder(dtype)
    f32 = _identity if dtype == "fp64" else ROUNDERS["fp32"]
    x = np.asarray(x, dtype=np.float64)
    wg, wu, wd = (np.asarray(a, dtype=np.float64) for a in (w_gate, w_up, w_down))
    T, k = np.asarray(ids).shape
    E = wg.shape[0]
    out = np.zeros((T, x.shape[1]))
    for t in range(T):
        acc = np.zeros(x.shape[1])
        for j in range(k):
            e = int(ids[t][j])
            if not 0 <= e < E:
                continue
            yj = _mlp(x[t:t + 1], wg[e], wu[e], wd[e], rnd)[0]
            acc = f32(acc + f32(yj * float(w[t][j])))
        out[t] = rnd(acc)
    if shared is not None:
        sg, su, sd = (np.asarray(a, dtype=np.float64) for a in shared)
        out = rnd(out + _mlp(x, sg, su, sd, rnd))
    return out


def tolerance(ref_absmax: float, dtype: str) -> float:
    """kernels/workspace/moe_dispatch/duipai.py:37-60: bf16 4 ULP-relative
    (2^-6 max|ref| + 1e-3), fp32 1e-5 * max(1, max|ref|)."""
    if dtype == "fp32":
        return 1e-5 * max(1.0, ref_absmax)
    return 2 ** -6 * ref_absmax + 1e-3


def fp64_gate(err_fused: float, err_stock: float, scale: float, dtype: str) -> bool:
    """kernels/workspace/moe_dispatch/duipai.py:88-116: against the fp64 truth,
    bf16 fused error <= max(1.5 x stock error, 2^-12 scale); fp32 relative 1e-5."""
    if dtype == "fp32":
        return err_fused <= 1e-5 * max(scale, 1.0)
    return err_fused <= max(err_stock * 1.5, 2 ** -12 * scale)
