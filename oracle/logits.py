"""Oracle of the lm_head epilogue (test infrastructure only).

softmax_argmax  probs = softmax(l) in fp64 over each row of fp32-cast
                logits, ids = the first index of the row maximum, conf = the
                probability there -- speculative_decoding/cache_aware.py:916-918
                (``F.softmax(logits.float())``, ``argmax``, ``gather``) and the
                verify pass's target_probs, cache_aware.py:1197-1198.
denoise_select  the unmasking step that follows, cache_aware.py:919-938:
                masked rows compete on conf, the n_unmask largest win (ties:
                the lower row; unmasked rows rank as -inf), winners take their
                argmax id, their step in step_map and their softmax row.

Pinned in tests against torch's CPU softmax / argmax / topk (library
routines) on tie-free data, and against closed forms: a uniform row gives
conf = 1 / V and id 0; repeated maxima give the first index; one dominant
logit gives conf -> 1; -inf entries carry zero probability.
"""
from __future__ import annotations

import numpy as np


def softmax_argmax(logits: np.ndarray):
    """logits [M, V] (any float dtype) -> (ids int64 [M], conf f64 [M], probs f64 [M, V])."""
    l64 = np.asarray(logits, dtype=np.float32).astype(np.float64)
    M, V = l64.shape
    ids = np.zeros(M, dtype=np.int64)
    conf = np.zeros(M, dtype=np.float64)
    probs = np.zeros((M, V), dtype=np.float64)
    for m in range(M):
        row = l64[m]
        mx = row.max()
        ids[m] = int(np.flatnonzero(row == mx)[0])   # first occurrence, as torch.argmax
        e = np.exp(row - mx)
        s = e.sum()
        probs[m] = e / s
        conf[m] = probs[m, ids[m]]
    return ids, conf, probs


def denoise_select(logits: np.ndarray, cur_ids: np.ndarray, mask_id: int, n_unmask: int, step: int,
                   step_map: np.ndarray | None = None, per_pos_probs: np.ndarray | None = None):
    """In-place on copies: returns (cur_ids', step_map', per_pos_probs', ids, conf)."""
    ids, conf, probs = softmax_argmax(logits)
    cur = np.array(cur_ids, dtype=np.int64, copy=True)
    M = cur.shape[0]
    key = np.where(cur == mask_id, conf, -np.inf)
    # descending key, equal keys by row: a stable sort of -key
    order = sorted(range(M), key=lambda m: (-key[m], m))
    top = order[:n_unmask]
    sm = None if step_map is None else np.array(step_map, dtype=np.int64, copy=True)
    pp = None if per_pos_probs is None else np.array(per_pos_probs, dtype=np.float64, copy=True)
    for m in top:
        cur[m] = ids[m]
        if sm is not None:
            sm[m] = step
        if pp is not None:
            pp[m] = probs[m]
    return cur, sm, pp, ids, conf
