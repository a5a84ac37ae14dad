"""Oracle of the multi-block verify layout, its attention mask and greedy
acceptance (test infrastructure only).

build_verify_sequence_multi  the verify sequence [prompt | accepted data |
        K x (draft data, draft mask)], speculative_decoding/verify.py:350-418.
multi_block_causal_mask      the visibility rule of
        sdar/new_attn_multi_block.py:22-183 (prompt block-causal, per-block
        step-causal data/mask pairing by within-block rank, later blocks see
        earlier blocks' data only, padding isolated), for one sequence.
cached_block_mask            the rows a cached forward actually runs -- a
        folded prefix block, a freely denoised block, K verify blocks -- over
        the cache's slot space (committed context, then scratch slots), derived
        from multi_block_causal_mask on the equivalent full sequence.
greedy_match_verify          speculative_decoding/mrs.py:111-146.

Pinned in tests against hand-worked layouts, the single-block vectorised rule
of speculative_decoding/cache_aware.py:1149-1180, and invariants (an identity
step map gives a lower-triangular data block; data never sees its own block's
earlier-step masks ...).
"""
from __future__ import annotations

import numpy as np


def build_verify_sequence_multi(prompt_ids, accepted_blocks, draft_blocks, step_maps, block_length, block_size,
                                mask_token_id, share_mask_position=True):
    """-> (input_ids, token_labels, block_ids, labels, position_ids), lists."""
    ids = list(prompt_ids)
    tl = [0] * len(ids)
    bi = [-1] * len(ids)
    lab = [-100] * len(ids)
    pos = list(range(len(ids)))
    cur = len(ids)
    for b, blk in enumerate(accepted_blocks):
        n = len(blk)
        ids += list(blk)
        tl += [1] * n
        bi += [b] * n
        lab += [-100] * n
        pos += list(range(cur, cur + n))
        cur += n
    M = len(accepted_blocks)
    for k, (d, sm) in enumerate(zip(draft_blocks, step_maps)):
        data_pos = list(range(cur, cur + block_length))
        cur += block_length
        ids += list(d)
        tl += [s + 1 if s >= 0 else block_size + 1 for s in sm]
        bi += [M + k] * block_length
        lab += [-100] * block_length
        pos += data_pos
        if share_mask_position:
            mpos = data_pos
        else:
            mpos = list(range(cur, cur + block_length))
            cur += block_length
        ids += [mask_token_id] * block_length
        tl += [block_size + 1] * block_length
        bi += [M + k] * block_length
        lab += list(d)
        pos += mpos
    return ids, tl, bi, lab, pos


def _times(tl: np.ndarray, bi: np.ndarray, block_size: int):
    """Per-token (type, time): type 0 prompt/pad, 1 data, 2 mask; a mask token
    takes the time of the data token of the same within-block rank."""
    L = tl.shape[0]
    is_data = (tl > 0) & (tl <= block_size)
    is_mask = tl == block_size + 1
    typ = np.where(is_data, 1, np.where(is_mask, 2, 0))
    time = tl.astype(np.float64)
    time[tl == -1] = np.inf
    time[tl == 0] = 0.0
    for b in sorted(set(bi[bi >= 0].tolist())):
        idx = np.flatnonzero(bi == b)
        data = [i for i in idx if typ[i] == 1]
        masks = [i for i in idx if typ[i] == 2]
        for r, i in enumerate(masks):
            if r < len(data):
                time[i] = time[data[r]]
    return typ, time


def multi_block_causal_mask(token_labels, block_ids, block_size: int, block_causal_prompt: bool = True) -> np.ndarray:
    """[L, L] bool, True = row may attend to column."""
    tl = np.asarray(token_labels, dtype=np.int64)
    bi = np.asarray(block_ids, dtype=np.int64)
    L = tl.shape[0]
    typ, time = _times(tl, bi, block_size)
    is_prompt = tl == 0
    is_pad = tl == -1
    ti, tj = time[:, None], time[None, :]
    yi, yj = typ[:, None], typ[None, :]
    bi_i, bi_j = bi[:, None], bi[None, :]
    if block_causal_prompt:
        pblk = (np.cumsum(is_prompt) - 1) // block_size
        rule_prompt = is_prompt[:, None] & is_prompt[None, :] & (pblk[None, :] <= pblk[:, None])
        rule_see_prompt = (~is_prompt[:, None]) & (~is_pad[:, None]) & is_prompt[None, :]
    else:
        rule_prompt = (is_prompt[:, None] & is_prompt[None, :]) | (is_prompt[:, None] & (typ == 2)[None, :])
        rule_see_prompt = np.broadcast_to(is_prompt[None, :], (L, L))
    same = (bi_i == bi_j) & (bi_i >= 0)
    dd = same & (yi == 1) & (yj == 1) & (tj <= ti)
    dm = same & (yi == 1) & (yj == 2) & (tj > ti)
    md = same & (yi == 2) & (yj == 1) & (tj < ti)
    mm = same & (yi == 2) & (yj == 2) & (tj >= ti)
    cross = (bi_i > bi_j) & (bi_j >= 0) & (yj == 1)
    m = rule_prompt | rule_see_prompt | dd | dm | md | mm | cross
    return m & ~is_pad[:, None] & ~is_pad[None, :]


def cached_block_mask(ctx_len: int, s0: int, n_cols: int, n_prefix: int, n_free: int, step_maps, block_length: int,
                      block_size: int) -> np.ndarray:
    """Rows [prefix | free block | K verify blocks (data, mask)] of a cached
    forward over slots: [0, ctx_len) committed context, then from s0 the
    scratch slots of these rows in row order.  The prefix is a committed block
    (accepted data); the free block is the block being denoised (it sees the
    context, the prefix and all of itself); verify blocks follow the
    multi-block rule.  -> [R, n_cols] bool.

    The prefix may hold several committed blocks (of ``block_length``):
    every later row sees all of them, and among themselves they are
    block-causal, as the reference's runner flushes committed blocks into the
    cache one block at a time (speculative_decoding/cache_aware.py:2324-2336,
    each flush one _extend_cache_graph call of a full block, 1202-1259: a
    block sees the context before it and all of itself)."""
    K = len(step_maps)
    R = n_prefix + n_free + 2 * K * block_length
    out = np.zeros((R, n_cols), dtype=bool)
    out[:, :ctx_len] = True
    # prefix: seen by every later row; block-causal among itself
    out[n_prefix:, s0:s0 + n_prefix] = True
    pb = np.arange(n_prefix) // block_length
    out[:n_prefix, s0:s0 + n_prefix] = pb[None, :] <= pb[:, None]
    # free block: its rows see themselves
    out[n_prefix:n_prefix + n_free, s0 + n_prefix:s0 + n_prefix + n_free] = True
    if K:
        # the verify rows as a full sequence: one context token standing for the
        # prompt, the prefix as accepted block 0, then the K draft blocks
        dummy = [0] * K * block_length
        _, tl, bi, _, _ = build_verify_sequence_multi(
            [7], [[1] * n_prefix] if n_prefix else [], [dummy[k * block_length:(k + 1) * block_length]
                                                        for k in range(K)],
            step_maps, block_length, block_size, mask_token_id=9)
        full = multi_block_causal_mask(tl, bi, block_size)
        v0 = 1 + n_prefix                                   # first verify token in the sequence
        rows = slice(n_prefix + n_free, R)
        c0 = s0 + n_prefix + n_free
        out[rows, c0:c0 + 2 * K * block_length] = full[v0:, v0:]
        # sanity: the verify rows see the context token and the whole prefix
        assert full[v0:, 0].all() and full[v0:, 1:v0].all()
    return out


def greedy_match_verify(draft_ids, target_argmax):
    """-> (accepted_ids, n_accepted, bonus or None): accept while the draft
    equals the target's argmax, commit the argmax at the first mismatch."""
    for pos, (d, t) in enumerate(zip(draft_ids, target_argmax)):
        if d != t:
            return list(draft_ids[:pos]) + [t], pos, t
    return list(draft_ids), len(draft_ids), None


def accept_blocks(draft_blocks, target_argmax, block_length, eos_ids=None):
    """K-block greedy acceptance with first-reject truncation,
    speculative_decoding/speculative_decode.py:895-953 (greedy verify,
    partial_block_fill = "draft_argmax"): -> (committed blocks, generated
    tokens, accepted count).  Block k's final ids come from
    greedy_match_verify; a short block is padded with the draft's own tokens
    from len(final) on; the loop stops after the first rejected block, or
    after a block whose final ids hold an id of ``eos_ids`` (:944-950)."""
    eos = set(eos_ids or ())
    committed, generated, n_acc = [], [], 0
    for k in range(len(draft_blocks)):
        final, n, _bonus = greedy_match_verify(draft_blocks[k], target_argmax[k])
        n_acc += n
        block = list(final)
        if len(block) < block_length:
            block += list(draft_blocks[k][len(block):block_length])
        committed.append(block)
        generated.extend(final)
        if n < block_length or any(t in eos for t in final):
            break
    return committed, generated, n_acc
