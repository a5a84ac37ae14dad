"""Pins the verify-layout oracle (CPU only): hand-worked step-causal blocks,
the single-block vectorised rule of speculative_decoding/cache_aware.py:
1149-1180 (equal to the generic rule whenever every position was drafted),
structural invariants of the multi-block rule, the verify sequence layout
and greedy acceptance.  Planted slips (mask time not paired by rank, later
blocks seeing earlier masks, strict instead of non-strict data order) fail."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import verify as over


def _block(step_map, bl=None, bs=None):
    bl = bl or len(step_map)
    bs = bs or bl
    m = over.cached_block_mask(0, 0, 2 * bl, 0, 0, [list(step_map)], bl, bs)
    return m[:, :2 * bl].astype(int)


def test_hand_worked_two_token_block():
    # position 1 unmasked at step 0, position 0 at step 1: data times [2, 1]
    got = _block([1, 0])
    want = np.array([[1, 1, 0, 0],     # D0 (t=2): data t<=2; masks t>2: none
                     [0, 1, 1, 0],     # D1 (t=1): D1; M0 (t=2 > 1)
                     [0, 1, 1, 0],     # M0 (t=2): data t<2 -> D1; masks t>=2 -> M0
                     [0, 0, 1, 1]])    # M1 (t=1): no data t<1; masks t>=1 -> M0, M1
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(6))
def test_single_block_vectorised_rule(seed):
    """cache_aware.py:1165-1173 with data and mask times both = step_map."""
    rng = np.random.default_rng(seed)
    bl = 4 + seed % 3
    step = rng.permutation(bl)
    t = step.astype(int)
    ti, tj = t[:, None], t[None, :]
    want = np.block([[tj <= ti, tj > ti], [tj < ti, tj >= ti]]).astype(int)
    assert np.array_equal(_block(step), want)


def test_identity_steps_are_triangular():
    g = _block(list(range(4)))
    D, DM, MD, MM = g[:4, :4], g[:4, 4:], g[4:, :4], g[4:, 4:]
    assert np.array_equal(D, np.tril(np.ones((4, 4), int)))
    assert np.array_equal(MM, np.triu(np.ones((4, 4), int)))
    assert np.array_equal(MD, np.tril(np.ones((4, 4), int), -1))
    assert np.array_equal(DM, np.triu(np.ones((4, 4), int), 1))


def test_cross_blocks_and_context():
    steps = [[0, 1, 2, 3], [3, 2, 1, 0], [1, 0, 3, 2]]
    ctx, s0, n_cols = 10, 16, 48
    m = over.cached_block_mask(ctx, s0, n_cols, 4, 0, steps, 4, 4)
    assert m.shape == (4 + 24, n_cols)
    assert m[:, :ctx].all() and not m[:, ctx:s0].any()
    assert m[:, s0:s0 + 4].all()                      # the prefix is seen by everyone
    assert not m[:4, s0 + 4:].any()                   # the prefix sees no verify token
    v = m[4:, s0 + 4:s0 + 28]
    for k in range(3):
        rows = slice(8 * k, 8 * k + 8)
        for k2 in range(3):
            data = v[rows, 8 * k2:8 * k2 + 4]
            masks = v[rows, 8 * k2 + 4:8 * k2 + 8]
            if k2 < k:
                assert data.all() and not masks.any()
            elif k2 > k:
                assert not data.any() and not masks.any()
    assert not m[:, s0 + 28:].any()


def test_several_committed_blocks_are_block_causal():
    """Three committed blocks folded in ahead of two verify blocks: each sees
    the context, itself and the blocks before it (the reference flushes
    committed blocks one at a time); every verify row sees all three."""
    steps = [[0, 1, 2, 3], [1, 0, 3, 2]]
    ctx, s0, n_cols = 20, 20, 64
    m = over.cached_block_mask(ctx, s0, n_cols, 12, 0, steps, 4, 4)
    assert m.shape == (12 + 16, n_cols)
    p = m[:12, s0:s0 + 12].astype(int)
    want = np.kron(np.tril(np.ones((3, 3), int)), np.ones((4, 4), int))
    assert np.array_equal(p, want)
    assert m[:, :ctx].all()
    assert m[12:, s0:s0 + 12].all()
    assert not m[:12, s0 + 12:].any()
    # one committed block: all of it, as before
    one = over.cached_block_mask(ctx, s0, n_cols, 4, 0, steps, 4, 4)
    assert one[:4, s0:s0 + 4].all()


def test_free_block_and_never_drafted():
    m = over.cached_block_mask(5, 8, 20, 4, 4, [], 4, 4)
    assert m[4:8, 8:16].all() and not m[:4, 12:16].any()
    # a never-drafted position is a mask token of the data segment: its rank
    # pairing shifts the mask segment, as in the generic rule
    g = _block([0, -1, 1, 2])
    assert g.shape == (8, 8)
    assert g[1, 1] == 1                               # a mask sees itself (t_j >= t_i)


def test_planted_mask_slips():
    step = [2, 0, 3, 1]
    good = _block(step)
    t = np.array(step) + 1
    # strict data order: a data token would not see itself
    strict = np.block([[t[None, :] < t[:, None], t[None, :] > t[:, None]],
                       [t[None, :] < t[:, None], t[None, :] >= t[:, None]]]).astype(int)
    assert not np.array_equal(strict, good)
    # masks timed by their own position (not by data-rank pairing) differ once
    # a position was never drafted
    sm = [0, -1, 1, 2]
    lab = np.array([s + 1 if s >= 0 else 5 for s in sm] + [5] * 4)
    typ = np.where(lab <= 4, 1, 2)
    tim = lab.copy()
    tim[4:] = [lab[p] if lab[p] <= 4 else 5 for p in range(4)]     # the slip
    ti, tj, yi, yj = tim[:, None], tim[None, :], typ[:, None], typ[None, :]
    slip = (((yi == 1) & (yj == 1) & (tj <= ti)) | ((yi == 1) & (yj == 2) & (tj > ti)) |
            ((yi == 2) & (yj == 1) & (tj < ti)) | ((yi == 2) & (yj == 2) & (tj >= ti))).astype(int)
    assert not np.array_equal(slip, _block(sm))
    steps = [[0, 1, 2, 3], [0, 1, 2, 3]]
    m = over.cached_block_mask(0, 0, 16, 0, 0, steps, 4, 4)
    assert not m[8:, 4:8].any()                       # block 1 never sees block 0's masks


def test_build_verify_sequence_multi_layout():
    ids, tl, bi, lab, pos = over.build_verify_sequence_multi(
        [11, 12, 13], [[21, 22, 23, 24]], [[31, 32, 33, 34], [41, 42, 43, 44]],
        [[0, 1, 2, 3], [3, -1, 1, 0]], 4, 4, mask_token_id=99)
    assert ids == [11, 12, 13, 21, 22, 23, 24, 31, 32, 33, 34, 99, 99, 99, 99, 41, 42, 43, 44, 99, 99, 99, 99]
    assert tl == [0, 0, 0, 1, 1, 1, 1, 1, 2, 3, 4, 5, 5, 5, 5, 4, 5, 2, 1, 5, 5, 5, 5]
    assert bi == [-1] * 3 + [0] * 4 + [1] * 8 + [2] * 8
    assert pos == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 7, 8, 9, 10, 11, 12, 13, 14, 11, 12, 13, 14]
    assert lab[11:15] == [31, 32, 33, 34] and lab[19:] == [41, 42, 43, 44]


def test_greedy_match_verify():
    assert over.greedy_match_verify([1, 2, 3, 4], [1, 2, 3, 4]) == ([1, 2, 3, 4], 4, None)
    assert over.greedy_match_verify([1, 2, 3, 4], [1, 2, 9, 4]) == ([1, 2, 9], 2, 9)
    assert over.greedy_match_verify([5, 2, 3, 4], [1, 2, 3, 4]) == ([1], 0, 1)
