"""Write the golden fixtures under tests/golden/ from closed forms.

    python tests/golden/make_golden.py

Nothing here runs the reference or the oracle.  Every expected value comes
from exact integer / rational arithmetic (Python ints and Fractions with
round-to-nearest-even to bf16 done on the exact value) or from brute-force
definitions (sorting with an explicit key, counting by loops):

  thin_int.npz    small-integer x, w: every fp32 partial sum is an exact
                  integer, so any summation order gives the exact sum; the
                  expected output is that sum rounded once to bf16 (and the
                  fp32 output is the sum itself).  Covers M in 1..32, odd K/N.
  thin_k1.npz     K = 1: y = bf16(x * w), the product of two bf16 is exact.
  align.npz       flat expert ids -> counts, offsets, padded offsets, stable
                  permutation, 16-padded slot table, per-tile experts, by
                  loops over the definition of the reference's _align.
  route.npz       logits with many exact ties -> top-k ids by sorting with key
                  (-logit, index); all-equal rows whose renormalised weights
                  are exactly scale / k.
  moe_int.npz     integer MoE layers built so every stage is exact: gate
                  outputs are integers in [49, 79] (silu(g) rounds to g), up
                  outputs small integers, h = bf16(g*u), down sums exact
                  integers, routing weights powers of two; the expected output
                  follows the reference's rounding points exactly.
"""
from __future__ import annotations

import os
import sys
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.numerics import bf16_round_int  # noqa: E402  (pure-integer rounding only)

BLOCK_M = 16


def _bf16_exact_array(vals) -> np.ndarray:
    return np.array([float(bf16_round_int(int(v) if isinstance(v, (int, np.integer)) else v))
                     for v in np.asarray(vals, dtype=object).reshape(-1)],
                    dtype=np.float64).reshape(np.shape(vals))


def make_thin_int(rng) -> dict:
    out = {}
    shapes = [(1, 64, 8), (4, 2048, 48), (7, 1000, 33), (16, 4096, 20), (32, 512, 40),
              (4, 8, 1), (3, 24, 130)]
    for i, (M, K, N) in enumerate(shapes):
        x = rng.integers(-4, 5, size=(M, K)).astype(np.int64)
        w = rng.integers(-4, 5, size=(N, K)).astype(np.int64)
        y = x @ w.T                                  # exact integers
        out[f"c{i}_x"] = x.astype(np.int8)
        out[f"c{i}_w"] = w.astype(np.int8)
        out[f"c{i}_y_fp32"] = y.astype(np.float64)   # |y| < 2^24: exact in fp32
        out[f"c{i}_y_bf16"] = _bf16_exact_array(y)
    # bias case: |acc| and |acc + bias| <= 256 stay exact in bf16
    M, K, N = 4, 16, 24
    x = rng.integers(-2, 3, size=(M, K)).astype(np.int64)
    w = rng.integers(-2, 3, size=(N, K)).astype(np.int64)
    b = rng.integers(-8, 9, size=(N,)).astype(np.int64)
    out["bias_x"], out["bias_w"], out["bias_b"] = x.astype(np.int8), w.astype(np.int8), b.astype(np.int8)
    out["bias_y"] = (x @ w.T + b[None, :]).astype(np.float64)
    out["n_cases"] = np.array(len(shapes))
    return out


def make_thin_k1(rng) -> dict:
    # bf16 values: 8 significant bits, random exponents
    def bf16_vals(n):
        mant = rng.integers(128, 256, size=n)
        exp = rng.integers(-20, 10, size=n)
        sign = rng.choice([-1, 1], size=n)
        return [sign[i] * Fraction(int(mant[i])) * Fraction(2) ** int(exp[i] - 7) for i in range(n)]
    M, N = 4, 96
    xs, ws = bf16_vals(M), bf16_vals(N)
    y = [[float(bf16_round_int(xs[m] * ws[n])) for n in range(N)] for m in range(M)]
    return {"x": np.array([float(v) for v in xs]).reshape(M, 1),
            "w": np.array([float(v) for v in ws]).reshape(N, 1),
            "y": np.array(y)}


def align_bruteforce(ids: list[int], E: int, n_tiles: int) -> dict:
    M = len(ids)
    key = [e if 0 <= e < E else E for e in ids]
    counts = [0] * E
    for e in key:
        if e < E:
            counts[e] += 1
    offsets, pad_offsets = [0], [0]
    for e in range(E):
        offsets.append(offsets[-1] + counts[e])
        pad_offsets.append(pad_offsets[-1] + (counts[e] + BLOCK_M - 1) // BLOCK_M * BLOCK_M)
    perm = sorted(range(M), key=lambda i: (key[i], i))
    slots = [-1] * (n_tiles * BLOCK_M)
    for e in range(E):
        members = [i for i in perm if key[i] == e]
        for r, i in enumerate(members):
            if pad_offsets[e] + r < len(slots):
                slots[pad_offsets[e] + r] = i
    tile_expert = []
    for t in range(n_tiles):
        row = t * BLOCK_M
        e = 0
        while e < E and pad_offsets[e + 1] <= row:   # first e whose padded end > row
            e += 1
        tile_expert.append(e)
    return {"counts": counts, "offsets": offsets, "pad_offsets": pad_offsets,
            "perm": perm, "slots": slots, "tile_expert": tile_expert}


def make_align(rng) -> dict:
    out = {}
    cases = []
    for T, k, E in [(4, 8, 256), (16, 8, 256), (64, 8, 256), (1, 8, 256), (4, 2, 8), (7, 3, 13),
                    (16, 1, 32), (32, 4, 64), (100, 8, 1024), (33, 6, 1), (5, 2, 3)]:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if k <= E else \
            rng.integers(0, E, size=(T, k))
        cases.append((T, k, E, ids))
    # concentrated: most slots on a few experts (one group spans many tiles)
    T, k, E = 64, 8, 256
    hot = rng.permutation(E)[:10]
    ids = np.stack([rng.choice(hot, size=k, replace=False) for _ in range(T)])
    cases.append((T, k, E, ids))
    # all tokens on one expert (k = 1), the reference's all_one_expert case
    cases.append((32, 1, 256, np.zeros((32, 1), dtype=np.int64)))
    # repeated expert within a token, and ids outside [0, E)
    cases.append((6, 4, 16, rng.integers(0, 4, size=(6, 4))))
    bad = rng.integers(0, 16, size=(9, 4))
    bad[0, 1], bad[3, 0], bad[8, 3] = -1, 16, 99
    cases.append((9, 4, 16, bad))
    for i, (T, k, E, ids) in enumerate(cases):
        flat = [int(v) for v in np.asarray(ids).reshape(-1)]
        M = len(flat)
        n_tiles = min(E, M) + (M + BLOCK_M - 1) // BLOCK_M
        ref = align_bruteforce(flat, E, n_tiles)
        out[f"c{i}_ids"] = np.asarray(ids, dtype=np.int64).reshape(T, k)
        out[f"c{i}_E"] = np.array(E)
        out[f"c{i}_n_tiles"] = np.array(n_tiles)
        for name, v in ref.items():
            out[f"c{i}_{name}"] = np.asarray(v, dtype=np.int32)
    out["n_cases"] = np.array(len(cases))
    return out


def make_route(rng) -> dict:
    out = {}
    cases = []
    for T, E, k in [(8, 256, 8), (5, 64, 4), (3, 13, 3), (4, 1024, 8), (2, 8, 8)]:
        lg = rng.integers(-3, 4, size=(T, E)).astype(np.float64)   # many exact ties
        cases.append((lg, k))
    for i, (lg, k) in enumerate(cases):
        T, E = lg.shape
        ids = [sorted(range(E), key=lambda e: (-lg[t, e], e))[:k] for t in range(T)]
        out[f"c{i}_logits"] = lg.astype(np.float32)
        out[f"c{i}_k"] = np.array(k)
        out[f"c{i}_ids"] = np.array(ids, dtype=np.int64)
    # all-equal rows: any score, renormalised over k picks, is exactly 1/k
    out["flat_logits"] = np.full((4, 32), 0.75, dtype=np.float32)
    out["flat_k"] = np.array(8)
    out["flat_ids"] = np.tile(np.arange(8), (4, 1)).astype(np.int64)
    out["flat_w_scale2.5"] = np.full((4, 8), 2.5 / 8)
    out["n_cases"] = np.array(len(cases))
    return out


def _mlp_exact(xrow, wg, wu, wd, rnd):
    """Exact per-token expert MLP with rounding `rnd` at the reference's points."""
    H = len(xrow)
    I = len(wg)
    g = [rnd(sum(int(xrow[h]) * int(wg[i][h]) for h in range(H))) for i in range(I)]
    u = [rnd(sum(int(xrow[h]) * int(wu[i][h]) for h in range(H))) for i in range(I)]
    # silu(g) == g exactly in fp32 and bf16 for integer g >= 49 (exp(-49) < 2^-70)
    assert all(gi >= 49 for gi in g)
    hh = [rnd(rnd(g[i]) * u[i]) for i in range(I)]
    return [rnd(sum(hh[i] * int(wd[n][i]) for i in range(I))) for n in range(len(wd))]


def make_moe_int(rng) -> dict:
    out = {}
    configs = [(5, 2, 8, 16, 8, False), (37, 3, 8, 32, 16, True), (4, 8, 256, 16, 8, True),
               (16, 1, 32, 24, 8, False), (3, 4, 6, 40, 24, True)]
    for ci, (T, k, E, H, I, with_shared) in enumerate(configs):
        x = rng.integers(-1, 2, size=(T, H))
        x[:, 0] = 1
        def gate(n_out):
            w = rng.integers(-1, 2, size=(n_out, H))
            w[:, 0] = 64
            return w
        wg = np.stack([gate(I) for _ in range(E)])
        wu = rng.integers(-2, 3, size=(E, I, H))
        wd = rng.integers(-1, 2, size=(E, H, I))
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
        wts = rng.choice([0.5, 1.0, 2.0], size=(T, k))
        shared = None
        if with_shared:
            Is = I
            shared = (gate(Is), rng.integers(-2, 3, size=(Is, H)), rng.integers(-1, 2, size=(H, Is)))
        exp = {}
        for dtype, rnd in (("bf16", bf16_round_int), ("fp32", lambda v: Fraction(v))):
            res = []
            for t in range(T):
                acc = Fraction(0)
                for j in range(k):
                    e = int(ids[t, j])
                    yj = _mlp_exact(x[t], wg[e], wu[e], wd[e], rnd)
                    if j == 0:
                        acc = [Fraction(0)] * H
                    acc = [acc[n] + yj[n] * Fraction(wts[t, j]) for n in range(H)]
                o = [rnd(a) for a in acc]
                if shared is not None:
                    ys = _mlp_exact(x[t], *shared, rnd)
                    o = [rnd(o[n] + ys[n]) for n in range(H)]
                res.append([float(v) for v in o])
            exp[dtype] = np.array(res)
        p = f"c{ci}_"
        out[p + "x"] = x.astype(np.int8)
        out[p + "w_gate"] = wg.astype(np.int8)
        out[p + "w_up"] = wu.astype(np.int8)
        out[p + "w_down"] = wd.astype(np.int8)
        out[p + "ids"] = ids.astype(np.int64)
        out[p + "w"] = wts.astype(np.float32)
        out[p + "y_bf16"] = exp["bf16"]
        out[p + "y_fp32"] = exp["fp32"]
        if shared is not None:
            out[p + "sh_gate"], out[p + "sh_up"], out[p + "sh_down"] = (s.astype(np.int8) for s in shared)
    out["n_cases"] = np.array(len(configs))
    return out


def main():
    rng = np.random.default_rng(20261201)
    for name, fn in (("thin_int", make_thin_int), ("thin_k1", make_thin_k1), ("align", make_align),
                     ("route", make_route), ("moe_int", make_moe_int)):
        data = fn(rng)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
