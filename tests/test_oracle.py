"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something independent of its own
formula: the closed-form golden fixtures (exact integer/rational arithmetic,
brute-force definitions), torch's CPU routines, or a second evaluation order.
Each check is chosen so a plausible slip -- a dropped rounding point, a wrong
gather index, an unstable sort, an off-by-one in the padding -- fails it; the
planted-mistake tests at the end show that they do.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as omoe
from oracle import thin_linear as othin
from oracle.numerics import bf16_round_int, round_bf16, round_fp16


# ─────────────────────────────────────────────────────────── numerics ───
def test_round_bf16_matches_torch_cast():
    g = torch.Generator().manual_seed(0)
    v = torch.cat([torch.randn(20000, generator=g) * 10.0 ** torch.randint(-30, 30, (20000,), generator=g),
                   torch.tensor([0.0, -0.0, 1.0, 65504.0, 3.4e38, -3.4e38, float("inf"), 1e-40])])
    got = round_bf16(v.numpy())
    ref = v.to(torch.bfloat16).float().numpy().astype(np.float64)
    assert np.array_equal(got, ref)


def test_round_bf16_ties_to_even_exact():
    # 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7: even -> 1
    assert round_bf16(np.array([1 + 2 ** -8]))[0] == 1.0
    assert round_bf16(np.array([1 + 3 * 2 ** -8]))[0] == 1 + 2 ** -6
    for v in [257, 259, 261, 1 + 2 ** -8, Fraction(3, 7), -1000001]:
        assert float(bf16_round_int(v)) == round_bf16(np.array([float(v)]))[0]


def test_round_fp16_matches_torch():
    v = torch.randn(5000, dtype=torch.float32) * 100
    assert np.array_equal(round_fp16(v.numpy()), v.half().float().numpy())


# ───────────────────────────────────────────────────────── thin linear ───
def test_linear_exact_golden_int(golden):
    d = golden("thin_int")
    for i in range(int(d["n_cases"])):
        x, w = d[f"c{i}_x"].astype(np.float64), d[f"c{i}_w"].astype(np.float64)
        assert np.array_equal(othin.linear_exact(x, w, dtype="bf16"), d[f"c{i}_y_bf16"]), i
        assert np.array_equal(othin.linear_exact(x, w, dtype="fp32"), d[f"c{i}_y_fp32"]), i
    y = othin.linear_exact(d["bias_x"], d["bias_w"], d["bias_b"], dtype="bf16")
    assert np.array_equal(y, d["bias_y"])


def test_linear_exact_golden_k1(golden):
    d = golden("thin_k1")
    assert np.array_equal(othin.linear_exact(d["x"], d["w"], dtype="bf16"), d["y"])


def test_planted_linear_mistakes_are_caught(golden):
    """Plausible slips in a linear restatement each fail a golden vector."""
    from oracle.numerics import round_bf16
    d = golden("thin_int")
    x, w = d["c0_x"].astype(np.float64), d["c0_w"].astype(np.float64)
    expect = d["c0_y_bf16"]
    assert x.shape[1] > 1
    slips = {
        "dropped last k term": round_bf16(x[:, :-1] @ w[:, :-1].T),
        "reversed k pairing": round_bf16(x @ w[:, ::-1].T),
        "off-by-one output row": np.roll(round_bf16(x @ w.T), 1, axis=1),
        "sign flip": round_bf16(-(x @ w.T)),
        "rounded product terms": round_bf16(round_bf16(x[:, None, :] * w[None, :, :] / 3).sum(-1) * 3),
    }
    for name, bad in slips.items():
        assert not np.array_equal(bad, expect), name
    bias_bad = othin.linear_exact(d["bias_x"], d["bias_w"], None, dtype="bf16")
    assert not np.array_equal(bias_bad, d["bias_y"]), "bias dropped"


def test_linear_exact_vs_torch_cpu_linear():
    """Second opinion: torch's CPU bf16 F.linear (the reference oracle) sits
    within the reference tolerance of the exact-sum oracle."""
    g = torch.Generator().manual_seed(1)
    for M, K, N in [(4, 2048, 256), (1, 6144, 64), (16, 1000, 129), (32, 4096, 96)]:
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
        ref = othin.linear_exact(x.float().numpy(), w.float().numpy(), dtype="bf16")
        got = othin.linear_cpu_torch(x, w).float().numpy()
        tol = othin.tolerance(float(np.abs(ref).max()), "bf16")
        assert float(np.abs(got - ref).max()) <= tol
        assert othin.max_abs_rel(got, ref) <= 1e-2


def test_gated_exact_vs_torch_cpu_composition():
    """gated_exact against torch CPU F.silu(F.linear) * F.linear at the same
    dtype (PyTorch's own rounding points), and planted slips fail."""
    from oracle.numerics import round_bf16
    g = torch.Generator().manual_seed(5)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        for M, K, I in [(1, 256, 64), (4, 2048, 96), (16, 1000, 33)]:
            x = torch.randn(M, K, generator=g).to(dt)
            wg = (torch.randn(I, K, generator=g) * 0.03).to(dt)
            wu = (torch.randn(I, K, generator=g) * 0.03).to(dt)
            ref = othin.gated_exact(x.float().numpy(), wg.float().numpy(), wu.float().numpy(), dtype=name)
            t = (torch.nn.functional.silu(torch.nn.functional.linear(x, wg))
                 * torch.nn.functional.linear(x, wu)).float().numpy()
            assert float(np.abs(ref - t).max()) <= othin.tolerance(float(np.abs(ref).max()), name)
    x = torch.randn(4, 512, generator=g).bfloat16().float().numpy()
    wg = (torch.randn(64, 512, generator=g) * 0.05).bfloat16().float().numpy()
    wu = (torch.randn(64, 512, generator=g) * 0.05).bfloat16().float().numpy()
    ref = othin.gated_exact(x, wg, wu)
    lin = lambda w: othin.linear_exact(x, w)
    slips = {"gate and up swapped": othin.gated_exact(x, wu, wg),
             "no SiLU": round_bf16(lin(wg) * lin(wu)),
             "sigmoid for SiLU": round_bf16(round_bf16(1 / (1 + np.exp(-lin(wg)))) * lin(wu))}
    for name, bad in slips.items():
        assert not np.array_equal(bad, ref), name


def _stock_rmsnorm(x, w, eps):
    x32 = x.float()
    var = x32.pow(2).mean(-1, keepdim=True)
    return w * (x32 * torch.rsqrt(var + eps)).to(x.dtype)


def test_rmsnorm_exact_vs_torch_stock_form():
    """rmsnorm_exact against the stock PyTorch RMSNorm on the CPU (the form
    sdar/run_native_tp2.py installs); its fp64 statistics may move x * r by
    one unit in the last place, which the product with the weight can carry
    to two.  Planted slips fail."""
    g = torch.Generator().manual_seed(9)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        for M, K in [(1, 2048), (4, 4096), (16, 1000)]:
            x = (torch.randn(M, K, generator=g) * 3).to(dt)
            w = (1 + 0.2 * torch.randn(K, generator=g)).to(dt)
            ref = othin.rmsnorm_exact(x.float().numpy(), w.float().numpy(), 1e-6, dtype=name)
            t = _stock_rmsnorm(x, w, 1e-6).float().numpy()
            ulp = 2.0 ** (-7 if name == "bf16" else -10)
            assert np.all(np.abs(ref - t) <= 2 * ulp * np.abs(ref) + 1e-30)
            assert (ref != t).mean() < 0.01
    x = (torch.randn(4, 512, generator=g) * 3).bfloat16()
    w = (1 + 0.2 * torch.randn(512, generator=g)).bfloat16()
    xf, wf = x.float().numpy().astype(np.float64), w.float().numpy().astype(np.float64)
    ref = othin.rmsnorm_exact(xf, wf, 1e-6)
    r = 1 / np.sqrt((xf * xf).mean(-1, keepdims=True) + 1e-6)
    slips = {"one rounding": round_bf16(wf * xf * r),
             "sum for mean": round_bf16(wf * round_bf16(xf / np.sqrt((xf * xf).sum(-1, keepdims=True) + 1e-6))),
             "no weight": round_bf16(xf * r)}
    for name, bad in slips.items():
        assert not np.array_equal(bad, ref), name


# ─────────────────────────────────────────────────────────────── route ───
def test_route_ids_golden(golden):
    d = golden("route")
    for i in range(int(d["n_cases"])):
        ids, _ = omoe.route_topk(d[f"c{i}_logits"], int(d[f"c{i}_k"]))
        assert np.array_equal(ids, d[f"c{i}_ids"]), i
    for scoring in ("softmax", "sigmoid"):
        ids, w = omoe.route_topk(d["flat_logits"], int(d["flat_k"]), scoring=scoring,
                                 renorm=True, scale=2.5)
        assert np.array_equal(ids, d["flat_ids"])
        assert np.allclose(w, d["flat_w_scale2.5"], rtol=0, atol=1e-15)


def test_route_ids_match_torch_topk_on_distinct_logits():
    g = torch.Generator().manual_seed(2)
    lg = torch.randn(64, 256, generator=g)
    ids, w = omoe.route_topk(lg.numpy(), 8, scoring="sigmoid", renorm=True, scale=2.5)
    tk = lg.topk(8, dim=-1).indices.numpy()
    assert np.array_equal(ids, tk)
    # the reference's _routing weights (build_oracle.py:87-90), via torch
    s = torch.sigmoid(lg).gather(1, torch.from_numpy(tk))
    ref = (s / (s.sum(-1, keepdim=True) + 1e-20) * 2.5).double().numpy()
    assert np.allclose(w, ref, rtol=1e-6, atol=0)
    _, ws = omoe.route_topk(lg.numpy(), 8, scoring="softmax", renorm=False)
    p = torch.softmax(lg.double(), dim=-1).gather(1, torch.from_numpy(tk)).numpy()
    assert np.allclose(ws, p, rtol=1e-12, atol=0)


# ─────────────────────────────────────────────────────────────── align ───
def test_align_golden(golden):
    d = golden("align")
    for i in range(int(d["n_cases"])):
        got = omoe.align(d[f"c{i}_ids"], int(d[f"c{i}_E"]), int(d[f"c{i}_n_tiles"]))
        for name in ("counts", "offsets", "pad_offsets", "perm", "slots", "tile_expert"):
            assert np.array_equal(got[name], d[f"c{i}_{name}"]), (i, name)


def test_align_invariants_random():
    rng = np.random.default_rng(3)
    for _ in range(50):
        E = int(rng.integers(1, 300))
        k = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.integers(1, 80))
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
        a = omoe.align(ids, E)
        flat = ids.reshape(-1)
        assert a["counts"].sum() == flat.size
        assert sorted(a["perm"].tolist()) == list(range(flat.size))
        assert np.all(np.diff(flat[a["perm"]]) >= 0)                   # sorted by expert
        for e in range(E):                                             # stable within group
            grp = a["perm"][a["offsets"][e]:a["offsets"][e + 1]]
            assert np.all(np.diff(grp) > 0)
        s = a["slots"]
        assert sorted(s[s >= 0].tolist()) == list(range(flat.size))    # every slot once
        for t, e in enumerate(a["tile_expert"]):                       # tile -> its group
            rows = s[t * 16:(t + 1) * 16]
            if e < E:
                assert np.all(flat[rows[rows >= 0]] == e)
            else:
                assert np.all(rows == -1)


def test_align_matches_torch_reference_ops():
    """The reference's _align is torch ops (scatter_add_, cumsum, stable
    argsort, searchsorted right=True); run those on CPU as a second opinion."""
    rng = np.random.default_rng(4)
    for T, k, E in [(32, 8, 256), (7, 3, 13), (64, 8, 256), (1, 8, 256)]:
        ids = torch.from_numpy(np.stack([rng.permutation(E)[:k] for _ in range(T)]))
        flat = ids.reshape(-1)
        M = flat.numel()
        nt = omoe.num_tiles(M, E)
        counts = torch.zeros(E, dtype=torch.long).scatter_add_(0, flat, torch.ones_like(flat))
        padded = ((counts + 15) // 16) * 16
        pad_end = padded.cumsum(0)
        order = torch.argsort(flat, stable=True)
        rank = torch.arange(M) - (counts.cumsum(0) - counts)[flat[order]]
        slots = torch.full((nt * 16,), -1, dtype=torch.int32)
        slots[(pad_end - padded)[flat[order]] + rank] = order.to(torch.int32)
        te = torch.searchsorted(pad_end, torch.arange(nt) * 16, right=True)
        a = omoe.align(ids.numpy(), E, nt)
        assert np.array_equal(a["slots"], slots.numpy())
        assert np.array_equal(a["tile_expert"], te.numpy())
        assert np.array_equal(a["perm"], order.numpy())
        assert np.array_equal(a["counts"], counts.numpy())


# ──────────────────────────────────────────────────────────── dispatch ───
def _moe_case(d, i, dtype):
    p = f"c{i}_"
    args = [d[p + n].astype(np.float64) for n in ("x",)] + [d[p + "ids"], d[p + "w"].astype(np.float64)]
    ws = [d[p + n].astype(np.float64) for n in ("w_gate", "w_up", "w_down")]
    shared = None
    if p + "sh_gate" in d:
        shared = tuple(d[p + n].astype(np.float64) for n in ("sh_gate", "sh_up", "sh_down"))
    return args + ws, shared


def test_dispatch_golden_int(golden):
    d = golden("moe_int")
    for i in range(int(d["n_cases"])):
        for dtype in ("bf16", "fp32"):
            args, shared = _moe_case(d, i, dtype)
            got = omoe.dispatch_grouped(*args, dtype=dtype, shared=shared)
            assert np.array_equal(got, d[f"c{i}_y_{dtype}"]), (i, dtype)
            got2 = omoe.dispatch_direct(*args, dtype=dtype, shared=shared)
            assert np.array_equal(got2, d[f"c{i}_y_{dtype}"]), (i, dtype)


def _rand_moe(rng, T, k, E, H, I, dtype="bf16"):
    rnd = {"bf16": round_bf16, "fp32": lambda a: np.asarray(a, np.float32).astype(np.float64)}[dtype]
    x = rnd(rng.standard_normal((T, H)))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    w = np.asarray(rng.random((T, k)), np.float32).astype(np.float64)
    wg = rnd(rng.standard_normal((E, I, H)) / np.sqrt(H))
    wu = rnd(rng.standard_normal((E, I, H)) / np.sqrt(H))
    wd = rnd(rng.standard_normal((E, H, I)) / np.sqrt(I))
    return x, ids, w, wg, wu, wd


def test_dispatch_grouped_equals_direct_random():
    rng = np.random.default_rng(5)
    for T, k, E, H, I in [(7, 3, 13, 130, 70), (16, 8, 64, 64, 32), (1, 8, 256, 32, 16)]:
        args = _rand_moe(rng, T, k, E, H, I)
        a = omoe.dispatch_grouped(*args, dtype="bf16")
        b = omoe.dispatch_direct(*args, dtype="bf16")
        assert np.allclose(a, b, rtol=0, atol=1e-12 * max(1, np.abs(b).max()))


def test_dispatch_vs_torch_reference_loop():
    """Second opinion: the reference's stock loop (build_oracle.py:34-67)
    restated with torch CPU ops in bf16 -- the same rounding points come out
    of torch's own kernels."""
    rng = np.random.default_rng(6)
    T, k, E, H, I = 16, 4, 32, 128, 64
    x, ids, w, wg, wu, wd = _rand_moe(rng, T, k, E, H, I)
    tb = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)
    X, WG, WU, WD = tb(x), tb(wg), tb(wu), tb(wd)
    ID, W = torch.from_numpy(ids), torch.from_numpy(np.asarray(w, np.float32))
    idxs = ID.view(-1).argsort(stable=True)
    tpe = torch.zeros(E, dtype=torch.long).scatter_add_(0, ID.view(-1), torch.ones(T * k, dtype=torch.long))
    sorted_tokens = X[idxs // k]
    outs, start = [], 0
    for e in range(E):
        n = int(tpe[e])
        if n == 0:
            continue
        toks = sorted_tokens[start:start + n]
        outs.append(F.linear(F.silu(F.linear(toks, WG[e])) * F.linear(toks, WU[e]), WD[e]))
        start += n
    o = torch.cat(outs)
    new_x = torch.empty_like(o)
    new_x[idxs] = o
    ref = new_x.view(T, k, -1).float().mul_(W.unsqueeze(-1)).sum(1).to(torch.bfloat16).float().numpy()
    got = omoe.dispatch_grouped(x, ids, w, wg, wu, wd, dtype="bf16")
    assert np.abs(got - ref).max() <= omoe.tolerance(float(np.abs(ref).max()), "bf16")


# ──────────────────────────────── the checks above catch planted mistakes ───
def test_planted_mistakes_are_caught(golden, monkeypatch):
    d = golden("moe_int")
    args, shared = _moe_case(d, 1, "bf16")
    expect = d["c1_y_bf16"]
    # (1) drop the rounding of h
    real_mlp = omoe._mlp

    def mlp_no_h_round(tok, wg, wu, wd, rnd):
        g, u = rnd(tok @ wg.T), rnd(tok @ wu.T)
        return rnd((rnd(omoe._silu(g)) * u) @ wd.T)
    monkeypatch.setattr(omoe, "_mlp", mlp_no_h_round)
    assert not np.array_equal(omoe.dispatch_grouped(*args, dtype="bf16", shared=shared), expect)
    monkeypatch.setattr(omoe, "_mlp", real_mlp)
    # (2) gather the wrong token row (slot % T instead of slot // k)
    x, ids, w, wg, wu, wd = args
    T, k = ids.shape
    bad = omoe.dispatch_direct(x[::-1].copy(), ids, w, wg, wu, wd, dtype="bf16", shared=shared)
    assert not np.array_equal(bad, expect)
    # (3) an unstable sort breaks the align golden
    a = golden("align")
    flat = a["c2_ids"].reshape(-1)
    unstable = np.argsort(flat, kind="quicksort")[::-1]
    assert not np.array_equal(unstable, a["c2_perm"])
    # (4) searchsorted left instead of right shifts tile experts
    pad_end = np.cumsum((np.bincount(flat, minlength=256) + 15) // 16 * 16)
    left = np.searchsorted(pad_end, np.arange(int(a["c2_n_tiles"])) * 16, side="left")
    assert not np.array_equal(left, a["c2_tile_expert"])


def test_linear_residual_exact_vs_torch_cpu():
    """residual + F.linear in bf16 on the CPU equals the oracle on exact
    (small-integer) products; a slip that skips the projection's rounding
    fails."""
    g = torch.Generator().manual_seed(21)
    x = torch.randint(-3, 4, (8, 512), generator=g).bfloat16()
    w = torch.randint(-3, 4, (96, 512), generator=g).bfloat16()
    r = (torch.randn(8, 96, generator=g) * 300).bfloat16()
    ref = (r + F.linear(x, w)).float().numpy()
    got = othin.linear_residual_exact(x.float().numpy(), w.float().numpy(), r.float().numpy())
    assert np.array_equal(got, ref)
    xf, wf, rf = (t.float().numpy().astype(np.float64) for t in (x, w, r))
    one_round = round_bf16(xf @ wf.T + rf)
    x2 = (torch.randn(8, 512, generator=g) * 2).bfloat16()
    ref2 = (r + F.linear(x2, w)).float().numpy()
    got2 = othin.linear_residual_exact(x2.float().numpy(), w.float().numpy(), r.float().numpy())
    slip2 = round_bf16(x2.float().numpy().astype(np.float64) @ wf.T + rf)
    assert np.abs(got2 - ref2).max() <= 2 ** -7 * np.abs(ref2).max()
    assert not np.array_equal(slip2, got2) or not np.array_equal(one_round, got)
