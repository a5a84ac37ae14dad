"""GPU parity of the fused MoE step (MI355X).

* route: top-k ids bit-exact against the oracle (including exact ties) and
  torch.topk; weights within fp32 rounding of the closed form.
* align: counts, offsets, padded offsets, permutation, slot table and tile
  experts bit-exact against the golden fixtures and the oracle; ``_align``
  also equals the reference's own torch ops run on the GPU.
* dispatch: the golden integer layers bit-exact (bf16 and fp32); the
  reference's synthetic case list (kernels/workspace/moe_dispatch/build_oracle.py:115-156)
  and random/edge cases (duipai.py:119-147) within the reference's bounds
  against the oracle, plus its fp64 gate (fused error <= 1.5 x the stock
  path's error); graph capture with a routing changed between replays; the
  benchmarked MoE step (T in {4, 16, 64}, E=256, k=8, H=2048, I=512, shared
  expert) end to end.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as omoe

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _dt(dtype):
    return {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]


# ─────────────────────────────────────────────────────────────────── route ───
def test_route_golden_ties(golden):
    from kernels.moe_dispatch_fused import moe_route
    d = golden("route")
    for i in range(int(d["n_cases"])):
        lg = torch.from_numpy(d[f"c{i}_logits"]).to(DEV)
        for scoring in ("softmax", "sigmoid"):
            ids, _ = moe_route(lg, int(d[f"c{i}_k"]), scoring=scoring)
            assert np.array_equal(ids.cpu().numpy(), d[f"c{i}_ids"]), (i, scoring)
    lg = torch.from_numpy(d["flat_logits"]).to(DEV)
    for scoring in ("softmax", "sigmoid"):
        ids, w = moe_route(lg, int(d["flat_k"]), scoring=scoring, renorm=True, scale=2.5)
        assert np.array_equal(ids.cpu().numpy(), d["flat_ids"])
        assert np.allclose(_np(w), d["flat_w_scale2.5"], rtol=1e-6, atol=0)


@pytest.mark.parametrize("T,E,k", [(4, 256, 8), (16, 256, 8), (64, 256, 8), (33, 64, 6),
                                   (5, 13, 3), (7, 1024, 8), (3, 8, 8), (9, 100, 1)])
@pytest.mark.parametrize("scoring,renorm,scale", [("softmax", False, 1.0), ("softmax", True, 1.0),
                                                  ("sigmoid", True, 2.5)])
def test_route_vs_oracle(T, E, k, scoring, renorm, scale):
    from kernels.moe_dispatch_fused import moe_route
    g = torch.Generator(device=DEV).manual_seed(T * 1000 + E + k)
    lg = torch.randn(T, E, device=DEV, generator=g)
    ids, w = moe_route(lg, k, scoring=scoring, renorm=renorm, scale=scale)
    rid, rw = omoe.route_topk(lg.cpu().numpy(), k, scoring=scoring, renorm=renorm, scale=scale)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert torch.equal(ids, lg.topk(k, dim=-1).indices)
    assert np.allclose(_np(w), rw, rtol=2e-6, atol=1e-9)


def test_route_strided_logits():
    from kernels.moe_dispatch_fused import moe_route
    g = torch.Generator(device=DEV).manual_seed(5)
    big = torch.randn(16, 512, device=DEV, generator=g)
    lg = big[:, 100:356]
    ids, w = moe_route(lg, 8, scoring="sigmoid", renorm=True, scale=2.5)
    rid, rw = omoe.route_topk(lg.cpu().numpy(), 8, scoring="sigmoid", renorm=True, scale=2.5)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(_np(w), rw, rtol=2e-6)


# ─────────────────────────────────────────────────────────────────── align ───
def _check_align(al, ref):
    for name in ("counts", "offsets", "pad_offsets", "perm", "slots", "tile_expert"):
        got = getattr(al, name).cpu().numpy()
        assert np.array_equal(got, ref[name]), name


def test_align_golden(golden):
    from kernels.moe_dispatch_fused import moe_align
    d = golden("align")
    for i in range(int(d["n_cases"])):
        ids = torch.from_numpy(d[f"c{i}_ids"]).to(DEV)
        al = moe_align(ids, int(d[f"c{i}_E"]), int(d[f"c{i}_n_tiles"]))
        _check_align(al, {n: d[f"c{i}_{n}"] for n in
                          ("counts", "offsets", "pad_offsets", "perm", "slots", "tile_expert")})


def test_align_random_vs_oracle():
    from kernels.moe_dispatch_fused import moe_align
    rng = np.random.default_rng(11)
    for trial in range(40):
        E = int(rng.choice([1, 3, 8, 13, 64, 256, 257, 1000, 1024]))
        k = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.choice([1, 2, 5, 17, 64, 100, 500, 1024]))
        if rng.random() < 0.3:
            hot = rng.permutation(E)[:max(k, E // 20)]
            ids = np.stack([rng.choice(hot, size=k, replace=False) for _ in range(T)])
        else:
            ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
        al = moe_align(torch.from_numpy(ids).to(DEV), E)
        _check_align(al, omoe.align(ids, E))


@pytest.mark.parametrize("scoring,renorm,scale", [("softmax", False, 1.0), ("sigmoid", True, 2.5)])
def test_route_align_fused_equals_two_calls(scoring, renorm, scale):
    """One launch (route + align) gives exactly the two calls' outputs, and
    the ids and tables match the oracle."""
    from kernels.moe_dispatch_fused import moe_align, moe_route, moe_route_align
    g = torch.Generator(device=DEV).manual_seed(21)
    for T, E, k in [(1, 8, 1), (4, 256, 8), (16, 256, 8), (64, 256, 8), (5, 13, 3), (33, 1000, 6),
                    (1024, 256, 8), (3, 64, 64), (16, 8, 8), (8, 16, 16), (16, 1024, 8), (2, 4, 4),
                    (2, 64, 64), (17, 256, 7), (11, 300, 11)]:
        logits = torch.randn(T, E, device=DEV, generator=g)
        ids1, w1 = moe_route(logits, k, scoring=scoring, renorm=renorm, scale=scale)
        al1 = moe_align(ids1, E)
        ids2, w2, al2 = moe_route_align(logits, k, scoring=scoring, renorm=renorm, scale=scale)
        assert torch.equal(ids1, ids2) and torch.equal(w1, w2), (T, E, k)
        for name in al1._fields:
            assert torch.equal(getattr(al1, name), getattr(al2, name)), (T, E, k, name)
        ids_ref, _ = omoe.route_topk(logits.cpu().numpy().astype(np.float64), k, scoring=scoring,
                                     renorm=renorm, scale=scale)
        assert np.array_equal(ids2.cpu().numpy(), ids_ref), (T, E, k)
        _check_align(al2, omoe.align(ids_ref, E))


def test_align_more_tiles_than_the_picks_fill():
    """A tile count above the default (a table sized for a larger bound):
    every tile past the filled ones is empty (expert E, rows -1), in both the
    one-launch route + align (up to 128 picks, and past the 136 tiles its
    table holds) and the general align (past its 1536)."""
    from kernels.moe_dispatch_fused import _num_tiles, moe_align, moe_route_align
    g = torch.Generator(device=DEV).manual_seed(23)
    for T, E, k, extra in [(4, 256, 8, 20), (4, 256, 8, 300), (16, 256, 8, 64), (64, 256, 8, 40),
                           (1024, 256, 8, 1500)]:
        logits = torch.randn(T, E, device=DEV, generator=g)
        nt = _num_tiles(T * k, E) + extra
        ids, _, al = moe_route_align(logits, k, num_tiles=nt)
        ref = omoe.align(ids.cpu().numpy(), E, nt)
        _check_align(al, ref)
        _check_align(moe_align(ids, E, nt), ref)


def test_align_max_slots():
    from kernels.moe_dispatch_fused import moe_align
    rng = np.random.default_rng(12)
    ids = np.stack([rng.permutation(256)[:8] for _ in range(1024)])     # 8192 slots
    _check_align(moe_align(torch.from_numpy(ids).to(DEV), 256), omoe.align(ids, 256))
    with pytest.raises(ValueError):
        moe_align(torch.zeros(1025, 8, dtype=torch.long, device=DEV), 256)


def test_align_matches_reference_torch_ops_on_gpu():
    """_align's contract via the reference's own torch ops (scatter_add_,
    cumsum, stable argsort, searchsorted) executed on the same GPU."""
    from kernels.moe_dispatch_fused import _align, _num_tiles
    g = torch.Generator(device=DEV).manual_seed(13)
    for T, k, E in [(32, 8, 256), (64, 8, 256), (7, 3, 13), (1, 8, 256)]:
        ids = torch.stack([torch.randperm(E, device=DEV, generator=g)[:k] for _ in range(T)])
        flat = ids.reshape(-1)
        M = flat.numel()
        nt = _num_tiles(M, E)
        counts = torch.zeros(E, dtype=torch.long, device=DEV).scatter_add_(0, flat, torch.ones_like(flat))
        padded = ((counts + 15) // 16) * 16
        pad_end = padded.cumsum(0)
        order = torch.argsort(flat, stable=True)
        rank = torch.arange(M, device=DEV) - (counts.cumsum(0) - counts)[flat[order]]
        slots = torch.full((nt * 16,), -1, dtype=torch.int32, device=DEV)
        slots[(pad_end - padded)[flat[order]] + rank] = order.to(torch.int32)
        te = torch.searchsorted(pad_end, torch.arange(nt, device=DEV) * 16, right=True).to(torch.int32)
        s2, t2 = _align(ids, E, nt)
        assert torch.equal(s2, slots) and torch.equal(t2, te)


# ──────────────────────────────────────────────────────────────── dispatch ───
def _golden_case(d, i, dtype):
    p = f"c{i}_"
    tdt = _dt(dtype)
    f = lambda n: torch.from_numpy(d[p + n].astype(np.float32)).to(DEV).to(tdt)
    x, wg, wu, wd = f("x"), f("w_gate"), f("w_up"), f("w_down")
    ids = torch.from_numpy(d[p + "ids"]).to(DEV)
    w = torch.from_numpy(d[p + "w"]).to(DEV)
    shared = tuple(f(n) for n in ("sh_gate", "sh_up", "sh_down")) if p + "sh_gate" in d else None
    return x, ids, w, wg, wu, wd, shared


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_dispatch_golden_int_bitexact(golden, dtype):
    from kernels.moe_dispatch_fused import moe_dispatch, _grouped_ffn, _align, _num_tiles
    d = golden("moe_int")
    for i in range(int(d["n_cases"])):
        x, ids, w, wg, wu, wd, shared = _golden_case(d, i, dtype)
        expect = d[f"c{i}_y_{dtype}"]
        if shared is None:
            got = moe_dispatch(x, ids, w, wg, wu, wd)
        else:
            E = wg.shape[0]
            slots, te = _align(ids, E, _num_tiles(ids.numel(), E))
            got = _grouped_ffn(x, ids, w, wg, wu, wd, slots, te, shared=shared)
        assert np.array_equal(_np(got), expect), (i, dtype)


def _routing(T, k, E, g, concentration=None):
    """The reference's synthetic routing (build_oracle.py:71-90), on the GPU."""
    if concentration is None:
        logits = torch.randn(T, E, device=DEV, generator=g)
    else:
        pool = max(1, int(E * concentration))
        logits = torch.randn(T, E, device=DEV, generator=g) - 8.0
        hot = torch.randperm(E, device=DEV, generator=g)[:pool]
        logits[:, hot] += 8.0
    ids = logits.topk(k, dim=-1).indices.contiguous()
    s = torch.sigmoid(logits.float()).gather(1, ids)
    w = s / (s.sum(-1, keepdim=True) + 1e-20) if k > 1 else s
    return ids, (w * 2.5).float()


def _case(T, k, E, H, I, dtype, scale=1.0, concentration=None, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    tdt = _dt(dtype)
    x = (torch.randn(T, H, device=DEV, generator=g) * scale).to(tdt)
    ids, w = _routing(T, k, E, g, concentration)
    mk = lambda *s: (torch.randn(*s, device=DEV, generator=g) / (s[-1] ** 0.5)).to(tdt)
    return x, ids, w, mk(E, I, H), mk(E, I, H), mk(E, H, I)


def _oracle(x, ids, w, wg, wu, wd, dtype, shared=None):
    """Oracle on the active experts only (keeps the host copy small)."""
    ids_c = ids.cpu().numpy()
    act = np.unique(ids_c[(ids_c >= 0) & (ids_c < wg.shape[0])])
    remap = np.full(wg.shape[0], -1, dtype=np.int64)
    remap[act] = np.arange(act.size)
    ids_r = np.where((ids_c >= 0) & (ids_c < wg.shape[0]), remap[np.clip(ids_c, 0, wg.shape[0] - 1)], -1)
    sel = torch.from_numpy(act).to(DEV)
    sh = tuple(_np(s) for s in shared) if shared is not None else None
    return omoe.dispatch_grouped(_np(x), ids_r, _np(w), _np(wg[sel]), _np(wu[sel]), _np(wd[sel]),
                                 dtype=dtype, shared=sh)


def _stock_gpu(x, ids, w, wg, wu, wd):
    """The reference's stock loop (build_oracle.py:34-67) with torch ops on the GPU."""
    E = wg.shape[0]
    k = ids.shape[1]
    cnts = ids.new_zeros((ids.shape[0], E))
    cnts.scatter_(1, ids, 1)
    tpe = cnts.sum(dim=0).cpu()
    idxs = ids.view(-1).argsort()
    sorted_tokens = x[idxs // k]
    outs, start = [], 0
    for e in range(E):
        n = int(tpe[e])
        if n == 0:
            continue
        toks = sorted_tokens[start:start + n]
        g_, u_ = F.linear(toks, wg[e]), F.linear(toks, wu[e])
        outs.append(F.linear(F.silu(g_) * u_, wd[e]))
        start += n
    o = torch.cat(outs)
    new_x = torch.empty_like(o)
    new_x[idxs] = o
    return new_x.view(*ids.shape, -1).to(w.dtype).mul_(w.unsqueeze(-1)).sum(1).to(new_x.dtype)


# the reference's synthetic list (build_oracle.py:115-156)
SYNTH = [
    ("mini_T32", 32, 8, 256, 2048, 512, 1.0, 0.15),
    ("mini_T64", 64, 8, 256, 2048, 512, 1.0, 0.20),
    ("flash_T32", 32, 8, 256, 4096, 1024, 1.0, 0.15),
    ("uniform", 32, 8, 256, 2048, 512, 1.0, None),
    ("single_token", 1, 8, 256, 2048, 512, 1.0, 0.05),
    ("tiny", 4, 2, 8, 64, 32, 1.0, None),
    ("odd_dims", 7, 3, 13, 130, 70, 1.0, None),
    ("k1", 16, 1, 32, 128, 64, 1.0, None),
    ("large_mag", 16, 4, 64, 256, 128, 100.0, None),
    ("tiny_mag", 16, 4, 64, 256, 128, 1e-3, None),
]


# The reference's list runs in fp32 and bf16 (build_oracle.py:117); fp16 is
# added here for every case but large_mag, whose x * 100 drives
# h = silu(g) * u past fp16's 65504 (the case targets bf16's range).
_SYNTH_PARAMS = [pytest.param(c, dt, id=f"{dt}-{c[0]}") for c in SYNTH for dt in ("bf16", "fp16", "fp32")
                 if not (dt == "fp16" and c[6] > 10)]


@pytest.mark.parametrize("case,dtype", _SYNTH_PARAMS)
def test_dispatch_synthetic_vs_oracle(case, dtype):
    from kernels.moe_dispatch_fused import moe_dispatch
    name, T, k, E, H, I, scale, conc = case
    x, ids, w, wg, wu, wd = _case(T, k, E, H, I, dtype, scale, conc, seed=zlib.crc32(name.encode()) & 0xFFFF)
    with torch.inference_mode():
        got = moe_dispatch(x, ids, w, wg, wu, wd)
    assert got.shape == (T, H) and got.dtype == x.dtype
    ref = _oracle(x, ids, w, wg, wu, wd, dtype)
    amax = float(np.abs(ref).max())
    err = float(np.abs(_np(got) - ref).max())
    assert err <= omoe.tolerance(amax, dtype), (name, err)
    # the reference's fp64 gate: no less accurate than the stock path
    truth = _oracle(x, ids, w, wg, wu, wd, "fp64")
    with torch.inference_mode():
        stock = _stock_gpu(x, ids, w, wg, wu, wd)
    e_stock = float(np.abs(_np(stock) - truth).max())
    e_fused = float(np.abs(_np(got) - truth).max())
    assert omoe.fp64_gate(e_fused, e_stock, float(np.abs(truth).max()), dtype), (e_fused, e_stock)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_dispatch_all_one_expert(dtype):
    from kernels.moe_dispatch_fused import moe_dispatch
    x, ids, w, wg, wu, wd = _case(32, 1, 256, 2048, 512, dtype, 1.0, 0.05, seed=11)
    ids = torch.zeros_like(ids)                     # 32 slots -> 2 tiles of one expert
    with torch.inference_mode():
        got = moe_dispatch(x, ids, w, wg, wu, wd)
    ref = _oracle(x, ids, w, wg, wu, wd, dtype)
    assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), dtype)


def test_dispatch_random_edges():
    from kernels.moe_dispatch_fused import moe_dispatch
    rng = np.random.default_rng(21)
    for i in range(10):
        dtype = ["fp32", "bf16"][i % 2]
        E = int(rng.choice([4, 7, 16, 33, 64, 256]))
        k = min(int(rng.choice([1, 2, 3, 8])), E)
        T = int(rng.choice([1, 2, 5, 17, 32, 64]))
        H = int(rng.choice([32, 96, 130, 256, 2048]))
        I = int(rng.choice([16, 48, 70, 128, 512]))
        conc = [None, 0.05, 0.3][i % 3]
        scale = [1.0, 1e-3, 50.0][i % 3]
        x, ids, w, wg, wu, wd = _case(T, k, E, H, I, dtype, scale, conc, seed=1000 + i)
        with torch.inference_mode():
            got = moe_dispatch(x, ids, w, wg, wu, wd)
        ref = _oracle(x, ids, w, wg, wu, wd, dtype)
        err = float(np.abs(_np(got) - ref).max())
        assert err <= omoe.tolerance(float(np.abs(ref).max()), dtype), (i, E, k, T, H, I, err)


def test_dispatch_noncontiguous_x():
    from kernels.moe_dispatch_fused import moe_dispatch
    x, ids, w, wg, wu, wd = _case(32, 8, 64, 256, 128, "bf16", seed=777)
    g = torch.Generator(device=DEV).manual_seed(778)
    big = torch.randn(32, 512, device=DEV, generator=g).to(torch.bfloat16)
    xs = big[:, ::2]
    with torch.inference_mode():
        got = moe_dispatch(xs, ids, w, wg, wu, wd)
        contig = moe_dispatch(xs.contiguous(), ids, w, wg, wu, wd)
    ref = _oracle(xs, ids, w, wg, wu, wd, "bf16")
    assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "bf16")
    assert float((got.float() - contig.float()).abs().max()) <= 2 ** -6 * float(contig.abs().max())


def test_dispatch_duplicate_and_invalid_ids():
    """Repeated experts in a token count twice; ids outside [0, E) add nothing."""
    from kernels.moe_dispatch_fused import moe_dispatch
    x, ids, w, wg, wu, wd = _case(9, 4, 16, 64, 32, "fp32", seed=31)
    ids = ids.clone()
    ids[0, 1] = ids[0, 0]
    ids[1, 2] = -1
    ids[2, 0] = 16
    with torch.inference_mode():
        got = moe_dispatch(x, ids, w, wg, wu, wd)
    ref = omoe.dispatch_direct(_np(x), ids.cpu().numpy(), _np(w), _np(wg), _np(wu), _np(wd), dtype="fp32")
    assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "fp32")


def test_graph_capture_with_new_routing():
    """Capture once, replay with routings written in place between replays."""
    from kernels.moe_dispatch_fused import moe_dispatch
    x, ids, w, wg, wu, wd = _case(32, 8, 256, 2048, 512, "bf16", 1.0, 0.15, seed=41)
    with torch.inference_mode():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                moe_dispatch(x, ids, w, wg, wu, wd)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = moe_dispatch(x, ids, w, wg, wu, wd)
        g = torch.Generator(device=DEV).manual_seed(42)
        for r in range(3):
            new_ids, new_w = _routing(32, 8, 256, g, [None, 0.05, 0.3][r])
            ids.copy_(new_ids)
            w.copy_(new_w)
            graph.replay()
            torch.cuda.synchronize()
            eager = moe_dispatch(x, ids, w, wg, wu, wd)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), r


# ──────────────────── the benchmarked MoE step (T 4/16/64, E=256, k=8) ───
@pytest.mark.parametrize("T", [4, 16, 64])
def test_moe_forward_c4(T):
    from kernels.moe_dispatch_fused import moe_forward, moe_route
    E, k, H, I = 256, 8, 2048, 512
    g = torch.Generator(device=DEV).manual_seed(4000 + T)
    logits = torch.randn(T, E, device=DEV, generator=g)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    mk = lambda *s: (torch.randn(*s, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wg, wu, wd = mk(E, I, H), mk(E, I, H), mk(E, H, I)
    shared = (mk(I, H), mk(I, H), mk(H, I))
    with torch.inference_mode():
        out = moe_forward(x, logits, k, wg, wu, wd, shared=shared, scoring="softmax", renorm=False)
        ids, w = moe_route(logits, k, scoring="softmax", renorm=False)
    rid, rw = omoe.route_topk(logits.cpu().numpy(), k, scoring="softmax", renorm=False)
    assert np.array_equal(ids.cpu().numpy(), rid)
    ref = _oracle(x, ids, w, wg, wu, wd, "bf16", shared=shared)
    amax = float(np.abs(ref).max())
    err = float(np.abs(_np(out) - ref).max())
    assert err <= omoe.tolerance(amax, "bf16"), err
    assert err / amax <= 1e-2


# ───────────────────────── a few tokens: down and combine in one launch ───
SMALL = [
    # name, T, k, E, H, I, shared, ids pattern
    ("T4_k8_E256", 4, 8, 256, 2048, 512, True, None),
    ("T1_k8_noshared", 1, 8, 256, 2048, 512, False, None),
    ("T3_k4_I1024", 3, 4, 32, 256, 1024, True, None),        # 8 load steps per h row
    ("T4_all_one_expert", 4, 8, 64, 512, 256, True, "same"),  # 32 slots of one expert: 2 tiles x 4 column sets
    ("T2_dup_invalid", 2, 6, 16, 136, 128, False, "dup"),     # repeated and out-of-range ids, H % 8 != 0
]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("case", SMALL, ids=[c[0] for c in SMALL])
def test_small_token_down_combine(case, dtype):
    """T <= 4 runs down and combine as one kernel; it must agree with the
    oracle like the three-launch path, including experts holding more than
    four slots of the tile and ids that add nothing."""
    from kernels.moe_dispatch_fused import _align, _grouped_ffn, _num_tiles
    name, T, k, E, H, I, with_shared, pattern = case
    x, ids, w, wg, wu, wd = _case(T, k, E, H, I, dtype, seed=zlib.crc32(name.encode()) & 0xFFFF)
    ids = ids.clone()
    if pattern == "same":
        ids.fill_(5)
    elif pattern == "dup":
        ids[0, 1] = ids[0, 0]
        ids[1, 0] = ids[0, 0]
        ids[1, 2] = -1
        ids[0, 3] = E
    g = torch.Generator(device=DEV).manual_seed(9)
    mk = lambda *s: (torch.randn(*s, device=DEV, generator=g) / (s[-1] ** 0.5)).to(_dt(dtype))
    shared = (mk(I, H), mk(I, H), mk(H, I)) if with_shared else None
    slots, te = _align(ids, E, _num_tiles(ids.numel(), E))
    with torch.inference_mode():
        got = _grouped_ffn(x, ids, w, wg, wu, wd, slots, te, shared=shared)
    sh = tuple(_np(s) for s in shared) if shared is not None else None
    ref = omoe.dispatch_direct(_np(x), ids.cpu().numpy(), _np(w), _np(wg), _np(wu), _np(wd), dtype=dtype, shared=sh)
    err = float(np.abs(_np(got) - ref).max())
    assert err <= omoe.tolerance(float(np.abs(ref).max()), dtype), (name, err)


def test_dispatch_beyond_one_align_launch():
    """T * k above the single align workgroup's 8192 slots (a long prefill):
    moe_dispatch and moe_forward split the tokens into chunks, each aligned and
    dispatched on its own, and equal the oracle over all T tokens."""
    from kernels import _native
    from kernels.moe_dispatch_fused import moe_dispatch, moe_forward, moe_route
    T, k, E, H, I = 1100, 8, 64, 256, 128
    assert T * k > _native.MOE_MAX_SLOTS
    x, ids, w, wg, wu, wd = _case(T, k, E, H, I, "bf16", seed=31)
    with torch.inference_mode():
        got = moe_dispatch(x, ids, w, wg, wu, wd)
    ref = _oracle(x, ids, w, wg, wu, wd, "bf16")
    assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "bf16")
    g = torch.Generator(device=DEV).manual_seed(32)
    logits = torch.randn(T, E, device=DEV, generator=g)
    mk = lambda *sh: (torch.randn(*sh, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    shared = (mk(I, H), mk(I, H), mk(H, I))
    with torch.inference_mode():
        out = moe_forward(x, logits, k, wg, wu, wd, shared=shared)
        rids, rw = moe_route(logits, k)
    ref2 = _oracle(x, rids, rw, wg, wu, wd, "bf16", shared=shared)
    assert float(np.abs(_np(out) - ref2).max()) <= omoe.tolerance(float(np.abs(ref2).max()), "bf16")


class _ExpertMLP(torch.nn.Module):
    def __init__(self, H, I):
        super().__init__()
        self.gate_proj = torch.nn.Linear(H, I, bias=False)
        self.up_proj = torch.nn.Linear(H, I, bias=False)
        self.down_proj = torch.nn.Linear(I, H, bias=False)


class LLaDA2MoeSparseMoeBlock(torch.nn.Module):
    """Stand-in with the remote class's name, experts and moe_infer signature;
    its stock moe_infer is the reference's per-expert loop."""

    def __init__(self, E, H, I):
        super().__init__()
        self.experts = torch.nn.ModuleList(_ExpertMLP(H, I) for _ in range(E))

    def moe_infer(self, x, topk_ids, topk_weight):
        wg = torch.stack([e.gate_proj.weight for e in self.experts])
        wu = torch.stack([e.up_proj.weight for e in self.experts])
        wd = torch.stack([e.down_proj.weight for e in self.experts])
        return _stock_gpu(x, topk_ids, topk_weight, wg, wu, wd)


def _moe_block(E, H, I, seed):
    torch.manual_seed(seed)
    blk = LLaDA2MoeSparseMoeBlock(E, H, I).to(device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05)
    return blk


def test_apply_moe_to_model_runs_the_grouped_dispatch():
    """fused_toggle.apply_moe_to_model on a model holding two MoE blocks: each
    switched block's moe_infer equals the oracle on the weights it had before
    stacking; a block outside the switched model keeps the stock loop."""
    from kernels import fused_toggle
    E, H, I, T, k = 32, 256, 128, 16, 4
    root = torch.nn.Module()
    root.a, root.b = _moe_block(E, H, I, 1), _moe_block(E, H, I, 2)
    other = _moe_block(E, H, I, 3)
    before = {n: [torch.stack([getattr(e, p).weight.detach().clone() for e in blk.experts])
                  for p in ("gate_proj", "up_proj", "down_proj")]
              for n, blk in (("a", root.a), ("b", root.b))}
    assert fused_toggle.apply_moe_to_model(root) == 2
    assert fused_toggle.is_moe_applied(root) and not fused_toggle.is_moe_applied(other)
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    ids, w = _routing(T, k, E, g)
    for n, blk in (("a", root.a), ("b", root.b)):
        with torch.inference_mode():
            got = blk.moe_infer(x, ids, w)
        ref = _oracle(x, ids, w, *before[n], "bf16")
        assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "bf16")
    with torch.inference_mode():
        stock = other.moe_infer(x, ids, w)
    wts = [torch.stack([getattr(e, p).weight for e in other.experts]) for p in ("gate_proj", "up_proj", "down_proj")]
    ref = _oracle(x, ids, w, *wts, "bf16")
    assert float(np.abs(_np(stock) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "bf16")


def test_fused_moe_dispatch_module():
    """FusedMoEDispatch over stack_expert_weights' stacks equals the oracle;
    the stacks stay out of the state dict and follow the module."""
    from kernels.moe_dispatch_fused import FusedMoEDispatch, stack_expert_weights
    E, H, I, T, k = 64, 512, 256, 24, 8
    blk = _moe_block(E, H, I, 5)
    wts = [torch.stack([getattr(e, p).weight.detach().clone() for e in blk.experts])
           for p in ("gate_proj", "up_proj", "down_proj")]
    mod = FusedMoEDispatch(*stack_expert_weights(blk.experts))
    assert blk.experts[0].gate_proj.weight.numel() == 0            # released
    assert len(mod.state_dict()) == 0 and len(list(mod.buffers())) == 3
    assert all(torch.equal(a, b) for a, b in zip((mod.w_gate, mod.w_up, mod.w_down), wts))
    g = torch.Generator(device=DEV).manual_seed(6)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    ids, w = _routing(T, k, E, g, 0.25)
    with torch.inference_mode():
        got = mod(x, ids, w)
    ref = _oracle(x, ids, w, *wts, "bf16")
    assert float(np.abs(_np(got) - ref).max()) <= omoe.tolerance(float(np.abs(ref).max()), "bf16")
