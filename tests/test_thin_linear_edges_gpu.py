"""GPU parity of the skinny linear on the reference's edge-case lists.

* the extremes of kernels/workspace/thin_linear/build_oracle.py:176-196
  (large x, large w, tiny values, mixed magnitudes, zero x, cancellation,
  deep K 32768 x 256);
* the hand-picked edges of kernels/workspace/thin_linear/duipai.py:113-126
  (single element, N=1, K=1, M=1, odd prime K, zeros, huge and denormal-ish
  magnitudes, transposed x, sliced and strided w, deep K 65536 x 64);
* its seeded random sweep (duipai.py:98-107): 24 shapes with M <= 16 and
  K, N <= 4096, one in four fp32, activations scaled by 10^[-3, 2];
* ``make_bench_fn`` (kernels/thin_linear_fused.py:418-419).

Each case is checked against the oracle (the fp64 sum rounded once to the
dtype) within the reference's bound (2^-7 max|ref| + 1e-3 for bf16,
1e-5 max(1, max|ref|) for fp32) and, where the output is not identically
zero, max-abs-rel <= 1e-2.  Shapes are fixed by seeds (the reference draws
them from the clock).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import thin_linear as othin

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def rnd(*shape, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def check(x, w, label):
    from kernels.thin_linear_fused import thin_linear
    dt = "fp32" if x.dtype == torch.float32 else "bf16"
    print(f"edge {label}: x{tuple(x.shape)} w{tuple(w.shape)} {dt}", flush=True)
    with torch.inference_mode():
        got = thin_linear(x, w)
    torch.cuda.synchronize()
    assert got.shape == (x.shape[0], w.shape[0]) and got.dtype == x.dtype
    ref = othin.linear_exact(x.double().cpu().numpy(), w.double().cpu().numpy(), dtype=dt)
    g = got.double().cpu().numpy()
    amax = float(np.abs(ref).max()) if ref.size else 0.0
    err = float(np.abs(g - ref).max()) if ref.size else 0.0
    assert err <= othin.tolerance(amax, dt), f"{label}: max err {err:.3e}"
    if amax > 0:
        assert othin.max_abs_rel(g, ref) <= 1e-2, label
    else:
        assert np.all(g == 0), label
    return got


# ─────────────────────────── build_oracle.py:176-196, the extreme cases ───
def _extreme(name):
    if name == "large_x":
        return rnd(4, 2048, scale=100.0, seed=1), rnd(2048, 2048, scale=0.02, seed=2)
    if name == "large_w":
        return rnd(4, 2048, seed=3), rnd(2048, 2048, scale=10.0, seed=4)
    if name == "tiny_vals":
        return rnd(4, 2048, scale=1e-3, seed=5), rnd(2048, 2048, scale=1e-3, seed=6)
    if name == "mixed_mag":
        x = rnd(4, 2048, seed=7) * torch.logspace(-4, 4, 2048, device=DEV).to(torch.bfloat16)
        return x, rnd(2048, 2048, scale=0.02, seed=8)
    if name == "zeros_x":
        return torch.zeros(4, 2048, device=DEV, dtype=torch.bfloat16), rnd(2048, 2048, scale=0.02, seed=9)
    if name == "cancellation":
        w = rnd(2048, 2048, scale=0.02, seed=10)
        w[:, 1::2] *= -1
        return rnd(4, 2048, seed=11).abs(), w
    if name == "deep_K":
        return rnd(4, 32768, seed=12), rnd(256, 32768, scale=0.005, seed=13)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["large_x", "large_w", "tiny_vals", "mixed_mag", "zeros_x",
                                  "cancellation", "deep_K"])
def test_reference_extremes(name):
    x, w = _extreme(name)
    check(x, w, f"extreme_{name}")


# ─────────────────────────────── duipai.py:113-126, the hand-picked edges ───
def _edge(name):
    if name == "single_element":
        return rnd(1, 1, seed=20), rnd(1, 1, seed=21)
    if name == "N1":
        return rnd(4, 2048, seed=22), rnd(1, 2048, scale=0.02, seed=23)
    if name == "K1":
        return rnd(4, 1, seed=24), rnd(2048, 1, scale=0.02, seed=25)
    if name == "M1":
        return rnd(1, 2048, seed=26), rnd(2048, 2048, scale=0.02, seed=27)
    if name == "K_odd_prime":
        return rnd(4, 1021, seed=28), rnd(769, 1021, scale=0.02, seed=29)
    if name == "all_zeros":
        return torch.zeros(4, 2048, device=DEV, dtype=torch.bfloat16), rnd(2048, 2048, scale=0.02, seed=30)
    if name == "huge_mag":
        return rnd(4, 2048, scale=1e3, seed=31), rnd(2048, 2048, scale=1e2, seed=32)
    if name == "denormal_ish":
        return rnd(4, 2048, scale=1e-6, seed=33), rnd(2048, 2048, scale=1e-6, seed=34)
    if name == "noncontig_x":
        return rnd(2048, 4, seed=35).t(), rnd(2048, 2048, scale=0.02, seed=36)
    big_w = rnd(4096, 2048, scale=0.02, seed=37)
    if name == "noncontig_w_slice":
        return rnd(4, 2048, seed=38), big_w[1024:3072]
    if name == "w_strided_view":
        return rnd(4, 2048, seed=39), big_w[::2]
    if name == "deep_K":
        return rnd(4, 65536, scale=0.1, seed=40), rnd(64, 65536, scale=0.005, seed=41)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["single_element", "N1", "K1", "M1", "K_odd_prime", "all_zeros",
                                  "huge_mag", "denormal_ish", "noncontig_x", "noncontig_w_slice",
                                  "w_strided_view", "deep_K"])
def test_duipai_edges(name):
    x, w = _edge(name)
    check(x, w, f"edge_{name}")


def test_deep_k_takes_the_split_path():
    """Both deep-K shapes leave most CUs idle with one workgroup per row tile,
    so the automatic plan splits K across workgroups (the ordered
    reduce launch runs), and the split result equals the unsplit one within
    the bound while staying bitwise repeatable."""
    from kernels.thin_linear_fused import pick_config, thin_linear
    for (M, K, N) in ((4, 32768, 256), (4, 65536, 64)):
        split = pick_config(M, N, K)[3]
        assert split > 1, (M, K, N, split)
        x, w = rnd(M, K, scale=0.1, seed=K), rnd(N, K, scale=0.005, seed=N)
        with torch.inference_mode():
            a = thin_linear(x, w)
            b = thin_linear(x, w)
            one = thin_linear(x, w, config=(16, 4, 256, 1))
        assert torch.equal(a, b)
        ref = othin.linear_exact(x.double().cpu().numpy(), w.double().cpu().numpy())
        for got in (a, one):
            err = float(np.abs(got.double().cpu().numpy() - ref).max())
            assert err <= othin.tolerance(float(np.abs(ref).max()), "bf16")


# ───────────────────────────────── duipai.py:98-107, the random sweep ───
def _sweep(n=24, seed=2024):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        M = int(rs.randint(1, 17))
        K = int(rs.randint(1, 4097))
        N = int(rs.randint(1, 4097))
        fp32 = i % 4 == 0
        sc = float(10.0 ** int(rs.randint(-3, 3)))
        out.append((i, M, K, N, fp32, sc))
    return out


@pytest.mark.parametrize("case", _sweep(), ids=lambda c: f"{c[1]}x{c[2]}x{c[3]}{'f32' if c[4] else ''}s{c[5]:g}")
def test_duipai_random_sweep(case):
    i, M, K, N, fp32, sc = case
    dt = torch.float32 if fp32 else torch.bfloat16
    check(rnd(M, K, dtype=dt, scale=sc, seed=100 + i), rnd(N, K, dtype=dt, scale=0.02, seed=200 + i),
          f"rand{i}")


# ─────────────────────────────────── make_bench_fn (thin_linear_fused.py:418-419) ───
def test_make_bench_fn_indexes_the_pool():
    from kernels.thin_linear_fused import make_bench_fn, thin_linear
    x = rnd(4, 2048, seed=50)
    pool = [rnd(4096, 2048, scale=0.02, seed=51 + i) for i in range(3)]
    fn = make_bench_fn(x, pool, None)
    with torch.inference_mode():
        for i in range(3):
            assert torch.equal(fn(i), thin_linear(x, pool[i]))


@pytest.mark.parametrize("M", [4, 16])
def test_int64_weight_offsets(M):
    """A weight past 2^31 elements (kernels/thin_linear_fused.py:311 switches
    its kernel to 64-bit offsets once N*K, M*K or M*N reaches 2^31): w is
    [1114112, 2048] bf16, 2.28e9 elements, 4.25 GiB, so its byte offsets pass
    2^32 from row 1048576 on.  The rows at the start, around the 2^31-element
    / 2^32-byte boundary and at the end are checked against the oracle; a
    32-bit offset would wrap the later ones onto the first rows."""
    from kernels.thin_linear_fused import thin_linear
    N, K = 1114112, 2048
    assert N * K >= 2 ** 31 and N * K * 2 > 2 ** 32
    print(f"int64 offsets: M={M} w[{N}, {K}] bf16", flush=True)
    w = torch.empty(N, K, device=DEV, dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(1234)
    for i in range(0, N, 131072):                        # bounded fp32 temporaries
        n = min(131072, N - i)
        w[i:i + n] = (torch.randn(n, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    x = rnd(M, K, seed=99)
    with torch.inference_mode():
        y = thin_linear(x, w)
    torch.cuda.synchronize()
    assert y.shape == (M, N)
    edge = 2 ** 31 // K                                  # first row past 2^31 elements (and 2^32 bytes)
    xs = x.double().cpu().numpy()
    for lo in (0, edge - 64, N - 128):
        rows = slice(lo, lo + 128)
        ref = othin.linear_exact(xs, w[rows].double().cpu().numpy())
        got = y[:, rows].double().cpu().numpy()
        err = float(np.abs(got - ref).max())
        assert err <= othin.tolerance(float(np.abs(ref).max()), "bf16"), (lo, err)
        assert othin.max_abs_rel(got, ref) <= 1e-2, lo
    # rows whose 32-bit byte offset would wrap onto the first rows differ from them
    assert not torch.equal(y[:, edge:edge + 128], y[:, :128])
    del w
    torch.cuda.empty_cache()
