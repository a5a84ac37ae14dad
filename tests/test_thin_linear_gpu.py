"""GPU parity of the skinny linear (MI355X).

Restates every case of the reference's kernels/thin_linear_fused_test.py
(deployed shapes x M, odd dims, fp32 IEEE, magnitudes, zeros, strided views,
leading dims, bias, grad mode, dtype mismatch, determinism at split_k 1/2/8,
dispatch fallback, tuned envelope, graph capture/replay, shared workspace,
toggle), against the same bound: live ``F.linear`` within 2^-7*max|ref|+1e-3
(bf16) / 1e-5*max(1, max|ref|) (fp32).  On top of that:

* bit-exact golden vectors (small-integer and K=1 cases, tests/golden/);
* the oracle (exact sum, rounded once) at the benchmarked shapes: the draft's
  gate_up, the draft set at M=4, the target set at M=16/32, within tolerance
  and the relative bar max-abs-rel <= 1e-2;
* size-independent properties at full size: bitwise determinism, row
  independence (a batch equals its rows computed alone), exact linearity in
  a power-of-two scale, strided view == contiguous copy.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import thin_linear as othin

pytestmark = pytest.mark.gpu

DEV = "cuda"
DEPLOYED = [(2048, 2048), (2048, 1024), (2048, 6144), (6144, 2048),
            (2048, 151936), (4096, 12288)]


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def tol(ref: torch.Tensor) -> float:
    if ref.dtype == torch.float32:
        return 1e-5 * max(1.0, float(ref.abs().max()))
    return 2 ** -7 * float(ref.abs().max()) + 1e-3


def rnd(*shape, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def assert_matches(x, w, **kw):
    from kernels.thin_linear_fused import thin_linear
    with torch.inference_mode():
        ref = F.linear(x, w)
        got = thin_linear(x, w, **kw)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    err = float((got.float() - ref.float()).abs().max())
    assert err <= tol(ref), f"max_err {err:.3e} > tol {tol(ref):.3e}"
    return err


# ───────────────────────────── the reference's cases (thin_linear_fused_test.py) ───
@pytest.mark.parametrize("K,N", DEPLOYED)
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_deployed_shapes(M, K, N):
    assert_matches(rnd(M, K, seed=M), rnd(N, K, scale=0.02, seed=K + N))


@pytest.mark.parametrize("K,N", [(1000, 1531), (2049, 129), (6143, 2047), (127, 65), (1, 1),
                                 (2048, 1), (3, 4096), (1021, 769)])
def test_odd_dims(K, N):
    assert_matches(rnd(4, K, seed=K), rnd(N, K, scale=0.02, seed=N))


def test_fp32_ieee():
    x = rnd(4, 2048, dtype=torch.float32)
    w = rnd(2048, 2048, scale=0.02, dtype=torch.float32, seed=3)
    err = assert_matches(x, w)
    ref_max = float(F.linear(x, w).abs().max())
    assert err / ref_max < 1e-5, f"relative {err / ref_max:.2e} is not fp32 accuracy"


@pytest.mark.parametrize("scale", [1e-6, 1e-3, 1.0, 1e2, 1e4])
def test_magnitudes(scale):
    assert_matches(rnd(4, 2048, scale=scale, seed=int(scale) + 1), rnd(2048, 2048, scale=0.02, seed=9))


def test_zeros_and_empty_contribution():
    from kernels.thin_linear_fused import thin_linear
    z = torch.zeros(4, 2048, device=DEV, dtype=torch.bfloat16)
    with torch.inference_mode():
        out = thin_linear(z, rnd(2048, 2048, scale=0.02))
    assert torch.all(out == 0)


def test_noncontiguous_x_and_w():
    assert_matches(rnd(2048, 4, seed=11).t(), rnd(2048, 2048, scale=0.02, seed=12))
    big = rnd(4096, 2048, scale=0.02, seed=13)
    assert_matches(rnd(4, 2048, seed=14), big[1024:3072])
    assert_matches(rnd(4, 2048, seed=15), big[::2])


def test_leading_dims_preserved():
    from kernels.thin_linear_fused import thin_linear
    x, w = rnd(2, 3, 2048, seed=16), rnd(512, 2048, scale=0.02, seed=17)
    with torch.inference_mode():
        got, ref = thin_linear(x, w), F.linear(x, w)
    assert got.shape == (2, 3, 512) == ref.shape
    assert float((got.float() - ref.float()).abs().max()) <= tol(ref)


@pytest.mark.parametrize("M", [4, 7, 9, 16, 32, 40, 48])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_bias_every_tile_kind(M, dtype):
    """The bias epilogue of every kernel (the GEMV at M <= 8; the 16-, 24- and
    32-row K-split tiles and the 64- to 128-row shared-activation tiles above),
    alone and through the split reduce, on a partial last row tile and token
    block.  The bias goes onto the rounded product, as the reference's
    ``y += bias`` (kernels/thin_linear_fused.py:343-344): bit-exact against
    the oracle on small-integer data, whose sums every order gets exactly,
    with products past the dtype's integer range so that one rounding and two
    differ; within the reference bound on random data."""
    from kernels.thin_linear_fused import thin_linear
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    K, N = 1000, 531
    g = torch.Generator().manual_seed(110 + M)
    scale = 3.0 if dtype == "bf16" else 15.0            # integer sums past 256 (bf16) / 2048 (fp16)
    xi = torch.randint(-3, 4, (M, K), generator=g).to(tdt)
    wi = (torch.randint(-3, 4, (N, K), generator=g) * scale).to(tdt)
    bi = (torch.randn(N, generator=g) * 3).to(tdt)
    want = othin.linear_exact(xi.float().numpy(), wi.float().numpy(), bi.float().numpy(), dtype=dtype)
    once = othin.linear_exact(xi.float().numpy(), wi.float().numpy(), dtype="fp32") + bi.float().numpy()
    once = torch.from_numpy(once).to(tdt).float().numpy()
    assert not np.array_equal(want, once)                # the case tells the two roundings apart
    x = rnd(M, K, dtype=tdt, seed=110 + M)
    w = rnd(N, K, dtype=tdt, scale=0.02, seed=111)
    b = rnd(N, dtype=tdt, scale=0.5, seed=112)
    ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), b.float().cpu().numpy(), dtype=dtype)
    amax = float(np.abs(ref).max())
    for rows in (4, 8, 16, 24, 32, 64, 96, 128):
        for split in (1, 3):
            cfg = (32, rows, 256, split)
            with torch.inference_mode():
                got_i = thin_linear(xi.to(DEV), wi.to(DEV), bi.to(DEV), config=cfg).float().cpu().numpy()
                got_t = thin_linear(x, w, b, config=cfg)
                assert torch.equal(got_t, thin_linear(x, w, config=cfg) + b)   # the torch add, bit for bit
                got = got_t.float().cpu().numpy()
            assert np.array_equal(got_i, want), (rows, split)
            err = float(np.abs(got - ref).max())
            assert err <= othin.tolerance(amax, dtype), (rows, split, err)


def test_bias_applied():
    from kernels.thin_linear_fused import thin_linear
    x, w = rnd(4, 512, seed=18), rnd(256, 512, scale=0.02, seed=19)
    b = rnd(256, scale=0.5, seed=20)
    with torch.inference_mode():
        got, ref = thin_linear(x, w, b), F.linear(x, w, b)
    assert float((got.float() - ref.float()).abs().max()) <= tol(ref)
    b32 = b.float()            # a bias of another dtype goes through torch's add
    with torch.inference_mode():
        got2 = thin_linear(x, w, b32)
    assert float((got2.float() - ref.float()).abs().max()) <= tol(ref)


def test_rejects_grad_mode():
    from kernels.thin_linear_fused import thin_linear
    x = rnd(4, 512, seed=21).requires_grad_(True)
    w = rnd(256, 512, scale=0.02, seed=22)
    with pytest.raises(RuntimeError, match="forward-only"):
        thin_linear(x, w)
    with torch.no_grad():
        thin_linear(x, w)


def test_dtype_mismatch_rejected():
    from kernels.thin_linear_fused import thin_linear
    with pytest.raises(TypeError):
        with torch.inference_mode():
            thin_linear(rnd(4, 512), rnd(256, 512, dtype=torch.float32))


@pytest.mark.parametrize("split_k", [1, 2, 8])
def test_reduction_is_deterministic(split_k):
    from kernels.thin_linear_fused import thin_linear
    x, w = rnd(4, 6144, seed=23), rnd(2048, 6144, scale=0.02, seed=24)
    cfg = (16, 32, 64, split_k)
    with torch.inference_mode():
        first = thin_linear(x, w, config=cfg)
        for _ in range(8):
            assert torch.equal(thin_linear(x, w, config=cfg), first)
        ref = F.linear(x, w)
        assert float((first.float() - ref.float()).abs().max()) <= tol(ref)


@pytest.mark.parametrize("M", [1, 4, 7, 9, 16, 24, 32, 33, 40, 48, 49])
def test_every_launch_shape(M):
    """Every rows / waves / split / block_k combination the planner accepts,
    on dims that leave partial tiles and a partial last k chunk."""
    from kernels.thin_linear_fused import thin_linear
    x, w = rnd(M, 1000, seed=31 + M), rnd(531, 1000, scale=0.02, seed=32)
    with torch.inference_mode():
        ref = F.linear(x, w)
        for rows in (4, 8, 16, 24, 32, 64, 96, 128):
            for waves in (2, 4, 8):
                for split in (1, 3):
                    for block_k in (256, 1024):
                        got = thin_linear(x, w, config=(16, rows, block_k, split), num_warps=waves)
                        err = float((got.float() - ref.float()).abs().max())
                        assert err <= tol(ref), (rows, waves, split, block_k, err)


def test_dispatch_falls_back_above_searched_M():
    from kernels.thin_linear_fused import ThinLinear, should_fuse
    lin = nn.Linear(2048, 2048, bias=False).to(DEV, torch.bfloat16).eval()
    tl_mod = ThinLinear(lin)
    assert should_fuse(4, 2048, 2048) and should_fuse(16, 2048, 2048)
    assert not should_fuse(32, 2048, 2048) and not should_fuse(96, 2048, 2048)
    with torch.inference_mode():
        for M, fused_expected in ((4, True), (16, True), (32, False), (96, False)):
            x = rnd(M, 2048, seed=M)
            got, ref = tl_mod(x), F.linear(x, lin.weight)
            if fused_expected:
                assert float((got.float() - ref.float()).abs().max()) <= tol(ref)
            else:
                assert torch.equal(got, ref), f"M={M} should have used F.linear"
        x3 = rnd(1, 96, 2048, seed=7)
        assert torch.equal(tl_mod(x3), F.linear(x3, lin.weight))
        x96 = rnd(96, 2048, seed=8)
        forced = ThinLinear(lin, always_fuse=True)(x96)
        ref96 = F.linear(x96, lin.weight)
        assert float((forced.float() - ref96.float()).abs().max()) <= tol(ref96)


def test_cuda_graph_capture_and_replay():
    from kernels.thin_linear_fused import thin_linear
    x, w = rnd(4, 2048, seed=25), rnd(2048, 2048, scale=0.02, seed=26)
    with torch.inference_mode():
        ref = F.linear(x, w)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                thin_linear(x, w)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = thin_linear(x, w)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert float((out.float() - ref.float()).abs().max()) <= tol(ref)
    with torch.inference_mode():
        x.mul_(2.0)
        g.replay()
        torch.cuda.synchronize()
        assert float((out.float() - F.linear(x, w).float()).abs().max()) <= tol(ref) * 2


def test_graph_capture_with_multiple_shapes_shares_workspace():
    from kernels.thin_linear_fused import thin_linear
    xs = [(rnd(4, 2048, seed=30), rnd(1024, 2048, scale=0.02, seed=31)),
          (rnd(4, 6144, seed=32), rnd(2048, 6144, scale=0.02, seed=33)),
          (rnd(4, 2048, seed=34), rnd(2048, 2048, scale=0.02, seed=35))]
    with torch.inference_mode():
        refs = [F.linear(x, w) for x, w in xs]
        eager = [thin_linear(x, w) for x, w in xs]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                for x, w in xs:
                    thin_linear(x, w)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs = [thin_linear(x, w) for x, w in xs]
        for _ in range(4):       # replays interleaved with eager work
            g.replay()
            torch.cuda.synchronize()
            for out, ref, e in zip(outs, refs, eager):
                assert float((out.float() - ref.float()).abs().max()) <= tol(ref)
                assert torch.equal(out, e)
            _ = [thin_linear(x, w) for x, w in xs]
            torch.cuda.synchronize()


class _Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(512, 512, bias=False)
        self.gate_proj = nn.Linear(512, 1024, bias=False)
        self.other = nn.Linear(512, 8, bias=False)

    def forward(self, x):
        return self.gate_proj(self.q_proj(x)), self.other(x)


def test_toggle_swaps_and_restores():
    from kernels import fused_toggle
    from kernels.thin_linear_fused import ThinLinear
    m = _Tiny().to(DEV, torch.bfloat16).eval()
    x = rnd(4, 512, seed=40)
    with torch.inference_mode():
        ref = m(x)
    assert fused_toggle.apply_to_model(m, True) == 2
    assert isinstance(m.q_proj, ThinLinear) and isinstance(m.other, nn.Linear)
    assert fused_toggle.apply_to_model(m, True) == 0
    with torch.inference_mode():
        got = m(x)
    for a, b in zip(got, ref):
        assert float((a.float() - b.float()).abs().max()) <= tol(b)
    assert fused_toggle.apply_to_model(m, False) == 2
    assert isinstance(m.q_proj, nn.Linear) and not fused_toggle.is_applied(m)


def test_toggle_warmup_runs_fused_modules():
    from kernels import fused_toggle
    m = nn.Module()
    m.q_proj = nn.Linear(2048, 2048, bias=False)
    m = m.to(DEV, torch.bfloat16).eval()
    fused_toggle.apply_to_model(m, True)
    fused_toggle.warmup(m, block_length=4)
    fused_toggle.apply_to_model(m, False)


# ──────────────────────────────────────────────── golden vectors (bit-exact) ───
def _t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(dtype)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_golden_integer_cases_bitexact(golden, dtype):
    from kernels.thin_linear_fused import thin_linear
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    d = golden("thin_int")
    with torch.inference_mode():
        for i in range(int(d["n_cases"])):
            x, w = _t(d[f"c{i}_x"], tdt), _t(d[f"c{i}_w"], tdt)
            expect = d[f"c{i}_y_{dtype}"]
            for cfg in (None, (16, 16, 256, 2), (16, 32, 256, 3)):
                got = thin_linear(x, w, config=cfg).float().cpu().numpy().astype(np.float64)
                assert np.array_equal(got, expect), (i, cfg)
        if dtype == "bf16":
            got = thin_linear(_t(d["bias_x"], tdt), _t(d["bias_w"], tdt), _t(d["bias_b"], tdt))
            assert np.array_equal(got.float().cpu().numpy(), d["bias_y"])


def test_golden_k1_bitexact(golden):
    from kernels.thin_linear_fused import thin_linear
    d = golden("thin_k1")
    with torch.inference_mode():
        got = thin_linear(_t(d["x"], torch.bfloat16), _t(d["w"], torch.bfloat16))
    assert np.array_equal(got.float().cpu().numpy().astype(np.float64), d["y"])


# ──────────────────────────────────────── oracle at the benchmarked shapes ───
def _oracle_check(M, K, N, seed):
    from kernels.thin_linear_fused import thin_linear
    x = rnd(M, K, seed=seed)
    w = rnd(N, K, scale=0.02, seed=seed + 1)
    with torch.inference_mode():
        got = thin_linear(x, w).float().cpu().numpy()
    ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype="bf16")
    amax = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= othin.tolerance(amax, "bf16"), (M, K, N, err)
    assert othin.max_abs_rel(got, ref) <= 1e-2
    return got


@pytest.mark.parametrize("M,K,N", [(4, 2048, 12288),                                   # C1
                                   (4, 2048, 4096), (4, 2048, 2048), (4, 6144, 2048),   # C2
                                   (16, 4096, 6144), (16, 4096, 4096), (16, 4096, 24576),
                                   (16, 12288, 4096), (32, 4096, 6144), (32, 4096, 4096),
                                   (32, 4096, 24576), (32, 12288, 4096),                # C3
                                   (36, 4096, 6144), (40, 4096, 4096), (44, 4096, 24576),
                                   (48, 12288, 4096)])        # C3 verify with committed blocks folded in
def test_oracle_baseline_shapes(M, K, N):
    _oracle_check(M, K, N, seed=M * 7 + K + N)


@pytest.mark.parametrize("M", [16, 32, 48])
def test_oracle_lm_head_target(M):
    _oracle_check(M, 4096, 151936, seed=99 + M)


XS_TILES = [(64, 2), (64, 4), (96, 4), (128, 4), (128, 8)]   # (rows per workgroup, waves)


@pytest.mark.parametrize("M", [9, 16, 17, 32, 33, 48])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_shared_activation_tiles_vs_oracle(M, dtype):
    """The 64-, 96- and 128-row tiles (waves split the rows and share each
    activation chunk through LDS) against the oracle, on the target's gate_up
    and qkv shapes and on dims that leave a partial row tile, a partial token
    block and a partial last k chunk; split 1, 2 and 3.  Bitwise stable across
    calls."""
    from kernels.thin_linear_fused import thin_linear, thin_linear_silu_mul
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    for K, N, split in [(4096, 24576, 1), (4096, 6144, 2), (1000, 531, 3)]:
        x = rnd(M, K, dtype=tdt, seed=70 + M + K)
        w = rnd(N, K, dtype=tdt, scale=0.02, seed=71 + N)
        ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype=dtype)
        amax = float(np.abs(ref).max())
        for rows, waves in XS_TILES:
            cfg = (32, rows, 256, split)
            with torch.inference_mode():
                got_t = thin_linear(x, w, config=cfg, num_warps=waves)
                assert torch.equal(thin_linear(x, w, config=cfg, num_warps=waves), got_t)
            got = got_t.float().cpu().numpy()
            err = float(np.abs(got - ref).max())
            assert err <= othin.tolerance(amax, dtype), (K, N, rows, waves, split, err)
            assert othin.max_abs_rel(got, ref) <= 1e-2
    # gated: the target MLP's gate and up halves (odd I at the other M)
    K, I = (4096, 12288) if M in (9, 32, 48) else (1000, 531)
    x = rnd(M, K, dtype=tdt, seed=80 + M)
    merged = rnd(2 * I, K, dtype=tdt, scale=0.02, seed=81)
    wg, wu = merged[:I], merged[I:]
    ref = othin.gated_exact(x.float().cpu().numpy(), wg.float().cpu().numpy(), wu.float().cpu().numpy(),
                            dtype=dtype)
    amax = float(np.abs(ref).max())
    for rows, waves in XS_TILES:
        with torch.inference_mode():
            got = thin_linear_silu_mul(x, wg, wu, config=(32, rows, 256, 1), num_warps=waves)
        got = got.float().cpu().numpy()
        assert float(np.abs(got - ref).max()) <= othin.tolerance(amax, dtype), (rows, waves)
        assert othin.max_abs_rel(got, ref) <= 1e-2


@pytest.mark.parametrize("M", [9, 16, 17, 32, 36, 48])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_partial_row_tiles_vs_oracle(M, dtype):
    """24-row tiles (two 16-row MFMA blocks, the second half-filled) against
    the oracle on the target's merged qkv shape and on dims that leave a
    partial last tile (531 = 22 x 24 + 3 rows) and a partial last k chunk.
    Waves split K the same way whatever the rows per workgroup, so every
    output is the same sum in the same order as with 32-row tiles: bit-equal."""
    from kernels.thin_linear_fused import thin_linear
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    for K, N in [(4096, 6144), (1000, 531)]:
        x = rnd(M, K, dtype=tdt, seed=90 + M + K)
        w = rnd(N, K, dtype=tdt, scale=0.02, seed=91 + N)
        ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype=dtype)
        amax = float(np.abs(ref).max())
        for waves in (2, 4, 8):
            for split in (1, 2):
                with torch.inference_mode():
                    got_t = thin_linear(x, w, config=(32, 24, 256, split), num_warps=waves)
                    full = thin_linear(x, w, config=(32, 32, 256, split), num_warps=waves)
                assert torch.equal(got_t, full), (K, N, waves, split)
                got = got_t.float().cpu().numpy()
                err = float(np.abs(got - ref).max())
                assert err <= othin.tolerance(amax, dtype), (K, N, waves, split, err)
                assert othin.max_abs_rel(got, ref) <= 1e-2


@pytest.mark.parametrize("M", [3, 5, 13, 17, 31, 33, 41, 48, 64, 96])
def test_oracle_other_row_counts(M):
    _oracle_check(M, 2048, 1536, seed=M)


@pytest.mark.parametrize("M", [1, 3, 4, 8, 9, 16, 32, 40])
def test_fp16_every_kernel(M):
    """fp16 through the GEMV (M <= 8), the LDS kernel (M > 8) and the strided
    path, against the oracle's exact sum rounded to fp16, within the
    reference's 16-bit bound."""
    from kernels.thin_linear_fused import thin_linear
    for K, N in [(2048, 2048), (1000, 531)]:
        x = rnd(M, K, dtype=torch.float16, seed=40 + M)
        w = rnd(N, K, dtype=torch.float16, scale=0.02, seed=41 + K)
        ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype="fp16")
        amax = float(np.abs(ref).max())
        with torch.inference_mode():
            for xv in (x, x.t().contiguous().t()):    # contiguous, then a strided view
                got = thin_linear(xv, w).float().cpu().numpy()
                err = float(np.abs(got - ref).max())
                assert err <= othin.tolerance(amax, "fp16"), (M, K, N, err)
                assert othin.max_abs_rel(got, ref) <= 1e-2


# ──────────────────────────────────────────── gated (SiLU-mul) projection ───
@pytest.mark.parametrize("M", [1, 4, 8, 9, 16, 32, 36, 48])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_silu_mul_vs_oracle(M, dtype):
    """thin_linear_silu_mul against the oracle's exact gated projection, on the
    draft MLP shape, odd dims, and the halves of a merged gate_up weight."""
    from kernels.thin_linear_fused import thin_linear_silu_mul
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    for K, I in [(2048, 6144), (1000, 531)]:
        x = rnd(M, K, dtype=tdt, seed=50 + M)
        merged = rnd(2 * I, K, dtype=tdt, scale=0.02, seed=51 + K)
        wg, wu = merged[:I], merged[I:]
        ref = othin.gated_exact(x.float().cpu().numpy(), wg.float().cpu().numpy(),
                                wu.float().cpu().numpy(), dtype=dtype)
        with torch.inference_mode():
            got = thin_linear_silu_mul(x, wg, wu).float().cpu().numpy()
        amax = float(np.abs(ref).max())
        err = float(np.abs(got - ref).max())
        assert err <= othin.tolerance(amax, dtype), (M, K, I, err)
        assert othin.max_abs_rel(got, ref) <= 1e-2


@pytest.mark.parametrize("M", [4, 16, 32, 40])
def test_silu_mul_every_launch_shape(M):
    from kernels.thin_linear_fused import thin_linear_silu_mul
    x = rnd(M, 1000, seed=60 + M)
    wg, wu = rnd(261, 1000, scale=0.03, seed=61), rnd(261, 1000, scale=0.03, seed=62)
    with torch.inference_mode():
        ref = F.silu(F.linear(x, wg)) * F.linear(x, wu)
        for rows in (8, 16, 32, 64, 96, 128):
            for waves in (2, 4, 8):
                for split in (1, 3):
                    got = thin_linear_silu_mul(x, wg, wu, config=(16, rows, 256, split), num_warps=waves)
                    err = float((got.float() - ref.float()).abs().max())
                    assert err <= tol(ref), (rows, waves, split, err)
        first = thin_linear_silu_mul(x, wg, wu, config=(16, 16, 256, 3))
        assert torch.equal(thin_linear_silu_mul(x, wg, wu, config=(16, 16, 256, 3)), first)


def test_silu_mul_fallbacks_and_errors():
    from kernels.thin_linear_fused import thin_linear_silu_mul
    x = rnd(4, 512, seed=70)
    wg, wu = rnd(64, 512, scale=0.03, seed=71), rnd(64, 512, scale=0.03, seed=72)
    with torch.inference_mode():
        ref = F.silu(F.linear(x, wg)) * F.linear(x, wu)
        for xv, g, u in [(x.t().contiguous().t(), wg, wu),                 # strided x
                         (x.float(), wg.float(), wu.float())]:              # fp32
            got = thin_linear_silu_mul(xv, g, u)
            r = F.silu(F.linear(xv, g)) * F.linear(xv, u)
            assert float((got.float() - r.float()).abs().max()) <= tol(r)
        assert thin_linear_silu_mul(x.view(2, 2, 512), wg, wu).shape == (2, 2, 64)
    with pytest.raises(TypeError):
        thin_linear_silu_mul(x, wg.float(), wu)
    with pytest.raises(ValueError):
        thin_linear_silu_mul(x, wg, wu[:32])
    with pytest.raises(RuntimeError, match="forward-only"):
        thin_linear_silu_mul(x.requires_grad_(True), wg, wu)


def test_gated_mlp_toggle_end_to_end():
    from kernels.fused_toggle import apply_gated_mlp_to_model

    class MLP(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(2048, 6144, bias=False)
            self.up_proj = nn.Linear(2048, 6144, bias=False)
            self.down_proj = nn.Linear(6144, 2048, bias=False)
            self.act_fn = nn.SiLU()

        def forward(self, x):
            return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))

    m = MLP().to(DEV, torch.bfloat16).eval()
    x = rnd(4, 2048, seed=80)
    with torch.inference_mode():
        stock = m(x)
        assert apply_gated_mlp_to_model(m) == 1
        fused = m(x)
        big = m(rnd(64, 2048, seed=81))            # outside the envelope: stock forward
        assert big.shape == (64, 2048)
        assert apply_gated_mlp_to_model(m, enable=False) == 1
        assert torch.equal(m(x), stock)
    assert float((fused.float() - stock.float()).abs().max()) <= tol(stock)


# ───────────────────────────────────────────────── RMSNorm and its prologue ───
def _norm_case(M, K, dtype, seed):
    x = rnd(M, K, dtype=dtype, scale=3.0, seed=seed)
    w = (1 + 0.2 * torch.randn(K, generator=torch.Generator(device=DEV).manual_seed(seed + 1),
                               device=DEV)).to(dtype)
    return x, w


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_rmsnorm_vs_oracle(dtype):
    from kernels.thin_linear_fused import thin_rmsnorm
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    ulp = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10, "fp32": 2.0 ** -20}[dtype]
    # 16-bit rows with K % 8 == 0 up to 8192 take the register-resident kernel
    # (1, 2, 3 or 4 chunks of 2048); K=77 and fp32 the element-wise one
    for M, K in [(1, 2048), (4, 2048), (32, 4096), (100, 1000), (3, 77), (5, 6144), (2, 8192), (3, 8200)]:
        x, w = _norm_case(M, K, tdt, seed=M + K)
        with torch.inference_mode():
            got = thin_rmsnorm(x, w, 1e-6).float().cpu().numpy()
        ref = othin.rmsnorm_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), 1e-6, dtype=dtype)
        assert np.all(np.abs(got - ref) <= 2 * ulp * np.abs(ref) + 1e-30), (M, K)   # 2 ulp: see the oracle test
    # rows of a wider buffer (16-byte aligned stride, then an odd one)
    for pad in (16, 3):
        xb, w = _norm_case(4, 2048 + pad, tdt, seed=pad)
        x, w = xb[:, :2048], w[:2048].contiguous()
        with torch.inference_mode():
            got = thin_rmsnorm(x, w, 1e-6).float().cpu().numpy()
        ref = othin.rmsnorm_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), 1e-6, dtype=dtype)
        assert np.all(np.abs(got - ref) <= 2 * ulp * np.abs(ref) + 1e-30), pad
    x, w = _norm_case(8, 512, tdt, seed=3)
    with torch.inference_mode():
        assert torch.equal(thin_rmsnorm(x, w, 1e-5), thin_rmsnorm(x, w, 1e-5))     # deterministic
        assert thin_rmsnorm(x.view(2, 4, 512), w, 1e-5).shape == (2, 4, 512)


@pytest.mark.parametrize("M", [1, 4, 6, 8, 16, 32, 36, 48])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_rmsnorm_linear_vs_oracle(M, dtype):
    """The fused norm + linear (norm inside the GEMV at M <= 8, a separate
    launch above) against the oracle's norm then exact linear."""
    from kernels.thin_linear_fused import thin_rmsnorm_linear, thin_rmsnorm_linear_silu_mul
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    for K, N in [(2048, 4096), (1000, 531)]:
        x, g = _norm_case(M, K, tdt, seed=90 + M)
        w = rnd(2 * N, K, dtype=tdt, scale=0.02, seed=91 + K)
        xn = othin.rmsnorm_exact(x.float().cpu().numpy(), g.float().cpu().numpy(), 1e-6, dtype=dtype)
        wn = w.float().cpu().numpy()
        with torch.inference_mode():
            y = thin_rmsnorm_linear(x, g, 1e-6, w[:N]).float().cpu().numpy()
            h = thin_rmsnorm_linear_silu_mul(x, g, 1e-6, w[:N], w[N:]).float().cpu().numpy()
        ref_y = othin.linear_exact(xn, wn[:N], dtype=dtype)
        ref_h = othin.gated_exact(xn, wn[:N], wn[N:], dtype=dtype)
        for got, ref in ((y, ref_y), (h, ref_h)):
            err = float(np.abs(got - ref).max())
            assert err <= othin.tolerance(float(np.abs(ref).max()), dtype), (M, K, N, err)
            assert othin.max_abs_rel(got, ref) <= 1e-2


def test_rmsnorm_linear_configs_bias_and_toggle():
    from kernels.fused_toggle import apply_rmsnorm_to_model
    from kernels.thin_linear_fused import thin_rmsnorm, thin_rmsnorm_linear
    x, g = _norm_case(4, 1000, torch.bfloat16, seed=7)
    w, b = rnd(333, 1000, scale=0.03, seed=8), rnd(333, scale=0.5, seed=9)
    with torch.inference_mode():
        ref = F.linear(thin_rmsnorm(x, g, 1e-6), w, b)
        for rows in (4, 8, 16, 32):
            for split in (1, 3):
                got = thin_rmsnorm_linear(x, g, 1e-6, w, b, config=(16, rows, 256, split))
                assert float((got.float() - ref.float()).abs().max()) <= tol(ref), (rows, split)

    class TinyRMSNorm(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.weight = nn.Parameter(torch.ones(n))
            self.variance_epsilon = 1e-6

        def forward(self, h):
            h32 = h.float()
            return self.weight * (h32 * torch.rsqrt(h32.pow(2).mean(-1, keepdim=True)
                                                    + self.variance_epsilon)).to(h.dtype)

    m = TinyRMSNorm(1000).to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(g)
        stock = m(x)
        assert apply_rmsnorm_to_model(m) == 1
        fused = m(x)
        apply_rmsnorm_to_model(m, enable=False)
    ulp = 2.0 ** -7
    assert torch.all((fused.float() - stock.float()).abs() <= 2 * ulp * stock.float().abs() + 1e-30)


# ───────────────────────────────────────────── size-independent properties ───
def test_properties_at_full_size():
    from kernels.thin_linear_fused import thin_linear
    with torch.inference_mode():
        for M, K, N in [(4, 2048, 12288), (32, 4096, 24576), (16, 12288, 4096)]:
            x = rnd(M, K, seed=200 + M)
            w = rnd(N, K, scale=0.02, seed=300 + M)
            y = thin_linear(x, w)
            assert torch.equal(thin_linear(x, w), y)                         # deterministic
            perm = torch.randperm(M, generator=torch.Generator().manual_seed(M))
            assert torch.equal(thin_linear(x[perm], w), y[perm])              # rows independent
            if M <= 4:   # one token or four: the same GEMV kernel and column set
                rows = torch.cat([thin_linear(x[i:i + 1], w) for i in range(M)])
                assert torch.equal(rows, y)
            assert torch.equal(thin_linear(x * 4, w), y * 4)                  # exact 2^k scaling
            wt = torch.empty(N, K + 64, device=DEV, dtype=w.dtype)
            wt[:, 32:32 + K] = w
            assert torch.equal(thin_linear(x, wt[:, 32:32 + K]), y)           # strided view


@pytest.mark.parametrize("M", [1, 4, 6, 8, 16, 32, 40, 48])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_linear_residual_vs_oracle(M, dtype):
    """residual + x w^T in one launch: bit-exact on small-integer data (every
    sum exact), within the reference bound on random data; in place; split K."""
    from kernels.thin_linear_fused import thin_linear, thin_linear_residual
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
    g = torch.Generator().manual_seed(M)
    K, N = 2048, 4096
    xi = torch.randint(-3, 4, (M, K), generator=g).to(dtype)
    wi = torch.randint(-3, 4, (N, K), generator=g).to(dtype)
    r = (torch.randn(M, N, generator=g) * 100).to(dtype)
    want = othin.linear_residual_exact(xi.float().numpy(), wi.float().numpy(), r.float().numpy(), dtype=name)
    with torch.inference_mode():
        got = thin_linear_residual(xi.to(DEV), wi.to(DEV), r.to(DEV))
    assert np.array_equal(got.float().cpu().numpy(), want)
    x = rnd(M, K, dtype=dtype, seed=M + 1)
    w = rnd(N, K, dtype=dtype, scale=0.02, seed=M + 2)
    res = rnd(M, N, dtype=dtype, seed=M + 3)
    with torch.inference_mode():
        ref = res + thin_linear(x, w)
        got = thin_linear_residual(x, w, res)
        assert torch.equal(got, ref)                          # the same rounding points as the two ops
        split = thin_linear_residual(x, w, res, config=(16, 16, 256, 4))
        assert float((split.float() - ref.float()).abs().max()) <= tol(ref)
        inplace = res.clone()
        thin_linear_residual(x, w, inplace, out=inplace)
        assert torch.equal(inplace, got)
