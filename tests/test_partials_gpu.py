"""Split-K partials summed by the launches that consume them, on the GPU.

``thin_linear_partials`` writes a projection's fp32 partials without the
reduce launch; ``reduce_residual_rmsnorm`` sums them into the residual stream
and applies the next RMSNorm, ``reduce_qkv_rope_cache`` sums them into the
q/k/v rows of the attention prologue.  Each consumer must give exactly what the
reduce-first sequence gives -- thin_linear's reduce (kernels/thin_linear_fused.py:
139-171: partials summed in split order, rounded to the dtype), the residual
add, the stock RMSNorm (sdar/run_native_tp2.py:42-47), qkv_rope_cache -- so the
checks are bit-equality with that sequence on the same partials, plus the
oracle (linear_residual_exact, rmsnorm_exact, linear_exact) within the
reference's bf16 bound (kernels/thin_linear_fused_test.py:28-32).  The last
test runs the decoder forward both ways at the verify's row counts.
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


def _np(t):
    return t.detach().double().cpu().numpy()


def split_sum(part):
    """The partials summed as thin_linear's reduce sums them: from 0 in split
    order above one partial (elementwise fp32 adds are exact IEEE ops)."""
    if part.shape[0] == 1:
        return part[0].clone()
    acc = torch.zeros_like(part[0])
    for s in range(part.shape[0]):
        acc = acc + part[s]
    return acc


@pytest.mark.parametrize("M", [9, 16, 32, 36, 48])
@pytest.mark.parametrize("split", [1, 2, 4])
def test_partials_sum_to_the_linear(M, split):
    from kernels.thin_linear_fused import thin_linear, thin_linear_partials
    K, N = 4096, 4096
    print(f"partials: M={M} split={split}", flush=True)
    x = rnd(M, K, seed=M)
    w = rnd(N, K, scale=0.02, seed=M + 1)
    cfg = (64, 16, 256, split)
    with torch.inference_mode():
        part = thin_linear_partials(x, w, config=cfg)
        ref = thin_linear(x, w, config=cfg)
    torch.cuda.synchronize()
    assert part.shape == (split, M, N) and part.dtype == torch.float32
    assert torch.equal(split_sum(part).to(torch.bfloat16), ref)
    want = othin.linear_exact(_np(x), _np(w))
    err = float(np.abs(_np(split_sum(part).to(torch.bfloat16)) - want).max())
    assert err <= othin.tolerance(float(np.abs(want).max()), "bf16")


@pytest.mark.parametrize("M,K,N,split,dtype", [
    (9, 4096, 4096, 1, torch.bfloat16),
    (16, 4096, 4096, 2, torch.bfloat16),
    (32, 12288, 4096, 4, torch.bfloat16),     # the target's down_proj into the next norm
    (36, 12288, 4096, 4, torch.bfloat16),
    (36, 4096, 4096, 1, torch.bfloat16),      # o_proj into the post-attention norm
    (48, 6144, 2048, 2, torch.bfloat16),      # the draft's hidden width
    (36, 2048, 6144, 3, torch.bfloat16),      # N past 4096 (three 2048-wide passes)
    (1, 2048, 2048, 1, torch.bfloat16),
    (36, 4096, 4096, 2, torch.float16),
])
def test_reduce_residual_rmsnorm_equals_reduce_then_norm(M, K, N, split, dtype):
    from kernels.thin_linear_fused import (reduce_residual_rmsnorm, thin_linear_partials, thin_linear_residual,
                                           thin_rmsnorm)
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    print(f"reduce+residual+norm: M={M} K={K} N={N} split={split} {name}", flush=True)
    x = rnd(M, K, dtype=dtype, seed=M + K)
    w = rnd(N, K, dtype=dtype, scale=0.02, seed=M + 7)
    res = rnd(M, N, dtype=dtype, seed=M + 8)
    gamma = (1 + 0.1 * rnd(N, dtype=torch.float32, seed=M + 9)).to(dtype)
    eps = 1e-6
    cfg = (64, 16, 256, split)
    with torch.inference_mode():
        part = thin_linear_partials(x, w, config=cfg)
        h_ref = thin_linear_residual(x, w, res, config=cfg)
        xn_ref = thin_rmsnorm(h_ref, gamma, eps)
        h, xn = reduce_residual_rmsnorm(part, res, gamma, eps)
        inplace = res.clone()
        h2, xn2 = reduce_residual_rmsnorm(part, inplace, gamma, eps, out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref) and torch.equal(xn, xn_ref)
    assert h2.data_ptr() == inplace.data_ptr() and torch.equal(h2, h_ref) and torch.equal(xn2, xn_ref)
    # against the oracle: the residual stream within the linear's bound, the
    # norm of the produced rows within 2 ulp of the oracle's norm of them
    want_h = othin.linear_residual_exact(_np(x), _np(w), _np(res), dtype=name)
    assert float(np.abs(_np(h) - want_h).max()) <= othin.tolerance(float(np.abs(want_h).max()), name)
    want_xn = othin.rmsnorm_exact(_np(h), _np(gamma), eps, dtype=name)
    ulp = 2.0 ** (-7 if name == "bf16" else -10)
    assert np.all(np.abs(_np(xn) - want_xn) <= 2 * ulp * np.maximum(np.abs(want_xn), 2.0 ** -14))


def test_reduce_residual_rmsnorm_rejects_bad_input():
    from kernels.thin_linear_fused import reduce_residual_rmsnorm
    part = torch.zeros(9, 4, 4096, device=DEV)
    res = torch.zeros(4, 4096, device=DEV, dtype=torch.bfloat16)
    g = torch.ones(4096, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="split"):
        reduce_residual_rmsnorm(part, res, g, 1e-6)
    with pytest.raises(ValueError, match="residual"):
        reduce_residual_rmsnorm(part[:2], res[:, :2048], g, 1e-6)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        reduce_residual_rmsnorm(torch.zeros(1, 4, 12, device=DEV), res[:, :12].contiguous(),
                                g[:12].contiguous(), 1e-6)


@pytest.mark.parametrize("M,split,dtype", [(36, 2, torch.bfloat16), (32, 1, torch.bfloat16), (12, 4, torch.bfloat16),
                                           (48, 2, torch.bfloat16), (36, 2, torch.float16)])
def test_reduce_qkv_rope_cache_equals_reduce_then_prologue(M, split, dtype):
    from kernels.attention_fused import (BlockKVCache, default_inv_freq, qkv_rope_cache, reduce_qkv_rope_cache,
                                         rope_tables)
    from kernels.thin_linear_fused import thin_linear, thin_linear_partials
    print(f"reduce+qkv_rope_cache: M={M} split={split} dtype={dtype}", flush=True)
    Hq, Hkv, D, H, eps = 32, 8, 128, 4096, 1e-6
    x = rnd(M, H, dtype=dtype, seed=M + 30)
    w = rnd((Hq + 2 * Hkv) * D, H, dtype=dtype, scale=0.02, seed=M + 31)
    qn = (1 + 0.1 * rnd(D, dtype=torch.float32, seed=M + 32)).to(dtype)
    kn = (1 + 0.1 * rnd(D, dtype=torch.float32, seed=M + 33)).to(dtype)
    cos, sin = rope_tables(default_inv_freq(device=DEV), 4096, dtype)
    pos = torch.arange(500, 500 + M, device=DEV)
    pos[1] = -1                                               # out of range: zero q row, no k write
    slots = torch.arange(900, 900 + M, device=DEV)
    slots2 = torch.arange(600, 600 + M, device=DEV)
    caches = [BlockKVCache(1, Hkv, 1024, 64, DEV, dtype=dtype) for _ in range(2)]
    cfg = (64, 24, 256, split)
    with torch.inference_mode():
        part = thin_linear_partials(x, w, config=cfg)
        q1 = reduce_qkv_rope_cache(part, Hq, qn, kn, eps, cos, sin, pos, slots, caches[0], 0, slots2=slots2)
        qkv = thin_linear(x, w, config=cfg)
        q2 = qkv_rope_cache(qkv, Hq, qn, kn, eps, cos, sin, pos, slots, caches[1], 0, slots2=slots2)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(caches[0].k_tiles[0], caches[1].k_tiles[0])
    assert torch.equal(caches[0].v_tiles[0], caches[1].v_tiles[0])
    assert float(q1[1].abs().max()) == 0.0
    assert float(caches[0].keys(0)[:, 901].abs().max()) == 0.0 and float(caches[0].keys(0)[:, 900].abs().max()) > 0


@pytest.mark.parametrize("tuned", [False, True], ids=["same_splits", "partials_table"])
@pytest.mark.parametrize("case", ["tiny", "sdar1p7b_2l"])
def test_decoder_partials_path_equals_reduce_first(case, tuned, monkeypatch):
    """SynthModel's forward above 8 rows, partials handed to their consumers,
    against the same model reducing every projection first, for a long prefix
    forward, the verify's 36 rows through block attention, and 12 rows at the
    end of the valid range through the one-launch attention.  With the
    reduce-first form's splits (the partials table emptied) logits and K/V
    caches are equal; with the partials table's own splits (other k-chunk
    sums) the logits agree within the composed bf16 bound, 2^-6 max + 1e-3."""
    import kernels.thin_linear_fused as tlf
    from speculative.model import ModelShape, SynthModel
    if not tuned:
        monkeypatch.setattr(tlf, "PARTIALS_RANGES", {})
    dims = {"tiny": dict(hidden=256, n_layers=2, n_q_heads=2, n_kv_heads=1, intermediate=512, vocab=1000),
            "sdar1p7b_2l": dict(hidden=2048, n_layers=2, n_q_heads=16, n_kv_heads=8, intermediate=6144,
                                vocab=8192)}[case]
    shape = ModelShape(**dims)
    models = [SynthModel(shape, DEV, seed=21, max_ctx=512, max_rows=64) for _ in range(2)]
    models[1].reduce_first = True
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, shape.vocab, (300,), generator=g).to(DEV)
    full = models[0].cache.full_len
    outs = []
    for mdl in models:
        o = []
        with torch.inference_mode():
            # 1) a 252-row prefix; 2) 36 cached rows at slots 252..287; 3) 12
            # rows at the end of a 300-slot valid range (the one-launch attention)
            for lo, hi, valid in ((0, 252, 252), (252, 288, 288), (288, 300, 300)):
                n = hi - lo
                mask = torch.zeros(n, full, dtype=torch.bool, device=DEV)
                mask[:, :valid] = torch.tril(torch.ones(n, valid, dtype=torch.bool, device=DEV), diagonal=lo)
                ar = torch.arange(lo, hi, device=DEV)
                o.append(mdl.forward(ids[lo:hi], ar, ar, mask, valid_len=valid, rows_at_end=True))
        torch.cuda.synchronize()
        outs.append(o)
    assert models[0].partials_path(36) and not models[1].partials_path(36)
    if not tuned:
        for a, b in zip(*outs):
            assert torch.equal(a, b)
        for lay in range(shape.n_layers):
            assert torch.equal(models[0].cache.k_tiles[lay], models[1].cache.k_tiles[lay])
            assert torch.equal(models[0].cache.v_tiles[lay], models[1].cache.v_tiles[lay])
        return
    for a, b in zip(*outs):
        ref = b.float()
        bound = 2.0 ** -6 * float(ref.abs().max()) + 1e-3
        assert float((a.float() - ref).abs().max()) <= bound
        top2 = ref.topk(2, dim=1).values
        clear = (top2[:, 0] - top2[:, 1]) > 2 * bound
        assert torch.equal(a.float().argmax(1)[clear], ref.argmax(1)[clear])
