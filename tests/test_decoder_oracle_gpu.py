"""Decoder composition on the GPU against a host oracle forward.

``SynthModel.forward`` (speculative/model.py) chains the kernels of one SDAR
decoder layer: RMSNorm + merged q/k/v, q/k norm + RoPE + cache write,
attention over the static cache, o_proj + residual, RMSNorm + gate/up +
SiLU.mul, down_proj + residual; then the final norm and the lm_head.  Here its
logits are compared with a forward composed on the host from the oracle's
per-op restatements -- ``rmsnorm_exact``, ``linear_exact``, ``gated_exact``,
``linear_residual_exact``, ``oracle.attention.qk_norm_rope`` and
``oracle.attention.attention`` -- following the reference's layer
(sdar/modeling_sdar.py:305-366: residual, input_layernorm, self_attn with
q_norm/k_norm before RoPE at 250-262, residual add, post_attention_layernorm,
mlp, residual add) and SDARMLP (113-119: down(act(gate(x)) * up(x))).

The GPU forward runs the way the runner runs it: a prefix forward writes the
context's K/V into the cache, then the last rows run as a cached forward that
reads them.  Forwards above 8 rows (every prefix here, and the 36-row case)
take the form that hands each projection's split-K partials to the launch
consuming them (speculative/model.py).  The oracle runs the whole sequence at once with the
block-causal prompt mask (blocks of 4).

Tolerance: max|got - ref| <= 2^-6 * max|ref| + 1e-3 on the logits of the
cached rows, the reference's bound for a composed bf16 path
(kernels/workspace/moe_dispatch/duipai.py:50-60; its single linear uses 2^-7).
The model is the random-init SynthModel with its embedding scaled by 1/16
and its q/k norm weights drawn apart, so that each of the terms below moves
the logits.  The test also plants three wiring mistakes in the oracle (gate and up
exchanged, q and k norm weights exchanged, the attention residual dropped)
and requires each to exceed the bound, so the bound does separate a correct
composition from a plausible wrong one.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import thin_linear as olin
from oracle.numerics import ROUNDERS

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def rope_tables_host(head_dim, theta, n_pos, dtype=torch.bfloat16):
    """cos/sin [n_pos, D] as SDARRotaryEmbedding.forward computes them (fp32
    outer product of positions and 1 / theta^(2i/D), halves duplicated,
    cos/sin in fp32, cast to the dtype), on the host."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    pos = torch.arange(n_pos, dtype=torch.float32)
    freqs = torch.outer(pos, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return _np(emb.cos().to(dtype)), _np(emb.sin().to(dtype))


def oracle_forward(model, ids, mask, cos, sin, plant=None, dt="bf16"):
    """Logits [n, V] of the whole sequence ``ids`` (positions 0..n-1) with the
    bool visibility ``mask`` [n, n], in dtype ``dt``; ``plant`` names a wiring
    mistake to make."""
    s = model.shape
    H, D, I = s.hidden, s.head_dim, s.intermediate
    Hq, Hkv = s.n_q_heads, s.n_kv_heads
    n = len(ids)
    h = _np(model.embed)[np.asarray(ids)]
    for L in model.layers:
        x = olin.rmsnorm_exact(h, _np(L.ln1), s.eps, dtype=dt)
        qkv = olin.linear_exact(x, _np(L.wqkv), dtype=dt)
        q = qkv[:, :Hq * D].reshape(n, Hq, D)
        k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(n, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].reshape(n, Hkv, D)
        qn, kn = _np(L.qn), _np(L.kn)
        if plant == "qk_norm_swapped":
            qn, kn = kn, qn
        q = oatt.qk_norm_rope(q, qn, s.eps, cos[:n], sin[:n], dtype=dt)
        k = oatt.qk_norm_rope(k, kn, s.eps, cos[:n], sin[:n], dtype=dt)
        a = oatt.attention(q, k.transpose(1, 0, 2), v.transpose(1, 0, 2), mask, 1.0 / np.sqrt(D))
        a = ROUNDERS[dt](a).reshape(n, Hq * D)       # SDPA's output in the dtype
        if plant == "no_attn_residual":
            h = olin.linear_exact(a, _np(L.wo), dtype=dt)
        else:
            h = olin.linear_residual_exact(a, _np(L.wo), h, dtype=dt)
        x = olin.rmsnorm_exact(h, _np(L.ln2), s.eps, dtype=dt)
        wg, wu = _np(L.wgu[:I]), _np(L.wgu[I:])
        if plant == "gate_up_swapped":
            wg, wu = wu, wg
        g = olin.gated_exact(x, wg, wu, dtype=dt)
        h = olin.linear_residual_exact(g, _np(L.wd), h, dtype=dt)
    return olin.linear_exact(olin.rmsnorm_exact(h, _np(model.lnf), s.eps, dtype=dt), _np(model.lm_head), dtype=dt)


CASES = {
    # the tiny SDAR-like decoder of the runner tests: 32-token context + 8 rows
    "tiny": (dict(hidden=256, n_layers=2, n_q_heads=2, n_kv_heads=1, intermediate=512, vocab=1000), 40, 8),
    # SDAR-1.7B widths (hidden 2048, 16 q / 8 KV heads of 128, intermediate
    # 6144), 2 layers, an 8192-id vocabulary (the lm_head's width does not
    # change the composition; 151936 would need 5 GB of fp64 host copies):
    # 248 context slots + 8 rows = 256 slots
    "sdar1p7b_2l": (dict(hidden=2048, n_layers=2, n_q_heads=16, n_kv_heads=8, intermediate=6144, vocab=8192),
                    256, 8),
    # the same model with 36 cached rows, the folded verify's count: above 8
    # rows the projections hand their split-K partials to the launches that
    # consume them (reduce + q/k norm + RoPE + cache write, reduce + residual
    # + RMSNorm)
    "sdar1p7b_2l_36rows": (dict(hidden=2048, n_layers=2, n_q_heads=16, n_kv_heads=8, intermediate=6144,
                                vocab=8192), 256, 36),
    # the tiny decoder in fp16, 12 cached rows (the one-launch attention above 8 rows)
    "tiny_fp16_12rows": (dict(hidden=256, n_layers=2, n_q_heads=2, n_kv_heads=1, intermediate=512, vocab=1000),
                         44, 12, torch.float16),
}


@pytest.mark.parametrize("case", list(CASES))
def test_decoder_forward_vs_oracle(case):
    from speculative.model import ModelShape, SynthModel
    dims, n, rows, *rest = CASES[case]
    dtype = rest[0] if rest else torch.bfloat16
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    print(f"decoder composition: {case}, {n} slots, {rows} cached rows, {dt}", flush=True)
    shape = ModelShape(**dims)
    model = SynthModel(shape, DEV, seed=11, max_ctx=n, max_rows=n, dtype=dtype)
    # Make every term of the composition visible in the logits: the embedding
    # scaled by 1/16 (exact in bf16) so the layers' residual contributions are
    # not buried under it, and q/k norm weights drawn apart (0.5 + U[0, 1))
    # so that exchanging them changes the attention.
    gen = torch.Generator(device=DEV).manual_seed(12)
    model.embed.mul_(1.0 / 16)
    for L in model.layers:
        L.qn.copy_(0.5 + torch.rand(shape.head_dim, generator=gen, device=DEV))
        L.kn.copy_(0.5 + torch.rand(shape.head_dim, generator=gen, device=DEV))
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, shape.vocab, (n,), generator=g)
    ar = torch.arange(n)
    blk = ar // 4
    vis = blk[None, :] <= blk[:, None]                  # the prompt's block-causal rule
    full = model.cache.full_len
    ctx = n - rows
    # 1) the context writes its K/V; 2) the last rows read them from the cache
    m0 = torch.zeros(ctx, full, dtype=torch.bool)
    m0[:, :ctx] = vis[:ctx, :ctx]
    a0 = ar[:ctx].to(DEV)
    model.forward(ids[:ctx].to(DEV), a0, a0, m0.to(DEV), valid_len=ctx, head=False, rows_at_end=True)
    m1 = torch.zeros(rows, full, dtype=torch.bool)
    m1[:, :n] = vis[ctx:]
    a1 = ar[ctx:].to(DEV)
    got = model.forward(ids[ctx:].to(DEV), a1, a1, m1.to(DEV), valid_len=n, rows_at_end=True)
    torch.cuda.synchronize()
    got = _np(got)

    cos, sin = rope_tables_host(shape.head_dim, shape.rope_theta, n, dtype)
    # the GPU's RoPE tables follow the same formula (fp32 cos/sin on the device
    # may land one bf16 step away from the host's on a rare argument)
    for dev_t, host_t in ((model.cos, cos), (model.sin, sin)):
        diff = np.abs(_np(dev_t[:n]) - host_t)
        assert diff.max() <= 2.0 ** -7 and (diff == 0).mean() > 0.99
    ref = oracle_forward(model, ids.tolist(), vis.numpy(), cos, sin, dt=dt)[ctx:]
    bound = 2.0 ** -6 * float(np.abs(ref).max()) + 1e-3
    err = float(np.abs(got - ref).max())
    print(f"  max|ref| {np.abs(ref).max():.4f}, max err {err:.5f}, bound {bound:.5f}", flush=True)
    assert err <= bound, (case, err, bound)
    # argmax agrees wherever the oracle's top two logits are further apart
    # than twice the bound
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * bound
    assert np.array_equal(got.argmax(1)[clear], ref.argmax(1)[clear])

    # planted mistakes in the oracle: each must fall outside the bound
    for plant in ("gate_up_swapped", "qk_norm_swapped", "no_attn_residual"):
        bad = oracle_forward(model, ids.tolist(), vis.numpy(), cos, sin, plant=plant, dt=dt)[ctx:]
        assert float(np.abs(bad - ref).max()) > bound, plant
