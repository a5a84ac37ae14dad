"""Pins the attention oracle (CPU only): against torch's CPU composition of
the reference's own ops (the stock RMSNorm, apply_rotary_pos_emb in bf16,
scaled_dot_product_attention with a bool mask and repeated KV heads) and
against closed forms.  Planted slips (rotate_half sign, a missing rounding
point, the wrong KV head for a query head) fail."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle.numerics import round_bf16


def _rotate_half(x):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def _torch_qk(x, w, eps, cos, sin):
    """modeling_sdar.py:250-262 on CPU: stock RMSNorm per head, then RoPE."""
    if w is not None:
        x32 = x.float()
        x = w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    c, s = cos[:, None, :], sin[:, None, :]
    return (x * c) + (_rotate_half(x) * s)


def _tables(pos, D=128, theta=1e6, dtype=torch.bfloat16):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    f = pos.float()[:, None] * inv[None, :]
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


@pytest.mark.parametrize("norm", [True, False])
def test_qk_norm_rope_vs_torch_cpu(norm):
    g = torch.Generator().manual_seed(1)
    M, H, D = 5, 6, 128
    x = (torch.randn(M, H, D, generator=g) * 2).bfloat16()
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16() if norm else None
    pos = torch.tensor([0, 1, 17, 600, 4095])
    cos, sin = _tables(pos)
    ref = _torch_qk(x, w, 1e-6, cos, sin).float().numpy()
    got = oatt.qk_norm_rope(x.float().numpy(), None if w is None else w.float().numpy(), 1e-6,
                            cos.float().numpy(), sin.float().numpy())
    ulp = 2.0 ** -7
    if norm:   # fp64 statistics may move x * r by an ulp (as for the RMSNorm oracle)
        assert np.all(np.abs(got - ref) <= 2 * ulp * np.abs(ref) + 1e-30)
        assert (got != ref).mean() < 0.01
    else:
        assert np.array_equal(got, ref)
    # position 0: cos = 1, sin = 0 -> the normed head itself
    x0 = got[0]
    normed = oatt.qk_norm_rope(x[:1].float().numpy(), None if w is None else w.float().numpy(), 1e-6,
                               np.ones((1, D)), np.zeros((1, D)))
    assert np.array_equal(x0, normed[0])


def test_attention_vs_torch_sdpa_cpu():
    g = torch.Generator().manual_seed(2)
    M, Hq, Hkv, L, D = 6, 8, 2, 77, 128
    q = torch.randn(M, Hq, D, generator=g)
    k = torch.randn(Hkv, L, D, generator=g)
    v = torch.randn(Hkv, L, D, generator=g)
    mask = torch.rand(M, L, generator=g) < 0.7
    mask[:, 0] = True
    scale = D ** -0.5
    kk = k.repeat_interleave(Hq // Hkv, dim=0)[None]
    vv = v.repeat_interleave(Hq // Hkv, dim=0)[None]
    ref = F.scaled_dot_product_attention(q.transpose(0, 1)[None], kk, vv, attn_mask=mask[None, None],
                                         scale=scale)[0].transpose(0, 1).numpy()
    got = oatt.attention(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), scale)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    M, Hq, Hkv, L, D = 3, 4, 2, 20, 128
    q = rng.standard_normal((M, Hq, D))
    k = rng.standard_normal((Hkv, L, D))
    v = rng.standard_normal((Hkv, L, D))
    one = np.zeros((M, L), dtype=bool)
    one[0, 5] = one[1, 19] = True                        # row 2: nothing visible
    out = oatt.attention(q, k, v, one, 0.1)
    assert np.allclose(out[0, 3], v[1, 5]) and np.allclose(out[1, 0], v[0, 19])
    assert np.all(out[2] == 0)
    keq = np.repeat(k[:, :1], L, axis=1)                 # equal keys: mean of the visible values
    vis = rng.random((M, L)) < 0.5
    vis[:, 0] = True
    out = oatt.attention(q, keq, v, vis, 0.3)
    for m in range(M):
        assert np.allclose(out[m, 1], v[0, vis[m]].mean(axis=0))
        assert np.allclose(out[m, 2], v[1, vis[m]].mean(axis=0))


def test_planted_attention_slips():
    g = torch.Generator().manual_seed(4)
    M, H, D = 2, 2, 128
    x = torch.randn(M, H, D, generator=g).bfloat16()
    cos, sin = _tables(torch.tensor([3, 9]))
    ref = _torch_qk(x, None, 1e-6, cos, sin).float().numpy()
    xf, c, s = x.float().numpy(), cos.float().numpy()[:, None], sin.float().numpy()[:, None]
    wrong_sign = round_bf16(round_bf16(xf * c) + round_bf16(np.concatenate([xf[..., 64:], -xf[..., :64]], -1) * s))
    one_round = round_bf16(xf * c + np.concatenate([-xf[..., 64:], xf[..., :64]], -1) * s)
    assert not np.array_equal(wrong_sign, ref)
    assert not np.array_equal(one_round, ref)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 4, D))
    k = rng.standard_normal((2, 9, D))
    v = rng.standard_normal((2, 9, D))
    good = oatt.attention(q, k, v, None, 0.1)
    swapped = oatt.attention(q, k[::-1].copy(), v[::-1].copy(), None, 0.1)   # hq -> the other KV head
    assert not np.allclose(good, swapped)
