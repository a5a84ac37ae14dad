"""Pins the lm_head-epilogue oracle (CPU only): torch's CPU softmax / argmax /
topk on tie-free rows, and closed forms for uniform rows, repeated maxima,
a dominant logit and -inf entries.  The planted-slip test at the end shows
that a first/last-index swap, an unnormalised confidence and a selection that
ignores the mask each fail one of these checks."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import logits as olog


def _torch_epilogue(l: torch.Tensor):
    probs = F.softmax(l.float(), dim=-1)
    ids = probs.argmax(dim=-1)
    conf = probs.gather(1, ids.unsqueeze(-1)).squeeze(-1)
    return ids, conf, probs


def _torch_denoise(l, cur, mask_id, n_u, step, step_map, ppp):
    """The reference's sequence, cache_aware.py:916-938, on CPU tensors."""
    ids, conf, probs = _torch_epilogue(l)
    is_masked = cur == mask_id
    masked_conf = torch.where(is_masked, conf, torch.full_like(conf, float("-inf")))
    _, top = masked_conf.topk(n_u)
    cur.scatter_(0, top, ids.gather(0, top))
    step_map.scatter_(0, top, torch.full_like(top, step))
    ppp.index_copy_(0, top, probs.index_select(0, top))
    return ids, conf


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_softmax_argmax_vs_torch_cpu(dtype):
    g = torch.Generator().manual_seed(3)
    l = (torch.randn(6, 3001, generator=g) * 3).to(dtype)
    ids, conf, probs = olog.softmax_argmax(l.float().numpy())
    rid, rconf, rprobs = _torch_epilogue(l)
    # torch.argmax takes the first maximum too; random bf16 rows may hold ties
    assert np.array_equal(ids, rid.numpy())
    np.testing.assert_allclose(conf, rconf.numpy(), rtol=2e-6)
    np.testing.assert_allclose(probs, rprobs.numpy(), rtol=2e-5, atol=1e-12)


def test_softmax_argmax_closed_forms():
    V = 1000
    uniform = np.full((1, V), 0.375, dtype=np.float32)
    ids, conf, probs = olog.softmax_argmax(uniform)
    assert ids[0] == 0 and conf[0] == pytest.approx(1.0 / V, rel=1e-12)
    ties = np.zeros((1, V), dtype=np.float32)
    ties[0, [700, 31, 402]] = 5.0
    ids, conf, _ = olog.softmax_argmax(ties)
    assert ids[0] == 31
    assert conf[0] == pytest.approx(np.exp(5.0) / (3 * np.exp(5.0) + V - 3), rel=1e-12)
    dom = np.zeros((1, V), dtype=np.float32)
    dom[0, 17] = 80.0
    ids, conf, _ = olog.softmax_argmax(dom)
    assert ids[0] == 17 and conf[0] == pytest.approx(1.0, abs=1e-30)
    neg = np.full((1, V), -np.inf, dtype=np.float32)
    neg[0, [5, 9]] = [1.0, 2.0]
    ids, conf, probs = olog.softmax_argmax(neg)
    assert ids[0] == 9 and probs[0, 0] == 0.0
    assert conf[0] == pytest.approx(np.exp(2.0) / (np.exp(1.0) + np.exp(2.0)), rel=1e-12)


@pytest.mark.parametrize("case", range(6))
def test_denoise_select_vs_torch_cpu(case):
    g = torch.Generator().manual_seed(100 + case)
    M, V, mask_id = [4, 4, 8, 16, 4, 32][case], 2000, 1999
    l = (torch.randn(M, V, generator=g) * 2).to(torch.bfloat16)
    cur = torch.randint(0, V - 1, (M,), generator=g)
    masked = torch.rand(M, generator=g) < 0.6
    masked[0] = True
    cur[masked] = mask_id
    n_masked = int(masked.sum())
    n_u = [1, n_masked, 2, 3, n_masked + 1 if n_masked < M else 1, 5][case]
    n_u = min(n_u, M)
    _, rconf, _ = _torch_epilogue(l)
    key = torch.where(cur == mask_id, rconf, torch.full_like(rconf, float("-inf")))
    finite = key[torch.isfinite(key)]
    assert finite.unique().numel() == finite.numel(), "tie-free case expected"
    if n_u > n_masked and M - n_masked > 1:
        pytest.skip("torch.topk order among -inf rows is unspecified")
    step_map = torch.full((M,), -1, dtype=torch.int64)
    ppp = torch.zeros(M, V)
    cur_ref = cur.clone()
    _torch_denoise(l, cur_ref, mask_id, n_u, 2, step_map, ppp)
    got_cur, got_sm, got_pp, _, _ = olog.denoise_select(
        l.float().numpy(), cur.numpy(), mask_id, n_u, 2, np.full(M, -1, dtype=np.int64), np.zeros((M, V)))
    assert np.array_equal(got_cur, cur_ref.numpy())
    assert np.array_equal(got_sm, step_map.numpy())
    np.testing.assert_allclose(got_pp, ppp.numpy(), rtol=2e-5, atol=1e-12)


def test_denoise_select_ties_and_fill():
    """Equal confidences go to the lower row; with fewer masked rows than
    n_unmask the rest come from the unmasked rows, lowest first."""
    V, mask_id = 50, 49
    l = np.zeros((4, V), dtype=np.float32)
    l[:, 3] = 4.0                                  # identical rows -> identical conf
    cur = np.array([mask_id, 7, mask_id, mask_id])
    got, _, _, ids, _ = olog.denoise_select(l, cur, mask_id, 2, 0)
    assert list(got) == [3, 7, 3, mask_id]
    got, _, _, _, _ = olog.denoise_select(l, np.array([7, mask_id, 8, 9]), mask_id, 3, 0)
    assert list(got) == [3, 3, 3, 9]


def test_planted_logits_mistakes_are_caught(monkeypatch):
    V = 1000
    ties = np.zeros((1, V), dtype=np.float32)
    ties[0, [700, 31, 402]] = 5.0
    # (1) last maximum instead of the first
    last = V - 1 - int(np.argmax(ties[0, ::-1]))
    assert last != 31
    # (2) conf = exp(max) unnormalised
    _, conf, _ = olog.softmax_argmax(ties)
    assert not np.isclose(np.exp(5.0), conf[0])
    # (3) a selection that ignores the mask picks an unmasked row
    g = torch.Generator().manual_seed(7)
    l = torch.randn(8, 300, generator=g) * 3
    _, rconf, _ = _torch_epilogue(l)
    cur = np.full(8, 299)
    best = int(torch.argmax(rconf))
    cur[best] = 5                                   # the most confident row is not masked
    got, _, _, _, _ = olog.denoise_select(l.numpy(), cur, 299, 1, 0)
    assert got[best] == 5 and (got != cur).sum() == 1
