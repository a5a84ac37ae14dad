"""GPU parity of the lm_head epilogue (MI355X): softmax statistics, argmax and
the draft's unmasking step (speculative_decoding/cache_aware.py:914-938,
1197-1198) against the oracle on the same logits.

ids and every integer side effect (cur_ids, step_map) are bit-exact; conf and
probs are fp32 softmax values within rtol 1e-5 of the fp64 oracle.  Cases:
the deployed vocabulary (151936) at the draft's 4 rows and the verify pass's
16/32 rows, small and ragged vocabularies, bf16/fp16/fp32, repeated maxima
placed in different workgroups' slices, -inf entries and an all -inf row,
strided rows, bitwise determinism, graph capture with replays, and the
lm_head chained in front (exact small-integer logits pin the argmax through
the linear).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import logits as olog
from oracle import thin_linear as othin

pytestmark = pytest.mark.gpu
DEV = "cuda"
VOCAB = 151936


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def rnd(*shape, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def check_rows(logits, ids, conf, probs=None):
    rid, rconf, rprobs = olog.softmax_argmax(logits.float().cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_allclose(conf.cpu().numpy(), rconf, rtol=1e-5, atol=0)
    if probs is not None:
        np.testing.assert_allclose(probs.cpu().numpy(), rprobs, rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("M,V", [(4, VOCAB), (16, VOCAB), (32, VOCAB), (1, 1), (3, 7), (5, 2049), (2, 300001)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_softmax_argmax_vs_oracle(M, V, dtype):
    from kernels.logits_fused import softmax_argmax
    print(f"softmax_argmax M={M} V={V} {dtype}", flush=True)
    l = rnd(M, V, dtype=dtype, scale=3.0, seed=M * 7 + V % 97)
    with torch.inference_mode():
        ids, conf, probs = softmax_argmax(l, return_probs=True)
    torch.cuda.synchronize()
    assert ids.dtype == torch.int64 and conf.dtype == torch.float32 and probs.shape == (M, V)
    check_rows(l, ids, conf, probs if V <= VOCAB else None)
    # the probabilities agree with torch's own softmax on the device
    ref = torch.softmax(l.float(), dim=-1)
    torch.testing.assert_close(probs, ref, rtol=1e-5, atol=1e-30)
    assert torch.equal(ids, ref.argmax(dim=-1))


def test_repeated_maxima_first_index():
    """Equal maxima in different slices (and inside one slice): the first wins."""
    from kernels.logits_fused import softmax_argmax
    M, V = 6, VOCAB
    l = rnd(M, V, scale=1.0, seed=3)
    spots = [[150000, 3, 77777], [2047, 2048], [151935, 151934], [0, 151935], [4096, 4095, 60000], [12345]]
    for m, pos in enumerate(spots):
        l[m, pos] = 9.0
    with torch.inference_mode():
        ids, conf = softmax_argmax(l)
    assert ids.tolist() == [min(p) for p in spots]
    check_rows(l, ids, conf)


def test_infinities():
    from kernels.logits_fused import softmax_argmax
    V = 5000
    l = torch.full((3, V), float("-inf"), device=DEV)
    l[0, [10, 4000]] = torch.tensor([1.0, 2.0], device=DEV)
    l[1] = rnd(V, dtype=torch.float32, seed=9)
    l[1, ::3] = float("-inf")
    with torch.inference_mode():
        ids, conf, probs = softmax_argmax(l, return_probs=True)
    ref = torch.softmax(l, dim=-1)
    assert ids[0].item() == 4000 and ids[1].item() == int(ref[1].argmax())
    torch.testing.assert_close(conf[:2], ref[:2].max(dim=-1).values, rtol=1e-5, atol=0)
    assert probs[0, 10].item() == pytest.approx(ref[0, 10].item(), rel=1e-5) and probs[0, 11].item() == 0.0
    # all -inf: id 0 and NaN confidence, as torch's softmax gives NaN rows
    assert ids[2].item() == 0 and torch.isnan(conf[2]) and torch.isnan(ref[2]).all()


def test_strided_rows_and_determinism():
    from kernels.logits_fused import softmax_argmax
    wide = rnd(8, VOCAB + 64, scale=2.0, seed=11)
    view = wide[:, 32:32 + VOCAB]
    with torch.inference_mode():
        a = softmax_argmax(view, return_probs=True)
        b = softmax_argmax(view.contiguous(), return_probs=True)
        c = softmax_argmax(view, return_probs=True)
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)
    check_rows(view, a[0], a[1])


def _denoise_case(M, V, seed, mask_frac=0.6):
    g = torch.Generator().manual_seed(seed)
    mask_id = V - 1
    cur = torch.randint(0, V - 1, (M,), generator=g)
    masked = torch.rand(M, generator=g) < mask_frac
    masked[0] = True
    cur[masked] = mask_id
    return cur, mask_id, int(masked.sum())


@pytest.mark.parametrize("M,V,n_u,seed", [(4, VOCAB, 1, 0), (4, VOCAB, 4, 1), (8, 5000, 3, 2),
                                          (16, VOCAB, 2, 3), (32, 3001, 7, 4), (64, 1000, 11, 5),
                                          (4, VOCAB, 0, 6)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_denoise_select_vs_oracle(M, V, n_u, seed, dtype):
    from kernels.logits_fused import denoise_select
    print(f"denoise_select M={M} V={V} n_u={n_u} {dtype}", flush=True)
    l = rnd(M, V, dtype=dtype, scale=2.0, seed=seed)
    cur, mask_id, n_masked = _denoise_case(M, V, seed)
    n_u = min(n_u, n_masked)
    step_map = torch.full((M,), -1, dtype=torch.int64)
    ppp = torch.zeros(M, V)
    exp_cur, exp_sm, exp_pp, exp_ids, exp_conf = olog.denoise_select(
        l.float().cpu().numpy(), cur.numpy(), mask_id, n_u, 3, step_map.numpy(), ppp.numpy())
    cur_d, sm_d, pp_d = cur.to(DEV), step_map.to(DEV), ppp.to(DEV)
    with torch.inference_mode():
        ids, conf = denoise_select(l, cur_d, mask_id, n_u, step=3, step_map=sm_d, per_pos_probs=pp_d)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), exp_ids)
    np.testing.assert_allclose(conf.cpu().numpy(), exp_conf, rtol=1e-5)
    assert np.array_equal(cur_d.cpu().numpy(), exp_cur)
    assert np.array_equal(sm_d.cpu().numpy(), exp_sm)
    np.testing.assert_allclose(pp_d.cpu().numpy(), exp_pp, rtol=1e-5, atol=1e-30)
    assert int((cur_d.cpu() != cur).sum()) <= n_u


def test_denoise_select_ties_fill_and_optional_outputs():
    from kernels.logits_fused import denoise_select
    V, mask_id = 4096, 4095
    l = torch.zeros(4, V, device=DEV, dtype=torch.bfloat16)
    l[:, 3] = 4.0
    cur = torch.tensor([mask_id, 7, mask_id, mask_id], device=DEV)
    with torch.inference_mode():
        denoise_select(l, cur, mask_id, 2)
    assert cur.tolist() == [3, 7, 3, mask_id]
    cur = torch.tensor([7, mask_id, 8, 9], device=DEV)
    with torch.inference_mode():
        denoise_select(l, cur, mask_id, 3)
    assert cur.tolist() == [3, 3, 3, 9]


def test_denoise_select_errors():
    from kernels.logits_fused import denoise_select, softmax_argmax
    l = rnd(65, 100)
    with pytest.raises(ValueError):
        denoise_select(l, torch.zeros(65, dtype=torch.int64, device=DEV), 99, 1)
    l = rnd(4, 100)
    with pytest.raises(ValueError):
        denoise_select(l, torch.zeros(4, dtype=torch.int64, device=DEV), 99, 5)
    with pytest.raises(ValueError):
        denoise_select(l, torch.zeros(4, dtype=torch.int32, device=DEV), 99, 1)
    with pytest.raises(TypeError):
        softmax_argmax(l.to(torch.float64))
    ids, conf = softmax_argmax(rnd(0, 100))
    assert ids.shape == (0,) and conf.shape == (0,)


def test_graph_capture_replays():
    """Both calls captured once, replayed on new logits with the program's own
    eager work between replays; every replay equals the eager result."""
    from kernels.logits_fused import denoise_select, softmax_argmax
    M, V, mask_id = 4, VOCAB, VOCAB - 1
    l_static = rnd(M, V, seed=20)
    cur0 = torch.tensor([mask_id, 5, mask_id, mask_id], device=DEV)
    cur = cur0.clone()
    sm = torch.full((M,), -1, dtype=torch.int64, device=DEV)
    pp = torch.zeros(M, V, device=DEV)
    with torch.inference_mode():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            softmax_argmax(l_static, return_probs=True)
            denoise_select(l_static, cur, mask_id, 2, 1, sm, pp)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = softmax_argmax(l_static, return_probs=True)
            sel = denoise_select(l_static, cur, mask_id, 2, 1, sm, pp)
        for r in range(3):
            l_static.copy_(rnd(M, V, seed=30 + r))
            cur.copy_(cur0)
            sm.fill_(-1)
            pp.zero_()
            g.replay()
            torch.cuda.synchronize()
            cur_e, sm_e, pp_e = cur0.clone(), torch.full_like(sm, -1), torch.zeros_like(pp)
            ref = softmax_argmax(l_static, return_probs=True)
            ref_sel = denoise_select(l_static, cur_e, mask_id, 2, 1, sm_e, pp_e)
            torch.cuda.synchronize()
            for a, b in zip(out, ref):
                assert torch.equal(a, b)
            for a, b in zip(sel, ref_sel):
                assert torch.equal(a, b)
            assert torch.equal(cur, cur_e) and torch.equal(sm, sm_e) and torch.equal(pp, pp_e)


def test_lm_head_argmax_exact_integer_logits():
    """Small-integer x and w make every logit exact, so the argmax through the
    lm_head is pinned bit-exactly by the oracle linear; ties included."""
    from kernels.logits_fused import lm_head_argmax
    g = torch.Generator().manual_seed(5)
    M, K, V = 4, 2048, VOCAB
    x = torch.randint(-2, 3, (M, K), generator=g).float()
    w = torch.randint(-2, 3, (V, K), generator=g, dtype=torch.int8).float()
    w[100] = w[40000]            # an exact tie between two vocabulary rows
    logits = othin.linear_exact(x.numpy(), w.numpy(), dtype="bf16")
    rid, rconf, _ = olog.softmax_argmax(logits)
    with torch.inference_mode():
        ids, conf = lm_head_argmax(x.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16))
    assert np.array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_allclose(conf.cpu().numpy(), rconf, rtol=1e-5)


def test_lm_head_argmax_deployed_shapes():
    from kernels.logits_fused import lm_head_argmax
    from kernels.thin_linear_fused import thin_linear
    for M, K in [(4, 2048), (32, 4096)]:
        x = rnd(M, K, seed=M)
        w = rnd(VOCAB, K, scale=0.02, seed=K)
        with torch.inference_mode():
            ids, conf, probs = lm_head_argmax(x, w, return_probs=True)
            logits = thin_linear(x, w)
        ref = torch.softmax(logits.float(), dim=-1)
        assert torch.equal(ids, ref.argmax(dim=-1))
        torch.testing.assert_close(probs, ref, rtol=1e-5, atol=1e-30)
        del w
