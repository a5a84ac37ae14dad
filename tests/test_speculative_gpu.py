"""GPU tests of the speculative step (tiny SDAR-like shapes): the cached
multi-block verify reproduces a full-sequence forward with the reference's
multi-block mask, the block mask kernel equals the oracle, and the runner's
iterations commit whole blocks, never commit mask ids, and advance the
context."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import verify as over

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


TINY = dict(hidden=256, n_layers=2, n_q_heads=2, n_kv_heads=1, intermediate=512, vocab=1000)


@pytest.mark.parametrize("case", [(0, 0, 0, 1, 4, 4, [[0, 1, 2, 3]]),
                                  (37, 40, 4, 4, 4, 4, []),
                                  (100, 100, 0, 0, 4, 4, [[3, 0, 2, 1], [0, 1, 2, 3], [1, 3, 0, 2], [2, 2, 1, 0]]),
                                  (9, 12, 4, 0, 2, 2, [[1, 0], [0, -1], [-1, -1]]),
                                  (64, 64, 4, 4, 8, 6, [[5, 4, 3, 2, 1, 0, 0, 1]])])
def test_block_mask_vs_oracle(case):
    from kernels.attention_fused import block_mask
    ctx, s0, n_prefix, n_free, bl, bs, steps = case
    n_cols = s0 + n_prefix + n_free + 2 * len(steps) * bl + 5
    sm = torch.tensor(steps, dtype=torch.int64, device=DEV).view(len(steps), bl) if steps else None
    got = block_mask(n_cols, ctx, s0, n_prefix, n_free, sm, bl, bs, device=DEV)
    want = over.cached_block_mask(ctx, s0, n_cols, n_prefix, n_free, steps, bl, bs)
    assert np.array_equal(got.cpu().numpy(), want)


def _models(seed=3, max_ctx=256):
    from speculative.model import ModelShape, SynthModel
    shape = ModelShape(**TINY)
    return (SynthModel(shape, DEV, seed, max_ctx, 64), SynthModel(shape, DEV, seed + 1, max_ctx, 64),
            shape)


def test_cached_verify_equals_full_sequence_forward():
    """The runner's verify (cached context, K x (data, mask) rows) against one
    forward of the whole verify sequence with the multi-block mask on a fresh
    model of the same weights."""
    from speculative.model import ModelShape, SynthModel
    from speculative.step import SpecRunner
    draft, target, shape = _models()
    V = shape.vocab
    runner = SpecRunner(draft, target, mask_token_id=V - 1)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, V - 1, (32,), generator=g)
    runner.prefill(prompt)
    for _ in range(2):                                  # grow the context past the prompt
        runner.step()
    ctx = runner.ctx
    runner.draft_blocks_()
    tgt = runner.verify_()
    g = runner._vg
    logits_v = target.forward(g.ids, g.pos, g.slots, g.mask, valid_len=target.cache.full_len,
                              valid_len_dev=g.valid)
    # the same sequence in full: prompt + committed blocks + the drafts
    drafts = runner.draft_blocks.cpu().tolist()
    steps = runner.step_maps.cpu().tolist()
    hist = runner.history_ids()
    assert len(hist) == ctx
    acc_blocks = [hist[i:i + 4] for i in range(32, ctx, 4)]
    ids, tl, bi, _, pos = over.build_verify_sequence_multi(prompt.tolist(), acc_blocks, drafts, steps, 4, 4, V - 1)
    mask = torch.from_numpy(over.multi_block_causal_mask(tl, bi, 4)).to(DEV)
    fresh = SynthModel(shape, DEV, 4, 256, 64)          # seed + 1 of _models(): the target's weights
    n = len(ids)
    full_mask = torch.zeros(n, fresh.cache.full_len, dtype=torch.bool, device=DEV)
    full_mask[:, :n] = mask
    ar = torch.arange(n, device=DEV)
    logits = fresh.forward(torch.tensor(ids, device=DEV), torch.tensor(pos, device=DEV), ar, full_mask,
                           valid_len=n)
    ref = logits[ctx:].float()
    err = float((logits_v.float() - ref).abs().max())
    assert err <= 0.02 * float(ref.abs().max()) + 1e-2, err
    # the graph's argmax of the mask rows equals the eager logits' argmax where no near-tie exists
    am = logits_v.float().argmax(-1).view(4, 2, 4)[:, 1]
    assert (am.cpu() == tgt.cpu()).float().mean() >= 0.9


def test_runner_iterations():
    from speculative.step import SpecRunner
    draft, target, shape = _models(seed=7)
    V = shape.vocab
    runner = SpecRunner(draft, target, mask_token_id=V - 1)
    prompt = torch.randint(0, V - 1, (40,), generator=torch.Generator().manual_seed(1))
    runner.prefill(prompt)
    for it in range(5):
        ctx0 = runner.ctx
        gen, n_acc = runner.step()
        assert 1 <= len(gen) <= 16 and 0 <= n_acc <= 16
        assert runner.ctx > ctx0 and (runner.ctx - ctx0) % 4 == 0
        assert V - 1 not in gen
        assert (runner.draft_blocks != V - 1).all()      # every position unmasked
        assert (runner.step_maps >= 0).all()
    # the step maps are permutations of the schedule's steps
    for row in runner.step_maps.cpu().tolist():
        assert sorted(row) == [0, 1, 2, 3]


def _run(pipelined, draft_seed, target_seed, iters=6, prompt_seed=2):
    from speculative.model import ModelShape, SynthModel
    from speculative.step import SpecRunner
    shape = ModelShape(**TINY)
    draft = SynthModel(shape, DEV, draft_seed, 256, 64)
    target = SynthModel(shape, DEV, target_seed, 256, 64)
    runner = SpecRunner(draft, target, mask_token_id=shape.vocab - 1, pipelined=pipelined)
    prompt = torch.randint(0, shape.vocab - 1, (32,), generator=torch.Generator().manual_seed(prompt_seed))
    runner.prefill(prompt)
    out = [runner.step() for _ in range(iters)]
    runner.finish()
    torch.cuda.synchronize()
    return out, runner


@pytest.mark.parametrize("same_weights", [True, False])
def test_pipelined_equals_sequential(same_weights):
    """The optimistic two-stream mode (the next iteration's drafts run beside
    the verify) commits exactly the tokens of the sequential runner, both when
    its drafts are used (draft = target weights: every block accepted) and
    when they are dropped (independent weights: rollback and redraft)."""
    ts = 5 if same_weights else 6
    seq, r_seq = _run(False, 5, ts)
    pip, r_pip = _run(True, 5, ts)
    assert pip == seq
    assert r_pip.history_ids() == r_seq.history_ids()
    assert r_pip.ctx == r_seq.ctx
    used, dropped = r_pip.stats["optimistic_used"], r_pip.stats["optimistic_dropped"]
    assert used + dropped == len(seq)
    if same_weights:
        assert used >= 1, r_pip.stats
    else:
        assert dropped >= 1, r_pip.stats
