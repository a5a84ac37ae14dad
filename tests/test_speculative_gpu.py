"""GPU tests of the speculative step: the block mask kernel equals the
oracle; the cached multi-block verify reproduces a full-sequence forward with
the reference's multi-block mask and equals an eager forward bit for bit;
every runner iteration's ids and acceptance equal the oracle's on the verify
logits it produced (tiny SDAR-like shapes and the SDAR-1.7B / SDAR-8B
benchmark shapes, with the extend in line, on a second stream and in the
optimistic pipelined mode)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import logits as olog
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
                                  (64, 64, 4, 4, 8, 6, [[5, 4, 3, 2, 1, 0, 0, 1]]),
                                  (20, 20, 12, 0, 4, 4, [[0, 1, 2, 3], [1, 0, 3, 2]]),
                                  (33, 40, 8, 4, 4, 4, [[2, 2, 0, 1]])])
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


@pytest.mark.parametrize("extra_blocks", [0, 2])
def test_cached_verify_equals_full_sequence_forward(extra_blocks):
    """The runner's verify -- cached context, the blocks the last acceptance
    committed folded in ahead of the K x (data, mask) rows, logits of the mask
    rows -- against one forward of the whole verify sequence with the
    multi-block mask on a fresh model of the same weights, and bit for bit
    against an eager forward of the same rows.  With ``extra_blocks`` two
    more committed blocks (fixed ids) join the last acceptance's, so several
    blocks are folded in at once (block-causal among themselves, as the
    reference flushes them one at a time)."""
    from kernels.logits_fused import softmax_argmax
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
    for b in range(extra_blocks):                       # more committed blocks, not yet in the target cache
        blk = [(97 * b + 13 * j) % (V - 1) for j in range(4)]
        runner._pending.append(blk)
        runner.history.extend(blk)
        runner.ctx += 4
        runner.last_block = torch.tensor(blk, dtype=torch.int64, device=DEV)
    ctx = runner.ctx
    n_folded = len(runner._pending)
    assert n_folded >= 1 + extra_blocks
    runner.draft_blocks_()
    tgt = runner.verify_().clone()
    torch.cuda.synchronize()
    g = runner.last_verify_graph
    c, bound = runner._verify_key
    assert c == n_folded and g.ids.numel() == 4 * c + 32
    logits_v = target.forward(g.ids, g.pos, g.slots, g.mask, valid_len=bound, valid_len_dev=g.valid,
                              head_rows=g.head_rows)
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
    ref = logits[ctx:].float().view(4, 2, 4, V)[:, 1].reshape(16, V)       # the mask rows
    err = float((logits_v.float() - ref).abs().max())
    # a fresh model's full-sequence forward runs other attention forms and row
    # counts (other reduction orders): equal within the bf16 rounding of 2 x 36
    # projections, not bit for bit
    assert err <= 0.02 * float(ref.abs().max()) + 1e-2, err
    # the verify graph against an eager forward of the same rows and bound: the
    # kernels are deterministic, so logits and ids are identical
    graph_logits = runner.last_verify_logits
    assert torch.equal(graph_logits, logits_v)
    am, _conf = softmax_argmax(logits_v)
    assert torch.equal(am.view(4, 4), tgt)


def check_iteration(runner, gen, n_acc, ctx0, hist0):
    """One runner iteration against the oracle: the verify's mask-row ids are
    the oracle's softmax argmax of the verify logits it produced, and the
    committed blocks, generated tokens and accepted count are the oracle's
    greedy acceptance (speculative_decode.py:895-953) of the drafts it
    checked against those ids."""
    K, bl = runner.K, runner.bl
    mask_rows = runner.last_verify_logits.float().cpu().numpy()       # [K * bl, V]: the mask rows
    assert mask_rows.shape[0] == K * bl
    ids, _, _ = olog.softmax_argmax(mask_rows)
    ids = ids.reshape(K, bl)
    graph_ids = runner.last_verify_ids.cpu().numpy()
    assert np.array_equal(graph_ids, ids)
    drafts = runner.last_verify_drafts.cpu().tolist()
    committed, generated, acc = over.accept_blocks(drafts, ids.tolist(), bl)
    assert gen == generated and n_acc == acc
    assert runner.ctx - ctx0 == bl * len(committed)
    assert runner.history_ids()[len(hist0):] == [t for b in committed for t in b]
    assert all(len(b) == bl for b in committed)


def test_runner_iterations():
    from speculative.step import SpecRunner
    draft, target, shape = _models(seed=7)
    V = shape.vocab
    runner = SpecRunner(draft, target, mask_token_id=V - 1)
    prompt = torch.randint(0, V - 1, (40,), generator=torch.Generator().manual_seed(1))
    runner.prefill(prompt)
    for it in range(5):
        ctx0, hist0 = runner.ctx, runner.history_ids()
        gen, n_acc = runner.step()
        assert 1 <= len(gen) <= 16 and 0 <= n_acc <= 16
        assert runner.ctx > ctx0 and (runner.ctx - ctx0) % 4 == 0
        assert V - 1 not in gen
        assert (runner.draft_blocks != V - 1).all()      # every position unmasked
        assert (runner.step_maps >= 0).all()
        check_iteration(runner, gen, n_acc, ctx0, hist0)
    # the step maps are permutations of the schedule's steps
    for row in runner.step_maps.cpu().tolist():
        assert sorted(row) == [0, 1, 2, 3]


def _run(pipelined, draft_seed, target_seed, iters=6, prompt_seed=2, fold=True, overlap=True):
    from speculative.model import ModelShape, SynthModel
    from speculative.step import SpecRunner
    shape = ModelShape(**TINY)
    draft = SynthModel(shape, DEV, draft_seed, 256, 64)
    target = SynthModel(shape, DEV, target_seed, 256, 64)
    runner = SpecRunner(draft, target, mask_token_id=shape.vocab - 1, pipelined=pipelined, fold=fold,
                        overlap=overlap)
    prompt = torch.randint(0, shape.vocab - 1, (32,), generator=torch.Generator().manual_seed(prompt_seed))
    runner.prefill(prompt)
    out = []
    for _ in range(iters):
        ctx0, hist0 = runner.ctx, runner.history_ids()
        gen, n_acc = runner.step()
        check_iteration(runner, gen, n_acc, ctx0, hist0)
        out.append((gen, n_acc))
    runner.finish()
    torch.cuda.synchronize()
    return out, runner


@pytest.mark.parametrize("same_weights", [True, False])
def test_pipelined_equals_sequential(same_weights):
    """The optimistic two-stream mode (the next iteration's drafts run beside
    the verify) commits exactly the tokens of the sequential runner, both when
    its drafts are used (draft = target weights: every block accepted) and
    when they are dropped (independent weights: rollback and redraft); every
    iteration of both equals the oracle's acceptance of its verify logits."""
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


def test_separate_extend_modes_agree():
    """The reference's separate extend of the committed blocks (fold=False), in
    line and on a second stream, commits the same tokens either way, with
    every iteration equal to the oracle's acceptance; with equal weights it
    extends four accepted blocks at once (block-causal among themselves)."""
    for ts in (5, 6):
        inline, r_in = _run(False, 5, ts, fold=False, overlap=False)
        side, r_side = _run(False, 5, ts, fold=False, overlap=True)
        assert inline == side and r_in.history_ids() == r_side.history_ids()


def test_speculative_step_at_sdar_shapes():
    """The end-to-end step at its benchmark shapes: random-init SDAR-1.7B
    draft and SDAR-8B target on one GPU, a 512-token prompt, 4-token blocks,
    4 denoise steps, 4 blocks per verify.  Three iterations each with the
    committed blocks folded into the next verify (the default), with the
    reference's separate extend in line and on a second stream, and in the
    optimistic pipelined mode: every iteration matches the oracle's argmax and
    acceptance on its own verify logits and commits whole blocks without the
    mask id.  Modes that run the same kernels on the same rows (folded and
    pipelined; extend in line and on a second stream) commit the same tokens;
    the folded and extend forms write the committed blocks' K/V from forwards
    of different row counts (other reduction orders), so their logits agree
    within bf16 rounding, not bit for bit, and their tokens are compared per
    iteration against the oracle instead."""
    from speculative.model import DRAFT_1P7B, TARGET_8B, SynthModel
    from speculative.step import SpecRunner
    from speculative.verify import MASK_TOKEN_ID
    print("sdar shapes: building the 1.7B draft and 8B target", flush=True)
    max_ctx = 512 + 16 * 8 + 64
    draft = SynthModel(DRAFT_1P7B, DEV, seed=11, max_ctx=max_ctx, max_rows=64)
    target = SynthModel(TARGET_8B, DEV, seed=12, max_ctx=max_ctx, max_rows=64)
    prompt = torch.randint(0, DRAFT_1P7B.vocab - 1, (512,), generator=torch.Generator().manual_seed(5))
    histories = {}
    try:
        for mode in ("fold", "inline", "overlap", "pipelined"):
            print(f"sdar shapes: mode {mode}", flush=True)
            runner = SpecRunner(draft, target, overlap=mode != "inline", pipelined=mode == "pipelined",
                                fold=mode in ("fold", "pipelined"))
            runner.prefill(prompt)
            for it in range(3):
                ctx0, hist0 = runner.ctx, runner.history_ids()
                gen, n_acc = runner.step()
                print(f"sdar shapes: {mode} iteration {it}: {len(gen)} tokens, {n_acc} accepted", flush=True)
                assert MASK_TOKEN_ID not in gen
                assert (runner.draft_blocks != MASK_TOKEN_ID).all()
                for row in runner.step_maps.cpu().tolist():
                    assert sorted(row) == [0, 1, 2, 3]
                check_iteration(runner, gen, n_acc, ctx0, hist0)
            runner.finish()
            torch.cuda.synchronize()
            histories[mode] = runner.history_ids()
    finally:
        del draft, target
        torch.cuda.empty_cache()
    assert histories["overlap"] == histories["inline"]
    assert histories["pipelined"] == histories["fold"]
