"""Greedy acceptance of K verified draft blocks, as the runner applies it on
the host after its one synchronisation per iteration.

Semantics of the reference's greedy branch (speculative_decoding/
speculative_decode.py:895-953 with mrs.py:111-146 greedy_match_verify and
partial_block_fill = "draft_argmax"): blocks are checked in order; inside a
block, draft tokens are accepted while they equal the target's argmax at
their position; the first mismatch contributes the target's token as the
bonus, the rest of that block is filled with the draft's own tokens, and no
later block is looked at.  A block whose committed-from ids (accepted drafts
and bonus) hold an end-of-sequence id also ends the loop (:944-950); the
runner passes none, as the reference's fixed-length benchmark mode
``--no_eos_stop`` does (:1007).

The verify sequence itself is never built on the host: the cached forward's
rows are the K draft blocks (data, mask) over the committed slots, and
``kernels.attention_fused.block_mask`` writes their mask rows on the GPU from
the step maps.
"""
from __future__ import annotations

MASK_TOKEN_ID = 151669


def accept_blocks(draft_blocks, target_ids, block_length, eos_ids=None):
    """-> (committed blocks, generated tokens, accepted draft count).

    ``draft_blocks`` and ``target_ids`` are K lists of ``block_length`` ids
    (the drafts and the target's argmax at the mask rows of each block).
    Every committed block is ``block_length`` long; ``generated`` is the
    accepted drafts plus the bonus token of the first rejected block.
    ``eos_ids``: end-of-sequence ids; the block that generates one is the
    last committed.
    """
    stop_ids = frozenset(eos_ids or ())
    committed, generated, n_acc = [], [], 0
    for draft, target in zip(draft_blocks, target_ids):
        draft, target = list(draft), list(target)
        agree = next((i for i, (d, t) in enumerate(zip(draft, target)) if d != t), len(draft))
        n_acc += agree
        if agree == len(draft):
            committed.append(draft[:block_length])
            generated.extend(draft)
            if stop_ids.isdisjoint(draft):
                continue
            break
        fixed = draft[:agree] + [target[agree]]
        generated.extend(fixed)
        committed.append((fixed + draft[agree + 1:])[:block_length])
        break
    return committed, generated, n_acc
