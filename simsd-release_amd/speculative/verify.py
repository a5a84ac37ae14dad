"""Multi-block verify: the sequence layout, the cached-forward mask and greedy
acceptance (speculative_decoding/verify.py:350-418, sdar/new_attn_multi_block.py:
22-183, speculative_decoding/mrs.py:111-146, speculative_decode.py:895-953).

``build_verify_sequence_multi`` and ``greedy_match_verify`` keep the
reference's signatures.  The cached forward does not materialise the full
[prompt | accepted | drafts] sequence: its rows are the K draft blocks (data,
mask) over the cache's committed slots, and ``kernels.attention_fused.
block_mask`` writes their mask rows on the GPU from the step maps.
"""
from __future__ import annotations

import torch

MASK_TOKEN_ID = 151669


def build_verify_sequence_multi(prompt_ids, accepted_blocks, draft_blocks, step_maps, block_length, block_size,
                                mask_token_id=MASK_TOKEN_ID, share_mask_position: bool = True):
    """[Prompt | Acc_0 data | ... | Draft_0 data, Draft_0 mask | ...]:
    -> (input_ids, token_labels, block_ids, labels, position_ids) lists.
    Token labels: 0 prompt, 1 accepted data, step + 1 draft data (block_size + 1
    when never drafted), block_size + 1 mask; mask positions repeat the data
    positions unless ``share_mask_position`` is False."""
    if len(draft_blocks) != len(step_maps) or not draft_blocks:
        raise ValueError("need one step map per draft block, at least one block")
    input_ids = list(prompt_ids)
    token_labels = [0] * len(input_ids)
    block_ids = [-1] * len(input_ids)
    labels = [-100] * len(input_ids)
    position_ids = list(range(len(input_ids)))
    cur = len(input_ids)
    for b, blk in enumerate(accepted_blocks):
        n = len(blk)
        input_ids.extend(blk)
        token_labels.extend([1] * n)
        block_ids.extend([b] * n)
        labels.extend([-100] * n)
        position_ids.extend(range(cur, cur + n))
        cur += n
    n_acc = len(accepted_blocks)
    for k, (draft, steps) in enumerate(zip(draft_blocks, step_maps)):
        data_pos = list(range(cur, cur + block_length))
        cur += block_length
        input_ids.extend(draft)
        token_labels.extend(s + 1 if s >= 0 else block_size + 1 for s in steps)
        block_ids.extend([n_acc + k] * block_length)
        labels.extend([-100] * block_length)
        position_ids.extend(data_pos)
        if share_mask_position:
            mask_pos = data_pos
        else:
            mask_pos = list(range(cur, cur + block_length))
            cur += block_length
        input_ids.extend([mask_token_id] * block_length)
        token_labels.extend([block_size + 1] * block_length)
        block_ids.extend([n_acc + k] * block_length)
        labels.extend(draft)
        position_ids.extend(mask_pos)
    return input_ids, token_labels, block_ids, labels, position_ids


def greedy_match_verify(draft_ids, draft_probs, target_probs, step_map, verify_order_mode="position"):
    """Accept draft[pos] while it equals argmax(target_probs[pos]); at the first
    mismatch commit the target's argmax as the bonus and stop.
    ``target_probs`` may be the [bl, V] probabilities or the [bl] argmax ids.
    -> (accepted_ids, n_accepted, bonus_token or None)."""
    if verify_order_mode != "position":
        raise ValueError("greedy_match_verify only supports verify_order_mode='position' "
                         f"(got {verify_order_mode!r})")
    if isinstance(target_probs, torch.Tensor) and target_probs.ndim == 2:
        target_argmax = target_probs.argmax(dim=-1).tolist()
    elif isinstance(target_probs, torch.Tensor):
        target_argmax = target_probs.tolist()
    else:
        target_argmax = list(target_probs)
    for pos, d in enumerate(draft_ids):
        if d != target_argmax[pos]:
            return list(draft_ids[:pos]) + [target_argmax[pos]], pos, target_argmax[pos]
    return list(draft_ids), len(draft_ids), None


def accept_blocks(draft_blocks, target_ids, block_length):
    """Greedy acceptance across K blocks with first-reject truncation
    (speculative_decode.py:895-953, greedy branch, partial_block_fill =
    "draft_argmax"): -> (committed blocks, generated tokens, accepted count).
    A rejected block is committed padded with the draft's own remaining tokens
    and ends the iteration."""
    committed, generated, n_acc = [], [], 0
    for k, draft in enumerate(draft_blocks):
        final, n, bonus = greedy_match_verify(draft, None, target_ids[k], None)
        n_acc += n
        block = list(final)
        if len(block) < block_length:
            block += list(draft[len(block):block_length])
        committed.append(block)
        generated.extend(final)
        if n < block_length:
            break
    return committed, generated, n_acc
