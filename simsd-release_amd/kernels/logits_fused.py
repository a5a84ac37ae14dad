"""The lm_head epilogue on MI355X: softmax statistics, argmax and the draft's
unmasking step over logits rows, in three small launches.

The reference runs these as a chain of torch ops after every lm_head call:

* the draft's block denoise body, speculative_decoding/cache_aware.py:914-938::

      probs = F.softmax(logits.float(), dim=-1)
      pred_ids = probs.argmax(dim=-1)
      confidence = probs.gather(1, pred_ids.unsqueeze(-1)).squeeze(-1)
      masked_conf = torch.where(cur_ids == mask_token_id, confidence, -inf)
      _, top_pos = masked_conf.topk(n_u)
      cur_ids.scatter_(0, top_pos, pred_ids.gather(0, top_pos))
      step_map.scatter_(0, top_pos, step_i)
      per_pos_probs.index_copy_(0, top_pos, probs.index_select(0, top_pos))

  -> ``denoise_select``;
* the target verify pass, cache_aware.py:1197-1198,
  ``target_probs = F.softmax(mask_logits.float(), dim=-1)`` (and greedy
  acceptance reads its argmax) -> ``softmax_argmax(..., return_probs=True)``.

``lm_head_argmax`` chains the skinny lm_head linear with it.

Semantics: ids are the first index of the row maximum (torch.argmax); conf is
the softmax probability of that entry, 1 / sum(exp(l - max)); probs rows are
exp(l - max) / sum in fp32.  The unmasking choice takes, among rows whose
current id is the mask id, the n_unmask largest conf, equal values going to
the lower row (torch.topk leaves that order open); rows that are not masked
rank as -inf and so are only taken when fewer than n_unmask rows are masked,
as in the reference.  All sums run in a fixed order (bit-reproducible); no
host sync, so the calls capture into a HIP graph.  NaN logits give
unspecified ids.
"""
from __future__ import annotations

import torch

from . import _native
from .thin_linear_fused import thin_linear

MAX_SELECT_ROWS = 64


def _rows(logits: torch.Tensor, what: str) -> tuple[torch.Tensor, int]:
    if logits.ndim != 2:
        raise ValueError(f"{what}: logits must be 2-D [rows, vocab], got {tuple(logits.shape)}")
    code = _native.DTYPE_CODES.get(logits.dtype)
    if code is None:
        raise TypeError(f"{what}: unsupported dtype {logits.dtype} (bf16, fp16 or fp32)")
    if logits.shape[1] == 0:
        raise ValueError(f"{what}: empty vocabulary")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    return logits, code


def _workspace(dev: torch.device, M: int, V: int) -> torch.Tensor:
    need = _native.lib().simsd_softmax_argmax_workspace_bytes(M, V)
    if need < 0:
        raise ValueError(f"bad logits shape [{M}, {V}]")
    return torch.empty(max(need, 256), device=dev, dtype=torch.uint8)


def softmax_argmax(logits: torch.Tensor, return_probs: bool = False):
    """ids = softmax(logits.float()).argmax(-1), conf = the probability at ids,
    and (``return_probs``) the fp32 softmax rows.

    logits: [M, V] bf16 / fp16 / fp32 (unit stride along V).
    -> (ids int64 [M], conf fp32 [M]) or (ids, conf, probs fp32 [M, V]).
    """
    logits, code = _rows(logits, "softmax_argmax")
    M, V = logits.shape
    dev = _native.require_device(logits)
    ids = torch.empty(M, device=dev, dtype=torch.int64)
    conf = torch.empty(M, device=dev, dtype=torch.float32)
    probs = torch.empty((M, V), device=dev, dtype=torch.float32) if return_probs else None
    if M > 0:
        ws = _workspace(dev, M, V)
        with _native.device_guard(dev):
            status = _native.lib().simsd_softmax_argmax(
                logits.data_ptr(), logits.stride(0), M, V, code, ids.data_ptr(), conf.data_ptr(),
                probs.data_ptr() if probs is not None else None, V if probs is not None else 0,
                ws.data_ptr(), ws.numel(), _native.stream_of(dev))
        _native.check(status, "softmax_argmax")
    return (ids, conf, probs) if return_probs else (ids, conf)


def denoise_select(logits: torch.Tensor, cur_ids: torch.Tensor, mask_token_id: int, n_unmask: int,
                   step: int = 0, step_map: torch.Tensor | None = None,
                   per_pos_probs: torch.Tensor | None = None):
    """One unmasking step of the draft's block denoise loop, in place.

    logits:        [M, V] lm_head output for the block's M <= 64 positions;
    cur_ids:       int64 [M] current ids of the block (unit stride; updated);
    step_map:      int64 [M] or None; rows unmasked now get ``step``;
    per_pos_probs: fp32 [M, V] or None; rows unmasked now get their softmax row.
    -> (pred_ids int64 [M], confidence fp32 [M]) for every row.
    """
    logits, code = _rows(logits, "denoise_select")
    M, V = logits.shape
    if M > MAX_SELECT_ROWS:
        raise ValueError(f"denoise_select: {M} rows exceed {MAX_SELECT_ROWS}")
    if not 0 <= n_unmask <= M:
        raise ValueError(f"denoise_select: n_unmask={n_unmask} outside [0, {M}]")
    dev = _native.require_device(logits, cur_ids, step_map, per_pos_probs)
    if cur_ids.dtype != torch.int64 or cur_ids.shape != (M,) or (M > 1 and cur_ids.stride(0) != 1):
        raise ValueError("denoise_select: cur_ids must be int64 [M] with unit stride")
    if step_map is not None and (step_map.dtype != torch.int64 or step_map.shape != (M,)
                                 or (M > 1 and step_map.stride(0) != 1)):
        raise ValueError("denoise_select: step_map must be int64 [M] with unit stride")
    if per_pos_probs is not None and (per_pos_probs.dtype != torch.float32
                                      or per_pos_probs.shape != (M, V) or per_pos_probs.stride(1) != 1):
        raise ValueError("denoise_select: per_pos_probs must be fp32 [M, V] with unit stride along V")
    ids = torch.empty(M, device=dev, dtype=torch.int64)
    conf = torch.empty(M, device=dev, dtype=torch.float32)
    if M == 0:
        return ids, conf
    ws = _workspace(dev, M, V)
    with _native.device_guard(dev):
        status = _native.lib().simsd_denoise_select(
            logits.data_ptr(), logits.stride(0), M, V, code, cur_ids.data_ptr(), int(mask_token_id),
            int(n_unmask), step_map.data_ptr() if step_map is not None else None, int(step),
            per_pos_probs.data_ptr() if per_pos_probs is not None else None,
            per_pos_probs.stride(0) if per_pos_probs is not None else 0,
            ids.data_ptr(), conf.data_ptr(), ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    _native.check(status, "denoise_select")
    return ids, conf


def lm_head_argmax(x: torch.Tensor, w: torch.Tensor, return_probs: bool = False):
    """Skinny lm_head (``thin_linear``, logits in x.dtype as the reference's
    lm_head returns them) followed by ``softmax_argmax``.
    x: [M, K], w: [V, K] -> (ids, conf[, probs])."""
    return softmax_argmax(thin_linear(x, w), return_probs=return_probs)
