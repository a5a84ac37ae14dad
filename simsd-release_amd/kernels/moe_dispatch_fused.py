"""Fused MoE expert dispatch for MI355X -- drop-in for kernels/moe_dispatch_fused.py.

Keeps the reference's public surface (kernels/moe_dispatch_fused.py:29-231):
``moe_dispatch(x, topk_ids, topk_weight, w_gate, w_up, w_down)``,
``stack_expert_weights``, ``FusedMoEDispatch``, ``BLOCK_M``, ``_align`` and
``_num_tiles``; adds the routing step the reference leaves to the remote
LLaDA2 gate (``moe_route``), the align outputs as a record (``moe_align``),
both in one launch (``moe_route_align``) and the whole step with a shared
expert (``moe_forward``).

Kernels (``csrc/moe.hip``, C ABI in ``include/simsd_kernels.h``):
  route    one wave per token: top-k over the E logits (ties -> lower index),
           softmax or sigmoid scores, optional renormalisation and scaling;
  align    one workgroup: LDS histogram, scans, a stable counting sort walked
           in slot order, the 16-row padded slot table and per-tile experts --
           integer, bit-exact, no host sync;
  gate_up  per (16-slot tile, 16 intermediate columns): the gate and up weight
           rows stream as two MFMA A blocks against the tile's gathered
           activation rows, and the epilogue writes h = silu(g) * u;
  down     per (tile, 64 hidden rows) on h;
  combine  fp32 weighted sum over each token's k experts in k order, then the
           shared expert's output added.
Every grid depends on (T, k, E, H, I) only; empty tiles exit at once, so the
step captures into a HIP graph.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _native

# Rows per tile (kernels/moe_dispatch_fused.py:29): each expert's group of
# slots is padded to a multiple of this in the align tables.
BLOCK_M = 16


def _num_tiles(M: int, E: int) -> int:
    """Worst-case tile count: every active group costs at least one tile."""
    return min(E, M) + (M + BLOCK_M - 1) // BLOCK_M


class MoeAlignment(NamedTuple):
    counts: torch.Tensor        # (E,) int32
    offsets: torch.Tensor       # (E+1,) int32, exclusive scan of counts
    pad_offsets: torch.Tensor   # (E+1,) int32, exclusive scan of 16-padded counts
    perm: torch.Tensor          # (T*k,) int32, slots sorted by expert (stable)
    slots: torch.Tensor         # (num_tiles*16,) int32, slot per padded row or -1
    tile_expert: torch.Tensor   # (num_tiles,) int32, expert per tile or E


def _flat_ids(topk_ids: torch.Tensor) -> torch.Tensor:
    flat = topk_ids.reshape(-1)
    if flat.dtype != torch.int64:
        flat = flat.to(torch.int64)
    return flat.contiguous()


def moe_align(topk_ids: torch.Tensor, E: int, num_tiles: int | None = None) -> MoeAlignment:
    """Sort the flat slots by expert and lay groups out on 16-row boundaries."""
    dev = _native.require_device(topk_ids)
    flat = _flat_ids(topk_ids)
    M = flat.numel()
    if not 0 < E <= _native.MOE_MAX_EXPERTS:
        raise ValueError(f"E={E} outside 1..{_native.MOE_MAX_EXPERTS}")
    if M > _native.MOE_MAX_SLOTS:
        raise ValueError(f"T*k={M} exceeds {_native.MOE_MAX_SLOTS} slots")
    if num_tiles is None:
        num_tiles = _num_tiles(M, E)
    i32 = dict(device=dev, dtype=torch.int32)
    al = MoeAlignment(
        counts=torch.empty(E, **i32), offsets=torch.empty(E + 1, **i32),
        pad_offsets=torch.empty(E + 1, **i32), perm=torch.empty(M, **i32),
        slots=torch.empty(num_tiles * BLOCK_M, **i32), tile_expert=torch.empty(num_tiles, **i32))
    lib = _native.lib()
    with _native.device_guard(dev):
        st = lib.simsd_moe_align(flat.data_ptr(), M, E, num_tiles, al.counts.data_ptr(),
                                 al.offsets.data_ptr(), al.pad_offsets.data_ptr(),
                                 al.perm.data_ptr(), al.slots.data_ptr(),
                                 al.tile_expert.data_ptr(), _native.stream_of(dev))
    _native.check(st, "moe_align")
    return al


def _align(topk_ids: torch.Tensor, E: int, num_tiles: int):
    """Sort slots by expert and lay each group out on BLOCK_M boundaries.

    Same contract as kernels/moe_dispatch_fused.py:93-132.  Returns
        slots       (num_tiles*BLOCK_M,) int32 -- original flat slot index, or -1
        tile_expert (num_tiles,)         int32 -- expert for the tile, or E (skip)
    """
    al = moe_align(topk_ids, E, num_tiles)
    return al.slots, al.tile_expert


_SCORING = {"softmax": _native.SCORE_SOFTMAX, "sigmoid": _native.SCORE_SIGMOID}


def moe_route(logits: torch.Tensor, k: int, scoring: str = "softmax", renorm: bool = True,
              scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k routing on the GPU: (topk_ids int64 (T, k), topk_weight fp32 (T, k)).

    ids are the k largest logits per row, largest first, ties to the lower
    expert index.  The weight of a pick is its score -- ``softmax`` over all E
    logits or ``sigmoid`` of the logit -- divided by the sum over the k picks
    (plus 1e-20) when ``renorm`` and k > 1, times ``scale``.  ``scoring="sigmoid",
    renorm=True, scale=2.5`` is the routing of
    kernels/workspace/moe_dispatch/build_oracle.py:71-90.
    """
    if logits.ndim != 2:
        raise ValueError(f"logits must be (T, E), got {tuple(logits.shape)}")
    if scoring not in _SCORING:
        raise ValueError(f"scoring must be one of {sorted(_SCORING)}, got {scoring!r}")
    dev = _native.require_device(logits)
    T, E = logits.shape
    if not 0 < k <= min(64, E):
        raise ValueError(f"need 0 < k <= min(64, E={E}), got k={k}")
    lg = logits
    if lg.dtype != torch.float32:
        lg = lg.float()
    if lg.stride(1) != 1:
        lg = lg.contiguous()
    ids = torch.empty((T, k), device=dev, dtype=torch.int64)
    w = torch.empty((T, k), device=dev, dtype=torch.float32)
    if T == 0:
        return ids, w
    lib = _native.lib()
    with _native.device_guard(dev):
        st = lib.simsd_moe_route_topk(lg.data_ptr(), T, E, lg.stride(0), k, _SCORING[scoring],
                                      int(bool(renorm)), float(scale), ids.data_ptr(),
                                      w.data_ptr(), _native.stream_of(dev))
    _native.check(st, "moe_route")
    return ids, w


def _grouped_ffn(x, topk_ids, topk_weight, w_gate, w_up, w_down, slots, tile_expert,
                 shared=None, out=None) -> torch.Tensor:
    T, H = x.shape
    k = topk_ids.shape[1]
    E, I, Hg = w_gate.shape
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")
    for name, wt, shape in (("w_gate", w_gate, (E, I, H)), ("w_up", w_up, (E, I, H)),
                            ("w_down", w_down, (E, H, I))):
        if tuple(wt.shape) != shape:
            raise ValueError(f"{name} must be {shape}, got {tuple(wt.shape)}")
        if wt.dtype != x.dtype:
            raise TypeError(f"{name} dtype {wt.dtype} != x dtype {x.dtype}")
    if topk_weight.shape != topk_ids.shape:
        raise ValueError("topk_weight and topk_ids must have the same shape")
    tw = topk_weight if topk_weight.dtype == torch.float32 else topk_weight.float()
    ids = topk_ids if topk_ids.dtype == torch.int64 else topk_ids.to(torch.int64)
    sg = su = sd = None
    Is = 0
    if shared is not None:
        sg, su, sd = shared
        Is = sg.shape[0]
        if tuple(sg.shape) != (Is, H) or tuple(su.shape) != (Is, H) or tuple(sd.shape) != (H, Is):
            raise ValueError("shared expert must be gate (Is, H), up (Is, H), down (H, Is)")
        if not (sg.dtype == su.dtype == sd.dtype == x.dtype):
            raise TypeError("shared expert dtype must match x")
    dev = _native.require_device(x, ids, tw, w_gate, w_up, w_down, slots, tile_expert,
                                 *(t for t in (sg, su, sd) if t is not None))
    if out is None:
        out = torch.empty((T, H), device=dev, dtype=x.dtype)
    if T == 0:
        return out
    lib = _native.lib()
    nbytes = lib.simsd_moe_workspace_bytes(T, k, H, I, Is, code)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    z = (None, 0, 0)
    sgp = (sg.data_ptr(), sg.stride(0), sg.stride(1)) if sg is not None else z
    sup = (su.data_ptr(), su.stride(0), su.stride(1)) if su is not None else z
    sdp = (sd.data_ptr(), sd.stride(0), sd.stride(1)) if sd is not None else z
    with _native.device_guard(dev):
        st = lib.simsd_moe_grouped_ffn(
            x.data_ptr(), x.stride(0), x.stride(1),
            w_gate.data_ptr(), *w_gate.stride(),
            w_up.data_ptr(), *w_up.stride(),
            w_down.data_ptr(), *w_down.stride(),
            *sgp, *sup, *sdp, Is,
            slots.data_ptr(), tile_expert.data_ptr(), tile_expert.numel(),
            ids.data_ptr(), ids.stride(0), ids.stride(1),
            tw.data_ptr(), tw.stride(0), tw.stride(1),
            out.data_ptr(), out.stride(0), out.stride(1),
            T, k, E, H, I, code, ws.data_ptr(), nbytes, _native.stream_of(dev))
    _native.check(st, "moe_grouped_ffn")
    return out


def moe_dispatch(x, topk_ids, topk_weight, w_gate, w_up, w_down):
    """Drop-in for ``LLaDA2MoeSparseMoeBlock.moe_infer`` on stacked weights.

    x           (T, H)    topk_ids (T, k) int64    topk_weight (T, k) fp32
    w_gate/up   (E, I, H)  w_down  (E, H, I)   -> (T, H)

    out_t = dtype( sum_j fp32(y_j) * w_j ), y_j = down_e(silu(gate_e(x_t)) * up_e(x_t))
    with the reference's dtype discipline (kernels/workspace/moe_dispatch/CONTRACT.md:26-40).
    """
    if x.ndim != 2 or topk_ids.ndim != 2:
        raise ValueError("x must be (T, H) and topk_ids (T, k)")
    E = w_gate.shape[0]
    T, k = topk_ids.shape
    rows = _chunk_rows(k)
    if T <= rows:
        slots, tile_expert = _align(topk_ids, E, _num_tiles(T * k, E))
        return _grouped_ffn(x, topk_ids, topk_weight, w_gate, w_up, w_down, slots, tile_expert)
    # More slots than one align workgroup sorts: token chunks of fixed size,
    # each aligned and dispatched on its own into its rows of one output.
    # Tokens are independent, so the result equals one dispatch over all T.
    out = torch.empty((T, x.shape[1]), device=x.device, dtype=x.dtype)
    for t0 in range(0, T, rows):
        t1 = min(T, t0 + rows)
        ids_c = topk_ids[t0:t1]
        slots, tile_expert = _align(ids_c, E, _num_tiles(ids_c.numel(), E))
        _grouped_ffn(x[t0:t1], ids_c, topk_weight[t0:t1], w_gate, w_up, w_down, slots,
                     tile_expert, out=out[t0:t1])
    return out


def _chunk_rows(k: int) -> int:
    """Tokens per align launch: the single align workgroup sorts at most
    MOE_MAX_SLOTS slots (T * k)."""
    return max(1, _native.MOE_MAX_SLOTS // max(int(k), 1))


# Up to this many tokens (one per wave of the single workgroup), routing and
# align run as one launch; beyond it, as two launches (routing in parallel).
FUSED_ROUTE_MAX_T = 16


def moe_route_align(logits: torch.Tensor, k: int, E: int | None = None, scoring: str = "softmax",
                    renorm: bool = True, scale: float = 1.0, num_tiles: int | None = None):
    """``moe_route`` followed by ``moe_align`` of its ids, in one launch.

    Returns (topk_ids, topk_weight, MoeAlignment), identical to the two calls
    in sequence.
    """
    if logits.ndim != 2:
        raise ValueError(f"logits must be (T, E), got {tuple(logits.shape)}")
    if scoring not in _SCORING:
        raise ValueError(f"scoring must be one of {sorted(_SCORING)}, got {scoring!r}")
    dev = _native.require_device(logits)
    T, El = logits.shape
    E = El if E is None else E
    if E != El:
        raise ValueError(f"E={E} but logits have {El} columns")
    if not 0 < E <= _native.MOE_MAX_EXPERTS:
        raise ValueError(f"E={E} outside 1..{_native.MOE_MAX_EXPERTS}")
    if not 0 < k <= min(64, E):
        raise ValueError(f"need 0 < k <= min(64, E={E}), got k={k}")
    M = T * k
    if M > _native.MOE_MAX_SLOTS:
        raise ValueError(f"T*k={M} exceeds {_native.MOE_MAX_SLOTS} slots")
    if num_tiles is None:
        num_tiles = _num_tiles(M, E)
    lg = logits
    if lg.dtype != torch.float32:
        lg = lg.float()
    if lg.stride(1) != 1:
        lg = lg.contiguous()
    ids = torch.empty((T, k), device=dev, dtype=torch.int64)
    w = torch.empty((T, k), device=dev, dtype=torch.float32)
    i32 = dict(device=dev, dtype=torch.int32)
    al = MoeAlignment(
        counts=torch.empty(E, **i32), offsets=torch.empty(E + 1, **i32),
        pad_offsets=torch.empty(E + 1, **i32), perm=torch.empty(M, **i32),
        slots=torch.empty(num_tiles * BLOCK_M, **i32), tile_expert=torch.empty(num_tiles, **i32))
    lib = _native.lib()
    with _native.device_guard(dev):
        st = lib.simsd_moe_route_align(
            lg.data_ptr(), T, E, lg.stride(0), k, _SCORING[scoring], int(bool(renorm)), float(scale),
            ids.data_ptr(), w.data_ptr(), num_tiles, al.counts.data_ptr(), al.offsets.data_ptr(),
            al.pad_offsets.data_ptr(), al.perm.data_ptr(), al.slots.data_ptr(),
            al.tile_expert.data_ptr(), _native.stream_of(dev))
    _native.check(st, "moe_route_align")
    return ids, w, al


def moe_forward(x, router_logits, k, w_gate, w_up, w_down, shared=None,
                scoring: str = "softmax", renorm: bool = True, scale: float = 1.0):
    """Route + dispatch + shared expert in one graph-capturable sequence.

    ``shared`` is ``(gate (Is, H), up (Is, H), down (H, Is))`` or None; its
    output is added to the routed output in x's dtype, as the LLaDA2 forward
    adds ``shared_experts(x)`` after ``moe_infer``.
    """
    E = w_gate.shape[0]
    T = router_logits.shape[0]
    if 0 < T <= FUSED_ROUTE_MAX_T and T * k <= _native.MOE_MAX_SLOTS:
        ids, w, al = moe_route_align(router_logits, k, E, scoring=scoring, renorm=renorm, scale=scale)
        return _grouped_ffn(x, ids, w, w_gate, w_up, w_down, al.slots, al.tile_expert, shared=shared)
    ids, w = moe_route(router_logits, k, scoring=scoring, renorm=renorm, scale=scale)
    rows = _chunk_rows(k)
    if T <= rows:
        slots, tile_expert = _align(ids, E, _num_tiles(ids.numel(), E))
        return _grouped_ffn(x, ids, w, w_gate, w_up, w_down, slots, tile_expert, shared=shared)
    out = torch.empty((T, x.shape[1]), device=x.device, dtype=x.dtype)
    for t0 in range(0, T, rows):
        t1 = min(T, t0 + rows)
        slots, tile_expert = _align(ids[t0:t1], E, _num_tiles((t1 - t0) * k, E))
        _grouped_ffn(x[t0:t1], ids[t0:t1], w[t0:t1], w_gate, w_up, w_down, slots, tile_expert,
                     shared=shared, out=out[t0:t1])
    return out


def stack_expert_weights(experts, free_originals: bool = True):
    """(w_gate (E,I,H), w_up (E,I,H), w_down (E,H,I)) from the experts of an
    MoE block (an ``nn.ModuleList`` of gate/up/down MLPs), the layout the
    grouped kernels stream.

    Behaviour of kernels/moe_dispatch_fused.py:195-217: one projection is
    stacked at a time, and with ``free_originals=True`` (destructive) each
    expert's weight is released as soon as it has been copied, so the extra
    memory never exceeds one projection's stack.  Each stack is allocated once
    and filled expert by expert; the result is contiguous.
    """
    experts = list(experts)
    if not experts:
        raise ValueError("stack_expert_weights needs at least one expert")
    out = []
    for proj in ("gate_proj", "up_proj", "down_proj"):
        first = getattr(experts[0], proj).weight.data
        stack = first.new_empty((len(experts), *first.shape))
        for e, mlp in enumerate(experts):
            lin = getattr(mlp, proj)
            stack[e].copy_(lin.weight.data)
            if free_originals:
                lin.weight.data = stack.new_empty(0)
        out.append(stack)
    return tuple(out)


class FusedMoEDispatch(torch.nn.Module):
    """``moe_dispatch`` as a module over stacked expert weights (the
    reference's isolated-signature wrapper, moe_dispatch_fused.py:220-231).
    The stacks are buffers that follow ``.to()`` but stay out of the
    state dict."""

    _NAMES = ("w_gate", "w_up", "w_down")

    def __init__(self, w_gate, w_up, w_down):
        super().__init__()
        for name, t in zip(self._NAMES, (w_gate, w_up, w_down)):
            self.register_buffer(name, t, persistent=False)

    def forward(self, x, topk_ids, topk_weight):
        stacks = [getattr(self, n) for n in self._NAMES]
        return moe_dispatch(x, topk_ids, topk_weight, *stacks)
