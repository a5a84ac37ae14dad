"""Opt-in switch that routes a model's projections and MoE experts through the MI355X kernels.

Public surface of kernels/fused_toggle.py (reference, lines 30-202), kept for
drop-in use: ``DEFAULT_TARGETS``, ``ALL_TARGETS``, ``apply_to_model``,
``is_applied``, the ``fused_linear`` context manager, ``warmup``,
``apply_moe_to_model`` and ``is_moe_applied``, with the same return values
and the same observable behaviour (idempotent switches, destructive expert
stacking, ``apply_moe_to_model(enable=False)`` raising).  Added here:
``apply_gated_mlp_to_model`` / ``is_gated_mlp_applied`` (gate and up
projections with SiLU-mul in one kernel), ``apply_rmsnorm_to_model`` (RMSNorm
in one launch) and ``expert_stacks``.

Design.  The model code is third-party (loaded through ``trust_remote_code``),
so nothing edits its call sites; every switch is a set of attribute patches
on module instances.  Each patch is recorded as (owner, attribute, previous
value) in a per-switch ledger keyed weakly by the model (owners are held
weakly too), so a switch is undone by replaying its ledger backwards, and a
model that is garbage collected takes its entry with it.  Nothing is patched on classes: an MoE
block gets an instance-level ``moe_infer`` bound to the grouped dispatch, so
blocks that were never switched keep the stock method untouched.

Default is off.  Switch before graph capture: a captured graph keeps the
forward that was installed when it was recorded.
"""
from __future__ import annotations

import types
import weakref
from typing import NamedTuple

import torch
import torch.nn as nn

from .thin_linear_fused import ThinLinear, reset_workspace

# Attribute names of the projections that are swapped by default.  lm_head is
# left out unless asked for (ALL_TARGETS): the logits epilogue has entry
# points of its own (kernels/logits_fused.py).
DEFAULT_TARGETS = (
    "q_proj", "k_proj", "v_proj", "o_proj",
    "gate_proj", "up_proj", "down_proj",
)
ALL_TARGETS = DEFAULT_TARGETS + ("lm_head",)

_UNSET = object()   # "the attribute was not in the instance dict before the patch"


class _Patch(NamedTuple):
    owner: "weakref.ref[nn.Module]"   # weak: the ledger must not keep its model alive
    attr: str
    before: object

    def undo(self) -> None:
        owner = self.owner()
        if owner is None:
            return
        if self.before is _UNSET:
            owner.__dict__.pop(self.attr, None)
        else:
            setattr(owner, self.attr, self.before)


class _Ledger:
    """Patches applied to each model by one switch, keyed weakly by the model."""

    def __init__(self):
        self._by_model: "weakref.WeakKeyDictionary[nn.Module, list[_Patch]]" = weakref.WeakKeyDictionary()

    def patches(self, model: nn.Module) -> list[_Patch]:
        return self._by_model.get(model, [])

    def add(self, model: nn.Module, patch: _Patch) -> None:
        self._by_model.setdefault(model, []).append(patch)

    def undo_all(self, model: nn.Module) -> int:
        done = self._by_model.pop(model, [])
        for p in reversed(done):
            p.undo()
        return len(done)


def _patch_attr(ledger: _Ledger, model: nn.Module, owner: nn.Module, attr: str, value) -> None:
    before = owner.__dict__.get(attr, _UNSET) if attr not in owner._modules else owner._modules[attr]
    ledger.add(model, _Patch(weakref.ref(owner), attr, before))
    setattr(owner, attr, value)


def _children_named(root: nn.Module, names, kind=nn.Linear):
    """(owner, attribute) of every child module of type ``kind`` held under
    one of ``names``, anywhere below root; each owner is visited once."""
    seen = {id(root)}
    todo = [root]
    while todo:
        owner = todo.pop()
        for attr, child in owner._modules.items():
            if child is None:
                continue
            if attr in names and isinstance(child, kind):
                yield owner, attr
            elif id(child) not in seen:
                seen.add(id(child))
                todo.append(child)


# ─────────────────────────────────────────────────────────────────────────────
# Projections -> ThinLinear (reference fused_toggle.py:52-104)
# ─────────────────────────────────────────────────────────────────────────────
_LINEARS = _Ledger()


def apply_to_model(model: nn.Module, enable: bool = True,
                   targets=DEFAULT_TARGETS,
                   config: tuple[int, int, int, int] | None = None) -> int:
    """Put ``ThinLinear`` in place of every ``nn.Linear`` held under one of
    ``targets`` (``enable=True``), or put the originals back (``enable=False``).

    ``ThinLinear`` aliases the original weight and bias, so the swap costs no
    memory and ``state_dict()`` is unchanged.  A second call in the same
    direction changes nothing.  Returns how many modules were swapped (or
    restored).
    """
    if not enable:
        n = _LINEARS.undo_all(model)
        if n:
            reset_workspace()
        return n
    if _LINEARS.patches(model):
        return 0
    sites = list(_children_named(model, frozenset(targets)))
    for owner, attr in sites:
        _patch_attr(_LINEARS, model, owner, attr, ThinLinear(owner._modules[attr], config=config))
    return len(sites)


def is_applied(model: nn.Module) -> bool:
    return bool(_LINEARS.patches(model))


class fused_linear:
    """``with fused_linear(model): ...`` -- swapped inside, restored on exit."""

    def __init__(self, model: nn.Module, enable: bool = True, **kw):
        self.model, self.enable, self.kw = model, enable, kw
        self.n = 0

    def __enter__(self):
        self.n = apply_to_model(self.model, self.enable, **self.kw)
        return self

    def __exit__(self, *exc):
        if self.enable:
            apply_to_model(self.model, False)
        return False


def warmup(model: nn.Module, block_length: int = 4, extra_M=()) -> None:
    """Exercise the swapped modules before any graph capture.

    The kernels are compiled ahead of time, so unlike the reference's Triton
    path (fused_toggle.py:107-133) there is nothing to JIT.  What a first call
    still does is load the library, which should not happen inside a
    capture.  One module per distinct (shape, dtype,
    device, config) is run at each token count the decode loop uses: 1,
    ``block_length``, ``2 * block_length``, the two prefill-size probes 96 and
    97, and ``extra_M``.
    """
    token_counts = sorted({1, block_length, 2 * block_length, 96, 97, *extra_M})
    kinds: dict[tuple, ThinLinear] = {}
    for mod in model.modules():
        if isinstance(mod, ThinLinear):
            w = mod.weight
            key = (tuple(w.shape), w.dtype, w.device, mod.config, mod.always_fuse, mod.bias is None)
            kinds.setdefault(key, mod)
    if not kinds:
        return
    with torch.inference_mode():
        for mod in kinds.values():
            w = mod.weight
            for m in token_counts:
                mod(torch.zeros(m, mod.in_features, device=w.device, dtype=w.dtype))
    if any(mod.weight.is_cuda for mod in kinds.values()):
        torch.cuda.synchronize()


# ─────────────────────────────────────────────────────────────────────────────
# LLaDA2 MoE blocks -> grouped dispatch (reference fused_toggle.py:148-202)
# ─────────────────────────────────────────────────────────────────────────────
_MOE_CLASS = "LLaDA2MoeSparseMoeBlock"
_STACKS = "_mi355_expert_stacks"


class ExpertStacks(NamedTuple):
    gate: torch.Tensor   # (E, I, H)
    up: torch.Tensor     # (E, I, H)
    down: torch.Tensor   # (E, H, I)


def expert_stacks(block: nn.Module) -> ExpertStacks | None:
    """The stacked expert weights a switched MoE block dispatches on, or None."""
    return block.__dict__.get(_STACKS)


def _grouped_moe_infer(self, x, topk_ids, topk_weight):
    from .moe_dispatch_fused import moe_dispatch
    return moe_dispatch(x, topk_ids, topk_weight, *self.__dict__[_STACKS])


def _moe_blocks(model: nn.Module):
    return [m for m in model.modules() if type(m).__name__ == _MOE_CLASS]


def apply_moe_to_model(model: nn.Module, enable: bool = True) -> int:
    """Make every LLaDA2 MoE block run ``moe_dispatch`` on stacked expert weights.

    Each block's experts are stacked once (``stack_expert_weights``, which
    releases the per-expert weights as it goes) and the block gets an
    instance-level ``moe_infer`` with the stock signature.  Blocks already
    switched are skipped.  Returns how many blocks were switched.  The
    released weights cannot be brought back, so ``enable=False`` raises
    ``NotImplementedError`` once any block is switched (and returns 0 when
    none is).
    """
    blocks = _moe_blocks(model)
    if not enable:
        if any(expert_stacks(b) is not None for b in blocks):
            raise NotImplementedError(
                "apply_moe_to_model cannot be undone: switching stacked the expert "
                "weights and released the per-expert copies, so the stock moe_infer "
                "has nothing left to run on. Reload the model instead.")
        return 0
    from .moe_dispatch_fused import stack_expert_weights

    n = 0
    for blk in blocks:
        if expert_stacks(blk) is not None:
            continue
        blk.__dict__[_STACKS] = ExpertStacks(*stack_expert_weights(blk.experts))
        blk.moe_infer = types.MethodType(_grouped_moe_infer, blk)
        n += 1
    return n


def is_moe_applied(model: nn.Module) -> bool:
    return any(expert_stacks(b) is not None for b in _moe_blocks(model))


# ─────────────────────────────────────────────────────────────────────────────
# SiLU-gated MLP blocks (gate_proj / up_proj / down_proj, modeling_sdar.py:113-119)
# ─────────────────────────────────────────────────────────────────────────────
_GATED = _Ledger()


def _is_silu(act) -> bool:
    if isinstance(act, nn.SiLU):
        return True
    return getattr(act, "__name__", "") == "silu" or type(act).__name__ in ("SiLU", "SiLUActivation")


def _gated_forward(mod: nn.Module, stock):
    from .thin_linear_fused import should_fuse, thin_linear_silu_mul

    def forward(x):
        wg, wu = mod.gate_proj.weight, mod.up_proj.weight
        M = x.numel() // x.shape[-1]
        if not should_fuse(M, 2 * wg.shape[0], wg.shape[1]):
            return stock(x)
        return mod.down_proj(thin_linear_silu_mul(x, wg, wu))
    return forward


def apply_gated_mlp_to_model(model: nn.Module, enable: bool = True) -> int:
    """Route SiLU-gated MLP blocks through ``thin_linear_silu_mul`` (or restore them).

    A block qualifies when it has ``gate_proj``, ``up_proj``, ``down_proj``
    (``nn.Linear`` or ``ThinLinear``) without bias on gate/up, and a SiLU
    ``act_fn``, as SDAR's and Qwen's MLPs do.  Its forward becomes
    ``down_proj(thin_linear_silu_mul(x, gate.weight, up.weight))`` when the
    merged gate_up shape is inside the fused envelope (``should_fuse(M, 2I,
    K)``), and the stock forward otherwise.  Idempotent both ways; returns
    how many blocks were switched or restored.
    """
    if not enable:
        return _GATED.undo_all(model)
    done = {id(p.owner()) for p in _GATED.patches(model)}
    n = 0
    for mod in model.modules():
        parts = [getattr(mod, p, None) for p in ("gate_proj", "up_proj", "down_proj")]
        if id(mod) in done or not all(p is not None and hasattr(p, "weight") for p in parts):
            continue
        if not _is_silu(getattr(mod, "act_fn", None)):
            continue
        if getattr(parts[0], "bias", None) is not None or getattr(parts[1], "bias", None) is not None:
            continue
        _patch_attr(_GATED, model, mod, "forward", _gated_forward(mod, mod.forward))
        n += 1
    return n


def is_gated_mlp_applied(model: nn.Module) -> bool:
    return bool(_GATED.patches(model))


# ─────────────────────────────────────────────────────────────────────────────
# RMSNorm modules (SDARRMSNorm and its kind: .weight, .variance_epsilon)
# ─────────────────────────────────────────────────────────────────────────────
_NORMS = _Ledger()


def _norm_forward(mod: nn.Module, stock):
    from .thin_linear_fused import thin_rmsnorm

    def forward(x):
        if x.device.type != "cuda" or mod.weight.dtype != x.dtype:
            return stock(x)
        return thin_rmsnorm(x, mod.weight, mod.variance_epsilon)
    return forward


def apply_rmsnorm_to_model(model: nn.Module, enable: bool = True) -> int:
    """Run every RMSNorm module (class name ending in ``RMSNorm`` with
    ``weight`` and ``variance_epsilon``) as one ``thin_rmsnorm`` launch instead
    of the stock five-op form.  Idempotent both ways; returns how many modules
    were switched or restored."""
    if not enable:
        return _NORMS.undo_all(model)
    done = {id(p.owner()) for p in _NORMS.patches(model)}
    n = 0
    for mod in model.modules():
        if id(mod) in done or not type(mod).__name__.endswith("RMSNorm"):
            continue
        if not (hasattr(mod, "weight") and hasattr(mod, "variance_epsilon")):
            continue
        _patch_attr(_NORMS, model, mod, "forward", _norm_forward(mod, mod.forward))
        n += 1
    return n
