"""Opt-in switch routing a model's ``nn.Linear`` / MoE calls through the MI355X kernels.

Same API and behaviour as kernels/fused_toggle.py (reference, lines 30-202):
``DEFAULT_TARGETS``, ``ALL_TARGETS``, ``apply_to_model``, ``is_applied``, the
``fused_linear`` context manager, ``warmup``, ``apply_moe_to_model`` and
``is_moe_applied``; added: ``apply_gated_mlp_to_model`` /
``is_gated_mlp_applied`` (gate and up projections with SiLU·mul in one
kernel) and ``apply_rmsnorm_to_model`` (RMSNorm in one launch).  The model code is third-party (loaded through
``trust_remote_code``), so the switch patches modules in place rather than
editing call sites: target linears are swapped for ``ThinLinear`` (which
aliases the original parameters), and LLaDA2's MoE block gets a class-level
``moe_infer`` that calls ``moe_dispatch`` on stacked expert weights.

Default is off.  Call it before graph capture: a captured graph keeps
whichever forward was installed when it was recorded.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .thin_linear_fused import ThinLinear, reset_workspace

# Leaf names of the projections to swap; lm_head is opt-in (ALL_TARGETS).
DEFAULT_TARGETS = (
    "q_proj", "k_proj", "v_proj", "o_proj",
    "gate_proj", "up_proj", "down_proj",
)
ALL_TARGETS = DEFAULT_TARGETS + ("lm_head",)

# id(model) -> {qualified name: original module}
_ORIGINALS: dict[int, dict[str, nn.Module]] = {}


def _targets_in(model: nn.Module, targets):
    for qualified, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and qualified.rsplit(".", 1)[-1] in targets:
            yield qualified, mod


def _replace(model: nn.Module, qualified: str, new: nn.Module) -> None:
    owner_path, _, leaf = qualified.rpartition(".")
    owner = model.get_submodule(owner_path) if owner_path else model
    setattr(owner, leaf, new)


def apply_to_model(model: nn.Module, enable: bool = True,
                   targets=DEFAULT_TARGETS,
                   config: tuple[int, int, int, int] | None = None) -> int:
    """Swap the target ``nn.Linear`` modules for ``ThinLinear`` (or restore them).

    Idempotent both ways; returns how many modules were swapped or restored.
    """
    key = id(model)
    if not enable:
        saved = _ORIGINALS.pop(key, None)
        if not saved:
            return 0
        for qualified, orig in saved.items():
            _replace(model, qualified, orig)
        reset_workspace()
        return len(saved)
    if key in _ORIGINALS:
        return 0
    saved = {}
    for qualified, mod in list(_targets_in(model, targets)):
        saved[qualified] = mod
        _replace(model, qualified, ThinLinear(mod, config=config))
    if saved:
        _ORIGINALS[key] = saved
    return len(saved)


def is_applied(model: nn.Module) -> bool:
    return id(model) in _ORIGINALS


class fused_linear:
    """Context-manager form::

        with fused_toggle.fused_linear(model):
            ...
    """

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
    """Run every swapped module once at each M the pipeline uses.

    The kernels are compiled ahead of time, so there is no JIT to trigger;
    what this still does is allocate the per-device split-K workspace and load
    the library before any graph capture, at M in {1, block_length,
    2*block_length, 96, 97, *extra_M} (the reference's sweep,
    kernels/fused_toggle.py:107-133).
    """
    Ms = {1, block_length, 2 * block_length, 96, 97, *extra_M}
    mods = [m for _, m in model.named_modules() if isinstance(m, ThinLinear)]
    with torch.inference_mode():
        for mod in mods:
            for M in sorted(Ms):
                mod(torch.zeros(M, mod.in_features, device=mod.weight.device,
                                dtype=mod.weight.dtype))
    if mods and mods[0].weight.is_cuda:
        torch.cuda.synchronize()


# ─────────────────────────────────────────────────────────────────────────────
# LLaDA2 MoE expert dispatch (moe_dispatch_fused.py)
# ─────────────────────────────────────────────────────────────────────────────
_MOE_ATTR = "_simsd_fused_moe"
_MOE_CLASS = "LLaDA2MoeSparseMoeBlock"


def apply_moe_to_model(model: nn.Module, enable: bool = True) -> int:
    """Switch LLaDA2 MoE blocks to the grouped dispatch.  Idempotent.

    Returns the number of blocks switched.  Stacking releases the per-expert
    weights, so ``enable=False`` cannot restore them and raises.
    """
    from .moe_dispatch_fused import moe_dispatch, stack_expert_weights

    n = 0
    for mod in model.modules():
        if mod.__class__.__name__ != _MOE_CLASS:
            continue
        if enable:
            if getattr(mod, _MOE_ATTR, None) is not None:
                continue
            setattr(mod, _MOE_ATTR, stack_expert_weights(mod.experts))
            n += 1
        elif getattr(mod, _MOE_ATTR, None) is not None:
            raise NotImplementedError(
                "apply_moe_to_model(enable=False) is not supported: stacking "
                "releases the per-expert weights so the layer's footprint stays "
                "flat. Reload the checkpoint to get the stock path back.")
    if n == 0:
        return 0

    cls = next(m.__class__ for m in model.modules() if m.__class__.__name__ == _MOE_CLASS)
    if not getattr(cls, "_simsd_moe_patched", False):
        stock = cls.moe_infer

        def moe_infer(self, x, topk_ids, topk_weight):
            packed = getattr(self, _MOE_ATTR, None)
            if packed is None:
                return stock(self, x, topk_ids, topk_weight)
            return moe_dispatch(x, topk_ids, topk_weight, *packed)

        cls.moe_infer = moe_infer
        cls._simsd_moe_stock = stock
        cls._simsd_moe_patched = True
    return n


def is_moe_applied(model: nn.Module) -> bool:
    return any(getattr(m, _MOE_ATTR, None) is not None for m in model.modules())


# ─────────────────────────────────────────────────────────────────────────────
# SiLU-gated MLP blocks (gate_proj / up_proj / down_proj, modeling_sdar.py:113-119)
# ─────────────────────────────────────────────────────────────────────────────
_GATED: dict[int, list[nn.Module]] = {}   # id(model) -> blocks whose forward is patched


def _is_silu(act) -> bool:
    if isinstance(act, nn.SiLU):
        return True
    return getattr(act, "__name__", "") == "silu" or act.__class__.__name__ in ("SiLU", "SiLUActivation")


def _gated_blocks(model: nn.Module):
    for mod in model.modules():
        parts = [getattr(mod, n, None) for n in ("gate_proj", "up_proj", "down_proj")]
        if all(p is not None and hasattr(p, "weight") for p in parts) and _is_silu(getattr(mod, "act_fn", None)):
            yield mod


def apply_gated_mlp_to_model(model: nn.Module, enable: bool = True) -> int:
    """Route SiLU-gated MLP blocks through ``thin_linear_silu_mul`` (or restore them).

    A block qualifies when it has ``gate_proj``, ``up_proj``, ``down_proj``
    (``nn.Linear`` or ``ThinLinear``) and a SiLU ``act_fn``, as SDAR's and
    Qwen's MLPs do.  Its forward becomes ``down_proj(thin_linear_silu_mul(x,
    gate.weight, up.weight))`` when the merged gate_up shape is inside the
    fused envelope (``should_fuse(M, 2I, K)``), and the stock forward
    otherwise.  No bias on gate/up (else the block is left alone).  Idempotent
    both ways; returns how many blocks were switched or restored.
    """
    from .thin_linear_fused import should_fuse, thin_linear_silu_mul

    key = id(model)
    if not enable:
        blocks = _GATED.pop(key, [])
        for mod in blocks:
            mod.__dict__.pop("forward", None)   # back to the class's forward
        return len(blocks)
    done = _GATED.setdefault(key, [])
    n = 0
    for mod in _gated_blocks(model):
        if any(m is mod for m in done):
            continue
        if getattr(mod.gate_proj, "bias", None) is not None or getattr(mod.up_proj, "bias", None) is not None:
            continue
        stock = mod.forward

        def forward(x, _mod=mod, _stock=stock):
            wg, wu = _mod.gate_proj.weight, _mod.up_proj.weight
            M = x.numel() // x.shape[-1]
            if not should_fuse(M, 2 * wg.shape[0], wg.shape[1]):
                return _stock(x)
            return _mod.down_proj(thin_linear_silu_mul(x, wg, wu))

        mod.forward = forward
        done.append(mod)
        n += 1
    return n


def is_gated_mlp_applied(model: nn.Module) -> bool:
    return bool(_GATED.get(id(model)))


# ─────────────────────────────────────────────────────────────────────────────
# RMSNorm modules (SDARRMSNorm and its kind: .weight, .variance_epsilon)
# ─────────────────────────────────────────────────────────────────────────────
_NORMS: dict[int, list[nn.Module]] = {}


def apply_rmsnorm_to_model(model: nn.Module, enable: bool = True) -> int:
    """Run every RMSNorm module (class name ending in ``RMSNorm`` with
    ``weight`` and ``variance_epsilon``) as one ``thin_rmsnorm`` launch instead
    of the stock five-op form.  Idempotent both ways; returns how many modules
    were switched or restored."""
    from .thin_linear_fused import thin_rmsnorm

    key = id(model)
    if not enable:
        mods = _NORMS.pop(key, [])
        for mod in mods:
            mod.__dict__.pop("forward", None)
        return len(mods)
    done = _NORMS.setdefault(key, [])
    n = 0
    for mod in model.modules():
        if not (mod.__class__.__name__.endswith("RMSNorm") and hasattr(mod, "weight")
                and hasattr(mod, "variance_epsilon")):
            continue
        if any(m is mod for m in done):
            continue
        stock = mod.forward

        def forward(x, _mod=mod, _stock=stock):
            if x.device.type != "cuda" or _mod.weight.dtype != x.dtype:
                return _stock(x)
            return thin_rmsnorm(x, _mod.weight, _mod.variance_epsilon)

        mod.forward = forward
        done.append(mod)
        n += 1
    return n
