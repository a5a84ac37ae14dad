"""Skinny-M ``F.linear`` for MI355X -- drop-in for kernels/thin_linear_fused.py.

Same public surface as the reference module (kernels/thin_linear_fused.py:57-419):
``thin_linear``, ``ThinLinear``, ``should_fuse``, ``pick_config``, ``TUNED``,
``_tuned_for``, ``_heuristic_config``, ``reset_workspace``, ``make_bench_fn`` and
the ``TARGET_CTAS`` / ``MAX_SPLIT_K`` / ``MIN_K_PER_SPLIT`` knobs, with the same
argument meaning and the same exceptions.  The arithmetic runs in a
hand-written gfx950 HIP kernel (``libsimsd_kernels.so``, C ABI in
``include/simsd_kernels.h``) instead of Triton.  Added on top:
``thin_linear_silu_mul``, an MLP's gate and up projections with the SiLU and
product in the same kernel; ``thin_linear_residual``, a projection with the
decoder layer's residual add in its epilogue; ``thin_rmsnorm`` (one launch)
and the RMSNorm prologue forms ``thin_rmsnorm_linear`` /
``thin_rmsnorm_linear_silu_mul``.

How the MI355X kernels work (``csrc/thin_gemm.hip``)
-----------------------------------------------------
At M <= 32 the op is a stream over the weight: arithmetic intensity is at most
~32 flop/byte against a ~312 flop/byte ridge, so HBM bandwidth is the bound,
and what matters is reading the weight once, in full cache lines, with enough
loads in flight.  All weight and activation reads go through buffer
descriptors whose hardware range check returns zeros past the tile, so the
load stream carries no branches.

* M <= 8 (bf16/fp16): ``v_mfma_f32_4x4x4_16b`` runs 16 independent 4x4x4
  products per instruction.  Lanes map to (weight row l%4, k chunk l/4), so
  one 16-byte load per lane covers 4 weight rows x 256 contiguous bytes, and
  the 4 output columns are the (up to 4) tokens -- nothing is padded.  The
  activations of a wave's K range sit in registers and serve every 4-row
  group, so the inner loop issues weight loads only.
* M > 8 (bf16/fp16): ``v_mfma_f32_16x16x32_bf16`` with 16 weight rows as the
  A operand and up to 16 tokens per block as the B operand.  The weight is
  still read as 4 rows x 256 contiguous bytes per instruction; each wave
  writes its 16- or 32-row tile through a padded LDS region and reads it back
  in the MFMA operand layout.  Several 256-byte k chunks are loaded per batch
  so enough bytes are in flight.
* fp32 and strided / unaligned views: the same 16x16 MFMA shape with the
  operands loaded straight in their MFMA layout (64 B of a row per lane
  group), element by element where the view is not vector-aligned.

A workgroup owns 4, 8, 16 or 32 weight rows and splits K over its waves,
which sum their fp32 partials in fixed order; narrow N uses fewer rows per
workgroup so every CU still gets work without a cross-workgroup reduction.
Above 8 tokens a workgroup may also own 64, 96 or 128 rows
(``thin_gemm_xs_kernel``): its waves then split the rows instead of K and
share each activation chunk, loaded once per workgroup into LDS, so the
activation bytes read from L2 per weight byte drop by the wave count.  An
explicit SPLIT_K > 1 splits K over workgroups too: fp32 partial tiles, then a
second launch sums them in split order.

Config tuples keep the reference's shape ``(BLOCK_M, BLOCK_N, BLOCK_K,
SPLIT_K[, num_warps, num_stages])`` and describe the MI355X kernels:
BLOCK_M is the token envelope (``TUNED``: dispatch for M up to 16 or 64) or
column-block width (heuristic: 4 or 8 for the GEMV, 16, 32 or 48 otherwise),
BLOCK_N the weight rows per workgroup (4, 8, 16, 24, 32, 64, 96 or 128; other
values round down to one of these; at least 16 above 8 tokens; 64, 96 and 128
apply above 8 tokens in bf16/fp16 and act as 32 elsewhere; 24 applies to the
ungated projection above 8 tokens and acts as 16 elsewhere), BLOCK_K the K elements of
activations a wave holds at once in the GEMV (256 or 1024),
SPLIT_K the workgroups along K, num_warps the waves per workgroup (2, 4 or 8);
num_stages is accepted and ignored.

Contract (reference CONTRACT, kernels/workspace/thin_linear/CONTRACT.md:26-91):
forward only; fp32 accumulation for bf16/fp16/fp32 inputs; deterministic
(fixed-order reductions, bit-identical across calls and graph replays); no
host sync, no value-dependent host branching and no allocation outside torch's
caching allocator, so it captures into a HIP graph.
"""
from __future__ import annotations

import torch

from . import _native

# Tuning knobs (kernels/thin_linear_fused.py:59-61).  MI355X has 256 CUs.
TARGET_CTAS = 256              # at least one workgroup on every CU
MAX_SPLIT_K = 16
MIN_K_PER_SPLIT = 512          # bf16 elements of every row per split (256 B per wave)
_ROWS = (4, 8, 16, 24, 32, 64, 96, 128)   # weight rows per workgroup the kernels are built for

_DEFAULT_WAVES = 4


def _next_pow2(n: int) -> int:
    n = max(int(n), 1)
    return 1 << (n - 1).bit_length()


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


# ─────────────────────────────────────────────────────────────────────────────
# Workspace (kernels/thin_linear_fused.py:173-190)
# ─────────────────────────────────────────────────────────────────────────────
# Split-K partial tiles (fp32) come from the torch caching allocator, one
# buffer per call.  The reference keeps one staging buffer per device and
# reuses it; here draft and target graphs replay on two streams at once (the
# speculative runner's overlap modes), and a captured graph keeps the address
# it was recorded with, so a shared buffer would be written by both at the
# same time.  Allocation per call costs host time only: inside a captured
# graph it is a fixed address in the graph's pool.
def _partials(dev: torch.device, nbytes: int) -> torch.Tensor:
    return torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)


def _scratch(dev: torch.device, nbytes: int) -> torch.Tensor:
    """A call's own scratch (the normalised rows of the RMSNorm + linear forms,
    plus their split-K partials)."""
    return _partials(dev, nbytes)


def reset_workspace() -> None:
    """Kept for the reference's API (kernels/thin_linear_fused.py:186-190).
    There is no cached staging buffer to drop: partials are per call."""
    return None


# ─────────────────────────────────────────────────────────────────────────────
# Configs (kernels/thin_linear_fused.py:193-262)
# ─────────────────────────────────────────────────────────────────────────────
# (K, N) -> (BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K, num_warps, num_stages).
# BLOCK_M is the largest M the entry covers.  Chosen by sweeping rows per
# workgroup x waves x split on one MI355X (M=4 for draft shapes, M=16 and 32
# for target shapes; bf16; HIP graph over a >= 1 GiB weight pool so the
# 256 MB MALL cannot serve repeats).  Entries not swept directly (separate
# gate/up, k/v and lm_head of the target) follow the nearest swept shape.
TUNED: dict[tuple[int, int], tuple[int, int, int, int, int, int]] = {
    # SDAR-1.7B draft projections (hidden 2048, 16 q / 8 kv heads, inter 6144)
    (2048, 2048): (16, 8, 1024, 1, 2, 2),     # q_proj, o_proj      4.0 us
    (2048, 1024): (16, 4, 1024, 1, 2, 2),     # k_proj, v_proj      3.2 us
    (2048, 6144): (16, 16, 256, 1, 4, 2),     # gate_proj, up_proj
    (6144, 2048): (16, 8, 256, 1, 8, 2),      # down_proj           6.6 us
    (2048, 151936): (16, 16, 256, 1, 4, 2),   # lm_head
    (2048, 4096): (16, 8, 256, 1, 4, 2),      # merged qkv          5.2 us
    (2048, 12288): (16, 16, 256, 1, 2, 2),    # merged gate+up     10.0 us
    # 8B-class target, verify rows M <= 64 (hidden 4096, 32 q / 8 kv, inter
    # 12288): K blocks of (4 data + 4 mask) rows, plus up to K committed
    # blocks folded in ahead of them (<= 48 rows at K = 4)
    (4096, 12288): (64, 32, 256, 1, 4, 2),    # gate_proj / up_proj
    (4096, 4096): (64, 16, 256, 1, 8, 2),     # q_proj, o_proj      8.7 / 11.2 us (M=16 / 32)
    (4096, 1024): (64, 16, 256, 4, 4, 2),     # k_proj, v_proj
    (4096, 6144): (64, 32, 256, 1, 4, 2),     # merged qkv         12.3 / 15.7 us
    (4096, 24576): (64, 32, 256, 1, 4, 2),    # merged gate+up     33.4 / 39.3 us
    (12288, 4096): (64, 16, 256, 1, 8, 2),    # down_proj          21.5 / 25.8 us
    (4096, 151936): (64, 32, 256, 1, 4, 2),   # lm_head
}

# Token ranges inside an entry's envelope where another geometry wins:
# (K, N) -> (((M_lo, M_hi), 6-tuple), ...), first match taken.  Same sweep as
# TUNED; 33-48 tokens is the verify with committed blocks folded in (one
# block at 36 rows), swept over rows x waves x split with 48-token column
# blocks.  Above 8 tokens these are the shared-activation tiles (64 weight rows
# per workgroup, waves splitting the rows) and, for the target's merged qkv,
# 24-row tiles (256 workgroups for its 6144 rows, where 32-row tiles leave 64
# CUs idle and 16-row tiles put two workgroups on half of them: 12.38 -> 11.62
# us at M=16, 15.81 -> 15.30 us at M=32); at 5-8 tokens the merged qkv with
# its RMSNorm prologue, where 16 rows per workgroup halve the workgroups that
# read both column sets' rows for the statistics (7.0-7.1 against 8.0-8.9 us
# with 8 rows; the plain projection moves by at most 0.4 us either way).
TUNED_RANGES: dict[tuple[int, int], tuple[tuple[tuple[int, int], tuple[int, int, int, int, int, int]], ...]] = {
    (2048, 4096): (((5, 8), (16, 16, 256, 1, 4, 2)),),      # merged qkv      7.1 us (M=8)
    (4096, 6144): (((9, 32), (32, 24, 256, 1, 4, 2)),       # merged qkv     11.6 / 15.3 us (M=16 / 32)
                   ((33, 48), (64, 24, 256, 2, 2, 2))),     #                17.7 / 18.3 us (M=36 / 48)
    (4096, 4096): (((33, 48), (64, 16, 256, 1, 4, 2)),),    # o_proj         12.7 / 13.1 us (M=36 / 48)
    (4096, 24576): (((33, 40), (64, 32, 256, 1, 2, 2)),     # gate+up (and the gated MLP) 45.3 us (M=36)
                    ((41, 48), (64, 96, 256, 1, 8, 2))),    #                46.2 us (M=48)
    (12288, 4096): (((9, 32), (32, 64, 256, 4, 4, 2)),      # down_proj   22.0 / 23.3 us (M=16 / 32)
                    ((33, 48), (64, 32, 256, 4, 2, 2))),    #             26.2 / 27.9 us (M=36 / 48)
    (4096, 151936): (((17, 32), (32, 64, 256, 1, 4, 2)),),  # lm_head      234 us (M=32)
}


def pick_config(M: int, N: int, K: int, itemsize: int = 2) -> tuple[int, int, int, int]:
    """(BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K) -- tuned where known, else heuristic."""
    full = _tuned_for(M, N, K)
    if full is not None:
        return full[0], full[1], full[2], full[3]
    return _heuristic_config(M, N, K, itemsize)


def _tuned_for(M: int, N: int, K: int):
    """The tuned 6-tuple, or None when this (M, K, N) is outside its envelope.

    An entry covers every M whose rounded-up block ``max(16, next_pow2(M))``
    fits its BLOCK_M: draft entries (BLOCK_M=16) stop at M=16, exactly the
    reference's rule (kernels/thin_linear_fused.py:232-242); target entries
    (BLOCK_M=64) extend to the multi-block verify with committed blocks folded
    in (32 rows plus up to 16).  Inside the
    envelope, the first ``TUNED_RANGES`` entry whose token range holds M
    takes over.
    """
    c = TUNED.get((K, N))
    if c is None or max(16, _next_pow2(max(M, 1))) > c[0]:
        return None
    for (lo, hi), cfg in TUNED_RANGES.get((K, N), ()):
        if lo <= M <= hi:
            return cfg
    return c


def _heuristic_config(M: int, N: int, K: int, itemsize: int = 2) -> tuple[int, int, int, int]:
    """Same rule as the library's automatic plan (``simsd_thin_linear_plan``).

    The most weight rows per workgroup (16, then 8, else 4) that still give
    every CU a workgroup (never below 16 for the 16x16 MFMA kernel above 8
    tokens); a split along K only when the tiles leave more than half the CUs
    idle.
    """
    if itemsize == 2 and M <= 8:        # 4x4x4 GEMV: 4 tokens per column set
        BLOCK_M, BLOCK_K = (4 if M <= 4 else 8), 256
    else:                               # 16x16 MFMA tiles: 1, 2 or (16-bit, 33..48 tokens) 3 column blocks
        BLOCK_M = 16 if M <= 16 else (48 if itemsize == 2 and 32 < M <= 48 else 32)
        BLOCK_K = (256 if BLOCK_M == 16 else 128) * 2 // itemsize
    m_tiles = _cdiv(M, BLOCK_M)
    BLOCK_N = 4
    for cand in (16, 8):
        if _cdiv(N, cand) * m_tiles >= TARGET_CTAS:
            BLOCK_N = cand
            break
    if itemsize == 2 and M > 8:
        BLOCK_N = 16
    tiles = _cdiv(N, BLOCK_N) * m_tiles
    split = 1
    if tiles < TARGET_CTAS // 2:
        split = _cdiv(TARGET_CTAS, tiles)
        split = max(1, min(split, MAX_SPLIT_K, (K * itemsize) // (MIN_K_PER_SPLIT * 2)))
    return BLOCK_M, BLOCK_N, BLOCK_K, split


def _rows_for(block_n: int) -> int:
    """The kernel's rows-per-workgroup for a requested BLOCK_N (round down)."""
    fit = [r for r in _ROWS if r <= max(int(block_n), _ROWS[0])]
    return fit[-1]


# ─────────────────────────────────────────────────────────────────────────────
# The op (kernels/thin_linear_fused.py:265-345)
# ─────────────────────────────────────────────────────────────────────────────
def thin_linear(x: torch.Tensor, w: torch.Tensor,
                bias: torch.Tensor | None = None,
                config: tuple[int, ...] | None = None,
                num_warps: int | None = None,
                num_stages: int | None = None) -> torch.Tensor:
    """`F.linear(x, w, bias)` for tiny M on the MI355X kernel.

    x: [..., K]  (leading dims are flattened, as `nn.Linear` does)
    w: [N, K]    (`nn.Linear.weight` layout)
    -> [..., N]
    """
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad):
        raise RuntimeError(
            "thin_linear is a forward-only inference kernel (contract mode="
            "inference); it has no backward. Call it under torch.no_grad() / "
            "torch.inference_mode(), or use F.linear for training.")
    if x.dtype != w.dtype:
        raise TypeError(f"dtype mismatch: x={x.dtype} w={w.dtype}")
    if w.ndim != 2:
        raise ValueError(f"w must be 2-D [N, K], got {tuple(w.shape)}")
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")

    out_shape = (*x.shape[:-1], w.shape[0])
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"K mismatch: x[..., {K}] vs w[{N}, {w.shape[1]}]")
    dev = _native.require_device(x2, w)

    if M == 0 or N == 0 or K == 0:
        y = torch.zeros((M, N), device=dev, dtype=x.dtype)
        if bias is not None:
            y += bias
        return y.view(out_shape)

    y = torch.empty((M, N), device=dev, dtype=x.dtype)

    if config is not None:
        block_n, block_k, split_k = int(config[1]), int(config[2]), int(config[3])
        waves = num_warps or _DEFAULT_WAVES
    else:
        tuned = _tuned_for(M, N, K)
        if tuned is not None:
            _, block_n, block_k, split_k, waves, _ = tuned
        else:
            _, block_n, block_k, split_k = _heuristic_config(M, N, K, x.element_size())
            waves = _DEFAULT_WAVES
        waves = num_warps or waves
    if split_k < 1:
        raise ValueError(f"SPLIT_K must be >= 1, got {split_k}")
    block_n = _rows_for(block_n)
    waves = 2 if waves <= 2 else (4 if waves <= 4 else 8)

    fuse_bias = (bias is not None and bias.dtype == x.dtype and bias.ndim == 1
                 and bias.shape[0] == N and bias.device == dev)
    lib = _native.lib()
    ws, ws_bytes = None, 0
    if split_k > 1:
        need = lib.simsd_thin_linear_workspace_bytes(M, N, K, code, block_n, split_k, waves)
        if need < 0:
            _native.check(-1, "thin_linear")
        ws = _partials(dev, need)
        ws_bytes = ws.numel()
    with _native.device_guard(dev):
        status = lib.simsd_thin_linear(
            x2.data_ptr(), x2.stride(0), x2.stride(1),
            w.data_ptr(), w.stride(0), w.stride(1),
            bias.data_ptr() if fuse_bias else None, bias.stride(0) if fuse_bias else 0,
            y.data_ptr(), y.stride(0), y.stride(1),
            M, N, K, code, block_n, block_k, split_k, waves,
            ws.data_ptr() if ws is not None else None, ws_bytes,
            _native.stream_of(dev))
    _native.check(status, "thin_linear")

    if bias is not None and not fuse_bias:
        y += bias
    return y.view(out_shape)


def _vec_rows(t: torch.Tensor) -> bool:
    """K-contiguous, 16-byte aligned rows (the fused kernels' operand form)."""
    es = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and (t.shape[-1] * es) % 16 == 0
            and (t.shape[0] == 1 or (t.stride(0) * es) % 16 == 0))


def thin_linear_silu_mul(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                         config: tuple[int, ...] | None = None,
                         num_warps: int | None = None) -> torch.Tensor:
    """``F.silu(F.linear(x, w_gate)) * F.linear(x, w_up)`` in one kernel.

    The gate and up projections of a SiLU-gated MLP (modeling_sdar.py:113-119)
    with the SiLU and the product in the epilogue: one pass over both weights
    and no [M, 2I] intermediate.  Rounding points as in PyTorch at the input
    dtype (each projection, the SiLU and the product rounded to it).  A merged
    gate_up weight [2I, K] is passed as its two halves (views, no copy).
    bf16/fp16 with K-contiguous 16-byte-aligned operands use the fused
    kernel; anything else runs the two projections through ``thin_linear``
    and the epilogue in PyTorch.  ``config`` is the merged (K, 2I) shape's.
    """
    if torch.is_grad_enabled() and (x.requires_grad or w_gate.requires_grad or w_up.requires_grad):
        raise RuntimeError(
            "thin_linear_silu_mul is a forward-only inference kernel; call it under "
            "torch.no_grad() / torch.inference_mode()")
    if not (x.dtype == w_gate.dtype == w_up.dtype):
        raise TypeError(f"dtype mismatch: x={x.dtype} w_gate={w_gate.dtype} w_up={w_up.dtype}")
    if w_gate.ndim != 2 or w_up.shape != w_gate.shape:
        raise ValueError(f"w_gate and w_up must both be [I, K], got {tuple(w_gate.shape)} "
                         f"and {tuple(w_up.shape)}")
    I, K = w_gate.shape
    if x.shape[-1] != K:
        raise ValueError(f"K mismatch: x[..., {x.shape[-1]}] vs w[{I}, {K}]")
    out_shape = (*x.shape[:-1], I)
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    dev = _native.require_device(x2, w_gate, w_up)
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")
    if M == 0 or I == 0:
        return torch.zeros(out_shape, device=dev, dtype=x.dtype)
    if (code == _native.DTYPE_CODES[torch.float32] or K == 0
            or not (_vec_rows(x2) and _vec_rows(w_gate) and _vec_rows(w_up))):
        g = thin_linear(x2, w_gate)
        return (torch.nn.functional.silu(g) * thin_linear(x2, w_up)).view(out_shape)

    h = torch.empty((M, I), device=dev, dtype=x.dtype)
    if config is not None:
        block_n, block_k, split_k = int(config[1]), int(config[2]), int(config[3])
        waves = num_warps or _DEFAULT_WAVES
    else:
        tuned = _tuned_for(M, 2 * I, K)
        if tuned is not None:
            _, block_n, block_k, split_k, waves, _ = tuned
        else:
            _, block_n, block_k, split_k = _heuristic_config(M, 2 * I, K, x.element_size())
            waves = _DEFAULT_WAVES
        waves = num_warps or waves
    if split_k < 1:
        raise ValueError(f"SPLIT_K must be >= 1, got {split_k}")
    block_n = _rows_for(block_n)
    waves = 2 if waves <= 2 else (4 if waves <= 4 else 8)
    lib = _native.lib()
    ws, ws_bytes = None, 0
    if split_k > 1:
        need = lib.simsd_thin_linear_workspace_bytes(M, 2 * I, K, code, block_n, split_k, waves)
        if need < 0:
            _native.check(-1, "thin_linear_silu_mul")
        ws = _partials(dev, need)
        ws_bytes = ws.numel()
    with _native.device_guard(dev):
        status = lib.simsd_thin_linear_silu_mul(
            x2.data_ptr(), x2.stride(0), x2.stride(1),
            w_gate.data_ptr(), w_gate.stride(0), w_gate.stride(1),
            w_up.data_ptr(), w_up.stride(0), w_up.stride(1),
            h.data_ptr(), h.stride(0), h.stride(1),
            M, I, K, code, block_n, block_k, split_k, waves,
            ws.data_ptr() if ws is not None else None, ws_bytes,
            _native.stream_of(dev))
    _native.check(status, "thin_linear_silu_mul")
    return h.view(out_shape)


def _launch_config(M: int, N_rows: int, K: int, itemsize: int, config, num_warps):
    """(block_n, block_k, split_k, waves) for a call: explicit config, else
    TUNED for (K, N_rows), else the heuristic."""
    if config is not None:
        block_n, block_k, split_k = int(config[1]), int(config[2]), int(config[3])
        waves = num_warps or _DEFAULT_WAVES
    else:
        tuned = _tuned_for(M, N_rows, K)
        if tuned is not None:
            _, block_n, block_k, split_k, waves, _ = tuned
        else:
            _, block_n, block_k, split_k = _heuristic_config(M, N_rows, K, itemsize)
            waves = _DEFAULT_WAVES
        waves = num_warps or waves
    if split_k < 1:
        raise ValueError(f"SPLIT_K must be >= 1, got {split_k}")
    return _rows_for(block_n), block_k, split_k, (2 if waves <= 2 else (4 if waves <= 4 else 8))


def thin_linear_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor,
                         out: torch.Tensor | None = None, config=None, num_warps=None) -> torch.Tensor:
    """``residual + thin_linear(x, w)`` in one launch (the decoder layer's
    ``hidden = residual + proj(...)``): the projection is rounded to the dtype,
    then added in the dtype, as PyTorch computes the two ops.  ``out`` may be
    ``residual`` itself (in place).  x: [M, K], w: [N, K], residual: [M, N]."""
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad or residual.requires_grad):
        raise RuntimeError("thin_linear_residual is a forward-only inference kernel; "
                           "call it under torch.no_grad() / torch.inference_mode()")
    if x.dtype != w.dtype or residual.dtype != x.dtype:
        raise TypeError(f"dtype mismatch: x={x.dtype} w={w.dtype} residual={residual.dtype}")
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")
    if x.ndim != 2 or w.ndim != 2 or w.shape[1] != x.shape[1]:
        raise ValueError(f"shapes: x {tuple(x.shape)}, w {tuple(w.shape)}")
    M, K = x.shape
    N = w.shape[0]
    if residual.shape != (M, N):
        raise ValueError(f"residual must be [{M}, {N}], got {tuple(residual.shape)}")
    dev = _native.require_device(x, w, residual, out)
    y = torch.empty((M, N), device=dev, dtype=x.dtype) if out is None else out
    if y.shape != (M, N) or y.dtype != x.dtype:
        raise ValueError(f"out must be [{M}, {N}] in {x.dtype}")
    if M == 0 or N == 0:
        return y
    if K == 0:
        y.copy_(residual)
        return y
    block_n, block_k, split_k, waves = _launch_config(M, N, K, x.element_size(), config, num_warps)
    lib = _native.lib()
    ws, ws_bytes = None, 0
    if split_k > 1:
        need = lib.simsd_thin_linear_workspace_bytes(M, N, K, code, block_n, split_k, waves)
        if need < 0:
            _native.check(-1, "thin_linear_residual")
        ws = _partials(dev, need)
        ws_bytes = ws.numel()
    with _native.device_guard(dev):
        status = lib.simsd_thin_linear_residual(
            x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), w.stride(0), w.stride(1),
            residual.data_ptr(), residual.stride(0), residual.stride(1),
            y.data_ptr(), y.stride(0), y.stride(1), M, N, K, code, block_n, block_k, split_k, waves,
            ws.data_ptr() if ws is not None else None, ws_bytes, _native.stream_of(dev))
    _native.check(status, "thin_linear_residual")
    return y


REDUCE_MAX_SPLIT = 8   # partials the consuming launches sum

# Geometries of thin_linear_partials where they differ from TUNED's:
# (K, N) -> (((M_lo, M_hi), 6-tuple), ...).  The partials pay no reduce
# launch of their own, so a split along K costs only the consumer's extra
# partial reads.  Swept on one MI355X over rows x waves x split, each point
# the partials launch plus its consumer (reduce + residual + RMSNorm, or
# reduce + q/k norm + RoPE + cache write) in a graph of 36 distinct weights:
# o_proj at 36 rows 16.6 -> 15.0 us, qkv at 32 rows 18.1 -> 16.5 us.
PARTIALS_RANGES: dict[tuple[int, int], tuple[tuple[tuple[int, int], tuple[int, int, int, int, int, int]], ...]] = {
    (4096, 6144): (((9, 48), (64, 24, 256, 2, 2, 2)),),          # merged qkv  14.0 / 16.5 / 18.8 / 19.5 us
    (4096, 4096): (((9, 16), (64, 16, 256, 2, 2, 2)),            # o_proj      11.1 us (M=16)
                   ((17, 32), (64, 64, 256, 4, 4, 2)),           #             12.8 us (M=32)
                   ((33, 40), (64, 32, 256, 4, 2, 2)),           #             15.0 us (M=36)
                   ((41, 48), (64, 32, 256, 2, 4, 2))),          #             15.7 us (M=48)
    (12288, 4096): (((9, 16), (64, 32, 256, 4, 2, 2)),           # down_proj   21.9 us (M=16)
                    ((17, 32), (64, 64, 256, 4, 4, 2)),          #             23.1 us (M=32)
                    ((33, 48), (64, 32, 256, 4, 2, 2))),         #             26.8 / 28.5 us (M=36 / 48)
}


def _partials_config(M: int, N: int, K: int):
    """The PARTIALS_RANGES 6-tuple for this call, or None (then TUNED's)."""
    for (lo, hi), cfg in PARTIALS_RANGES.get((K, N), ()):
        if lo <= M <= hi:
            return cfg
    return None


def thin_linear_partials(x: torch.Tensor, w: torch.Tensor, config=None, num_warps=None) -> torch.Tensor:
    """The split-K partials of ``x @ w.T`` without their reduce: fp32
    [split, M, N], partial s the sum over k-chunk s of the plan (the tuned
    split, at most 8; 1 is one partial over the whole K).  For the launches
    that sum them while doing work of their own -- ``reduce_residual_rmsnorm``
    and ``attention_fused.reduce_qkv_rope_cache`` -- so a projection splits
    K at no extra launch (the reference's split-K staging,
    kernels/thin_linear_fused.py:139-171, summed by its own launch)."""
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad):
        raise RuntimeError("thin_linear_partials is a forward-only inference kernel")
    if x.dtype != w.dtype:
        raise TypeError(f"dtype mismatch: x={x.dtype} w={w.dtype}")
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")
    if x.ndim != 2 or w.ndim != 2 or w.shape[1] != x.shape[1]:
        raise ValueError(f"shapes: x {tuple(x.shape)}, w {tuple(w.shape)}")
    M, K = x.shape
    N = w.shape[0]
    dev = _native.require_device(x, w)
    if config is None and x.element_size() == 2:
        cfg = _partials_config(M, N, K)
        if cfg is not None:
            config, num_warps = cfg[:4], num_warps or cfg[4]
    block_n, block_k, split_k, waves = _launch_config(M, N, K, x.element_size(), config, num_warps)
    split_k = max(1, min(split_k, REDUCE_MAX_SPLIT))
    part = torch.empty((split_k, M, N), device=dev, dtype=torch.float32)
    if M == 0 or N == 0:
        return part
    if K == 0:
        return part.zero_()
    with _native.device_guard(dev):
        status = _native.lib().simsd_thin_linear_partials(
            x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), w.stride(0), w.stride(1),
            part.data_ptr(), part.numel() * 4, M, N, K, code, block_n, block_k, split_k, waves,
            _native.stream_of(dev))
    _native.check(status, "thin_linear_partials")
    return part


def reduce_residual_rmsnorm(part: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                            out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The decoder layer's residual add and the next RMSNorm on a projection
    given as its partials (``thin_linear_partials``), in one launch:
    ``h = residual + proj`` (the projection's sum rounded to the dtype, then
    the dtype add) and ``xn = weight * (h * rsqrt(mean(h^2) + eps)).to(dtype)``
    (the stock RMSNorm), bit-identical to ``thin_linear_residual`` followed by
    ``thin_rmsnorm``.  ``out`` (the h buffer) may be ``residual`` itself.
    bf16/fp16, N % 8 == 0, N <= 8192.  -> (h, xn)."""
    if part.dtype != torch.float32 or part.ndim != 3 or not part.is_contiguous():
        raise ValueError("reduce_residual_rmsnorm: partials must be contiguous fp32 [split, M, N]")
    split, M, N = part.shape
    code = _native.DTYPE_CODES.get(residual.dtype)
    if code is None or residual.dtype == torch.float32:
        raise TypeError(f"reduce_residual_rmsnorm: dtype must be bf16 or fp16, got {residual.dtype}")
    if residual.shape != (M, N) or residual.stride(1) != 1:
        raise ValueError(f"reduce_residual_rmsnorm: residual must be [{M}, {N}] with unit column stride")
    if weight.shape != (N,) or weight.dtype != residual.dtype:
        raise ValueError(f"reduce_residual_rmsnorm: weight must be [{N}] in {residual.dtype}")
    if not 1 <= split <= REDUCE_MAX_SPLIT:
        raise ValueError(f"reduce_residual_rmsnorm: split {split} outside 1..{REDUCE_MAX_SPLIT}")
    dev = _native.require_device(part, residual, weight, out)
    h = torch.empty((M, N), device=dev, dtype=residual.dtype) if out is None else out
    if h.shape != (M, N) or h.dtype != residual.dtype or h.stride(1) != 1:
        raise ValueError(f"reduce_residual_rmsnorm: out must be [{M}, {N}] in {residual.dtype}")
    xn = torch.empty((M, N), device=dev, dtype=residual.dtype)
    if M == 0 or N == 0:
        return h, xn
    g = weight.contiguous()
    with _native.device_guard(dev):
        status = _native.lib().simsd_reduce_residual_rmsnorm(
            part.data_ptr(), split, part.numel() * 4, residual.data_ptr(), residual.stride(0),
            h.data_ptr(), h.stride(0), g.data_ptr(), float(eps), xn.data_ptr(), xn.stride(0), M, N, code,
            _native.stream_of(dev))
    _native.check(status, "reduce_residual_rmsnorm")
    return h, xn


def _norm_args(x: torch.Tensor, weight: torch.Tensor):
    if weight.ndim != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"RMSNorm weight must be [{x.shape[-1]}], got {tuple(weight.shape)}")
    if weight.dtype != x.dtype:
        raise TypeError(f"RMSNorm weight dtype {weight.dtype} != x dtype {x.dtype}")
    code = _native.DTYPE_CODES.get(x.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {x.dtype} (bf16, fp16 or fp32)")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2, weight.contiguous(), code


def thin_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm in one launch: ``weight * (x * rsqrt(mean(x^2) + eps)).to(x.dtype)``
    with the fp32 statistics and the rounding points of the stock PyTorch
    form (SDARRMSNorm, sdar/modeling_sdar.py:74-92; sdar/run_native_tp2.py:42-47)."""
    x2, g, code = _norm_args(x, weight)
    dev = _native.require_device(x2, g)
    M, K = x2.shape
    y = torch.empty((M, K), device=dev, dtype=x.dtype)
    if M == 0:
        return y.view(x.shape)
    with _native.device_guard(dev):
        st = _native.lib().simsd_rmsnorm(x2.data_ptr(), x2.stride(0), g.data_ptr(), float(eps),
                                         y.data_ptr(), y.stride(0), M, K, code, _native.stream_of(dev))
    _native.check(st, "rmsnorm")
    return y.view(x.shape)


def thin_rmsnorm_linear(x: torch.Tensor, weight: torch.Tensor, eps: float, w: torch.Tensor,
                        bias: torch.Tensor | None = None, config=None, num_warps=None) -> torch.Tensor:
    """``thin_linear(thin_rmsnorm(x, weight, eps), w, bias)``; at <= 8 tokens the
    norm runs inside the GEMV and the normalised rows never reach memory
    (unless the output is lm_head-sized: then every workgroup's statistics
    pass would cost more than a separate norm launch)."""
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad):
        raise RuntimeError("thin_rmsnorm_linear is a forward-only inference kernel")
    if w.ndim != 2 or w.shape[1] != x.shape[-1]:
        raise ValueError(f"w must be [N, {x.shape[-1]}], got {tuple(w.shape)}")
    if w.dtype != x.dtype:
        raise TypeError(f"dtype mismatch: x={x.dtype} w={w.dtype}")
    x2, g, code = _norm_args(x, weight)
    dev = _native.require_device(x2, g, w)
    (M, K), N = x2.shape, w.shape[0]
    out_shape = (*x.shape[:-1], N)
    if M == 0 or N == 0:
        return torch.zeros(out_shape, device=dev, dtype=x.dtype)
    block_n, block_k, split_k, waves = _launch_config(M, N, K, x.element_size(), config, num_warps)
    fuse_bias = (bias is not None and bias.dtype == x.dtype and bias.ndim == 1
                 and bias.shape[0] == N and bias.device == dev)
    lib = _native.lib()
    need = lib.simsd_rmsnorm_linear_workspace_bytes(M, N, K, code, block_n, split_k, waves)
    if need < 0:
        _native.check(-1, "rmsnorm_thin_linear")
    ws = _scratch(dev, need)
    y = torch.empty((M, N), device=dev, dtype=x.dtype)
    with _native.device_guard(dev):
        st = lib.simsd_rmsnorm_thin_linear(
            x2.data_ptr(), x2.stride(0), 1, g.data_ptr(), float(eps),
            w.data_ptr(), w.stride(0), w.stride(1),
            bias.data_ptr() if fuse_bias else None, bias.stride(0) if fuse_bias else 0,
            y.data_ptr(), y.stride(0), y.stride(1), M, N, K, code, block_n, block_k, split_k, waves,
            ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    _native.check(st, "rmsnorm_thin_linear")
    if bias is not None and not fuse_bias:
        y += bias
    return y.view(out_shape)


def thin_rmsnorm_linear_silu_mul(x: torch.Tensor, weight: torch.Tensor, eps: float,
                                 w_gate: torch.Tensor, w_up: torch.Tensor,
                                 config=None, num_warps=None) -> torch.Tensor:
    """``thin_linear_silu_mul(thin_rmsnorm(x, weight, eps), w_gate, w_up)``: an
    MLP block's norm, gate and up projections, SiLU and product; at <= 8
    tokens in one kernel.  bf16/fp16 with vector-aligned weights; other
    inputs go through the two separate ops."""
    if torch.is_grad_enabled() and (x.requires_grad or w_gate.requires_grad or w_up.requires_grad):
        raise RuntimeError("thin_rmsnorm_linear_silu_mul is a forward-only inference kernel")
    if not (x.dtype == w_gate.dtype == w_up.dtype):
        raise TypeError(f"dtype mismatch: x={x.dtype} w_gate={w_gate.dtype} w_up={w_up.dtype}")
    if w_gate.ndim != 2 or w_up.shape != w_gate.shape or w_gate.shape[1] != x.shape[-1]:
        raise ValueError(f"w_gate and w_up must both be [I, {x.shape[-1]}]")
    x2, g, code = _norm_args(x, weight)
    dev = _native.require_device(x2, g, w_gate, w_up)
    (M, K), I = x2.shape, w_gate.shape[0]
    out_shape = (*x.shape[:-1], I)
    if M == 0 or I == 0:
        return torch.zeros(out_shape, device=dev, dtype=x.dtype)
    if code == _native.DTYPE_CODES[torch.float32] or not (_vec_rows(w_gate) and _vec_rows(w_up)):
        return thin_linear_silu_mul(thin_rmsnorm(x2, g, eps), w_gate, w_up).view(out_shape)
    block_n, block_k, split_k, waves = _launch_config(M, 2 * I, K, x.element_size(), config, num_warps)
    lib = _native.lib()
    need = lib.simsd_rmsnorm_linear_workspace_bytes(M, 2 * I, K, code, block_n, split_k, waves)
    if need < 0:
        _native.check(-1, "rmsnorm_thin_linear_silu_mul")
    ws = _scratch(dev, need)
    h = torch.empty((M, I), device=dev, dtype=x.dtype)
    with _native.device_guard(dev):
        st = lib.simsd_rmsnorm_thin_linear_silu_mul(
            x2.data_ptr(), x2.stride(0), 1, g.data_ptr(), float(eps),
            w_gate.data_ptr(), w_gate.stride(0), w_gate.stride(1),
            w_up.data_ptr(), w_up.stride(0), w_up.stride(1),
            h.data_ptr(), h.stride(0), h.stride(1), M, I, K, code, block_n, block_k, split_k, waves,
            ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    _native.check(st, "rmsnorm_thin_linear_silu_mul")
    return h.view(out_shape)


def should_fuse(M: int, N: int, K: int) -> bool:
    """Is the fused kernel the production choice for this shape?

    Only inside a tuned entry's envelope (M <= 16 for draft shapes, M <= 32
    for target shapes), as in kernels/thin_linear_fused.py:348-377.  Outside it
    ``ThinLinear`` hands the call to ``F.linear`` (hipBLASLt), which is
    bit-exactly the stock path -- prefill must reproduce the stock KV cache.
    """
    return _tuned_for(M, N, K) is not None


class ThinLinear(torch.nn.Module):
    """`nn.Linear` drop-in that routes the forward through `thin_linear`.

    Holds a *reference* to the original module's parameters (no copy), so
    swapping it in costs no memory and `state_dict()` round-trips unchanged.
    Falls back to `F.linear` outside the tuned envelope (see `should_fuse`).
    """

    def __init__(self, linear: torch.nn.Linear,
                 config: tuple[int, int, int, int] | None = None,
                 always_fuse: bool = False):
        super().__init__()
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.weight = linear.weight
        self.bias = linear.bias
        self.config = config
        self.always_fuse = always_fuse

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        M = x.numel() // x.shape[-1]
        if (self.config is not None or self.always_fuse
                or should_fuse(M, self.out_features, self.in_features)):
            return thin_linear(x, self.weight, self.bias, config=self.config)
        return torch.nn.functional.linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, fused=mi355x-skinny-mfma "
                f"(tuned envelope only unless always_fuse)")


# ─────────────────────────────────────────────────────────────────────────────
# Bench hook (kernels/thin_linear_fused.py:418-419)
# ─────────────────────────────────────────────────────────────────────────────
def make_bench_fn(x, pool, sh):
    return lambda i: thin_linear(x, pool[i])
