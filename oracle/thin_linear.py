"""Oracle of the skinny linear (test infrastructure only).

The reference's correctness target is ``torch.nn.functional.linear``
(``ref_thin_linear``, kernels/workspace/thin_linear/CONTRACT.md:31-38): for
bf16/fp16 inputs an fp32-accumulated product rounded once to the input dtype,
plus bias (``y += bias`` after the GEMM, kernels/thin_linear_fused.py:343-344).

``linear_exact``      y = dtype( sum_k x[m,k] w[n,k] ) with the sum in fp64
                      (exact for fixture-sized integer data, within fp64
                      rounding otherwise) -- the closed form.
``linear_cpu_torch``  torch's CPU ``F.linear`` in the input dtype -- the
                      reference's own oracle run on the host; also the timed
                      CPU path of the benchmark.
``gated_exact``       silu(x w_gate^T) * (x w_up^T) with the rounding points of
                      a bf16/fp16 SDARMLP (modeling_sdar.py:113-119): each
                      projection, the SiLU and the product rounded to the dtype.
``rmsnorm_exact``     the stock RMSNorm (sdar/run_native_tp2.py:42-47): the
                      mean of squares in fp64, x * r rounded to the dtype, times
                      the weight, rounded again.
``linear_residual_exact``  residual + linear_exact(x, w): the projection
                      rounded to the dtype, then the dtype add (the decoder
                      layer's ``hidden = residual + proj(...)``).
``tolerance``         the reference's bounds (thin_linear_fused_test.py:28-32).
"""
from __future__ import annotations

import numpy as np

from .numerics import ROUNDERS


def linear_exact(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None,
                 dtype: str = "bf16") -> np.ndarray:
    """x [M, K], w [N, K] (values already representable in `dtype`) -> [M, N].

    Follows kernels/thin_linear_fused.py:265-345: flatten handled by the
    caller, product then bias, result in the input dtype.
    """
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    y = ROUNDERS[dtype](x64 @ w64.T)
    if bias is not None:
        y = ROUNDERS[dtype](y + np.asarray(bias, dtype=np.float64)[None, :])
    return y


def gated_exact(x: np.ndarray, w_gate: np.ndarray, w_up: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """h = rnd(rnd(silu(g)) * u) with g = linear_exact(x, w_gate), u = linear_exact(x, w_up);
    the SiLU in fp64 (v / (1 + e^-v)) before its rounding."""
    rnd = ROUNDERS[dtype]
    g = linear_exact(x, w_gate, dtype=dtype)
    u = linear_exact(x, w_up, dtype=dtype)
    return rnd(rnd(g / (1.0 + np.exp(-g))) * u)


def rmsnorm_exact(x: np.ndarray, weight: np.ndarray, eps: float, dtype: str = "bf16") -> np.ndarray:
    """rnd(weight * rnd(x * r)), r = 1 / sqrt(mean(x^2) + eps) per row."""
    rnd = ROUNDERS[dtype]
    x64 = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + eps)
    return rnd(np.asarray(weight, dtype=np.float64) * rnd(x64 * r))


def linear_residual_exact(x: np.ndarray, w: np.ndarray, residual: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """rnd(rnd(x w^T) + residual), the add formed in fp32 as the dtype's add."""
    y = linear_exact(x, w, dtype=dtype)
    s = (y + np.asarray(residual, dtype=np.float64)).astype(np.float32).astype(np.float64)
    return ROUNDERS[dtype](s)


def linear_cpu_torch(x, w, bias=None):
    """torch CPU ``F.linear`` (the reference oracle ``ref_thin_linear``)."""
    import torch
    import torch.nn.functional as F

    with torch.inference_mode():
        return F.linear(x, w, bias)


def tolerance(ref_absmax: float, dtype: str) -> float:
    """Pointwise bound vs the reference: bf16/fp16 2^-7*max|ref| + 1e-3,
    fp32 1e-5*max(1, max|ref|) (kernels/thin_linear_fused_test.py:28-32)."""
    if dtype == "fp32":
        return 1e-5 * max(1.0, ref_absmax)
    return 2 ** -7 * ref_absmax + 1e-3


def max_abs_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref| (the parity bar of the bf16 linear is <= 1e-2)."""
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.abs(ref).max()) if ref.size else 0.0
    err = float(np.abs(np.asarray(got, dtype=np.float64) - ref).max()) if ref.size else 0.0
    return err / den if den > 0 else err
