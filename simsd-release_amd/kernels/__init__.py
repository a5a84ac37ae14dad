"""SimSD matmul hot path on MI355X: the ``kernels`` package of the reference,
re-implemented over hand-written gfx950 HIP kernels (libsimsd_kernels.so).

Modules keep the reference's names so callers switch by path alone:
``kernels.thin_linear_fused``, ``kernels.moe_dispatch_fused``,
``kernels.fused_toggle``.
"""
