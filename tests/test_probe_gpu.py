"""The measurement probes behind bench.py --workload floor and gemv_valu: the
empty launch runs; the read probe covers every workgroup of a ragged grid at
every geometry (each writes its fold; all-zero rows fold to zero) and refuses
bad geometry; the VALU form of the M <= 4 linear matches the oracle."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


@pytest.mark.parametrize("rows_per_wg", [4, 8, 16])
@pytest.mark.parametrize("waves", [1, 2, 4, 8])
def test_read_probe_covers_every_workgroup(rows_per_wg, waves):
    from kernels import _native
    lib = _native.lib()
    rows, row_bytes = 1003, 4096
    buf = torch.zeros(rows * row_bytes // 2, dtype=torch.bfloat16, device=DEV)
    wgs = -(-rows // rows_per_wg)
    sink = torch.full((wgs + 1,), -1, dtype=torch.int32, device=DEV)
    s = _native.stream_of(torch.device(DEV))
    _native.check(lib.simsd_probe_empty(s), "probe_empty")
    _native.check(lib.simsd_probe_read(buf.data_ptr(), rows, row_bytes, rows_per_wg, waves, sink.data_ptr(),
                                       sink.numel(), s), "probe_read")
    torch.cuda.synchronize()
    assert (sink[:wgs] == 0).all() and int(sink[wgs]) == -1


def test_read_probe_rejects_bad_geometry():
    from kernels import _native
    lib = _native.lib()
    buf = torch.zeros(4096, dtype=torch.bfloat16, device=DEV)
    sink = torch.zeros(64, dtype=torch.int32, device=DEV)
    s = _native.stream_of(torch.device(DEV))
    assert lib.simsd_probe_read(buf.data_ptr(), 8, 1024, 32, 2, sink.data_ptr(), 64, s) == -1
    assert lib.simsd_probe_read(buf.data_ptr(), 8, 1024, 4, 3, sink.data_ptr(), 64, s) == -1
    assert lib.simsd_probe_read(buf.data_ptr(), 8, 1000, 4, 2, sink.data_ptr(), 64, s) == -1
    assert lib.simsd_probe_read(buf.data_ptr(), 64, 128, 4, 2, sink.data_ptr(), 8, s) == -1


@pytest.mark.parametrize("M", [1, 3, 4])
def test_valu_gemv_probe_vs_oracle(M):
    """The VALU form of the M <= 4 linear computes the same product as the
    product path: against the oracle's exact sum (bf16 tolerance and the
    1e-2 max-abs-rel bar) at the C1/C2 shapes and at ragged ones (N not a
    multiple of the row tile, K not a multiple of the 512-element chunk), at
    every geometry; bitwise stable across calls."""
    import numpy as np
    from kernels import _native
    from oracle import thin_linear as othin
    lib = _native.lib()
    s = _native.stream_of(torch.device(DEV))
    g = torch.Generator(device=DEV).manual_seed(M)
    for K, N in [(2048, 12288), (2048, 2048), (6144, 2048), (1000, 531), (8, 17)]:
        x = torch.randn(M, K, generator=g, device=DEV).bfloat16()
        w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).bfloat16()
        ref = othin.linear_exact(x.float().cpu().numpy(), w.float().cpu().numpy(), dtype="bf16")
        amax = float(np.abs(ref).max())
        for rows in (8, 16):
            for waves in (2, 4, 8):
                y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
                _native.check(lib.simsd_probe_gemv_valu(x.data_ptr(), K, w.data_ptr(), K, y.data_ptr(), N, M, N, K,
                                                        rows, waves, s), "probe_gemv_valu")
                y2 = torch.empty_like(y)
                _native.check(lib.simsd_probe_gemv_valu(x.data_ptr(), K, w.data_ptr(), K, y2.data_ptr(), N, M, N, K,
                                                        rows, waves, s), "probe_gemv_valu")
                torch.cuda.synchronize()
                assert torch.equal(y, y2)
                got = y.float().cpu().numpy()
                err = float(np.abs(got - ref).max())
                assert err <= othin.tolerance(amax, "bf16"), (K, N, rows, waves, err)
                assert othin.max_abs_rel(got, ref) <= 1e-2


def test_valu_gemv_probe_rejects_bad_shapes():
    from kernels import _native
    lib = _native.lib()
    s = _native.stream_of(torch.device(DEV))
    x = torch.zeros(8, 8192, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 8192, dtype=torch.bfloat16, device=DEV)
    y = torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV)
    p = (x.data_ptr(), 8192, w.data_ptr(), 8192, y.data_ptr(), 64)
    assert lib.simsd_probe_gemv_valu(*p, 5, 64, 2048, 16, 4, s) == -1      # M > 4
    assert lib.simsd_probe_gemv_valu(*p, 4, 64, 8192, 16, 4, s) == -1      # K past the staged rows
    assert lib.simsd_probe_gemv_valu(*p, 4, 64, 2044, 16, 4, s) == -1      # K % 8
    assert lib.simsd_probe_gemv_valu(*p, 4, 64, 2048, 4, 4, s) == -1       # rows per workgroup
    assert lib.simsd_probe_gemv_valu(*p, 4, 64, 2048, 16, 3, s) == -1      # waves
