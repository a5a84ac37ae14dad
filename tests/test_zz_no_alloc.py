"""simsd_thin_linear_noalloc, the allocation-free form of simsd_thin_linear,
called through the C ABI: two calls in a row (the second smaller, so it runs
over what the first left in the library's static scratch array) each equal
simsd_thin_linear with a caller workspace bit for bit and the oracle within
the reference's bf16 bound; explicit splits make both calls use the scratch
array.  A plan that needs more scratch than the array holds is refused."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import thin_linear as othin

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _rnd(*shape, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(torch.bfloat16)


def _args(x, w, y):
    return (x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), w.stride(0), w.stride(1), None, 0,
            y.data_ptr(), y.stride(0), y.stride(1), x.shape[0], w.shape[0], x.shape[1], 0)


def test_noalloc_equals_workspace_entry_point():
    from kernels import _native
    lib = _native.lib()
    stream = _native.stream_of(torch.device(DEV))
    # (M, N, K, rows per workgroup, split): a larger call, then a smaller one
    for M, N, K, rows, split in ((8, 3000, 8192, 8, 8), (3, 700, 4096, 4, 4)):
        print(f"noalloc M={M} N={N} K={K} split={split}", flush=True)
        x, w = _rnd(M, K, seed=M), _rnd(N, K, scale=0.02, seed=N)
        need = lib.simsd_thin_linear_workspace_bytes(M, N, K, 0, rows, split, 4)
        assert 0 < need <= lib.simsd_thin_linear_noalloc_max_scratch_bytes()
        ws = torch.empty(need, device=DEV, dtype=torch.uint8)
        y_ws = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        y_na = torch.full((M, N), float("nan"), device=DEV, dtype=torch.bfloat16)
        _native.check(lib.simsd_thin_linear(*_args(x, w, y_ws), rows, 0, split, 4, ws.data_ptr(), need, stream),
                      "thin_linear")
        _native.check(lib.simsd_thin_linear_noalloc(*_args(x, w, y_na), rows, 0, split, 4, stream),
                      "thin_linear_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ws)
        ref = othin.linear_exact(x.double().cpu().numpy(), w.double().cpu().numpy())
        err = float(np.abs(y_na.double().cpu().numpy() - ref).max())
        assert err <= othin.tolerance(float(np.abs(ref).max()), "bf16")
        assert othin.max_abs_rel(y_na.double().cpu().numpy(), ref) <= 1e-2


def test_noalloc_refuses_oversized_scratch():
    from kernels import _native
    lib = _native.lib()
    cap = lib.simsd_thin_linear_noalloc_max_scratch_bytes()
    M, N, K, split = 32, 24576, 4096, 16
    assert lib.simsd_thin_linear_workspace_bytes(M, N, K, 0, 32, split, 4) > cap
    x, w = _rnd(M, K), _rnd(N, K, scale=0.02)
    y = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    st = lib.simsd_thin_linear_noalloc(*_args(x, w, y), 32, 0, split, 4, _native.stream_of(torch.device(DEV)))
    assert st == -1
    assert b"static maximum" in lib.simsd_last_error_string()
