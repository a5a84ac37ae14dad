"""The measurement probes behind bench.py --workload floor: the empty launch
runs, and the read probe covers every workgroup of a ragged grid at every
geometry (each writes its fold; all-zero rows fold to zero), and refuses bad
geometry."""
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
