"""ullm_hip_stream_read, the read-floor calibration kernel used by bench.py:
it reads every byte once and leaves the sink alone unless the XOR fold of
the data hits its sentinel."""
import ctypes as C

import pytest
import torch

from ullm_amd import _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4 << 20, 1024), ((1 << 20) + 48, 7)])
def test_stream_read_runs_and_keeps_sink(nbytes, grid):
    dev = torch.device("cuda")
    src = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    sink = torch.full((grid,), -1, dtype=torch.int32, device=dev)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    L.check(L.lib().ullm_hip_stream_read(C.c_void_p(src.data_ptr()), nbytes, grid,
                                         C.c_void_p(sink.data_ptr()), st))
    torch.cuda.synchronize()
    assert (sink == -1).all()


def test_stream_read_sentinel_is_written():
    """Data folding to the sentinel 0x9e3779b9 is reported by its workgroup:
    the loads are live (the compiler cannot drop them)."""
    dev = torch.device("cuda")
    src = torch.zeros(64 * 4, dtype=torch.int32, device=dev)  # 1 KiB, one workgroup
    src[0] = torch.tensor(0x9E3779B9, dtype=torch.int64).to(torch.int32)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    L.check(L.lib().ullm_hip_stream_read(C.c_void_p(src.data_ptr()), src.numel() * 4, 1,
                                         C.c_void_p(sink.data_ptr()), st))
    torch.cuda.synchronize()
    assert int(sink[0]) & 0xFFFFFFFF == 0x9E3779B9
