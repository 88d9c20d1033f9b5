"""The streaming-read calibration kernel behind bench.py's plain_read figures:
it reads, writes nothing (the sink keeps its value unless the checksum hits
its impossible marker) and rejects misaligned arguments."""
import pytest
import torch

from serving import _native

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_stream_read_reads_and_writes_nothing():
    lib = _native.lib()
    buf = torch.arange(1 << 20, dtype=torch.int32, device=DEV)
    sink = torch.full((4,), 7, dtype=torch.int32, device=DEV)
    sp = torch.cuda.current_stream().cuda_stream
    for grid in (1, 64, 4096):
        _native.check(lib.pkv_stream_read(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), grid,
                                          sp), "stream_read")
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7, 7, 7]
    assert torch.equal(buf, torch.arange(1 << 20, dtype=torch.int32, device=DEV))


def test_stream_read_rejects_bad_arguments():
    lib = _native.lib()
    buf = torch.zeros(64, dtype=torch.int32, device=DEV)
    sp = torch.cuda.current_stream().cuda_stream
    assert lib.pkv_stream_read(buf.data_ptr() + 4, 64, None, 16, sp) == _native.PKV_ERR_INVALID
    assert lib.pkv_stream_read(buf.data_ptr(), 60, None, 16, sp) == _native.PKV_ERR_INVALID
    assert lib.pkv_stream_read(buf.data_ptr(), 64, None, 0, sp) == _native.PKV_ERR_INVALID
    assert lib.pkv_stream_read(None, 64, None, 16, sp) == _native.PKV_ERR_INVALID
    assert lib.pkv_stream_read(buf.data_ptr(), 0, None, 16, sp) == 0
