"""strata_bench_read (the plain-read floor helper bench.py measures the GEMV
set against) through the C ABI: it reads without writing, and rejects
arguments outside its contract."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_bench_read_reads_without_writing_and_checks_arguments(dev):
    from lokahi_amd import _abi
    from lokahi_amd.ops import _ctx, _stream
    lib = _abi.load()
    buf = torch.arange(1 << 20, dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    for wpc, u in ((1, 4), (4, 8), (16, 16)):
        _abi.check(lib.strata_bench_read(_ctx(0), buf.data_ptr(), buf.numel() * 4 - 48, wpc, u,
                                         sink.data_ptr(), _stream(0)))
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    for nbytes, wpc, u in ((0, 4, 8), (100, 4, 8), (4096, 0, 8), (4096, 17, 8), (4096, 4, 3)):
        rc = lib.strata_bench_read(_ctx(0), buf.data_ptr(), nbytes, wpc, u, sink.data_ptr(),
                                   _stream(0))
        assert rc == _abi.STRATA_EINVAL, (nbytes, wpc, u)
