"""tv_stream_read, the streaming-read measurement helper (include/tv_bench.h)."""

import ctypes

import pytest

from tinyvllm_amd import _lib


def test_rejects_bad_arguments_on_the_host():
    lib = _lib.load()
    assert lib.tv_stream_read(None, 1024, 0, 4, 8, 0, None, None) == _lib.TV_EINVAL
    fake = ctypes.c_void_p(1 << 20)      # never dereferenced: validation fails first
    assert lib.tv_stream_read(fake, 1000, 0, 4, 8, 0, fake, None) == _lib.TV_EINVAL      # not a multiple of 16
    assert lib.tv_stream_read(fake, 1024, 0, 4, 0, 0, fake, None) == _lib.TV_EINVAL      # no work-groups
    assert lib.tv_stream_read(fake, 1024, 0, 3, 8, 1, fake, None) == _lib.TV_EINVAL      # unsupported depth
    assert b"loads_in_flight" in lib.tv_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("nt", [0, 1])
@pytest.mark.parametrize("u", [4, 8])
@pytest.mark.parametrize("contiguous", [0, 1])
def test_reads_without_writing(nt, u, contiguous):
    import torch
    lib = _lib.load()
    buf = torch.full((1 << 20,), 3, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    # 1 MiB + a tail that is not a multiple of the grid's stride
    n = (1 << 20) - 16 * 7
    rc = lib.tv_stream_read(ctypes.c_void_p(buf.data_ptr()), n, nt, u, 64, contiguous, ctypes.c_void_p(sink.data_ptr()),
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0, lib.tv_last_error()
    assert int(sink.abs().sum()) == 0
