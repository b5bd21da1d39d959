"""The HBM calibration kernels behind the bench's measured peak (aspire_bandwidth_probe)."""

import pytest
import torch

from aspire_amd import _lib
from helpers import say

pytestmark = pytest.mark.gpu


def _probe(mode, src, nbytes, dst, dst_bytes, wgs, depth=4):
    return _lib.lib().aspire_bandwidth_probe(mode, _lib.ptr(src), nbytes, _lib.ptr(dst), dst_bytes, wgs, depth,
                                             _lib.stream_of(src))


@pytest.mark.parametrize("wgs,depth", [(1, 4), (7, 16), (2048, 1), (300, 2), (33, 8)])
def test_copy_probe_copies_every_byte(gpu, wgs, depth):
    """The copy mode moves every 16-byte chunk exactly once, whatever the grid (a grid larger
    than the buffer's chunks, one that does not divide it, one workgroup), and writes nothing
    past ``bytes``."""
    say("bandwidth probe copy", wgs, depth)
    n = (1 << 20) + 3 * 1024
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device=gpu)
    dst = torch.zeros(n + 4096, dtype=torch.uint8, device=gpu)
    _lib.check(_probe(1, src, n, dst, dst.numel(), wgs, depth), "copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:n], src)
    assert not dst[n:].any()


def test_read_probe_runs_and_checks_its_sink(gpu):
    """The streaming read runs over a buffer that is not a multiple of the grid's rows in
    flight; a sink smaller than workgroups * 1024 bytes (or than the bytes of a copy) and sizes
    that are not whole 1 KiB rows are refused on the host."""
    say("bandwidth probe read")
    n = 37 * 1024 * 1024 + 5 * 1024
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device=gpu)
    sink = torch.zeros(512 * 1024, dtype=torch.uint8, device=gpu)
    for depth in (1, 2, 4, 8, 16):
        _lib.check(_probe(0, src, n, sink, sink.numel(), 512, depth), "read")
    torch.cuda.synchronize()
    assert _probe(0, src, n, sink, sink.numel(), 512, 3) == _lib.ASPIRE_ERR_INVALID
    assert _probe(0, src, n, sink, sink.numel(), 513) == _lib.ASPIRE_ERR_INVALID
    assert _probe(0, src, n - 16, sink, sink.numel(), 512) == _lib.ASPIRE_ERR_INVALID
    assert _probe(1, src, n, sink, sink.numel(), 512) == _lib.ASPIRE_ERR_INVALID
