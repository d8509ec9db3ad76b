"""The measurement exports (include/pk_hip.h: pk_hip_empty_dev,
pk_hip_stream_read_dev, pk_hip_mfma_rate_dev), which bench.py times the
launch floor, the read floor and both published peaks with: they run, the
streaming read reaches every 16 bytes it is given (the unrolled part of its
grid-stride loop and the rest), and their argument checks refuse."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAGIC = 0x9E3779B9      # a read folds to it only where the buffer holds it


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch
    assert torch.cuda.is_available()
    return torch


def test_stream_read_reaches_every_piece(hip, torch):
    """One word set to the fold's constant and every other byte zero: the
    thread that reads it writes the sink. 600 MB is past four grid strides
    of the largest grid (32768 workgroups of 256 threads, 16 bytes each), so
    the four-load rounds and the remainder both run; the word is put at the
    first piece, a round's boundary, the middle, the last piece, and a
    count of bytes that stops short of it must leave the sink alone."""
    n16 = 4 * 32768 * 256 + 4 * 32768 * 64 + 3
    buf = torch.zeros((n16 * 4,), dtype=torch.int32, device="cuda")
    sink = torch.zeros((4,), dtype=torch.int32, device="cuda")
    magic = np.array([MAGIC], dtype=np.uint32).view(np.int32)[0]
    for piece in (0, 4 * 32768 * 256 - 1, 4 * 32768 * 256, n16 // 2, n16 - 1):
        say("stream read", n16, piece)
        buf[4 * piece + 1] = int(magic)
        sink.zero_()
        hip.stream_read_dev(buf, sink)
        torch.cuda.synchronize()
        assert int(sink[0].item()) == int(magic), piece
        sink.zero_()
        hip.stream_read_dev(buf, sink, nbytes=16 * piece)
        torch.cuda.synchronize()
        assert int(sink[0].item()) == 0, piece
        buf[4 * piece + 1] = 0
    with pytest.raises(hip.PkHipError):
        hip._check(hip.lib().pk_hip_stream_read_dev(hip._dptr(buf), 64, None, None))


def test_empty_and_mfma_rate_run(hip, torch):
    """The empty launch and the matrix cores' rate run to the end on the
    stream they are given (nothing in their sums meets the constant, so the
    sink stays zero), and a NULL sink is refused before any launch."""
    sink = torch.zeros((4,), dtype=torch.int32, device="cuda")
    say("empty, mfma rate")
    hip.empty_dev()
    hip.mfma_rate_dev(512, 64, sink)
    hip.mfma_rate_dev(0, 64, sink)          # no workgroups: nothing launched
    torch.cuda.synchronize()
    assert int(sink[0].item()) == 0
    with pytest.raises(hip.PkHipError):
        hip._check(hip.lib().pk_hip_mfma_rate_dev(8, 8, None, None))
