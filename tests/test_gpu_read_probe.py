"""wal_read_probe, the bench's read-bandwidth calibration: it reads exactly
the bytes asked for (the XOR of its per-wave partials equals the XOR of every
32-bit word in the range, on ragged sizes and grids larger than the data) and
refuses bad arguments on the host."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from wal2026_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid,block", [(16, 1, 64), (4096 + 48, 3, 128), (29_360_128, 256, 512),
                                               (1 << 20, 4096, 256)])
def test_read_probe_reads_every_word(nbytes, grid, block, gpu_device):
    g = torch.Generator().manual_seed(nbytes)
    host = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, generator=g)
    buf = host.to(gpu_device)
    partial = torch.zeros(grid * block // 64, dtype=torch.int32, device=gpu_device)
    stream = torch.cuda.current_stream()
    _lib.check(_lib.lib().wal_read_probe(buf.data_ptr(), nbytes, partial.data_ptr(), grid, block,
                                         stream.cuda_stream))
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    got = np.bitwise_xor.reduce(partial.cpu().numpy().view(np.uint32))
    assert got == want


def test_read_probe_argument_errors(gpu_device):
    lib = _lib.lib()
    buf = torch.zeros(64, dtype=torch.int32, device=gpu_device)
    partial = torch.zeros(64, dtype=torch.int32, device=gpu_device)
    p, q = buf.data_ptr(), partial.data_ptr()
    assert lib.wal_read_probe(p, 17, q, 1, 64, None) == _lib.EINVAL           # not a multiple of 16
    assert lib.wal_read_probe(p + 4, 16, q, 1, 64, None) == _lib.EINVAL       # misaligned
    assert lib.wal_read_probe(p, 16, q, 1, 96, None) == _lib.EINVAL           # block not a multiple of 64
    assert lib.wal_read_probe(p, 16, q, 1 << 16, 1024, None) == _lib.EINVAL   # strides past 32 bits
    assert lib.wal_read_probe(None, 16, q, 1, 64, None) == _lib.EINVAL
