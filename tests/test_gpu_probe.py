"""The streaming-read probe (ep_read_probe): every byte of the buffer is
read exactly once -- the XOR of the per-workgroup sink words equals the XOR
of the buffer's 32-bit words -- for ragged sizes and grids."""
import numpy as np
import pytest
import torch

from epure.kernels import _abi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096, 3), (1 << 20, 256), ((1 << 20) + 48, 7),
                                         (8650784, 256)])
def test_probe_reads_every_word_once(nbytes, grid):
    words = np.random.Generator(np.random.PCG64(nbytes)).integers(
        0, 2 ** 32, nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(words.view(np.int32)).to(DEV)
    sink = torch.full((grid,), -1, dtype=torch.int32, device=DEV)
    rc = _abi.lib.ep_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), grid,
                                _abi.stream_handle(DEV))
    assert rc == 0, _abi.last_error()
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(words)


def test_probe_declines_unaligned_sizes():
    buf = torch.zeros(64, dtype=torch.int32, device=DEV)
    sink = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert _abi.lib.ep_read_probe(buf.data_ptr(), 20, sink.data_ptr(), 1,
                                  _abi.stream_handle(DEV)) > 0
