"""The bench line's streaming-read probe (libpega_hbm_probe.so) reads every byte it is
timed on: each thread's XOR of the 16-byte pieces it loads equals the same fold in numpy
(workgroup b takes the b-th contiguous chunk, thread t the pieces t, t + 256, ... of it)."""
import ctypes
import os

import numpy as np
import pytest
import torch

from conftest import ROOT

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pieces,grid", [(4096, 4), (100_000, 7), (1 << 20, 1024)])
def test_hbm_probe_reads_every_piece(pieces, grid):
    lib = ctypes.CDLL(os.path.join(ROOT, "pegainfer_amd", "libpega_hbm_probe.so"))
    fn = lib.pega_hbm_read_probe
    fn.argtypes = [ctypes.c_void_p, ctypes.c_ulonglong, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    g = np.random.default_rng(pieces)
    words = g.integers(0, 2 ** 32, size=pieces * 4, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).cuda()
    out = torch.zeros(grid * 256, dtype=torch.int32, device="cuda")
    assert fn(src.data_ptr(), pieces * 16, out.data_ptr(), grid,
              torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    piece_xor = np.bitwise_xor.reduce(words.reshape(pieces, 4), axis=1)
    chunk = -(-pieces // grid)
    want = np.zeros(grid * 256, np.uint32)
    for b in range(grid):
        part = piece_xor[b * chunk:min((b + 1) * chunk, pieces)]
        padded = np.zeros(-(-part.size // 256) * 256, np.uint32)  # x ^ 0 = x
        padded[:part.size] = part
        if padded.size:
            want[b * 256:(b + 1) * 256] = np.bitwise_xor.reduce(padded.reshape(-1, 256), axis=0)
    assert np.array_equal(got, want)
