"""The read-bandwidth probes the bench's read ceiling is timed with (GPU):
every workgroup stores the XOR of exactly the words it was given, so the
probes read every word of the buffer once, in both shapes (contiguous runs
per workgroup, 32 KiB chunks in grid-stride order), including workgroups
left with nothing to read."""
import ctypes

import numpy as np
import pytest

from promptboot_amd import sampler as s
from tests.conftest import to_dev

pytestmark = pytest.mark.gpu

CHUNK_F4 = 256 * 8  # 16-byte groups per grid-stride chunk (32 KiB)


def expected(words: np.ndarray, blocks: int, grid_stride: bool) -> np.ndarray:
    g4 = words[: len(words) // 4 * 4].reshape(-1, 4)
    n4 = len(g4)
    out = np.zeros(blocks, np.uint32)
    if grid_stride:
        for c in range((n4 + CHUNK_F4 - 1) // CHUNK_F4):
            out[c % blocks] ^= np.bitwise_xor.reduce(g4[c * CHUNK_F4:(c + 1) * CHUNK_F4].ravel())
    else:
        per = (n4 + blocks - 1) // blocks
        for g in range(blocks):
            part = g4[g * per:min((g + 1) * per, n4)]
            if len(part):
                out[g] = np.bitwise_xor.reduce(part.ravel())
    return out


@pytest.mark.parametrize("grid_stride", [False, True])
@pytest.mark.parametrize("n_words,blocks", [(1 << 20, 64), (1_000_004, 37), (4096, 300),
                                            (3 * CHUNK_F4 * 4 * 7 + 12, 5)])
def test_read_probe_reads_every_word_once(grid_stride, n_words, blocks):
    import torch

    rng = np.random.default_rng([n_words, blocks])
    words = rng.integers(0, 1 << 32, n_words, dtype=np.uint64).astype(np.uint32)
    d_in = to_dev(words)
    d_out = torch.full((blocks,), -559038737, dtype=torch.int32, device="cuda:0")  # 0xdeadbeef
    fn = s.lib().pb_device_read_probe_grid_stride if grid_stride else s.lib().pb_device_read_probe
    st = fn(ctypes.c_void_p(d_in.data_ptr()), n_words, ctypes.c_void_p(d_out.data_ptr()), blocks,
            None)
    torch.cuda.synchronize()
    assert st == s.OK
    got = d_out.cpu().numpy().view(np.uint32)
    assert (got == expected(words, blocks, grid_stride)).all()
