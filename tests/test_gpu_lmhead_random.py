"""Seeded random LM-head steps against the oracle (GPU).

Each seed draws a head format (Q4_0 or Q8_0), a hidden width, a batch size
either side of the narrow/one-pass limit of 64 rows, weight scales from a
random range (with signed zeros, fp16 subnormals and, in some heads,
infinite or NaN scales in a few blocks), hidden states at a random scale
(with zero rows, rows whose activation scale leaves fp16's range, and rows
holding a non-finite value) and histories that hold each row's best ids.
The step runs with and without a logits buffer; the logits are compared bit
for bit with the oracle's head (NaN positions as a set), and both runs'
records with the oracle sampler on those logits.
"""
import numpy as np
import pytest

from promptboot_amd import sampler as s
from tests.test_gpu_lmhead_onepass import check

pytestmark = pytest.mark.gpu

V = s.VOCAB


def random_head(rng, blocks: int, q8: bool) -> np.ndarray:
    width = 34 if q8 else 18
    head = np.empty((V, blocks, width), np.uint8)
    lo = 10.0 ** rng.uniform(-4.0, -1.0)
    scales = rng.uniform(lo, lo * rng.uniform(1.5, 20.0), (V, blocks)).astype(np.float16)
    bits = scales.view(np.uint16)
    n = max(1, V * blocks // 1000)
    pick = lambda k: (rng.integers(0, V, k), rng.integers(0, blocks, k))
    bits[pick(n)] |= 0x8000                                   # negative scales
    bits[pick(n)] = rng.choice([0x0000, 0x8000, 0x0001, 0x03FF, 0x7BFF], n)  # zeros, subnormals, max
    if rng.random() < 0.3:                                    # non-finite scales in a few blocks
        bits[pick(3)] = rng.choice([0x7C00, 0xFC00, 0x7E00], 3)
    head[:, :, 0:2] = bits.view(np.uint8).reshape(V, blocks, 2)
    head[:, :, 2:] = rng.integers(0, 256, (V, blocks, width - 2), dtype=np.uint8)
    return head.reshape(-1)


def random_step(seed: int) -> dict:
    rng = np.random.default_rng([seed, 7])
    q8 = bool(rng.random() < 0.5)
    cols = int(rng.choice([32, 96, 896, 896, 2048]))
    rows = int(rng.choice([1, 2, 5, 16, 33, 64, 65, 96, 129]))
    hidden = (rng.standard_normal((rows, cols)) * 10.0 ** rng.uniform(-3.0, 2.0)).astype(np.float32)
    hidden[rng.random(rows) < 0.1] = 0.0
    huge = rng.random(rows) < 0.05  # activation scale past fp16's range
    hidden[huge, int(rng.integers(0, cols))] = np.float32(1e7)
    nonfinite = bool(rng.random() < 0.3)
    if nonfinite:
        r = int(rng.integers(0, rows))
        hidden[r, int(rng.integers(0, cols))] = rng.choice([np.nan, np.inf, -np.inf])
    hist = rng.integers(0, V, (rows, 256), dtype=np.uint64).astype(np.uint32)
    hl = rng.integers(0, 257, rows).astype(np.uint32)
    r24 = rng.integers(0, 1 << 24, rows).astype(np.uint32)
    return dict(head=random_head(rng, cols // 32, q8), hidden=hidden, hist=hist, hist_len=hl,
                random_24=r24, q8=q8)


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    b.reserve(129, 2048)
    yield b
    b.close()


@pytest.mark.parametrize("seed", range(12))
def test_random_lmhead_step_matches_oracle(smp, seed):
    c = random_step(seed)
    check(smp, c["head"], c["hidden"], c["hist"], c["hist_len"], c["random_24"], q8=c["q8"],
          nan_rows_ok=True)
