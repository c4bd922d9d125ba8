"""Element orders that drive the streaming threshold hardest, vs the oracle (GPU).

The sampler filters one pass over the row against a running threshold and
stages every float4 that reaches it.  These rows are built so that the stage
fills, flushes in the middle of chunks and merges over and over:

* ascending values: every element beats everything before it;
* descending values: the threshold settles on the first chunk;
* a sawtooth of period 1000: the top value ties 152 times, so the top-20 is
  decided by ids alone;
* 25 ones in a row of zeros: ties straddle rank 20;
* ascending values whose 30 largest ids are all in the history: the penalty
  reorders the top after the raw filter.

Every output (token, top-20 ids and values, weights, probabilities, kept,
rank, flags, error record) must equal the oracle's, for every slice plan.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from tests.conftest import assert_rows_equal
from tests.test_gpu_batch import run_gpu

pytestmark = pytest.mark.gpu

V = s.VOCAB


@pytest.fixture(scope="module")
def sampler():
    smp = s.BatchSampler(0)
    yield smp
    smp.close()


def ordered_rows(rng):
    ids = np.arange(V, dtype=np.float32)
    rows = [ids * np.float32(1e-3),                       # ascending
            -ids * np.float32(1e-3),                      # descending
            (np.arange(V) % 1000).astype(np.float32),     # sawtooth, 152-way top tie
            np.zeros(V, np.float32),                      # 25 tied ones
            ids * np.float32(1e-3)]                       # ascending, top ids penalised
    rows[3][rng.choice(V, 25, replace=False)] = 1.0
    hist = np.zeros((len(rows), 64), np.uint32)
    hl = np.zeros(len(rows), np.uint32)
    hist[4, :30] = np.arange(V - 30, V, dtype=np.uint32)
    hl[4] = 30
    for r in range(3):  # a few random history ids on the others
        hist[r, :8] = rng.integers(0, V, 8, dtype=np.uint32)
        hl[r] = 8
    logits = np.stack(rows)
    r24 = rng.integers(0, 1 << 24, len(rows), dtype=np.uint32)
    return dict(logits=logits, hist=hist, hist_len=hl, random_24=r24)


@pytest.mark.parametrize("segments", [0, 1, 3, 32])
def test_adversarial_orders_match_the_oracle(sampler, segments):
    w = ordered_rows(np.random.default_rng(7))
    got = run_gpu(sampler, w, segments)
    tok, det, err, _ = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"],
                                      threads=5)
    assert_rows_equal(*got, tok, det, err)
    assert (got[2]["status"] == 0).all()
    # spot-check the constructions
    assert det["ids"][0].tolist() == list(range(V - 1, V - 21, -1))   # ascending
    assert det["ids"][1].tolist() == list(range(20))                  # descending
    assert (det["ids"][2] == np.arange(20) * 1000 + 999).all()        # sawtooth ties by id
    assert not set(det["ids"][4].tolist()) & set(range(V - 30, V))    # penalised tops drop out
