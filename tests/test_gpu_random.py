"""Seeded random batches through pb_sample_batch against the oracle (GPU).

Each seed draws one batch from a family of shapes and value distributions
that the fixed workloads do not cover together: batch sizes either side of
the tile selection's 192-row limit, padded logits strides (padding holding
NaN), history strides from 1 to 2,048 ids (multiples of 4 and not), lengths
past the stride (clamped), no history at all, forced slice plans, and logits
that are Gaussian at any scale, quantised into heavy ties, a handful of
distinct values, large enough for the penalty to overflow to -inf,
subnormal, or dominated by spikes, with error rows (non-finite logits,
history ids >= vocab) sprinkled in.  Every output field is compared bit for
bit with the oracle on the same inputs (lengths clamped to the stride, as
the library's header specifies).
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from tests.conftest import assert_rows_equal, to_dev

pytestmark = pytest.mark.gpu

V = s.VOCAB


def random_case(seed: int, rows: int | None = None) -> dict:
    """One random batch (numpy, host side): logits [B, ld] float32, history
    [B, hist_ld] uint32 or None, lengths, uniforms and the slice plan.  `rows`
    replaces the drawn batch size (the other draws follow from the seed)."""
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 2, 7, 33, 64, 65, 127, 191, 192, 193, 256, 300]))
    B = B if rows is None else rows
    ld = V + int(rng.choice([0, 0, 4, 12]))
    kind = int(rng.integers(0, 6))
    shape = (B, V)
    if kind == 0:
        x = rng.normal(0.0, rng.uniform(0.02, 6.0), shape)
    elif kind == 1:
        q = float(rng.choice([1.0, 4.0, 16.0]))
        x = np.round(rng.normal(0.0, 2.0, shape) * q) / q
    elif kind == 2:
        x = rng.integers(-3, 3, shape).astype(np.float64)
    elif kind == 3:
        x = np.clip(rng.normal(0.0, 1e38, shape), -3.4e38, 3.4e38)
    elif kind == 4:
        x = rng.normal(0.0, 1e-40, shape)
    else:
        x = rng.normal(0.0, 1.0, shape)
        for r in range(B):
            k = int(rng.integers(1, 30))
            x[r, rng.choice(V, k, replace=False)] += rng.uniform(5.0, 45.0, k)
    lg = np.full((B, ld), np.nan, np.float32)
    lg[:, :V] = x.astype(np.float32)
    # signed zeros in some rows
    for r in rng.choice(B, max(1, B // 8), replace=False):
        idx = rng.choice(V, 64, replace=False)
        lg[r, idx] = np.where(rng.random(64) < 0.5, np.float32(0.0), np.float32(-0.0))
    # error rows: a non-finite logit
    if rng.random() < 0.5:
        for r in rng.choice(B, max(1, B // 10), replace=False):
            lg[r, int(rng.integers(0, V))] = rng.choice([np.nan, np.inf, -np.inf])
    hist_ld = int(rng.choice([0, 1, 3, 16, 300, 1023, 1024, 2048]))
    if hist_ld == 0:
        hist = hist_len = None
    else:
        hist = rng.integers(0, V, (B, hist_ld), dtype=np.uint64).astype(np.uint32)
        # histories that hold each row's best ids, so the penalty reorders the top
        top = np.argsort(-lg[:, :V], axis=1, kind="stable")[:, :64].astype(np.uint32)
        take = min(hist_ld, 64)
        rows = rng.random(B) < 0.5
        hist[rows, :take] = top[rows, :take]
        hist_len = rng.integers(0, hist_ld + 1, B).astype(np.uint32)
        past = rng.random(B) < 0.1
        hist_len[past] = hist_ld + rng.integers(1, 100, int(past.sum()))
        if rng.random() < 0.5:  # error rows: an id >= vocab inside the length
            for r in rng.choice(B, max(1, B // 10), replace=False):
                if hist_len[r] > 0:
                    hist[r, int(rng.integers(0, min(hist_len[r], hist_ld)))] = V + int(rng.integers(0, 1000))
    return dict(logits=lg, hist=hist, hist_len=hist_len,
                random_24=rng.integers(0, 1 << 24, B).astype(np.uint32),
                segments=int(rng.choice([0, 0, 0, 1, 3, 7])))


def run_gpu(smp, c):
    import torch

    B = c["logits"].shape[0]
    smp.set_segments(c["segments"])
    hist = None if c["hist"] is None else to_dev(c["hist"])
    hl = None if c["hist"] is None else to_dev(c["hist_len"])
    token = torch.empty(B, dtype=torch.int32, device="cuda:0")
    det = torch.empty((B, s.DETAIL_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    err = torch.empty((B, s.ERROR_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    smp.sample(to_dev(c["logits"]), to_dev(c["random_24"]), hist, hl, token=token, detail=det,
               err=err)
    torch.cuda.synchronize()
    smp.set_segments(0)
    return (token.cpu().numpy().view(np.uint32), det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(B),
            err.cpu().numpy().view(s.ERROR_DTYPE).reshape(B))


def run_oracle(c):
    hl = None
    if c["hist"] is not None:
        hl = np.minimum(c["hist_len"], c["hist"].shape[1]).astype(np.uint32)
    tok, det, err, _ = o.sample_batch(c["logits"], c["hist"], hl, c["random_24"], threads=16)
    return tok, det, err


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    yield b
    b.close()


@pytest.mark.parametrize("seed", range(32))
def test_random_batch_matches_oracle(smp, seed):
    c = random_case(seed)
    assert_rows_equal(*run_gpu(smp, c), *run_oracle(c))
