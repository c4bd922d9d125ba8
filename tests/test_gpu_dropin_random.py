"""Seeded random calls of the single-row drop-ins against the oracle (GPU).

Each seed draws a row from the random batch generator's distributions and a
history (empty, short, long with repeats, holding the row's best ids, with an
id >= vocab), a `seen` scratch that is clear, dirty (some history ids' bits
already set) or short, and a generator seed.  pb_sample_token_with_repetition
must give the oracle's status, error tuple, token, penalised row, returned
scratch and generator state (all untouched on an error); pb_sample_token,
pb_greedy_token and pb_top_logits_8 the oracle's results on the same row.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from tests.test_gpu_random import random_case

pytestmark = pytest.mark.gpu

V = s.VOCAB


def random_call(seed: int) -> dict:
    rng = np.random.default_rng([seed, 11])
    c = random_case(seed, rows=1)
    row = np.ascontiguousarray(c["logits"][0, :V]).view(np.uint32).copy()
    kind = int(rng.integers(0, 5))
    if kind == 0:
        hist = np.zeros(0, np.uint32)
    elif kind == 1:
        hist = rng.integers(0, V, int(rng.integers(1, 40)), dtype=np.uint64).astype(np.uint32)
    elif kind == 2:  # long, with repeats
        base = rng.integers(0, V, 500, dtype=np.uint64).astype(np.uint32)
        hist = rng.choice(base, int(rng.integers(1000, 40000)))
    else:  # the row's best ids, some repeated
        top = np.argsort(-row.view(np.float32), kind="stable")[:50].astype(np.uint32)
        hist = rng.choice(top, int(rng.integers(1, 120)))
    hist = np.ascontiguousarray(hist, np.uint32)
    if len(hist) and rng.random() < 0.08:
        hist[int(rng.integers(0, len(hist)))] = V + int(rng.integers(0, 5000))
    seen_len = s.SEEN_BYTES if rng.random() < 0.9 else int(rng.integers(0, s.SEEN_BYTES))
    seen = np.zeros(seen_len, np.uint8)
    if len(hist) and seen_len == s.SEEN_BYTES and rng.random() < 0.3:  # dirty scratch
        for t in rng.choice(hist, min(len(hist), 8)):
            if t < V:
                seen[t >> 3] |= np.uint8(1 << (t & 7))
    return dict(row=row, hist=hist, seen=seen, seed=int(rng.integers(0, 2**63)))


@pytest.mark.parametrize("seed", range(24))
def test_random_drop_in_matches_oracle(seed):
    c = random_call(seed)
    g_row, r_row = c["row"].copy(), c["row"].copy()
    g_seen, r_seen = c["seen"].copy(), c["seen"].copy()
    gs, rs = s.SamplingState(c["seed"]), o.SamplingState(c["seed"])
    st, rt, rerr = o.sample_token_with_repetition(r_row, c["hist"], r_seen, rs)
    try:
        t = s.sample_token_with_repetition(g_row, c["hist"], g_seen, gs)
        gst, gerr = 0, None
    except s.InferenceError as e:
        t, gst, gerr = None, e.status, e.tuple()
    assert gst == st
    if st == 0:
        assert t == rt
    else:
        assert gerr == rerr.tuple()
    assert (g_row == r_row).all() and (g_seen == r_seen).all()
    assert (gs.state(), gs.draws()) == (rs.state(), rs.draws())
    # the other drop-ins on the untouched row
    row = c["row"]
    gs2, rs2 = s.SamplingState(c["seed"]), o.SamplingState(c["seed"])
    st2, rt2, rerr2 = o.sample_token(row, rs2)
    try:
        assert s.sample_token(row, gs2) == rt2 and st2 == 0
    except s.InferenceError as e:
        assert e.status == st2 and e.tuple() == rerr2.tuple()
    assert (gs2.state(), gs2.draws()) == (rs2.state(), rs2.draws())
    st3, rt3, rerr3 = o.greedy_token(row)
    try:
        assert s.greedy_token(row) == rt3 and st3 == 0
    except s.InferenceError as e:
        assert e.status == st3 and e.tuple() == rerr3.tuple()
