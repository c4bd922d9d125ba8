"""Draws that land exactly on a step of the cumulative distribution, and rows
whose penalised top-20 holds -inf, through every device path (GPU).

The reference keeps the first top-p prefix that is not below the cutoff
(fp32_sse2.rs:1826-1834) and draws the first survivor whose binary32 prefix
is strictly greater than the target (:1836-1845): a target exactly on a step
goes to the next survivor.  The rows:

* two ids tied at the top, uniform 1/2: the target 1.0 equals the first
  prefix, so rank 1; with 1/2 - 2^-24 rank 0, with 1/2 + 2^-24 rank 1;
* 24 ids tied at the top: weights 1, total 20, and the cutoff 16 equals the
  16th prefix (kept 16); uniforms k/16 put the target on the integer k
  (rank k), k/16 -+ 2^-24 one uniform step either side (ranks k-1 and k);
* every logit at -3.4e38 and every id in the history: the penalty overflows
  them all to -inf, max - max is NaN and so is every weight, the total and
  the target (kept 1, rank 0, the lowest id);
* the same with 5 ids left out of the history: weights 1 x 5 and 0 x 15,
  kept 4, the target 2.0 on the second step (rank 2);
* the same with 25 ids left out: 20 ties of finite values, target 8.

The paths: pb_sample_batch through the tile selection (up to 192 rows) and
through the slice plans of one and seven slices per row, the single-row
drop-ins on host memory, and the fused Q4_0 LM head (narrow and wide GEMM)
on a head whose 24 tied vocabulary rows are identical.  Every output is
compared with the oracle bit for bit: token, top-20 ids and values, weights,
probabilities, kept, rank, flags and the error record.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import assert_rows_equal, to_dev
from tests.test_gpu_batch import run_gpu
from tests.test_gpu_lmhead import run_head

pytestmark = pytest.mark.gpu

V = s.VOCAB
HUGE = np.float32(-3.4e38)  # times 1.1 overflows to -inf


def step_uniforms():
    """(uniform, expected rank) pairs on and beside the integer steps of a
    24-way tie (kept 16, target = 16 u)."""
    out = []
    for k in range(16):
        out.append((k << 20, k))
        if k > 0:
            out.append(((k << 20) - 1, k - 1))
        out.append(((k << 20) + 1, k))
    return out


def boundary_rows(seed=3):
    """The rows of the module docstring; returns the workload dict and the
    expected (kept, rank) of each row, worked out by hand."""
    rng = np.random.default_rng(seed)
    rows, hists, r24, want = [], [], [], []
    base = rng.standard_normal((4, V), dtype=np.float32) - np.float32(20.0)
    # two leaders
    two = base[0].copy()
    two[[500, 77_000]] = np.float32(10.0)
    for u, rank in (((1 << 23), 1), ((1 << 23) - 1, 0), ((1 << 23) + 1, 1)):
        rows.append(two)
        hists.append(rng.integers(0, 400, 20).astype(np.uint32))
        r24.append(u)
        want.append((2, rank))
    # 24-way tie
    tie = base[1].copy()
    tie[np.sort(rng.choice(np.arange(1000, V), 24, replace=False))] = np.float32(5.0)
    for u, rank in step_uniforms():
        rows.append(tie)
        hists.append(rng.integers(0, 900, 30).astype(np.uint32))
        r24.append(u)
        want.append((16, rank))
    # -inf rows: the whole vocabulary, all but 5, all but 25 ids in the history
    full = np.full(V, HUGE)
    for left_out, u, expect in ((0, 12_345, (1, 0)), (5, 1 << 23, (4, 2)),
                                (25, 1 << 23, (16, 8))):
        keep = rng.choice(V, left_out, replace=False)
        h = np.setdiff1d(np.arange(V, dtype=np.uint32), keep)
        rows.append(full)
        hists.append(rng.permutation(h).astype(np.uint32))
        r24.append(u)
        want.append(expect)
    B = len(rows)
    hist = np.zeros((B, V), np.uint32)
    hist_len = np.zeros(B, np.uint32)
    for i, h in enumerate(hists):
        hist[i, :len(h)] = h
        hist_len[i] = len(h)
    seeds = np.array([workloads.seed_for_draw(u, i) for i, u in enumerate(r24)], np.uint64)
    w = dict(logits=np.stack(rows), hist=hist, hist_len=hist_len,
             random_24=np.array(r24, np.uint32), seeds=seeds)
    assert (workloads.next_24_stream(seeds) == w["random_24"]).all()
    return w, np.array(want, np.uint32)


@pytest.fixture(scope="module")
def rows():
    w, want = boundary_rows()
    ref = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"], threads=16)
    tok, det, err, _ = ref
    # the oracle's verdicts are the ones worked out by hand
    assert (err["status"] == 0).all()
    assert (det["kept"] == want[:, 0]).all() and (det["rank"] == want[:, 1]).all()
    nan_row = len(want) - 3
    assert (det["weight_bits"][nan_row] == 0xFFC00000).all()  # x86's default NaN
    assert tok[nan_row] == 0
    return w, ref[:3]


@pytest.fixture(scope="module")
def sampler():
    smp = s.BatchSampler(0)
    yield smp
    smp.close()


@pytest.mark.parametrize("segments", [0, 1, 7])
def test_batch_paths_match_the_oracle_on_steps_and_nan_weights(sampler, rows, segments):
    w, ref = rows
    got = run_gpu(sampler, w, segments)
    assert_rows_equal(*got, *ref)
    # the constructions reach the flags: exact steps and the cutoff on a prefix
    assert (got[1]["flags"][:3] == 1).all()
    assert (got[1]["flags"][3:3 + len(step_uniforms())] & 2).all()


def test_drop_ins_match_the_oracle_on_steps_and_nan_weights(rows):
    w, (rtok, _, _) = rows
    for i in range(len(rtok)):
        hist = w["hist"][i, :w["hist_len"][i]]
        seed = int(w["seeds"][i])
        g, r = w["logits"][i].view(np.uint32).copy(), w["logits"][i].view(np.uint32).copy()
        gs, rs = s.SamplingState(seed), o.SamplingState(seed)
        seen = np.zeros(s.SEEN_BYTES, np.uint8)
        t = s.sample_token_with_repetition(g, hist, seen, gs)
        st, rt, _ = o.sample_token_with_repetition(r, hist, np.zeros(o.SEEN_BYTES, np.uint8), rs)
        assert st == 0 and t == rt == rtok[i], (i, t, rt)
        assert (g == r).all(), i  # the in-place penalty, -inf included
        assert gs.state() == rs.state() and gs.draws() == 1
        assert not seen.any()
        if w["hist_len"][i] < 64:  # no penalty: sample_token on the raw row
            gs2, rs2 = s.SamplingState(seed), o.SamplingState(seed)
            raw = w["logits"][i].view(np.uint32)
            st2, rt2, _ = o.sample_token(raw, rs2)
            assert st2 == 0 and s.sample_token(raw, gs2) == rt2


def tied_head(w, tied):
    """make_lmhead's Q4_0 head with the rows of `tied` made identical: every
    nibble 15 (weight +7) under the scale 0.02, so that with positive hidden
    states they are the largest logits of every row, exactly equal."""
    q4 = w["q4"].reshape(V, workloads.HIDDEN // 32, 18).copy()
    q4[tied, :, 0:2] = np.array([0.02], np.float16).view(np.uint8)
    q4[tied, :, 2:] = 0xFF
    return q4.reshape(-1)


@pytest.mark.parametrize("nrows", [40, 72])  # the narrow and the wide GEMM
def test_lmhead_selection_on_exact_steps(sampler, nrows):
    import torch

    w = workloads.make_lmhead(rows=nrows)
    rng = np.random.default_rng(nrows)
    tied = np.sort(rng.choice(np.arange(V // 2, V), 24, replace=False))
    head = tied_head(w, tied)
    hidden = np.abs(w["hidden"]) + np.float32(1.0)
    hist = w["hist"].copy()
    hist[np.isin(hist, tied)] = 1
    pairs = step_uniforms()
    r24 = np.array([pairs[i % len(pairs)][0] for i in range(nrows)], np.uint32)
    sampler.reserve(nrows, workloads.HIDDEN)
    packed = sampler.pack_lmhead(torch.from_numpy(head).to("cuda:0"))
    glog, gtok, gdet, gerr = run_head(sampler, packed, hidden, hist, w["hist_len"], r24)
    rlog = o.lmhead_logits(hidden, head, V, workloads.HIDDEN, threads=16)
    assert (glog == rlog).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, w["hist_len"], r24, threads=16)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)
    assert (rdet["kept"] == 16).all() and (np.isin(rdet["ids"][:, :16], tied)).all()
    assert (rdet["rank"] == [pairs[i % len(pairs)][1] for i in range(nrows)]).all()
