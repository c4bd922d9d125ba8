"""Concurrent callers (GPU), every result bit-exact against the oracle.

The library's threading contract (include/pbsample.h): one context's batched
calls share its workspace, so they are ordered on one stream, and its host
side takes the context's lock, so host threads may share a context; different
contexts are independent, on any streams; the single-row drop-ins serialise
on the per-device default context.  Covered here:

* two contexts whose calls are enqueued alternately on two streams, the
  streams never synchronised with each other (the tile selection at 32 rows
  and the slice plan at 256 rows);
* four host threads sharing one context and one stream;
* four host threads calling the single-row drop-in at once, each with its own
  row, history, scratch and sampling state.
"""
import threading

import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import assert_rows_equal, to_dev

pytestmark = pytest.mark.gpu


def _outputs(torch, rows):
    return (torch.empty(rows, dtype=torch.int32, device="cuda:0"),
            torch.empty((rows, s.DETAIL_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0"),
            torch.empty((rows, s.ERROR_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0"))


def _host(out, rows):
    tok, det, err = out
    return (tok.cpu().numpy().view(np.uint32), det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(rows),
            err.cpu().numpy().view(s.ERROR_DTYPE).reshape(rows))


@pytest.mark.parametrize("name,rows", [("small", 64), ("flat", 512)])
def test_two_contexts_on_two_streams(name, rows):
    import torch

    w = workloads.make(name, rows=rows)
    half = rows // 2
    parts = [slice(0, half), slice(half, rows)]
    samplers = [s.BatchSampler(0), s.BatchSampler(0)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    inputs = [tuple(to_dev(w[k][p]) for k in ("logits", "hist", "hist_len", "random_24"))
              for p in parts]
    steps = 6
    outs = [[_outputs(torch, half) for _ in range(steps)] for _ in parts]
    for smp in samplers:
        smp.reserve(half)
    torch.cuda.synchronize()
    for i in range(steps):
        for k, smp in enumerate(samplers):
            logits, hist, hl, r24 = inputs[k]
            tok, det, err = outs[k][i]
            smp.sample(logits, r24, hist, hl, token=tok, detail=det, err=err, stream=streams[k])
    torch.cuda.synchronize()
    rtok, rdet, rerr, _ = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"],
                                         threads=16)
    for k, p in enumerate(parts):
        for i in range(steps):
            assert_rows_equal(*_host(outs[k][i], half), rtok[p], rdet[p], rerr[p])
    for smp in samplers:
        smp.close()


def test_threads_share_one_context():
    import torch

    w = workloads.make("small")
    rows = w["logits"].shape[0]
    smp = s.BatchSampler(0)
    smp.reserve(rows)
    logits, hist, hl, r24 = (to_dev(w[k]) for k in ("logits", "hist", "hist_len", "random_24"))
    threads, calls = 4, 5
    outs = [[_outputs(torch, rows) for _ in range(calls)] for _ in range(threads)]
    torch.cuda.synchronize()
    failures = []

    def worker(t):
        try:
            for c in range(calls):
                tok, det, err = outs[t][c]
                smp.sample(logits, r24, hist, hl, token=tok, detail=det, err=err)
        except Exception as e:  # reported by the main thread
            failures.append(e)

    pool = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for th in pool:
        th.start()
    for th in pool:
        th.join()
    torch.cuda.synchronize()
    assert not failures, failures
    rtok, rdet, rerr, _ = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"],
                                         threads=16)
    for t in range(threads):
        for c in range(calls):
            assert_rows_equal(*_host(outs[t][c], rows), rtok, rdet, rerr)
    smp.close()


def test_drop_ins_from_threads():
    w = workloads.make("small", rows=8)
    threads = 4
    results = [None] * threads
    failures = []

    def worker(t):
        try:
            got = []
            for r in (t, t + threads):
                row = np.ascontiguousarray(w["logits"][r]).view(np.uint32).copy()
                prompt = np.ascontiguousarray(w["hist"][r, :w["hist_len"][r]])
                seen = np.zeros(s.SEEN_BYTES, np.uint8)
                state = s.SamplingState(int(w["seeds"][r]))
                tok = s.sample_token_with_repetition(row, prompt, seen, state)
                got.append((r, tok, row, state.draws(), bool(seen.any())))
            results[t] = got
        except Exception as e:  # reported by the main thread
            failures.append(e)

    pool = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for th in pool:
        th.start()
    for th in pool:
        th.join()
    assert not failures, failures
    for got in results:
        for r, tok, row, draws, seen_left in got:
            want_row = np.ascontiguousarray(w["logits"][r]).view(np.uint32).copy()
            prompt = np.ascontiguousarray(w["hist"][r, :w["hist_len"][r]])
            state = o.SamplingState(int(w["seeds"][r]))
            st, want, _ = o.sample_token_with_repetition(want_row, prompt,
                                                         np.zeros(o.SEEN_BYTES, np.uint8), state)
            assert st == 0 and tok == want
            assert (row == want_row).all()  # the penalty applied in place, as the oracle's
            assert draws == state.draws() == 1 and not seen_left
