"""The batched entry points of a reserved context under HIP graph capture.

pb_context_reserve sizes the workspace at set-up, so pb_sample_batch,
pb_lmhead_q8_sample_batch and pb_decode_step only launch kernels: each is
captured once into a graph and replayed several times, with new inputs
uploaded and eager launches of the library run between the replays, and
every replay is checked against the oracle (tokens, top-20 detail, logits
and the decode loop's contexts and states bit for bit).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import hip
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import assert_rows_equal

pytestmark = pytest.mark.gpu

V = s.VOCAB
DW = s.DETAIL_DTYPE.itemsize // 4
EW = s.ERROR_DTYPE.itemsize // 4


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    b.reserve(64, workloads.HIDDEN)
    yield b
    b.close()


def capture_sample(smp, w, rows):
    d = hip.DeviceArray.from_numpy
    bufs = dict(logits=d(w["logits"][:rows]), hist=d(w["hist"][:rows]),
                hl=d(w["hist_len"][:rows]), r24=d(w["random_24"][:rows]),
                token=hip.DeviceArray(rows, np.uint32), det=hip.DeviceArray((rows, DW), np.uint32),
                err=hip.DeviceArray((rows, EW), np.uint32))
    stream = hip.Stream()
    graph = hip.Graph(stream)
    graph.begin()
    smp.sample(bufs["logits"], bufs["r24"], bufs["hist"], bufs["hl"], token=bufs["token"],
               detail=bufs["det"], err=bufs["err"], stream=stream)
    graph.end()
    return graph, stream, bufs


def replay_and_check(smp, graph, stream, bufs, w, rows, replay):
    u = workloads.next_24_stream(np.arange(rows, dtype=np.uint64) * 977 + replay)
    bufs["r24"].upload(u)
    graph.launch()
    stream.synchronize()
    got = (bufs["token"].numpy(), bufs["det"].numpy().view(s.DETAIL_DTYPE).reshape(rows),
           bufs["err"].numpy().view(s.ERROR_DTYPE).reshape(rows))
    want = o.sample_batch(w["logits"][:rows], w["hist"][:rows], w["hist_len"][:rows], u,
                          threads=16)[:3]
    assert_rows_equal(*got, *want)
    # eager work of the library between replays, on the null stream
    other = hip.DeviceArray(rows, np.uint32)
    smp.sample(bufs["logits"], bufs["r24"], bufs["hist"], bufs["hl"], token=other)
    assert (other.numpy() == got[0]).all()
    other.free()


# 64 rows take the tile selection (tile words, then the selection); a forced
# plan of seven slices per row and 200 rows (two slices per row) the slice
# plan (segment_kernel, then finish_kernel through the slice records)
@pytest.mark.parametrize("rows,segments", [(64, 0), (64, 7), (200, 0)])
def test_sample_batch_replays(smp, rows, segments):
    w = workloads.make("small", rows=rows)
    smp.set_segments(segments)
    try:
        smp.reserve(rows)
        graph, stream, bufs = capture_sample(smp, w, rows)
        for replay in range(4):
            replay_and_check(smp, graph, stream, bufs, w, rows, replay)
        graph.close()
    finally:
        smp.set_segments(0)


def test_replays_survive_a_growing_reserve():
    """A graph captured on a context's slice workspace replays correctly after
    pb_context_reserve has outgrown that workspace: the old one stays
    allocated until the context is destroyed."""
    rows = 16
    w = workloads.make("small", rows=rows)
    b = s.BatchSampler(0, segments=5)
    try:
        b.reserve(rows)
        graph, stream, bufs = capture_sample(b, w, rows)
        replay_and_check(b, graph, stream, bufs, w, rows, 0)
        b.reserve(64)                    # a larger slice workspace
        b.reserve(64, workloads.HIDDEN)  # and the LM head's
        for replay in range(1, 4):
            replay_and_check(b, graph, stream, bufs, w, rows, replay)
        graph.close()
    finally:
        b.close()


def test_lmhead_q8_replays(smp):
    rows = 3
    w = workloads.make_lmhead(rows=rows)
    head = workloads.make_q8_head()
    packed = smp.pack_lmhead(hip.DeviceArray.from_numpy(head), q8=True)
    d = hip.DeviceArray.from_numpy
    hidden, hist, hl, r24 = d(w["hidden"]), d(w["hist"]), d(w["hist_len"]), d(w["random_24"])
    token = hip.DeviceArray(rows, np.uint32)
    det = hip.DeviceArray((rows, DW), np.uint32)
    logits = hip.DeviceArray((rows, V), np.uint32)
    stream = hip.Stream()
    graph = hip.Graph(stream)
    graph.begin()
    smp.lmhead_sample(packed, hidden, r24, hist, hl, token=token, detail=det, logits=logits,
                      stream=stream, q8=True)
    graph.end()
    rng = np.random.default_rng(3)
    for replay in range(3):
        x = rng.standard_normal((rows, workloads.HIDDEN), dtype=np.float32)
        hidden.upload(x)
        graph.launch()
        stream.synchronize()
        rlog = o.lmhead_logits(x, head, V, workloads.HIDDEN, threads=16, q8=True)
        assert (logits.numpy() == rlog).all(), replay
        rtok, rdet, rerr, _ = o.sample_batch(rlog, w["hist"], w["hist_len"], w["random_24"],
                                             threads=16)
        assert_rows_equal(token.numpy(), det.numpy().view(s.DETAIL_DTYPE).reshape(rows),
                          np.zeros(rows, s.ERROR_DTYPE), rtok, rdet, rerr)
        # an eager single-row drop-in between replays
        assert s.greedy_token(rlog[0]) == int(np.argmax(rlog[0].view(np.float32)))
    graph.close()


def test_lmhead_one_pass_replays(smp):
    """70 rows through the Q4_0 head without a logits buffer (one pass: the
    selection recomputes tiles from the head) under capture, replayed with
    new hidden states."""
    rows = 70
    w = workloads.make_lmhead(rows=rows)
    smp.reserve(rows, workloads.HIDDEN)
    packed = smp.pack_lmhead(hip.DeviceArray.from_numpy(w["q4"]))
    d = hip.DeviceArray.from_numpy
    hidden, hist, hl, r24 = d(w["hidden"]), d(w["hist"]), d(w["hist_len"]), d(w["random_24"])
    token = hip.DeviceArray(rows, np.uint32)
    det = hip.DeviceArray((rows, DW), np.uint32)
    stream = hip.Stream()
    graph = hip.Graph(stream)
    graph.begin()
    smp.lmhead_sample(packed, hidden, r24, hist, hl, token=token, detail=det, stream=stream)
    graph.end()
    rng = np.random.default_rng(4)
    for replay in range(3):
        x = rng.standard_normal((rows, workloads.HIDDEN), dtype=np.float32)
        hidden.upload(x)
        graph.launch()
        stream.synchronize()
        rlog = o.lmhead_logits(x, w["q4"], V, workloads.HIDDEN, threads=16)
        rtok, rdet, rerr, _ = o.sample_batch(rlog, w["hist"], w["hist_len"], w["random_24"],
                                             threads=16)
        assert_rows_equal(token.numpy(), det.numpy().view(s.DETAIL_DTYPE).reshape(rows),
                          np.zeros(rows, s.ERROR_DTYPE), rtok, rdet, rerr)
    graph.close()
    packed.free()


def test_decode_step_replays(smp):
    rng = np.random.default_rng(8)
    prompts = [workloads.zipf_ids(rng, n) for n in (30, 7, 120, 2)]
    seeds, limits = [0x0123_4567_89AB_CDEF, 1, 2, 3], [12, 3, 12, 12]
    dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
    oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
    rows = len(prompts)
    logits = hip.DeviceArray((rows, V), np.uint32)
    stream = hip.Stream()
    graph = hip.Graph(stream)
    e = s._Error()
    graph.begin()
    st = s.lib().pb_decode_step(smp._ctx, ctypes.c_void_p(logits.data_ptr()), V, V, rows,
                                *dec._ptrs(), ctypes.c_void_p(stream.handle), ctypes.byref(e))
    graph.end()
    assert st == s.OK
    for step in range(14):
        x = np.stack([rng.normal(0, 2.5, V).astype(np.float32) for _ in range(rows)])
        x[:, s.IM_END] = 30.0 if step >= 9 else x[:, s.IM_END]
        x = x.view(np.uint32)
        want = [d.step(x[r]) for r, d in enumerate(oracle_rows)]
        logits.upload(x)
        before = dec._draw()
        graph.launch()
        stream.synchronize()
        got = dec._settle(before)
        assert [int(t) for t in got] == [s.NO_TOKEN if t is None else t for t in want], step
        if not dec.active():
            break
    states = dec.sampling_states()
    for r, d in enumerate(oracle_rows):
        assert dec.contexts()[r].tolist() == d.working
        assert (states[r].state(), states[r].draws()) == (d.state.state(), d.state.draws())
    graph.close()
