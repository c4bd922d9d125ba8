"""pb_sample_batch_noalloc through the C ABI: the same outputs as pb_sample_batch
(bit for bit, tokens, top-20 detail and error records) when its workspace is
the library's static device array instead of the context's.

Consecutive calls share the array, and each is checked against
pb_sample_batch on the same inputs and against the oracle:

* the tile selection (up to 192 rows: tile words, then the selection):
  192 rows, then 64, 9 and 1, each smaller than the one before, so the
  array still holds the previous call's words past the rows in use;
* the automatic slice plan (193 to 255 rows: two slices per row, the slice
  records, then the merge): 250 rows (500 records), then 200 (400 records)
  on the first call's records;
* a forced plan of seven slices: 64 rows (448 records), then 33 (231).

A slice plan forced past the array's 21,705 records is refused before
anything is enqueued.
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


def run(fn, ctx, w, rows):
    d = hip.DeviceArray.from_numpy
    logits, hist = d(w["logits"][:rows]), d(w["hist"][:rows])
    hl, r24 = d(w["hist_len"][:rows]), d(w["random_24"][:rows])
    token = hip.DeviceArray(rows, np.uint32)
    det = hip.DeviceArray((rows, DW), np.uint32)
    err = hip.DeviceArray((rows, EW), np.uint32)
    e = s._Error()
    p = lambda a: ctypes.c_void_p(a.data_ptr())
    st = fn(ctx, p(logits), V, V, rows, p(hist), w["hist"].shape[1], p(hl), p(r24), p(token),
            p(det), p(err), None, ctypes.byref(e))
    assert st == s.OK, (st, list(e.tuple() if hasattr(e, "tuple") else []))
    hip.synchronize()
    return (token.numpy(), det.numpy().view(s.DETAIL_DTYPE).reshape(rows),
            err.numpy().view(s.ERROR_DTYPE).reshape(rows))


def check_calls(ctx, w, sequence):
    for rows in sequence:
        want = run(s.lib().pb_sample_batch, ctx, w, rows)
        got = run(s.lib().pb_sample_batch_noalloc, ctx, w, rows)
        assert_rows_equal(*got, *want)
        rtok, rdet, rerr, _ = o.sample_batch(w["logits"][:rows], w["hist"][:rows],
                                             w["hist_len"][:rows], w["random_24"][:rows],
                                             threads=16)
        assert_rows_equal(*got, rtok, rdet, rerr)
        assert (got[2]["status"] != s.OK).sum() == (1 if rows > 5 else 0)


def test_noalloc_matches_pb_sample_batch_on_consecutive_calls():
    w = workloads.make("small", rows=250)
    w["hist"][5, 7] = V + 9              # one row fails on its history
    ctx = ctypes.c_void_p()
    assert s.lib().pb_context_create(0, ctypes.byref(ctx)) == s.OK
    try:
        assert s.lib().pb_segments_for_rows(250) == s.lib().pb_segments_for_rows(200) == 2
        check_calls(ctx, w, (192, 64, 9, 1))      # tile selection
        check_calls(ctx, w, (250, 200))           # automatic slice plan, stale records
        s.lib().pb_context_set_segments(ctx, 7)   # forced plan: pb_sample_batch needs a reserve
        e = s._Error()
        assert s.lib().pb_context_reserve(ctx, 64, 0, ctypes.byref(e)) == s.OK
        check_calls(ctx, w, (64, 33))
    finally:
        s.lib().pb_context_destroy(ctx)


def test_noalloc_refuses_a_plan_past_its_array():
    rows = 680                                    # 680 x 32 = 21,760 records
    w = workloads.make("small", rows=8)
    ctx = ctypes.c_void_p()
    assert s.lib().pb_context_create(0, ctypes.byref(ctx)) == s.OK
    try:
        s.lib().pb_context_set_segments(ctx, 32)
        d = hip.DeviceArray.from_numpy
        # full-size buffers, although nothing may read them
        logits = hip.DeviceArray((rows, V), np.uint32)
        hist = hip.DeviceArray((rows, w["hist"].shape[1]), np.uint32)
        hl = hip.DeviceArray.zeros(rows, np.uint32)
        r24 = hip.DeviceArray.zeros(rows, np.uint32)
        token = d(np.full(rows, 7, np.uint32))
        e = s._Error()
        p = lambda a: ctypes.c_void_p(a.data_ptr())
        st = s.lib().pb_sample_batch_noalloc(ctx, p(logits), V, V, rows, p(hist),
                                             w["hist"].shape[1], p(hl), p(r24), p(token), None,
                                             None, None, ctypes.byref(e))
        assert st == s.CAPACITY and e.status == s.CAPACITY
        assert e.available == 192 * 2374 * 8 and e.needed == rows * 32 * (20 * 8 + 8)
        hip.synchronize()
        assert (token.numpy() == 7).all()  # nothing was enqueued
        for a in (logits, hist, hl, r24, token):
            a.free()
    finally:
        s.lib().pb_context_destroy(ctx)
