"""pb_sample_batch_noalloc through the C ABI: the same outputs as pb_sample_batch
(bit for bit, tokens, top-20 detail and error records) when its slice
workspace is the library's static device array instead of the context's.

Two calls in a row on the same array, the second with a smaller batch (the
array keeps the first call's records; nothing may depend on them), then a
one-row call, each against pb_sample_batch on the same inputs and against the
oracle.  A slice plan forced past the array's 1,024 records is refused before
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


def test_noalloc_matches_pb_sample_batch_on_consecutive_calls():
    w = workloads.make("small")          # 64 rows: 16 slices each, 1,024 records
    w["hist"][5, 7] = V + 9              # one row fails on its history
    ctx = ctypes.c_void_p()
    assert s.lib().pb_context_create(0, ctypes.byref(ctx)) == s.OK
    try:
        for rows in (64, 9, 1):          # 1,024 then 288 then 32 records
            want = run(s.lib().pb_sample_batch, ctx, w, rows)
            got = run(s.lib().pb_sample_batch_noalloc, ctx, w, rows)
            assert_rows_equal(*got, *want)
            rtok, rdet, rerr, _ = o.sample_batch(w["logits"][:rows], w["hist"][:rows],
                                                 w["hist_len"][:rows], w["random_24"][:rows],
                                                 threads=16)
            assert_rows_equal(*got, rtok, rdet, rerr)
            assert (got[2]["status"] != s.OK).sum() == (1 if rows > 5 else 0)
    finally:
        s.lib().pb_context_destroy(ctx)


def test_noalloc_refuses_a_plan_past_its_array():
    w = workloads.make("small", rows=64)
    ctx = ctypes.c_void_p()
    assert s.lib().pb_context_create(0, ctypes.byref(ctx)) == s.OK
    try:
        s.lib().pb_context_set_segments(ctx, 32)   # 64 x 32 = 2,048 records
        d = hip.DeviceArray.from_numpy
        logits, hl, r24 = d(w["logits"]), d(w["hist_len"]), d(w["random_24"])
        hist = d(w["hist"])
        token = hip.DeviceArray.from_numpy(np.full(64, 7, np.uint32))
        e = s._Error()
        p = lambda a: ctypes.c_void_p(a.data_ptr())
        st = s.lib().pb_sample_batch_noalloc(ctx, p(logits), V, V, 64, p(hist), w["hist"].shape[1],
                                             p(hl), p(r24), p(token), None, None, None,
                                             ctypes.byref(e))
        assert st == s.CAPACITY and e.status == s.CAPACITY
        assert e.available == 1024 * (20 * 8 + 8) and e.needed == 2048 * (20 * 8 + 8)
        assert (token.numpy() == 7).all()  # nothing was enqueued
    finally:
        s.lib().pb_context_destroy(ctx)
