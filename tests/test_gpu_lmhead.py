"""Fused Q4_0 LM head + sampler vs the oracle (GPU).

The logits must be bit-identical to the oracle's restatement of
inference_prepare_q8 + inference_q4_matvec_rows_prepared
(fp32_sse2.rs:956-983, 1217-1248), and every sampler output bit-identical to
the oracle's sampler on those logits.  Covers batches that are not multiples
of the 64-row wave tile, two 256-row groups, all-zero hidden states (every
logit ties), and the error rows.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import assert_rows_equal, to_dev

pytestmark = pytest.mark.gpu

V = s.VOCAB


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def head(smp):
    w = workloads.make_lmhead(rows=300)
    import torch

    q4 = torch.from_numpy(w["q4"]).to("cuda:0")
    packed = smp.pack_lmhead(q4)
    torch.cuda.synchronize()
    return w, packed


def test_mfma_fragment_layout():
    import torch

    out = torch.zeros(32 * 32, dtype=torch.int32, device="cuda:0")
    st = s.lib().pb_device_mfma_selftest(ctypes.c_void_p(out.data_ptr()),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    i = np.arange(32)[:, None]
    k = np.arange(32)[None, :]
    a = (7 * i + 3 * k) % 17 - 8
    b = (5 * i + 11 * k) % 15 - 7  # b[k][j] with k as row index
    want = a @ b
    assert (out.cpu().numpy().reshape(32, 32) == want).all()


def run_head(smp, packed, hidden, hist, hist_len, r24):
    import torch

    B = hidden.shape[0]
    token = torch.empty(B, dtype=torch.int32, device="cuda:0")
    det = torch.empty((B, s.DETAIL_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    err = torch.empty((B, s.ERROR_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    logits = torch.empty((B, V), dtype=torch.int32, device="cuda:0")
    smp.lmhead_sample(packed, to_dev(hidden), to_dev(r24), to_dev(hist), to_dev(hist_len),
                      token=token, detail=det, err=err, logits=logits)
    torch.cuda.synchronize()
    return (logits.cpu().numpy().view(np.uint32), token.cpu().numpy().view(np.uint32),
            det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(B),
            err.cpu().numpy().view(s.ERROR_DTYPE).reshape(B))


def oracle_head(w, hidden, rows):
    logits = o.lmhead_logits(hidden, w["q4"], V, workloads.HIDDEN, threads=16)
    tok, det, err, _ = o.sample_batch(logits, w["hist"][:rows], w["hist_len"][:rows],
                                      w["random_24"][:rows], threads=16)
    return logits, tok, det, err


@pytest.mark.parametrize("rows", [5, 64, 300])
def test_head_logits_and_draws_are_bit_exact(smp, head, rows):
    w, packed = head
    hidden = w["hidden"][:rows]
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, w["hist"][:rows],
                                      w["hist_len"][:rows], w["random_24"][:rows])
    rlog, rtok, rdet, rerr = oracle_head(w, hidden, rows)
    bad = np.argwhere(glog != rlog)
    assert bad.size == 0, (bad[:5], glog[tuple(bad[0])], rlog[tuple(bad[0])])
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)
    # logits within 1e-3 relative of a float64 head is implied; spot-check it
    assert np.isfinite(glog.view(np.float32)).all()


def test_zero_hidden_states_tie_every_logit(smp, head):
    w, packed = head
    hidden = np.zeros((3, workloads.HIDDEN), np.float32)
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, w["hist"][:3], w["hist_len"][:3],
                                      w["random_24"][:3])
    assert (glog == 0).all()
    rlog, rtok, rdet, rerr = oracle_head(w, hidden, 3)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)


def test_error_rows(smp, head):
    w, packed = head
    hidden = w["hidden"][:4].copy()
    hist = w["hist"][:4].copy()
    hl = w["hist_len"][:4].copy()
    hidden[1, 100] = np.inf          # every logit of row 1 is non-finite
    hist[2, 3] = V + 7               # bad history id
    hidden[3, 5] = np.nan            # NaN is ignored by the Q8 max; quant -> 0
    hist[3, 0] = V                   # so row 3 fails on its history id
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, hist, hl, w["random_24"][:4])
    rlog = o.lmhead_logits(hidden, w["q4"], V, workloads.HIDDEN, threads=16)
    bad = np.argwhere((glog != rlog) & ~np.isnan(rlog.view(np.float32)))
    assert bad.size == 0
    assert (np.isnan(glog.view(np.float32)) == np.isnan(rlog.view(np.float32))).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, hl, w["random_24"][:4], threads=4)
    assert gerr["status"].tolist() == rerr["status"].tolist() == [0, 7, 3, 3]
    assert (gerr["detail"] == rerr["detail"]).all()
    assert gerr["available"][2] == V + 7 and gerr["available"][3] == V
    assert (gtok == rtok).all()
    assert (gdet[0]["ids"] == rdet[0]["ids"]).all()
