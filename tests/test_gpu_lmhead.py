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


def run_head(smp, packed, hidden, hist, hist_len, r24, q8=False, cols=workloads.HIDDEN):
    import torch

    B = hidden.shape[0]
    token = torch.empty(B, dtype=torch.int32, device="cuda:0")
    det = torch.empty((B, s.DETAIL_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    err = torch.empty((B, s.ERROR_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    logits = torch.empty((B, V), dtype=torch.int32, device="cuda:0")
    smp.lmhead_sample(packed, to_dev(hidden), to_dev(r24), to_dev(hist), to_dev(hist_len),
                      token=token, detail=det, err=err, logits=logits, q8=q8, cols=cols)
    torch.cuda.synchronize()
    return (logits.cpu().numpy().view(np.uint32), token.cpu().numpy().view(np.uint32),
            det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(B),
            err.cpu().numpy().view(s.ERROR_DTYPE).reshape(B))


def oracle_head(w, hidden, rows):
    logits = o.lmhead_logits(hidden, w["q4"], V, workloads.HIDDEN, threads=16)
    tok, det, err, _ = o.sample_batch(logits, w["hist"][:rows], w["hist_len"][:rows],
                                      w["random_24"][:rows], threads=16)
    return logits, tok, det, err


# up to 64 rows the head runs lm_gemm_narrow_kernel (one 16-row tile per wave up
# to 32 rows, two above), beyond that lm_gemm_kernel: both sides of each switch
@pytest.mark.parametrize("rows", [1, 2, 5, 16, 17, 32, 33, 64, 65, 129, 300])
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


def _set_scales(q4, edits):
    """q4: [V, blocks, 18] uint8; edits: {(id, block): fp16 bits}."""
    for (v, b), bits in edits.items():
        q4[v, b, 0] = bits & 0xFF
        q4[v, b, 1] = bits >> 8


@pytest.mark.parametrize("rows", [4, 160])
def test_special_weight_and_activation_scales(smp, head, rows):
    """Edge scales through both epilogue forms of the head.  Finite scales
    (signed zeros, +-1, fp16 subnormals, +-65504) sit in tiles that take the
    fused multiply-add form; +-inf and NaN sit in tiles of their own, which
    take the subtract-then-multiply form (inf * 0 = NaN as in the reference).
    The hidden rows give activation scales that are normal, fp16-subnormal,
    zero for one block, and infinite (amax / 127 above fp16's range).
    Logits are compared bit for bit with the oracle, NaN positions as a set."""
    import torch

    w, _ = head
    blocks = workloads.HIDDEN // 32
    q4 = w["q4"].reshape(V, blocks, 18).copy()
    finite = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x0001, 0x03FF, 0x7BFF, 0xFBFF]
    edits = {}
    for j, bits in enumerate(finite):   # tiles 10 .. 17, assorted ids and blocks
        edits[(64 * (10 + j) + 5 * j + 1, (3 * j) % blocks)] = bits
        edits[(64 * (10 + j) + 63, blocks - 1)] = bits
    for j, bits in enumerate([0x7C00, 0xFC00, 0x7E00]):  # tiles 100 .. 102
        edits[(64 * (100 + j) + 7 * j, j)] = bits
    edits[(64 * 103 + 40, blocks - 1)] = 0x7C00          # inf in the last block only
    _set_scales(q4, edits)
    packed = smp.pack_lmhead(torch.from_numpy(q4.reshape(-1)).to("cuda:0"))
    rng = np.random.default_rng(5)
    hidden = np.empty((4, workloads.HIDDEN), np.float32)
    hidden[0] = rng.standard_normal(workloads.HIDDEN)
    hidden[1] = rng.standard_normal(workloads.HIDDEN) * np.float32(1e-4)   # subnormal fp16 scales
    hidden[2] = rng.standard_normal(workloads.HIDDEN)
    hidden[2, 64:96] = 0.0                                                # one all-zero block
    hidden[3] = rng.standard_normal(workloads.HIDDEN) * np.float32(1e7)    # amax / 127 -> inf
    hidden = np.tile(hidden, (rows // 4, 1))  # 160 rows: the wide kernel
    glog, _, _, _ = run_head(smp, packed, hidden, w["hist"][:rows], w["hist_len"][:rows],
                             w["random_24"][:rows])
    rlog = o.lmhead_logits(hidden, q4.reshape(-1), V, workloads.HIDDEN, threads=16)
    gnan = np.isnan(glog.view(np.float32))
    rnan = np.isnan(rlog.view(np.float32))
    assert (gnan == rnan).all()
    bad = np.argwhere((glog != rlog) & ~rnan)
    assert bad.size == 0, (bad[:5], glog[tuple(bad[0])], rlog[tuple(bad[0])])
    # the edits really reach special values: inf and NaN columns exist
    assert rnan[0].any() and np.isinf(rlog.view(np.float32)[0]).any()


def _top_histories(rlog, rows):
    """Histories made of each row's best ids, so that the penalty lowers the
    largest value of the tiles that decide the row's top-20: the top 20, the
    top 64, every id of the tiles holding the top 5, every other id of the
    top 40, and the top 3 repeated (the penalty applies once per unique id)."""
    hists = []
    for r in range(rows):
        top = np.argsort(-rlog[r].view(np.float32), kind="stable")[:64].astype(np.uint32)
        kind = r % 5
        if kind == 0:
            ids = top[:20]
        elif kind == 1:
            ids = top
        elif kind == 2:
            tiles = np.unique(top[:5] // 64)
            ids = (tiles[:, None] * 64 + np.arange(64, dtype=np.uint32)).reshape(-1)
        elif kind == 3:
            ids = top[:40:2]
        else:
            ids = np.repeat(top[:3], 7)
        hists.append(ids.astype(np.uint32))
    ld = max(len(h) for h in hists)
    hist = np.zeros((rows, ld), np.uint32)
    hl = np.zeros(rows, np.uint32)
    for r, h in enumerate(hists):
        hist[r, :len(h)] = h
        hl[r] = len(h)
    return hist, hl


def test_history_holds_the_best_ids(smp, head):
    """Every tile maximum that decides a row's top-20 is a penalised value."""
    w, packed = head
    rows = 40
    hidden = w["hidden"][:rows]
    rlog = o.lmhead_logits(hidden, w["q4"], V, workloads.HIDDEN, threads=16)
    hist, hl = _top_histories(rlog, rows)
    r24 = w["random_24"][:rows]
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, hist, hl, r24)
    assert (glog == rlog).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, hl, r24, threads=16)
    assert (rerr["status"] == 0).all()
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)


@pytest.mark.parametrize("rows", [1, 140])
def test_one_tile_holds_the_best_ids(smp, head, rows):
    """All 64 ids of one tile get the weights of row 0's best id: row 0's
    top-20 are 20 tied ids of that tile (lowest ids first), and more elements
    reach the first round's threshold than it keys at once, so the select
    takes its general path; through the narrow and the wide GEMM."""
    import torch

    w, _ = head
    hidden = w["hidden"][:rows]
    q4 = w["q4"].reshape(V, workloads.HIDDEN // 32, 18).copy()
    rlog0 = o.lmhead_logits(hidden[:1], w["q4"], V, workloads.HIDDEN, threads=16)
    best = int(np.argmax(rlog0[0].view(np.float32)))
    tile = (best // 64 + 1000) % (V // 64)
    q4[tile * 64:(tile + 1) * 64] = q4[best]
    q4 = q4.reshape(-1)
    packed = smp.pack_lmhead(torch.from_numpy(q4).to("cuda:0"))
    torch.cuda.synchronize()
    rlog = o.lmhead_logits(hidden, q4, V, workloads.HIDDEN, threads=16)
    r0 = rlog[0].view(np.float32)
    assert (r0[tile * 64:(tile + 1) * 64] == r0.max()).all()
    r24 = w["random_24"][:rows]
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, w["hist"][:rows], w["hist_len"][:rows], r24)
    assert (glog == rlog).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, w["hist"][:rows], w["hist_len"][:rows], r24, threads=16)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)
    top = rdet[0]["ids"]
    assert ((top >= tile * 64) & (top < tile * 64 + 64)).sum() >= 10


def test_every_logit_negative(smp):
    """A head whose logits are all negative: the tile maxima are negative, so
    the penalty multiplies by 1.1 instead of dividing."""
    import torch

    rows, cols = 10, workloads.HIDDEN
    rng = np.random.default_rng(23)
    blocks = cols // 32
    # nibbles 0..7 are quants -8..-1; with positive activations every dot is negative
    lo = rng.integers(0, 8, (V, blocks, 16), dtype=np.uint8)
    hi = rng.integers(0, 8, (V, blocks, 16), dtype=np.uint8)
    q4 = np.zeros((V, blocks, 18), np.uint8)
    q4[:, :, 2:] = lo | (hi << 4)
    sc = rng.uniform(0.001, 0.02, (V, blocks)).astype(np.float16).view(np.uint16)
    q4[:, :, 0] = sc & 0xFF
    q4[:, :, 1] = sc >> 8
    packed = smp.pack_lmhead(torch.from_numpy(q4.reshape(-1)).to("cuda:0"))
    hidden = rng.uniform(0.5, 2.0, (rows, cols)).astype(np.float32)
    rlog = o.lmhead_logits(hidden, q4.reshape(-1), V, cols, threads=16)
    assert (rlog.view(np.float32) < 0).all()
    hist, hl = _top_histories(rlog, rows)
    r24 = (np.arange(rows, dtype=np.uint32) * 1_234_567) & 0xFFFFFF
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, hist, hl, r24)
    assert (glog == rlog).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, hl, r24, threads=16)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)


@pytest.mark.parametrize("rows", [3, 140])
def test_widest_hidden_state(smp, rows):
    """cols = 2048, the widest the head accepts: logits bit-exact through the
    narrow kernel (3 rows) and the wide one (140 rows, whose per-block scales
    then take 96 KB of the workgroup's LDS)."""
    import torch

    cols = 2048
    rng = np.random.default_rng(11)
    blocks = cols // 32
    q4 = rng.integers(0, 256, (V, blocks, 18), dtype=np.uint8)
    sc = rng.uniform(0.001, 0.02, (V, blocks)).astype(np.float16).view(np.uint16)
    q4[:, :, 0] = sc & 0xFF
    q4[:, :, 1] = sc >> 8
    packed = smp.pack_lmhead(torch.from_numpy(q4.reshape(-1)).to("cuda:0"), cols=cols)
    hidden = rng.standard_normal((rows, cols)).astype(np.float32)
    r24 = np.arange(rows, dtype=np.uint32) * 977
    token = torch.empty(rows, dtype=torch.int32, device="cuda:0")
    logits = torch.empty((rows, V), dtype=torch.int32, device="cuda:0")
    smp.lmhead_sample(packed, to_dev(hidden), to_dev(r24), token=token, logits=logits, cols=cols)
    torch.cuda.synchronize()
    glog = logits.cpu().numpy().view(np.uint32)
    rlog = o.lmhead_logits(hidden, q4.reshape(-1), V, cols, threads=16)
    assert (glog == rlog).all()
    rtok, _, _, _ = o.sample_batch(rlog, np.zeros((rows, 1), np.uint32),
                                   np.zeros(rows, np.uint32), r24, threads=4)
    assert (token.cpu().numpy().view(np.uint32) == rtok).all()
