"""Fused Q8_0 LM head + sampler vs the oracle (GPU).

The model's own output head is Q8_0 (tensor 290, model.rs:817-818).  The
logits must be bit-identical to the oracle's restatement of
inference_prepare_q8 + inference_q8_matvec_rows_prepared
(fp32_sse2.rs:956-983, 1251-1280), whose epilogue multiplies the two scales
first, and every sampler output bit-identical to the oracle's sampler on those
logits.  Covers the reference's own dots.bin row, batches that are not
multiples of the wave tile, two 256-row groups, the int8 extremes, special
scales, error rows, histories of each row's best ids, and the decode loop.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import GOLDEN, assert_rows_equal, to_dev
from tests.test_gpu_lmhead import _top_histories, run_head

pytestmark = pytest.mark.gpu

V = s.VOCAB
BLOCKS = workloads.HIDDEN // 32


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def head(smp):
    import torch

    w = workloads.make_lmhead(rows=300)
    q8 = workloads.make_q8_head()
    packed = smp.pack_lmhead(torch.from_numpy(q8).to("cuda:0"), q8=True)
    torch.cuda.synchronize()
    return w, q8, packed


def oracle_logits(hidden, q8, cols=workloads.HIDDEN):
    return o.lmhead_logits(hidden, q8, V, cols, threads=16, q8=True)


def test_the_references_dots_row_on_the_device(smp):
    """tests.rs:4139-4198: two 64-column blocks whose Q8_0 matvec is the
    pinned word 0x44388000 (dots.bin).  Id 0 of a 64-column head holds that
    row; the others are random."""
    import torch

    cols = 64
    rng = np.random.default_rng(31)
    q8 = np.empty((V, 2, 34), np.uint8)
    sc = rng.uniform(0.001, 0.02, (V, 2)).astype(np.float16).view(np.uint16)
    q8[:, :, 0] = sc & 0xFF
    q8[:, :, 1] = sc >> 8
    q8[:, :, 2:] = rng.integers(0, 256, (V, 2, 32), dtype=np.uint8)
    for block in range(2):
        q8[0, block, 0:2] = [0x00, 0x3C]
        q8[0, block, 2:] = (np.arange(32) % 17 - 8).astype(np.int8).view(np.uint8)
    x = np.array([float((i % 31) - 15) for i in range(64)], np.float32)
    x[31], x[63] = 127.0, -127.0
    packed = smp.pack_lmhead(torch.from_numpy(q8.reshape(-1)).to("cuda:0"), cols=cols, q8=True)
    hidden = x[None, :]
    glog, _, _, gerr = run_head(smp, packed, hidden, np.zeros((1, 1), np.uint32),
                                np.zeros(1, np.uint32), np.array([123], np.uint32), q8=True,
                                cols=cols)
    dots = np.fromfile(GOLDEN / "q4_q8_dots.bin", dtype="<u4")
    assert int(glog[0, 0]) == int(dots[1]) == 0x44388000
    assert (glog == oracle_logits(hidden, q8.reshape(-1), cols)).all()


@pytest.mark.parametrize("rows", [1, 2, 5, 16, 17, 32, 33, 64, 65, 129, 300])
def test_q8_head_logits_and_draws_are_bit_exact(smp, head, rows):
    w, q8, packed = head
    hidden = w["hidden"][:rows]
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, w["hist"][:rows],
                                      w["hist_len"][:rows], w["random_24"][:rows], q8=True)
    rlog = oracle_logits(hidden, q8)
    bad = np.argwhere(glog != rlog)
    assert bad.size == 0, (bad[:5], glog[tuple(bad[0])], rlog[tuple(bad[0])])
    rtok, rdet, rerr, _ = o.sample_batch(rlog, w["hist"][:rows], w["hist_len"][:rows],
                                         w["random_24"][:rows], threads=16)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)


@pytest.mark.parametrize("rows", [5, 160])
def test_int8_extremes_and_special_scales(smp, head, rows):
    """Weights of -128 and 127 against saturated activations (the largest
    dots, |dot| up to 2^19), and weight scales of signed zero, +-1, fp16
    subnormals, +-65504, +-inf and NaN; hidden rows with normal, fp16-subnormal,
    zero and infinite activation scales.  NaN positions compared as a set."""
    import torch

    w, q8, _ = head
    h = q8.reshape(V, BLOCKS, 34).copy()
    h[64 * 5:64 * 6, :, 2:] = np.where(np.arange(32) % 2 == 0, 0x80, 0x7F).astype(np.uint8)
    specials = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x0001, 0x03FF, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00,
                0x7E00]
    for j, bits in enumerate(specials):
        v, b = 64 * (20 + j) + 3 * j, (5 * j) % BLOCKS
        h[v, b, 0] = bits & 0xFF
        h[v, b, 1] = bits >> 8
    packed = smp.pack_lmhead(torch.from_numpy(h.reshape(-1)).to("cuda:0"), q8=True)
    rng = np.random.default_rng(7)
    hidden = np.empty((5, workloads.HIDDEN), np.float32)
    hidden[0] = rng.standard_normal(workloads.HIDDEN)
    hidden[1] = rng.standard_normal(workloads.HIDDEN) * np.float32(1e-4)
    hidden[2] = rng.standard_normal(workloads.HIDDEN)
    hidden[2, 64:96] = 0.0
    hidden[3] = rng.standard_normal(workloads.HIDDEN) * np.float32(1e7)
    hidden[4] = np.where(np.arange(workloads.HIDDEN) % 2 == 0, -3.0, 3.0)  # |q| = 127 everywhere
    hidden = np.tile(hidden, (rows // 5, 1))  # 160 rows: the wide kernel
    glog, _, _, _ = run_head(smp, packed, hidden, w["hist"][:rows], w["hist_len"][:rows],
                             w["random_24"][:rows], q8=True)
    rlog = oracle_logits(hidden, h.reshape(-1))
    gnan = np.isnan(glog.view(np.float32))
    rnan = np.isnan(rlog.view(np.float32))
    assert (gnan == rnan).all()
    bad = np.argwhere((glog != rlog) & ~rnan)
    assert bad.size == 0, (bad[:5], glog[tuple(bad[0])], rlog[tuple(bad[0])])
    assert rnan[0].any() and np.isinf(rlog.view(np.float32)[0]).any()


def test_error_rows(smp, head):
    w, q8, packed = head
    hidden = w["hidden"][:4].copy()
    hist = w["hist"][:4].copy()
    hl = w["hist_len"][:4].copy()
    hidden[1, 100] = np.inf          # every logit of row 1 is non-finite
    hist[2, 3] = V + 7               # bad history id
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, hist, hl, w["random_24"][:4],
                                      q8=True)
    rlog = oracle_logits(hidden, q8)
    assert (np.isnan(glog.view(np.float32)) == np.isnan(rlog.view(np.float32))).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, hl, w["random_24"][:4], threads=4)
    assert gerr["status"].tolist() == rerr["status"].tolist() == [0, 7, 3, 0]
    assert (gerr["detail"] == rerr["detail"]).all()
    assert (gtok == rtok).all()
    assert (gdet[0]["ids"] == rdet[0]["ids"]).all() and (gdet[3]["ids"] == rdet[3]["ids"]).all()


def test_history_holds_the_best_ids(smp, head):
    w, q8, packed = head
    rows = 30
    hidden = w["hidden"][:rows]
    rlog = oracle_logits(hidden, q8)
    hist, hl = _top_histories(rlog, rows)
    r24 = w["random_24"][:rows]
    glog, gtok, gdet, gerr = run_head(smp, packed, hidden, hist, hl, r24, q8=True)
    assert (glog == rlog).all()
    rtok, rdet, rerr, _ = o.sample_batch(rlog, hist, hl, r24, threads=16)
    assert_rows_equal(gtok, gdet, gerr, rtok, rdet, rerr)


def test_q8_decode_steps_match_the_oracle_loop(smp, head):
    import torch

    _, q8, packed = head
    rng = np.random.default_rng(9)
    prompts = [workloads.zipf_ids(rng, n) for n in (20, 7, 33)]
    seeds, limits = [4, 5, 6], [5, 8, 5]
    oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
    dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
    try:
        for step in range(9):
            hidden = np.stack([
                np.random.default_rng([r, step, d.working[-1], 8]).normal(0, 1, workloads.HIDDEN)
                for r, d in enumerate(oracle_rows)]).astype(np.float32)
            logits = oracle_logits(hidden, q8)
            want = [d.step(logits[r]) for r, d in enumerate(oracle_rows)]
            got = dec.lmhead_step(packed, to_dev(hidden), q8=True)
            assert got.tolist() == [s.NO_TOKEN if t is None else t for t in want], step
            if not dec.active():
                break
        for r, d in enumerate(oracle_rows):
            assert dec.contexts()[r].tolist() == d.working
            assert dec.sampling_states()[r].draws() == d.state.draws()
    finally:
        dec.close()


@pytest.mark.parametrize("rows", [3, 140])
def test_widest_hidden_state_q8(smp, rows):
    """cols = 2048, the widest the head accepts: the packed Q8_0 head is then
    330 MB, the largest byte offsets the GEMMs' weight and scale loads take.
    Logits bit-exact through the narrow kernel (3 rows) and the wide one
    (140 rows), and tokens equal to the oracle sampler's."""
    import torch

    cols = 2048
    rng = np.random.default_rng(12)
    blocks = cols // 32
    q8 = rng.integers(0, 256, (V, blocks, 34), dtype=np.uint8)
    sc = rng.uniform(0.0005, 0.004, (V, blocks)).astype(np.float16).view(np.uint16)
    q8[:, :, 0] = sc & 0xFF
    q8[:, :, 1] = sc >> 8
    packed = smp.pack_lmhead(torch.from_numpy(q8.reshape(-1)).to("cuda:0"), cols=cols, q8=True)
    hidden = rng.standard_normal((rows, cols)).astype(np.float32)
    r24 = np.arange(rows, dtype=np.uint32) * 977
    token = torch.empty(rows, dtype=torch.int32, device="cuda:0")
    logits = torch.empty((rows, V), dtype=torch.int32, device="cuda:0")
    smp.lmhead_sample(packed, to_dev(hidden), to_dev(r24), token=token, logits=logits, cols=cols,
                      q8=True)
    torch.cuda.synchronize()
    glog = logits.cpu().numpy().view(np.uint32)
    rlog = oracle_logits(hidden, q8.reshape(-1), cols)
    assert (glog == rlog).all()
    rtok, _, _, _ = o.sample_batch(rlog, np.zeros((rows, 1), np.uint32),
                                   np.zeros(rows, np.uint32), r24, threads=4)
    assert (token.cpu().numpy().view(np.uint32) == rtok).all()
