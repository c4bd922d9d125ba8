"""Batched device sampler vs the oracle, row by row, every output bit-exact (GPU).

Covers the workloads of promptboot_amd.workloads (B=1, 64, adversarial
B=1024 cases, a B=4096 slice of full-context histories), the small batches'
path through the tile words and the LM head's selection, the
single-workgroup path (one slice per row) and the multi-slice path with the
cross-slice merge (forced slice plans), error rows, and the in-place penalty
variant.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads
from tests.conftest import assert_rows_equal, to_dev

pytestmark = pytest.mark.gpu

V = s.VOCAB


@pytest.fixture(scope="module")
def sampler():
    smp = s.BatchSampler(0)
    yield smp
    smp.close()


def run_gpu(smp, w, segments=0, rows=None):
    import torch

    smp.set_segments(segments)
    B = w["logits"].shape[0] if rows is None else rows
    logits = to_dev(w["logits"][:B])
    hist = to_dev(w["hist"][:B])
    hl = to_dev(w["hist_len"][:B])
    r24 = to_dev(w["random_24"][:B])
    token = torch.empty(B, dtype=torch.int32, device="cuda:0")
    det = torch.empty((B, s.DETAIL_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    err = torch.empty((B, s.ERROR_DTYPE.itemsize // 4), dtype=torch.int32, device="cuda:0")
    smp.sample(logits, r24, hist, hl, token=token, detail=det, err=err)
    torch.cuda.synchronize()
    smp.set_segments(0)
    return (token.cpu().numpy().view(np.uint32), det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(B),
            err.cpu().numpy().view(s.ERROR_DTYPE).reshape(B))


def run_oracle(w, rows=None):
    B = w["logits"].shape[0] if rows is None else rows
    tok, det, err, _ = o.sample_batch(w["logits"][:B], w["hist"][:B], w["hist_len"][:B],
                                      w["random_24"][:B], threads=16)
    return tok, det, err


@pytest.mark.parametrize("name,rows", [("single", None), ("small", None), ("flat", 256),
                                       ("ties", 256), ("dominant", 256), ("half", 128)])
@pytest.mark.parametrize("segments", [0, 1, 7])
def test_batch_matches_oracle(sampler, name, rows, segments):
    w = workloads.make(name, rows=rows)
    got = run_gpu(sampler, w, segments)
    want = run_oracle(w)
    assert_rows_equal(*got, *want)
    assert (got[2]["status"] == 0).all()


def test_large_rows_with_full_context_histories(sampler):
    w = workloads.make("large", rows=512)
    assert w["hist"].shape[1] == 32768 and w["hist_len"].max() > 30000
    got = run_gpu(sampler, w)
    want = run_oracle(w)
    assert_rows_equal(*got, *want)


def test_rows_past_the_first_residency_round_run_longest_history_first(sampler):
    """Past the workgroups the GPU holds at once (1,024 on MI355X), one-slice
    batches take the remaining rows longest history first, ranked in groups of
    4,096 rows.  5,300 rows with lengths spread over 0..32,768 (some zero, some
    past the stride and clamped) span two such groups; every row is sampled
    exactly once and bit-exact against the oracle (the outputs start as 0xff
    bytes, so a row left out or sampled into the wrong slot shows)."""
    import torch

    B, L = 5300, 32768
    rng = np.random.default_rng(20260101)
    logits = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.5)
    hist = rng.integers(0, V, (B, L), dtype=np.uint32)
    hl = rng.integers(0, L + 1, B).astype(np.uint32)
    hl[::89] = 0
    hl[5::97] = L + 7
    r24 = rng.integers(0, 1 << 24, B).astype(np.uint32)
    token = torch.full((B,), -1, dtype=torch.int32, device="cuda:0")
    det = torch.full((B, s.DETAIL_DTYPE.itemsize // 4), -1, dtype=torch.int32, device="cuda:0")
    err = torch.full((B, s.ERROR_DTYPE.itemsize // 4), -1, dtype=torch.int32, device="cuda:0")
    sampler.sample(to_dev(logits), to_dev(r24), to_dev(hist), to_dev(hl), token=token, detail=det,
                   err=err)
    torch.cuda.synchronize()
    got = (token.cpu().numpy().view(np.uint32), det.cpu().numpy().view(s.DETAIL_DTYPE).reshape(B),
           err.cpu().numpy().view(s.ERROR_DTYPE).reshape(B))
    tok, rdet, rerr, _ = o.sample_batch(logits, hist, np.minimum(hl, L).astype(np.uint32), r24,
                                        threads=16)
    assert_rows_equal(*got, tok, rdet, rerr)
    assert (got[2]["status"] == 0).all()


@pytest.mark.parametrize("name,rows", [("large", 192), ("ties", 128), ("flat", 128),
                                       ("dominant", 64)])
def test_small_batches_take_the_tile_selection(sampler, name, rows):
    """Up to 192 rows the automatic plan samples through the tile words and the
    LM head's selection: full-context histories (whose penalties push some
    rows' top-20 below the first round's threshold, into a second round or
    the general selection) and the adversarial rows, bit-exact."""
    w = workloads.make(name, rows=rows)
    got = run_gpu(sampler, w)
    want = run_oracle(w)
    assert_rows_equal(*got, *want)


@pytest.mark.parametrize("segments", [1, 2, 5, 64])
def test_segment_counts_agree(sampler, segments):
    w = workloads.make("small", rows=16)
    assert_rows_equal(*run_gpu(sampler, w, segments), *run_oracle(w))


def test_error_rows_and_precedence(sampler):
    w = workloads.make("small", rows=12)
    lg, hist, hl = w["logits"], w["hist"], w["hist_len"]
    lg[1, 151_935] = np.nan                       # last element
    lg[2, 0] = np.inf                             # first element
    lg[3, [90_000, 7, 150_000]] = [np.nan, -np.inf, np.inf]  # first index wins
    hist[4, 5] = V                                # first bad id position wins
    hist[4, 9] = V + 100
    hl[4] = max(hl[4], 10)
    lg[5, 100] = np.nan                           # non-finite beats a bad id
    hist[5, 0] = 0xFFFFFFFF
    hl[6] = min(hl[6], hist.shape[1] - 1)
    hist[6, hl[6]] = V + 1                        # beyond the length: ignored
    lg[7, :] = np.float32(-3.4e38)                # penalty overflows to -inf
    lg[8, :] = 0.0                                # all ties
    lg[8, ::2] = np.float32(-0.0)
    lg[9, :] = np.float32(1e-42)                  # subnormal logits
    lg[10, 1000:1040] = np.float32(7.0)           # a tie block at the top
    for segments in (0, 1, 3, 64):
        assert_rows_equal(*run_gpu(sampler, w, segments), *run_oracle(w))
    tok, det, err = run_gpu(sampler, w)
    assert err["status"].tolist()[:6] == [0, 7, 7, 7, 3, 7]
    assert err["detail"][3] == (7 << 32) | 7 and err["available"][4] == V
    assert (tok[1:6] == s.NO_TOKEN).all()
    assert (det[1:6]["ids"] == 0xFFFFFFFF).all()


def test_bad_ids_deep_in_full_context_histories(sampler):
    """Ids >= vocab at every batch boundary of a 32,768-id history: the end of
    the first batch of 4,096 ids and the start of the second, the start of
    the batches requested two at a time after them, the last position, and
    one just past a row's length (ignored).  The first bad position decides
    the error (its id is the record's `available`); a non-finite logit
    still wins.  Tile selection (8 rows) and both slice plans, against the
    oracle."""
    w = workloads.make("large", rows=8)
    lg, hist, hl = w["logits"], w["hist"], w["hist_len"]
    assert hist.shape[1] == 32768
    hl[:] = 32768
    hist[0, [5000, 20000]] = [V + 1, V + 2]       # the first one wins
    hist[1, 32767] = V + 3                        # the last position
    hist[2, [8192, 30000]] = [V + 4, 0xFFFFFFFF]  # first batch of the first pair
    hist[3, 4096] = V + 5                         # first id of the second batch
    hl[4] = 9000
    hist[4, 9000] = V + 6                         # past the length: ignored
    hist[5, 12345] = V + 7
    lg[5, 77] = np.nan                            # non-finite beats a bad id
    hl[7] = 4097
    hist[7, 4096] = V + 8                         # the row's last position
    hist[7, 4095] = V + 9                         # ... after an earlier one
    for segments in (0, 1, 7):
        assert_rows_equal(*run_gpu(sampler, w, segments), *run_oracle(w))
    tok, det, err = run_gpu(sampler, w)
    assert err["status"].tolist() == [3, 3, 3, 3, 0, 7, 0, 3]
    assert err["available"][[0, 1, 2, 3, 7]].tolist() == [V + 1, V + 3, V + 4, V + 5, V + 9]
    assert tok[4] != s.NO_TOKEN and tok[6] != s.NO_TOKEN


def test_inplace_variant_penalises_like_the_reference(sampler):
    import torch

    w = workloads.make("small", rows=24)
    w["logits"][3, 17] = np.nan  # a failing row must stay untouched
    B = 24
    logits = to_dev(w["logits"])
    seen = torch.zeros((B, s.SEEN_BYTES), dtype=torch.uint8, device="cuda:0")
    token = torch.empty(B, dtype=torch.int32, device="cuda:0")
    sampler.sample(logits, to_dev(w["random_24"]), to_dev(w["hist"]), to_dev(w["hist_len"]),
                   token=token, inplace=True, seen=seen)
    torch.cuda.synchronize()
    rtok, _, rerr, pen = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"],
                                        threads=8, want_penalized=True)
    got = logits.cpu().numpy().view(np.uint32)
    assert (token.cpu().numpy().view(np.uint32) == rtok).all()
    ok = rerr["status"] == 0
    assert (got[ok] == pen[ok]).all()
    assert (got[~ok] == w["logits"][~ok].view(np.uint32)).all()
    assert not seen.cpu().numpy().any()


def test_rows_are_independent_of_batch_neighbours(sampler):
    w = workloads.make("small", rows=64)
    full = run_gpu(sampler, w)
    for r in (0, 17, 63):
        one = {k: (v[r:r + 1] if isinstance(v, np.ndarray) else v) for k, v in w.items()}
        single = run_gpu(sampler, one)
        assert single[0][0] == full[0][r]
        assert (single[1][0]["ids"] == full[1][r]["ids"]).all()


def test_sample_rows_is_transactional_per_row(sampler):
    w = workloads.make("small", rows=6)
    w["logits"][2, 5] = np.inf
    states = [s.SamplingState(int(x)) for x in w["seeds"]]
    tok, det, err = sampler.sample_rows(to_dev(w["logits"]), to_dev(w["hist"]),
                                        to_dev(w["hist_len"]), states)
    draws = [st.draws() for st in states]
    assert draws == [1, 1, 0, 1, 1, 1]
    assert states[2] == s.SamplingState(int(w["seeds"][2]))
    rtok, _, _, _ = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"])
    assert (tok == rtok).all()


def test_best_logits_in_the_last_tiles_of_the_row(sampler):
    """The row's last six 64-id tiles fall in the last tile-words workgroup,
    whose other lanes read the row's last tile again (clamped) and store
    nothing.  Rows whose maximum is the last id, whose whole top-20 is the
    last tile, or whose maximum sits just inside or just before those six
    tiles: through the batch (logits in HBM) and through the drop-in (logits
    read from host memory), both bit-exact against the oracle."""
    w = workloads.make("small", rows=4)
    lg = w["logits"].view(np.float32)
    V = lg.shape[1]
    lg[0, V - 1] = 60.0
    lg[1, V - 64:V - 44] = 50.0 + np.arange(20, dtype=np.float32)
    lg[2, V - 6 * 64] = 55.0
    lg[3, V - 6 * 64 - 1] = 55.0
    got = run_gpu(sampler, w)
    want = run_oracle(w)
    assert_rows_equal(*got, *want)
    for r in range(4):
        hist = np.ascontiguousarray(w["hist"][r, :w["hist_len"][r]])
        g = lg[r].view(np.uint32).copy()
        ref = g.copy()
        gseen = np.zeros(s.SEEN_BYTES, np.uint8)
        rseen = gseen.copy()
        gs, rs = s.SamplingState(100 + r), o.SamplingState(100 + r)
        t = s.sample_token_with_repetition(g, hist, gseen, gs)
        _, rt, _ = o.sample_token_with_repetition(ref, hist, rseen, rs)
        assert t == rt and (g == ref).all() and not gseen.any(), r


@pytest.mark.parametrize("rows", [1, 64, 192])
def test_tile_selection_on_padded_rows_and_an_odd_history_stride(sampler, rows):
    """The tile selection (up to 192 rows) on logits rows padded to ld = V + 4,
    whose padding holds NaN that must never be read, and on a history matrix
    whose stride of 1,023 ids is not a multiple of 4 (the scalar history
    loads), bit-exact against the oracle."""
    w = workloads.make("small", rows=rows)
    lg = np.full((rows, V + 4), np.nan, np.float32)
    lg[:, :V] = w["logits"]
    hl = np.minimum(w["hist_len"], 1023).astype(np.uint32)
    hl[0] = 1023
    padded = dict(logits=lg, hist=np.ascontiguousarray(w["hist"][:, :1023]), hist_len=hl,
                  random_24=w["random_24"])
    got = run_gpu(sampler, padded)
    assert_rows_equal(*got, *run_oracle(padded))
    assert (got[2]["status"] == 0).all()


@pytest.mark.parametrize("name,rows,segments", [("small", 64, 0), ("flat", 256, 0), ("small", 64, 7)])
def test_history_lengths_past_the_stride_are_clamped(sampler, name, rows, segments):
    """A history length above hist_ld counts as hist_ld ids (the header's
    contract for every batched entry point): lengths of hist_ld + 1, far past
    it and 0xffffffff give the oracle's results on the clamped lengths, on the
    tile selection, the one-slice plan and a forced seven-slice plan."""
    w = workloads.make(name, rows=rows)
    ld = w["hist"].shape[1]
    long = w["hist_len"].copy()
    long[0::3] = ld + 1
    long[1::3] = ld + 12345
    long[2] = 0xFFFFFFFF
    got = run_gpu(sampler, dict(w, hist_len=long), segments=segments)
    want = run_oracle(dict(w, hist_len=np.minimum(long, ld).astype(np.uint32)))
    assert_rows_equal(*got, *want)
    assert (got[2]["status"] == 0).all()
