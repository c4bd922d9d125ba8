"""Pins the oracle where the reference holds no vector: checks fixed by the
mathematics, chosen so that a dropped term, a wrong index or a swapped
operand in the restatement fails one of them.

- expf: within 1 ulp of correctly rounded exp over its whole finite range
  (a dropped polynomial term or ln2_lo costs tens to thousands of ulps).
- top-20: equals a stable descending sort (-0 == +0, ties by ascending id).
- weights/probabilities: an independent float64 softmax over the survivors.
- top-p: `kept` is the smallest prefix whose mass reaches 0.8 of the total.
- draw: over evenly spaced uniforms the rank frequencies follow the
  survivors' probabilities, the map is monotone, u=0 picks rank 0.
"""
import numpy as np
import pytest

from oracle import oracle as o

V = o.VOCAB
K = o.TOP_K


def as_u32(x):
    return np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in representable binary32 steps between non-negative floats."""
    return np.abs(a.astype(np.int64) - b.astype(np.int64))


def correctly_rounded_exp(xs: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore", under="ignore"):
        return np.exp(xs.astype(np.float64)).astype(np.float32).view(np.uint32)


@pytest.mark.parametrize("lo,hi", [(-103.9, -87.0), (-87.0, -1.0), (-1.0, 1.0), (1.0, 88.7)])
def test_expf_within_one_ulp_of_correctly_rounded(lo, hi):
    rng = np.random.default_rng(1234)
    xs = rng.uniform(lo, hi, 20000).astype(np.float32)
    xs = np.concatenate([xs, np.float32([lo, hi])]).astype(np.float32)
    got = np.array([o.expf_bits(int(b)) for b in xs.view(np.uint32)], np.uint32)
    want = correctly_rounded_exp(xs)
    d = ulp_distance(got, want)
    assert d.max() <= 1, (xs[d.argmax()], hex(got[d.argmax()]), hex(want[d.argmax()]))
    # the method is mostly exactly rounded; a wrong constant would shift this
    assert (d == 0).mean() > 0.8


def test_expf_tiny_and_special_inputs():
    tiny = np.float32([1e-8, -1e-8, 2**-20, -(2**-20), 1e-30, 0.0])
    for x in tiny:
        assert o.expf_bits(int(as_u32([x])[0])) == int(as_u32([np.float32(1.0) + x])[0])
    assert o.expf_bits(0x7FC00000) == 0x7FC00000  # NaN passes through
    assert o.expf_bits(0xFF800000) == 0            # exp(-inf) = 0
    assert o.expf_bits(0x7F800000) == 0x7F800000   # exp(+inf) = inf


def stable_topk(values: np.ndarray, k=K) -> np.ndarray:
    v = values.astype(np.float32).copy()
    v[v == 0] = 0.0  # -0 ties with +0
    return np.argsort(-v, kind="stable")[:k]


def make_rows(rng, kind, n=12):
    rows = []
    for _ in range(n):
        if kind == "normal":
            r = rng.normal(0, 2.5, V).astype(np.float32)
            r[rng.choice(V, 5, replace=False)] += rng.uniform(8, 15, 5).astype(np.float32)
        elif kind == "flat":
            r = rng.normal(0, 0.1, V).astype(np.float32)
        elif kind == "ties":
            r = (np.round(rng.normal(0, 2.5, V) * 4) / 4).astype(np.float32)
        elif kind == "zeros":
            r = np.where(rng.random(V) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
            r[rng.choice(V, 7, replace=False)] = np.float32(-1.0)
        elif kind == "negative":
            r = rng.normal(-60, 0.5, V).astype(np.float32)
        rows.append(r)
    return rows


@pytest.mark.parametrize("kind", ["normal", "flat", "ties", "zeros", "negative"])
def test_topk_is_stable_descending_sort(kind):
    rng = np.random.default_rng(["normal", "flat", "ties", "zeros", "negative"].index(kind) + 100)
    for row in make_rows(rng, kind, 6):
        tok, det = o.sample_top_k_top_p(row, 123456)
        assert det["ids"].tolist() == stable_topk(row).tolist()
        assert (det["value_bits"] == as_u32(row)[det["ids"]]).all()
        assert det["token"] == tok == det["ids"][det["rank"]]


@pytest.mark.parametrize("kind", ["normal", "flat", "ties"])
def test_probabilities_match_float64_softmax(kind):
    rng = np.random.default_rng(7)
    for row in make_rows(rng, kind, 8):
        _, det = o.sample_top_k_top_p(row, 99)
        kept = int(det["kept"])
        v = row[det["ids"]].astype(np.float64)
        w = np.exp((v - v[0]) / 0.7)
        p = w[:kept] / w[:kept].sum()
        got = det["probs"][:kept].astype(np.float64)
        assert np.allclose(got, p, rtol=1e-5, atol=0), (got, p)
        assert (det["probs"][kept:] == 0).all()
        assert det["weight_bits"][0] == 0x3F800000  # w[0] = exp(0) = 1 exactly


@pytest.mark.parametrize("kind", ["normal", "flat", "ties"])
def test_top_p_kept_is_minimal_prefix(kind):
    rng = np.random.default_rng(11)
    for row in make_rows(rng, kind, 8):
        _, det = o.sample_top_k_top_p(row, 5)
        if det["flags"] & o.FLAG_CUTOFF_BOUNDARY:
            continue
        w = det["weight_bits"].view(np.float32).astype(np.float64)
        prefix = np.cumsum(w)
        need = 0.8 * prefix[-1]
        kept = int(det["kept"])
        expected = int(np.argmax(prefix >= need)) + 1 if (prefix >= need).any() else K
        assert kept == expected
        # closed form: kept == 1 exactly when w[0] alone reaches the cutoff
        assert (kept == 1) == (1.0 >= need)


def test_draw_frequencies_follow_probabilities():
    """Small-vocabulary row so every uniform is cheap: sweep 2^14 evenly spaced
    24-bit uniforms; rank frequencies must equal the survivors' probabilities
    to within the sweep resolution, and the rank must be monotone in u."""
    rng = np.random.default_rng(3)
    row = rng.normal(0, 0.3, 64).astype(np.float32)
    n = 1 << 14
    ranks = []
    det0 = None
    for i in range(n):
        r24 = (i << 10) | 0x1FF
        tok, det = o.sample_top_k_top_p(row, r24)
        ranks.append(int(det["rank"]))
        det0 = det
    ranks = np.array(ranks)
    kept = int(det0["kept"])
    assert kept > 3
    assert (np.diff(ranks) >= 0).all()
    freq = np.bincount(ranks, minlength=K)[:kept] / n
    assert np.abs(freq - det0["probs"][:kept]).max() < 2.0 / n + 1e-6
    assert o.sample_top_k_top_p(row, 0)[1]["rank"] == 0
    assert o.sample_top_k_top_p(row, 0xFFFFFF)[1]["rank"] == kept - 1


def test_random_24_uses_low_24_bits_only():
    rng = np.random.default_rng(5)
    row = rng.normal(0, 0.3, 64).astype(np.float32)
    for r in (0, 123, 0xABCDEF, 0xFFFFFF):
        a = o.sample_top_k_top_p(row, r)[0]
        b = o.sample_top_k_top_p(row, r | 0xFF000000)[0]
        assert a == b


def test_batch_driver_equals_single_calls():
    rng = np.random.default_rng(21)
    B = 5
    logits = rng.normal(0, 2.5, (B, V)).astype(np.float32)
    hist = rng.integers(0, 2000, (B, 64)).astype(np.uint32)
    hist_len = np.array([0, 1, 17, 64, 33], np.uint32)
    r24 = rng.integers(0, 1 << 24, B).astype(np.uint32)
    logits[3, 100] = np.nan
    hist[4, 5] = V + 3
    tok, det, err, pen = o.sample_batch(logits, hist, hist_len, r24, threads=2,
                                        want_penalized=True)
    for r in range(B):
        st, t, _, d = _single(logits[r], hist[r, :hist_len[r]], r24[r])
        assert err[r]["status"] == st
        if st == 0:
            assert tok[r] == t and (det[r]["ids"] == d["ids"]).all()
            assert (pen[r] == row_after(logits[r], hist[r, :hist_len[r]])).all()
        else:
            assert tok[r] == 0xFFFFFFFF
    assert err[3]["status"] == 7 and err[3]["detail"] == (7 << 32) | 100
    assert err[4]["status"] == 3 and err[4]["available"] == V + 3


def _single(row_f32, hist, r24):
    """Penalty then top-k/top-p with a given uniform, via the single-row API."""
    row = as_u32(row_f32).copy()
    # validation precedence as in sample_token_with_repetition
    bad = np.flatnonzero((row & 0x7F800000) == 0x7F800000)
    if bad.size:
        return 7, 0, None, None
    if (np.asarray(hist) >= V).any():
        return 3, 0, None, None
    o.apply_repetition_penalty(row, hist, np.zeros(o.SEEN_BYTES, np.uint8))
    t, d = o.sample_top_k_top_p(row, int(r24))
    return 0, t, None, d


def row_after(row_f32, hist):
    row = as_u32(row_f32).copy()
    o.apply_repetition_penalty(row, hist, np.zeros(o.SEEN_BYTES, np.uint8))
    return row


def test_draw_on_exact_cdf_step_goes_to_next_survivor():
    """Two tied leaders (w = [1, 1], rest underflow to 0): top-p keeps both
    (1 < 0.8*2 <= 2), kept_total = 2, and u = 2^23/2^24 = 0.5 gives target
    exactly 1.0 = the first CDF step.  The reference's strict `>`
    (fp32_sse2.rs:1840) passes over it to rank 1; `>=` would stop at rank 0."""
    row = np.full(64, -1000.0, np.float32)
    row[[10, 30]] = 5.0
    tok, det = o.sample_top_k_top_p(row, 1 << 23)
    assert det["kept"] == 2 and det["ids"][:2].tolist() == [10, 30]
    assert det["weight_bits"][:2].tolist() == [0x3F800000, 0x3F800000]
    assert tok == 30 and det["rank"] == 1
    assert det["flags"] & o.FLAG_DRAW_BOUNDARY
    # one step below the boundary stays on rank 0
    assert o.sample_top_k_top_p(row, (1 << 23) - 1)[0] == 10


def _kept_rule(weights_f32: np.ndarray, accumulate_f32: bool) -> int:
    total = np.float32(0) if accumulate_f32 else 0.0
    for w in weights_f32:
        total = np.float32(total + w) if accumulate_f32 else total + float(w)
    cutoff = np.float32(np.float32(total) * np.float32(0.8))
    prefix = 0.0
    for i, w in enumerate(weights_f32):
        prefix += float(w)
        if not cutoff > np.float32(prefix):
            return i + 1
    return K


def test_top_p_total_accumulates_in_float64():
    """fp32_sse2.rs:1820-1824 sums the weights in binary64.  Rows whose top-20
    sit within 2^-13 of the leader have weights 1 + x exactly (the tiny-input
    branch of expf), so the weights are known without the oracle.  For the
    deficit pairs (e, f) below a binary32 running sum moves the cutoff across
    prefix 16; the oracle must follow the binary64 rule."""
    decisive = 0
    for e in (23, 29, 41, 77, 151):
        for f in range(int(e * 0.85), int(e * 1.05) + 1):
            row = np.full(40, -1000.0, np.float32)
            row[0] = 0.0
            row[1:16] = -np.float32(e * 1e-7)
            row[16:20] = -np.float32(f * 1e-7)
            top = row[stable_topk(row)]
            x = (top - top[0]) / np.float32(0.7)
            w = (np.float32(1.0) + x.astype(np.float32)).astype(np.float32)
            _, det = o.sample_top_k_top_p(row, 1)
            assert (det["weight_bits"] == w.view(np.uint32)).all()
            k64, k32 = _kept_rule(w, False), _kept_rule(w, True)
            assert det["kept"] == k64
            decisive += k64 != k32
    assert decisive >= 5
