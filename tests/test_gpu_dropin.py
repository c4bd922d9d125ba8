"""The reference's sampler unit tests, run through the GPU drop-ins (C ABI).

Mirrors crates/promptboot-core/src/tests.rs:368-599 and the exact host
oracle's first sampled token (fixtures/inference/exact-host-oracle.txt:14),
calling pb_sample_token_with_repetition / pb_sample_token / pb_greedy_token /
pb_top_logits_8 through promptboot_amd.sampler.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from tests.test_oracle_known_answers import fbits, filled

pytestmark = pytest.mark.gpu

V = s.VOCAB


def test_real_hello_row_draws_9707_and_penalises_like_the_oracle(known, qwen_cases):
    e = known["exact_host_oracle"]
    logits, prompt = qwen_cases["hello"]
    gpu_logits = logits.copy()
    ref_logits = logits.copy()
    state = s.SamplingState(e["seed"])
    seen = np.zeros(s.SEEN_BYTES, np.uint8)
    token = s.sample_token_with_repetition(gpu_logits, prompt, seen, state)
    assert token == e["first_sampled_token"] == 9707
    assert state.draws() == 1
    ref_state = o.SamplingState(e["seed"])
    o.sample_token_with_repetition(ref_logits, prompt, np.zeros(o.SEEN_BYTES, np.uint8),
                                   ref_state)
    assert state.state() == ref_state.state()
    assert (gpu_logits == ref_logits).all()
    assert not seen.any()


@pytest.mark.parametrize("case", ["hello", "arithmetic", "color"])
def test_real_rows_match_oracle_for_many_draws(qwen_cases, case):
    logits, prompt = qwen_cases[case]
    for seed in (1, 2, 3, 0xFEEDFACEDEADBEEF, 0x0123456789ABCDEF):
        g, r = logits.copy(), logits.copy()
        gs, rs = s.SamplingState(seed), o.SamplingState(seed)
        history = list(prompt)
        for _ in range(3):
            # the history grows by each drawn token, as in the generation loop
            # (validate_inference.rs:796-810); the row keeps its penalties
            t = s.sample_token_with_repetition(g, history, np.zeros(s.SEEN_BYTES, np.uint8), gs)
            st, rt, _ = o.sample_token_with_repetition(r, history, np.zeros(o.SEEN_BYTES, np.uint8), rs)
            assert st == 0 and t == rt
            assert (g == r).all()
            history.append(t)
        assert gs.state() == rs.state() and gs.draws() == rs.draws() == 3


@pytest.mark.parametrize("case", ["hello", "arithmetic", "color"])
def test_real_rows_top8_and_greedy_match_llama_cpp(known, qwen_cases, case):
    c = known["cases"][case]
    logits, _ = qwen_cases[case]
    assert s.top_logits_8(logits).tolist() == c["step0_top8"]
    assert s.greedy_token(logits) == c["step0_selected_id"]


def test_sampling_is_seeded_bounded_and_transactional(known):
    b = known["unit"]["bounded_row"]
    logits = filled(b["fill"])
    for token in range(b["count"]):
        logits[token] = fbits(np.float32(b["start"]) - np.float32(token) * np.float32(b["step"]))
    first = s.SamplingState(b["seed"])
    second = first.copy()
    for _ in range(b["draws"]):
        a = s.sample_token(logits, first)
        assert a == s.sample_token(logits, second)
        assert a < b["selected_below"]
    assert first == second and first.draws() == 8
    assert first.state() == known["unit"]["prng"]["state_after"]
    assert s.SamplingState(0).state() == known["unit"]["prng"]["zero_seed_state"]

    before = first.copy()
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token(logits[:-1], first)
    assert ex.value.status == s.CAPACITY and first == before
    logits[17] = fbits(float("nan"))
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token(logits, first)
    assert ex.value.status == s.NONFINITE_OUTPUT and first == before
    assert ex.value.detail == (7 << 32) | 17


def test_penalty_applies_once_per_seen_token_and_clears_scratch(known):
    p = known["unit"]["penalty"]
    logits = filled(p["fill"], p["set"])
    seen = np.zeros(s.SEEN_BYTES, np.uint8)
    state = s.SamplingState(p["seed"])
    s.sample_token_with_repetition(logits, p["history"], seen, state)
    assert logits[7] == fbits(np.float32(11.0) / np.float32(1.1))
    assert logits[9] == fbits(np.float32(-2.0) * np.float32(1.1))
    assert logits[12] == fbits("-0.0")
    assert not seen.any()
    assert state.draws() == 1

    before = logits.copy()
    before_state = state.copy()
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token_with_repetition(logits, p["bad_token_history"], seen, state)
    assert ex.value.tuple() == [3, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, V, V, 2 << 32]
    assert (logits == before).all() and not seen.any() and state == before_state


def test_all_zero_row_with_penalty_matches_oracle(known):
    """The penalty test row is 151,933 zeros: every rank ties, so the top-20
    is decided by the id order alone."""
    p = known["unit"]["penalty"]
    for seed in range(1, 9):
        g = filled(p["fill"], p["set"])
        r = g.copy()
        gs, rs = s.SamplingState(seed), o.SamplingState(seed)
        t = s.sample_token_with_repetition(g, p["history"], np.zeros(s.SEEN_BYTES, np.uint8), gs)
        _, rt, _ = o.sample_token_with_repetition(r, p["history"], np.zeros(o.SEEN_BYTES, np.uint8), rs)
        assert t == rt and (g == r).all()


def test_dominant_eos_row(known):
    d = known["unit"]["dominant"]
    logits = filled(d["fill"], [(d["eos"], d["eos_value"]), (d["zero_at"], 0.0)])
    for seed in d["seeds"]:
        state = s.SamplingState(seed)
        assert s.sample_token(logits, state) == d["eos"]
        assert state.draws() == 1


def test_error_tuples_and_precedence(known):
    t = known["unit"]["error_tuples"]
    g = known["unit"]["greedy_tie"]
    logits = filled(g["fill"], g["set"])
    assert s.greedy_token(logits) == g["expected"]
    for bad, want in ((logits[:-1], t["short"]), (np.zeros(V + 1, np.uint32), t["long"])):
        with pytest.raises(s.InferenceError) as ex:
            s.greedy_token(bad)
        assert ex.value.tuple() == want
    logits[11] = fbits(float("nan"))
    with pytest.raises(s.InferenceError) as ex:
        s.greedy_token(logits)
    assert ex.value.tuple() == t["nan_at_11"]

    # non-finite beats a short scratch, which beats a bad history id
    # (inference.rs:925-953)
    row = filled(0.5)
    row[99_999] = fbits(float("-inf"))
    state = s.SamplingState(3)
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token_with_repetition(row, [V + 5], np.zeros(10, np.uint8), state)
    assert ex.value.status == s.NONFINITE_OUTPUT and ex.value.detail == (7 << 32) | 99_999
    row[99_999] = fbits(1.0)
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token_with_repetition(row, [V + 5], np.zeros(10, np.uint8), state)
    assert ex.value.tuple() == [4, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, s.SEEN_BYTES, 10, (4 << 32) | 2]
    with pytest.raises(s.InferenceError) as ex:
        s.sample_token_with_repetition(row, [3, V + 5, V + 9], np.zeros(s.SEEN_BYTES, np.uint8),
                                       state)
    assert ex.value.tuple() == [3, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, V, V + 5, 2 << 32]
    assert state.draws() == 0


def test_top8_stable_signed_zero_and_transactional(known):
    t = known["unit"]["top8_stable"]
    logits = filled(t["fill"], t["set"])
    out = s.top_logits_8(logits)
    assert out[:, 0].tolist() == t["expected_tokens"]
    sentinel = np.tile(np.array([0xFEEDFACE, 0xDEADBEEF], np.uint32), 8).reshape(8, 2)
    keep = sentinel.copy()
    with pytest.raises(s.InferenceError):
        s.top_logits_8(logits[:-1], keep)
    logits[t["inf_at"]] = fbits(float("inf"))
    with pytest.raises(s.InferenceError) as ex:
        s.top_logits_8(logits, keep)
    assert ex.value.detail == (7 << 32) | t["inf_at"]
    assert (keep == sentinel).all()

    z = known["unit"]["top8_signed_zero"]
    out = s.top_logits_8(filled(z["fill"], z["set"]))
    assert out[:, 0].tolist() == z["expected_tokens"]
    assert out[0, 1] == fbits("-0.0") and out[1, 1] == fbits(0.0)


def test_preset_seen_bits_follow_the_reference_dedupe():
    """Ids whose scratch bit is already set are skipped by the penalty and the
    history bits are cleared afterwards (fp32_sse2.rs:1856-1875)."""
    rng = np.random.default_rng(9)
    base = rng.normal(0, 2.5, V).astype(np.float32).view(np.uint32)
    hist = rng.integers(0, 3000, 400).astype(np.uint32)
    top = np.argsort(-base.view(np.float32))[:30].astype(np.uint32)
    hist = np.concatenate([hist, top])
    seen0 = np.zeros(s.SEEN_BYTES, np.uint8)
    for tok in list(top[::3]) + [5, 77_777]:
        seen0[tok // 8] |= 1 << (tok % 8)
    g, r = base.copy(), base.copy()
    gseen, rseen = seen0.copy(), seen0.copy()
    gs, rs = s.SamplingState(11), o.SamplingState(11)
    t = s.sample_token_with_repetition(g, hist, gseen, gs)
    _, rt, _ = o.sample_token_with_repetition(r, hist, rseen, rs)
    assert t == rt and (g == r).all() and (gseen == rseen).all()


def test_staging_grows_then_shorter_and_empty_histories():
    """A 40,000-id history outgrows the drop-in's staging (sized at context
    creation for 32,768 ids, the context limit); then a short history and an
    empty one follow on the regrown buffers.  Each call has preset scratch
    bits: with an empty history the scratch comes back exactly as it went in."""
    rng = np.random.default_rng(17)
    base = rng.normal(0, 2.5, V).astype(np.float32).view(np.uint32)
    top = np.argsort(-base.view(np.float32))[:40].astype(np.uint32)
    long_hist = np.concatenate([rng.integers(0, V, 39_960).astype(np.uint32), top])
    seen0 = np.zeros(s.SEEN_BYTES, np.uint8)
    for tok in list(top[::4]) + [9, 150_000]:
        seen0[tok // 8] |= 1 << (tok % 8)
    gs, rs = s.SamplingState(21), o.SamplingState(21)
    for hist in (long_hist, top[:25], np.zeros(0, np.uint32)):
        g, r = base.copy(), base.copy()
        gseen, rseen = seen0.copy(), seen0.copy()
        t = s.sample_token_with_repetition(g, hist, gseen, gs)
        _, rt, _ = o.sample_token_with_repetition(r, hist, rseen, rs)
        assert t == rt and (g == r).all() and (gseen == rseen).all()
        assert gs.state() == rs.state() and gs.draws() == rs.draws()
    assert (gseen == seen0).all()


def test_mapped_and_copied_staging_alternate():
    """Calls with a clear scratch (the row, scalars and history read from the
    mapped pinned staging, the token, records and penalised values written
    back into it) alternate with calls whose scratch has bits set (one copy
    each way and a write-back launch), on histories that grow the staging
    between them.  Every call matches the oracle."""
    rng = np.random.default_rng(23)
    gs, rs = s.SamplingState(5), o.SamplingState(5)
    for i, n in enumerate((300, 300, 70_000, 70_000, 17, 0, 1, 1)):
        base = rng.normal(0, 2.5, V).astype(np.float32).view(np.uint32)
        top = np.argsort(-base.view(np.float32))[:20].astype(np.uint32)
        hist = np.concatenate([rng.integers(0, V, n).astype(np.uint32), top[:min(n, 20)]])
        seen0 = np.zeros(s.SEEN_BYTES, np.uint8)
        if i % 2:
            for tok in list(top[::3]) + [5]:
                seen0[tok // 8] |= 1 << (tok % 8)
        g, r = base.copy(), base.copy()
        gseen, rseen = seen0.copy(), seen0.copy()
        t = s.sample_token_with_repetition(g, hist, gseen, gs)
        _, rt, _ = o.sample_token_with_repetition(r, hist, rseen, rs)
        assert t == rt and (g == r).all() and (gseen == rseen).all(), (i, n)
        assert gs.state() == rs.state() and gs.draws() == rs.draws()
