"""Pins the CPU oracle to every known answer the reference holds for the sampler.

Sources: crates/promptboot-core/src/tests.rs:368-599 (sampler unit tests),
fixtures/analytic/expf-edge.u32le, fixtures/inference/exact-host-oracle.txt
and fixtures/reference/model/*/{prompt_final_logits.f32le,steps.json}
(copied as data into tests/golden/ by tests/golden/make_golden.py).
"""
import numpy as np
import pytest

from oracle import oracle as o
from tests.conftest import GOLDEN

V = o.VOCAB


def fbits(x) -> int:
    if isinstance(x, str):
        x = float(x)
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def filled(fill, sets=()):
    row = np.full(V, fbits(fill), dtype=np.uint32)
    for token, value in sets:
        row[token] = fbits(value)
    return row


# ---- PRNG (inference.rs:779-810; tests.rs:424-441; exact-host-oracle.txt:15-16) ----

def test_prng_state_after_eight_draws(known):
    p = known["unit"]["prng"]
    s = o.SamplingState(p["seed"])
    for _ in range(p["draws"]):
        s.next_24()
    assert s.state() == p["state_after"]
    assert s.draws() == 8


def test_prng_state_after_exact_host_oracle_draws(known):
    e = known["exact_host_oracle"]
    s = o.SamplingState(e["seed"])
    for _ in range(e["final_draws"]):
        s.next_24()
    assert e["final_draws"] == e["sampled_token_count"] == 41
    assert s.state() == e["final_state"]


def test_prng_zero_seed_replacement(known):
    assert o.SamplingState(0).state() == known["unit"]["prng"]["zero_seed_state"]
    assert o.SamplingState(0).draws() == 0


def test_prng_outputs_are_24_bit():
    s = o.SamplingState(0xFEEDFACEDEADBEEF)
    vals = [s.next_24() for _ in range(4096)]
    assert max(vals) < (1 << 24)
    # 4096 uniform 24-bit draws: every top nibble bucket is hit.
    assert len({v >> 20 for v in vals}) == 16


def test_policy_constants(known):
    p = known["unit"]["policy"]
    assert (p["temperature_milli"], p["top_k"], p["top_p_milli"],
            p["repetition_penalty_milli"]) == (700, o.TOP_K, 800, 1100)
    # binary32 constants of fp32_sse2.rs:1792-1795, 1855 are the nearest floats
    assert fbits(0.7) == 0x3F333333
    assert fbits(0.8) == 0x3F4CCCCD
    assert fbits(1.1) == 0x3F8CCCCD


# ---- expf (fp32_sse2.rs:404-469; tests.rs:3293-3309) ----

def test_expf_edge_pairs():
    pairs = np.fromfile(GOLDEN / "expf_edge.u32le", dtype="<u4").reshape(-1, 2)
    assert pairs.shape == (16, 2)
    for index, (inp, expected) in enumerate(pairs):
        actual = o.expf_bits(int(inp))
        if expected & 0x7FFFFFFF == 0 or expected & 0x7F800000 == 0x7F800000:
            assert actual == expected, index
        else:
            assert abs(int(actual) - int(expected)) <= 1, (index, hex(actual), hex(expected))


# ---- repetition penalty (fp32_sse2.rs:1848-1876; tests.rs:468-492) ----

def test_penalty_once_per_seen_token_and_clears_scratch(known):
    p = known["unit"]["penalty"]
    logits = filled(p["fill"], p["set"])
    seen = np.zeros(o.SEEN_BYTES, np.uint8)
    s = o.SamplingState(p["seed"])
    st, _, _ = o.sample_token_with_repetition(logits, p["history"], seen, s)
    assert st == 0
    assert logits[7] == fbits(np.float32(11.0) / np.float32(1.1))
    assert logits[9] == fbits(np.float32(-2.0) * np.float32(1.1))
    assert logits[12] == fbits("-0.0")
    assert not seen.any()
    assert s.draws() == 1
    # every other word is bit-identical
    untouched = np.ones(V, bool)
    untouched[[7, 9, 12]] = False
    assert (logits[untouched] == 0).all()

    before = logits.copy()
    before_state = s.copy()
    st, _, err = o.sample_token_with_repetition(logits, p["bad_token_history"], seen, s)
    assert st == 3
    assert err.tuple() == [3, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, V, V, (2 << 32) | 0]
    assert (logits == before).all()
    assert not seen.any()
    assert s == before_state


def test_short_seen_is_capacity_error_and_transactional():
    logits = filled(0.0)
    seen = np.zeros(o.SEEN_BYTES - 1, np.uint8)
    s = o.SamplingState(5)
    st, _, err = o.sample_token_with_repetition(logits, [1, 2], seen, s)
    # inference.rs:926-938
    assert err.tuple() == [4, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, o.SEEN_BYTES, o.SEEN_BYTES - 1,
                           (4 << 32) | 2]
    assert s.draws() == 0 and (logits == fbits(0.0)).all()


# ---- draw (fp32_sse2.rs:1786-1846; tests.rs:424-466, 494-505) ----

def test_dominant_eos_row_collapses_top_p(known):
    d = known["unit"]["dominant"]
    logits = filled(d["fill"], [(d["eos"], d["eos_value"]), (d["zero_at"], 0.0)])
    for seed in d["seeds"]:
        s = o.SamplingState(seed)
        st, tok, _ = o.sample_token(logits, s)
        assert (st, tok, s.draws()) == (0, d["eos"], 1)


def test_bounded_row_is_seeded_and_bounded(known):
    b = known["unit"]["bounded_row"]
    logits = filled(b["fill"])
    for token in range(b["count"]):
        logits[token] = fbits(np.float32(b["start"]) - np.float32(token) * np.float32(b["step"]))
    first = o.SamplingState(b["seed"])
    second = first.copy()
    for _ in range(b["draws"]):
        st1, t1, _ = o.sample_token(logits, first)
        st2, t2, _ = o.sample_token(logits, second)
        assert st1 == st2 == 0 and t1 == t2 and t1 < b["selected_below"]
    assert first == second and first.draws() == 8
    assert first.state() == known["unit"]["prng"]["state_after"]

    before = first.copy()
    st, _, err = o.sample_token(logits[:-1], first)
    assert st == 4 and first == before
    logits[17] = fbits(float("nan"))
    st, _, err = o.sample_token(logits, first)
    assert st == 7 and first == before


def test_real_hello_row_known_answer(known, qwen_cases):
    """exact-host-oracle.txt:14: sampled_tokens[0] = 9707 from the hello prompt
    logits with the prompt as history and seed 0x0123456789abcdef
    (validate_inference.rs:767-794)."""
    e = known["exact_host_oracle"]
    logits, prompt = qwen_cases[e["first_token_case"]]
    logits = logits.copy()
    seen = np.zeros(o.SEEN_BYTES, np.uint8)
    s = o.SamplingState(e["seed"])
    st, tok, _, det = o.sample_token_with_repetition(logits, prompt, seen, s, want_detail=True)
    assert (st, tok, s.draws()) == (0, e["first_sampled_token"], 1)
    # 9707 is in the prompt, so it was penalised, yet it still holds most mass.
    assert 9707 in set(prompt.tolist())
    assert det["ids"][0] == 9707


@pytest.mark.parametrize("case", ["hello", "arithmetic", "color"])
def test_real_rows_top8_and_greedy_match_llama_cpp(known, qwen_cases, case):
    """steps.json step 0 holds llama.cpp's top-8 (id, bits) and greedy id of the
    same logits row; top_logits_8 and greedy_token (inference.rs:814-881) must
    reproduce them exactly."""
    c = known["cases"][case]
    logits, _ = qwen_cases[case]
    st, out, _ = o.top_logits_8(logits)
    assert st == 0
    assert out.reshape(8, 2).tolist() == c["step0_top8"]
    st, g, _ = o.greedy_token(logits)
    assert (st, g) == (0, c["step0_selected_id"])
    assert logits[g] == c["step0_selected_logit_bits"]


# ---- errors (inference.rs:226-264, 737-757; tests.rs:368-418) ----

def test_greedy_ties_and_error_tuples(known):
    g = known["unit"]["greedy_tie"]
    logits = filled(g["fill"], g["set"])
    assert o.greedy_token(logits)[:2] == (0, g["expected"])
    t = known["unit"]["error_tuples"]
    assert o.greedy_token(logits[:-1])[2].tuple() == t["short"]
    assert o.greedy_token(np.zeros(V + 1, np.uint32))[2].tuple() == t["long"]
    logits[11] = fbits(float("nan"))
    assert o.greedy_token(logits)[2].tuple() == t["nan_at_11"]


def test_top8_stable_transactional_and_inf(known):
    t = known["unit"]["top8_stable"]
    logits = filled(t["fill"], t["set"])
    st, out, _ = o.top_logits_8(logits)
    assert st == 0
    assert out.reshape(8, 2)[:, 0].tolist() == t["expected_tokens"]
    assert out.reshape(8, 2)[:2, 1].tolist() == [fbits(9.0)] * 2
    sentinel = np.tile(np.array([0xFEEDFACE, 0xDEADBEEF], np.uint32), 8)
    keep = sentinel.copy()
    st, out, _ = o.top_logits_8(logits[:-1], keep)
    assert st == 4 and (keep == sentinel).all()
    logits[t["inf_at"]] = fbits(float("inf"))
    st, out, err = o.top_logits_8(logits, keep)
    assert st == 7 and err.domain == 19 and err.detail == (7 << 32) | t["inf_at"]
    assert (keep == sentinel).all()


def test_top8_orders_negatives_and_signed_zero_by_token(known):
    t = known["unit"]["top8_signed_zero"]
    logits = filled(t["fill"], t["set"])
    st, out, _ = o.top_logits_8(logits)
    pairs = out.reshape(8, 2)
    assert pairs[:, 0].tolist() == t["expected_tokens"]
    assert pairs[0, 1] == fbits("-0.0") and pairs[1, 1] == fbits(0.0)
