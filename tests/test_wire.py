"""Wire formats: word files, logits checkpoint hashes and the exact host oracle
record (crates/promptboot-core/examples/validate_inference.rs:74-81, 597-649).

Pinned by the reference's own record, fixtures/inference/exact-host-oracle.txt
(copied as tests/golden/exact_host_oracle.txt): the parser must read it and
the encoder must reproduce it byte for byte; its checkpoint hashes must equal
the hashes of the Qwen logits rows; its seed, 41 draws and final state must
agree with the PRNG; and its first sampled token must be the sampler's
answer on the hello row.
"""
import pathlib

import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import wire

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
TEXT = (GOLDEN / "exact_host_oracle.txt").read_text()


def test_reference_record_round_trips_byte_for_byte():
    rec = wire.ExactOracle.parse(TEXT)
    assert rec.encode() == TEXT
    assert rec.seed == 0x0123_4567_89AB_CDEF
    assert rec.logit_words == s.VOCAB
    assert rec.sampling_policy.encode() == s.SAMPLING_POLICY
    assert len(rec.checkpoints) == 9
    assert len(rec.sampled_tokens) == rec.sampler_draws == 41
    assert rec.sampled_tokens[0] == 9707 and rec.sampled_tokens[-1] == s.IM_END


def test_record_state_is_the_prng_after_its_draws():
    rec = wire.ExactOracle.parse(TEXT)
    st = o.SamplingState(rec.seed)
    for _ in range(rec.sampler_draws):
        st.next_24()
    assert (st.state(), st.draws()) == (rec.sampler_state, rec.sampler_draws)


def test_checkpoint_hashes_match_the_logits_rows():
    rec = dict(wire.ExactOracle.parse(TEXT).checkpoints)
    for case in ("hello", "arithmetic", "color"):
        words = wire.read_words(GOLDEN / f"qwen_{case}_logits.f32le")
        assert words.size == s.VOCAB
        assert wire.words_sha256(words) == rec[f"fixture_{case}"]
    # the first conversation turn samples from the hello row
    assert rec["conversation_first_hello"] == rec["fixture_hello"]


def test_first_sampled_token_from_the_hashed_row():
    rec = wire.ExactOracle.parse(TEXT)
    logits = wire.read_logits_rows(GOLDEN / "qwen_hello_logits.f32le")[0].copy()
    prompt = wire.read_words(GOLDEN / "qwen_hello_prompt.u32le")
    assert prompt.size == 30
    state = o.SamplingState(rec.seed)
    seen = np.zeros(o.SEEN_BYTES, np.uint8)
    st, tok, _ = o.sample_token_with_repetition(logits, prompt, seen, state)
    assert st == 0 and tok == rec.sampled_tokens[0] and state.draws() == 1


def test_encode_of_a_new_record(tmp_path):
    rng = np.random.default_rng(3)
    row = rng.normal(0, 2.5, s.VOCAB).astype(np.float32)
    rec = wire.ExactOracle(seed=42)
    rec.checkpoint("step0", row)
    rec.sampled_tokens = [5, 6, s.IM_END]
    rec.sampler_state, rec.sampler_draws = 0x1234, 3
    text = rec.encode()
    assert text.splitlines()[2] == "seed=000000000000002a"
    assert text.splitlines()[4].startswith("checkpoint=step0 sha256=")
    assert text.endswith("sampled_tokens=5,6,151645\nsampler_state=0000000000001234\n"
                         "sampler_draws=3\n")
    assert wire.ExactOracle.parse(text) == rec
    with pytest.raises(ValueError):
        rec.checkpoint("short", row[:10])


@pytest.mark.parametrize("mutate", [
    lambda t: t.replace("schema=1", "schema=2"),
    lambda t: t.replace("seed=0123456789abcdef", "seed=0123456789ABCDEF"),
    lambda t: t.rstrip("\n"),
    lambda t: t + "extra=1\n",
    lambda t: t.replace(" sha256=097a", " sha256=097A"),
    lambda t: t.replace("sampler_draws=41", "sampler_draws=041"),
    lambda t: "\n".join(line for line in t.split("\n") if not line.startswith("sampler_state")),
])
def test_parse_rejects_non_canonical_text(mutate):
    with pytest.raises(ValueError):
        wire.ExactOracle.parse(mutate(TEXT))


def test_word_files_keep_every_bit_pattern(tmp_path):
    words = np.array([0, 0x80000000, 0x7FC00001, 0xFF800000, 0x00000001, 0x3F800000,
                      0xFFFFFFFF], np.uint32)
    p = tmp_path / "row.f32le"
    wire.write_words(p, words)
    assert p.read_bytes()[:8] == bytes([0, 0, 0, 0, 0, 0, 0, 0x80])
    assert (wire.read_words(p) == words).all()
    wire.write_words(p, words.view(np.float32))
    assert (wire.read_words(p) == words).all()
    p.write_bytes(b"\x00" * 6)
    with pytest.raises(ValueError):
        wire.read_words(p)
    wire.write_words(p, np.zeros(s.VOCAB + 1, np.uint32))
    with pytest.raises(ValueError):
        wire.read_logits_rows(p)
    with pytest.raises(TypeError):
        wire.write_words(p, np.zeros(3, np.int64))
