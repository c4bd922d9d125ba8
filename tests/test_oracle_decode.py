"""The decode-loop restatement (oracle.DecodeRow, src/model_repl.rs:928-1150),
pinned without a model:

* known answer: the hello turn's first step gives 9707 with one draw
  (fixtures/inference/exact-host-oracle.txt:14-16) and the context grows by it;
* the generated tokens are part of the next step's history: a constructed
  row whose winner flips only when the previous pick is penalised;
* an end-of-sequence piece (151643 or 151645) is stored as 151645 and ends
  the turn (model_repl.rs:1099-1103, 1119-1150; validate_inference.rs:806-813);
* the generation limit ends the turn (model_repl.rs:928);
* a sampler error ends the turn with no append and no draw;
* the sampling_draws evidence of the REPL harness
  (tests/integration/repl/run_model_repl_qemu.py:1195-1202): one state per
  boot, draws grow by exactly the sampled tokens of each turn and not at all
  on a turn that fails its first sample.
"""
import pathlib

import numpy as np

from oracle import oracle as o

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
V = o.VOCAB
SEED = 0x0123_4567_89AB_CDEF


def row_with(fill: float, pairs) -> np.ndarray:
    r = np.full(V, fill, np.float32)
    for i, v in pairs:
        r[i] = v
    return r.view(np.uint32)


def test_hello_first_step_known_answer():
    logits = np.fromfile(GOLDEN / "qwen_hello_logits.f32le", dtype="<u4")
    prompt = np.fromfile(GOLDEN / "qwen_hello_prompt.u32le", dtype="<u4")
    d = o.DecodeRow(prompt, SEED, limit=128)
    before = logits.copy()
    assert d.step(logits) == 9707
    assert (logits == before).all()  # the caller's row is not mutated by the loop
    assert d.state.draws() == 1 and d.generated == 1 and d.active()
    assert d.working == [int(t) for t in prompt] + [9707]


def test_generated_tokens_are_penalised_on_the_next_step():
    # 30 vs 28.6: 30 wins (kept = 1).  Once 30's token is in the context it is
    # penalised to 27.27 and 28.6 wins (kept = 1 again).  A loop that forgot the
    # generated tokens would pick id 100 twice.
    logits = row_with(-100.0, [(100, 30.0), (200, 28.6)])
    d = o.DecodeRow([1, 2, 3], 7, limit=8)
    assert d.step(logits) == 100
    assert d.step(logits) == 200
    assert d.working == [1, 2, 3, 100, 200] and d.state.draws() == 2


def test_end_of_text_is_stored_as_im_end_and_ends_the_turn():
    for eos in (o.END_OF_TEXT, o.IM_END):
        d = o.DecodeRow([5, 6], 1, limit=8)
        assert d.step(row_with(-100.0, [(eos, 10.0)])) == eos
        assert d.working == [5, 6, o.IM_END] and d.reason == "EOS"
        assert d.step(row_with(-100.0, [(9, 10.0)])) is None
        assert d.state.draws() == 1 and d.tokens == [eos]


def test_generation_limit_ends_the_turn():
    d = o.DecodeRow([5], 2, limit=3)
    for k in range(3):
        assert d.step(row_with(-100.0, [(10 + k, 10.0)])) == 10 + k
    assert d.reason == "LIMIT" and d.working == [5, 10, 11, 12]
    assert d.step(row_with(-100.0, [(20, 10.0)])) is None and d.state.draws() == 3
    assert o.DecodeRow([5], 2, limit=0).reason == "LIMIT"


def test_sampler_error_ends_the_turn_without_a_draw():
    d = o.DecodeRow([5, 6], 3, limit=8)
    assert d.step(row_with(-100.0, [(9, 10.0)])) == 9
    bad = row_with(-100.0, [(9, 10.0)])
    bad[11] = 0x7FC00000
    assert d.step(bad) is None
    assert d.reason == "ERROR" and d.working == [5, 6, 9] and d.state.draws() == 1
    assert d.error == [7, 19, 0xFFFFFFFF, 0, 0xFFFFFFFF, 0, 0x7FC00000, (7 << 32) | 11]
    d = o.DecodeRow([5, o.VOCAB], 3, limit=8)  # bad history id
    assert d.step(row_with(-100.0, [(9, 10.0)])) is None
    assert d.error[0] == 3 and d.error[6] == o.VOCAB and d.state.draws() == 0


def test_sampling_draws_evidence_across_turns():
    state = o.SamplingState(SEED)
    # turn 1: three tokens up to its limit
    t1 = o.DecodeRow([1, 2], 0, limit=3, state=state)
    for k in range(3):
        t1.step(row_with(-100.0, [(40 + k, 10.0)]))
    assert state.draws() == len(t1.tokens) == 3
    # turn 2: fails at its first sample: no draw
    t2 = o.DecodeRow(t1.working, 0, limit=3, state=state)
    bad = row_with(-100.0, [(9, 10.0)])
    bad[0] = 0x7F800000
    t2.step(bad)
    assert t2.reason == "ERROR" and state.draws() == 3
    # turn 3: ends on end-of-sequence at its second token
    t3 = o.DecodeRow(t1.working, 0, limit=16, state=state)
    t3.step(row_with(-100.0, [(50, 10.0)]))
    t3.step(row_with(-100.0, [(o.IM_END, 10.0)]))
    assert t3.reason == "EOS" and state.draws() == 5
    ref = o.SamplingState(SEED)
    for _ in range(5):
        ref.next_24()
    assert state == ref
