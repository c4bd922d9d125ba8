"""The sampled hello turn of the exact host oracle, with stand-in continuations.

The reference samples its first turn from the real hello logits, then from
the model's next logits after each token (validate_inference.rs:767-824).
With no model here, step k > 0 uses a seeded stand-in row that depends on the
previous token: N(0, 2.5^2) with five ids derived from that token boosted by
U(8, 15), the end-of-sequence ids held at -30 until step 40 and <|im_end|> at
+60 at step 40.  The turn therefore ends after exactly 41 draws, as the
reference's recorded turn does, so its final SamplingState must be the
reference record's (the state depends only on the seed and the draw count).
"""
import pathlib

import numpy as np

from oracle import oracle as o
from promptboot_amd import wire

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
V = o.VOCAB
EOS_STEP = 40
STEP_CHECKPOINT = "decode_step_"


def hello():
    logits = wire.read_logits_rows(GOLDEN / "qwen_hello_logits.f32le")[0].copy()
    prompt = wire.read_words(GOLDEN / "qwen_hello_prompt.u32le")
    return logits, prompt


def next_logits(step: int, prev: int) -> np.ndarray:
    rng = np.random.default_rng([7, step, prev])
    x = rng.normal(0.0, 2.5, V).astype(np.float32)
    ids = (prev * 7919 + np.arange(5) * 104_729 + step) % V
    x[ids] += rng.uniform(8.0, 15.0, 5).astype(np.float32)
    x[o.IM_END] = x[o.END_OF_TEXT] = np.float32(-30.0)
    if step >= EOS_STEP:
        x[o.IM_END] = np.float32(60.0)
    return x.view(np.uint32)


def oracle_record(seed: int = 0x0123_4567_89AB_CDEF, max_tokens: int = 128) -> wire.ExactOracle:
    """The record the oracle's restatement of the turn produces."""
    logits, prompt = hello()
    rec = wire.ExactOracle(seed=seed)
    rec.checkpoint("conversation_first_hello", logits)
    row = o.DecodeRow(prompt, seed, max_tokens)
    step = 0
    while True:
        tok = row.step(logits)
        assert tok is not None, (row.reason, row.error)
        rec.sampled_tokens.append(tok)
        if tok in (o.IM_END, o.END_OF_TEXT):
            break
        step += 1
        logits = next_logits(step, tok)
        rec.checkpoint(f"{STEP_CHECKPOINT}{step}", logits)
    rec.sampler_state = row.state.state()
    rec.sampler_draws = row.state.draws()
    return rec
