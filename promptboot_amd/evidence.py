"""The exact host oracle record of a sampled turn, produced on the device.

The reference's harness writes an evidence record of its first sampled
conversation turn (crates/promptboot-core/examples/validate_inference.rs:
767-824): the first turn's logits are checkpointed by their SHA-256, every
sampled token is listed, and the boot's SamplingState (state and draw count)
is recorded once the turn ends on an end-of-sequence piece
(ExactOracle::encode, :611-649).  `sampled_turn_record` runs the same turn
through the device decode loop (DecodeBatch, one row) and returns that record
in the reference's format (promptboot_amd.wire.ExactOracle).

There is no model here: the caller supplies the first logits row (for the
reference, the prefill's output) and a function giving each next row from the
step and the previous token (the reference's engine.decode_selected).
"""
from __future__ import annotations

from typing import Callable, Sequence

import numpy as np

from . import hip
from . import sampler as s
from .wire import ExactOracle

REFERENCE_SEED = 0x0123_4567_89AB_CDEF  # validate_inference.rs:774
REFERENCE_MAX_TOKENS = 128              # validate_inference.rs:775


def sampled_turn_record(prompt: Sequence[int], first_logits, next_logits: Callable[[int, int], np.ndarray],
                        seed: int = REFERENCE_SEED, max_tokens: int = REFERENCE_MAX_TOKENS,
                        first_checkpoint: str = "conversation_first_hello",
                        step_checkpoint: str | None = None,
                        sampler: "s.BatchSampler | None" = None) -> ExactOracle:
    """Samples one turn on the device and returns its evidence record.

    Step 0 samples from `first_logits` (checkpointed as `first_checkpoint`);
    step k > 0 from next_logits(k, previous token) (checkpointed as
    f"{step_checkpoint}{k}" when a prefix is given).  Every step samples with
    the whole working context as history (prompt + the turn so far, an
    end-of-sequence piece stored as <|im_end|>), one draw per sampled token.
    The turn ends on an end-of-sequence piece; reaching `max_tokens` first
    raises, as the reference's harness asserts, and so does a sampler error.
    """
    record = ExactOracle(seed=seed)
    dec = s.DecodeBatch([np.asarray(prompt, np.uint32)], [seed], [max_tokens], sampler=sampler)
    try:
        logits = np.asarray(first_logits)
        if logits.dtype == np.float32:
            logits = logits.view(np.uint32)
        record.checkpoint(first_checkpoint, logits)
        row = hip.DeviceArray((1, s.VOCAB), np.uint32)
        step = 0
        while True:
            row.upload(logits.reshape(1, s.VOCAB))
            token = int(dec.step(row)[0])
            if token == s.NO_TOKEN:
                errs = dec.errors()
                if int(errs[0]["status"]) != s.OK:
                    raise s.InferenceError(errs[0])
                raise RuntimeError(f"the turn reached its limit of {max_tokens} tokens before "
                                   "an end-of-sequence piece")
            record.sampled_tokens.append(token)
            if token in (s.IM_END, s.END_OF_TEXT):
                break
            step += 1
            logits = np.asarray(next_logits(step, token))
            if logits.dtype == np.float32:
                logits = logits.view(np.uint32)
            if step_checkpoint is not None:
                record.checkpoint(f"{step_checkpoint}{step}", logits)
        state = dec.sampling_states()[0]
        record.sampler_state = state.state()
        record.sampler_draws = state.draws()
        return record
    finally:
        dec.close()
