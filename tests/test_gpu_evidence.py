"""The evidence record produced on the device (promptboot_amd.evidence:
DecodeBatch over the hello turn) is byte for byte the record the oracle's
restatement of the same turn produces, and shares the reference record's
first token, final sampler state and draw count (41 draws)."""
import pytest

from promptboot_amd import evidence, wire
from tests import evidence_case as ev

pytestmark = pytest.mark.gpu


def test_device_turn_record_is_the_oracles_byte_for_byte():
    logits, prompt = ev.hello()
    got = evidence.sampled_turn_record(prompt, logits, ev.next_logits,
                                       step_checkpoint=ev.STEP_CHECKPOINT)
    want = ev.oracle_record()
    assert got.encode() == want.encode()
    ref = wire.ExactOracle.parse((ev.GOLDEN / "exact_host_oracle.txt").read_text())
    assert got.sampled_tokens[0] == ref.sampled_tokens[0] == 9707
    assert (got.sampler_state, got.sampler_draws) == (ref.sampler_state, ref.sampler_draws)
