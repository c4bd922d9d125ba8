"""The oracle's record of the sampled hello turn with stand-in continuations
agrees with the reference's exact host oracle record on everything the
stand-ins leave unchanged: the seed, the policy, the first logits checkpoint
(the hello row's hash), the first sampled token (9707), and the sampler state
and draw count after the turn's 41 draws."""
from promptboot_amd import wire
from tests import evidence_case as ev

REF = wire.ExactOracle.parse((ev.GOLDEN / "exact_host_oracle.txt").read_text())


def test_oracle_turn_record_matches_the_reference_where_it_must():
    rec = ev.oracle_record()
    assert rec.seed == REF.seed and rec.sampling_policy == REF.sampling_policy
    assert rec.checkpoints[0] == ("conversation_first_hello",
                                  dict(REF.checkpoints)["conversation_first_hello"])
    assert len(rec.checkpoints) == ev.EOS_STEP + 1
    assert rec.sampled_tokens[0] == REF.sampled_tokens[0] == 9707
    assert len(rec.sampled_tokens) == REF.sampler_draws == 41
    assert rec.sampled_tokens[-1] == ev.o.IM_END
    assert (rec.sampler_state, rec.sampler_draws) == (REF.sampler_state, REF.sampler_draws)
    # the record is in the reference's canonical text form
    assert wire.ExactOracle.parse(rec.encode()).encode() == rec.encode()
