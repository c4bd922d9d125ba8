"""Decode-loop steps on the GPU (pb_decode_step, pb_lmhead_decode_step) in
lockstep with the oracle's restatement of the REPL loop (oracle.DecodeRow,
src/model_repl.rs:928-1150).

There is no model here, so a seeded stand-in produces each step's logits
from the row's previous token (the next logits depend on what was sampled, so
any divergence shows up as a wrong token at the next step).  Every step
compares tokens; at the end the working contexts, the per-row
SamplingStates (draw counts included), the stop reasons and the error
records must be identical.  Rows cover end-of-sequence on both ids, the
generation limit, a non-finite logit mid-turn, a bad id in the prompt, and a
row that starts with no room left.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from promptboot_amd import workloads

pytestmark = pytest.mark.gpu

V = s.VOCAB
REASON = {s.ROW_EOS: "EOS", s.ROW_LIMIT: "LIMIT", s.ROW_ERROR: "ERROR"}


def stand_in_logits(row: int, step: int, prev: int, eos_after: int | None,
                    eos_id: int = s.IM_END) -> np.ndarray:
    """Next-token logits of a seeded stand-in model: N(0, 2.5^2), five ids
    derived from the previous token boosted by U(8, 15), and an
    end-of-sequence logit pushed up from step `eos_after` on."""
    rng = np.random.default_rng([row, step, prev])
    x = rng.normal(0.0, 2.5, V).astype(np.float32)
    ids = (prev * 7919 + np.arange(5) * 104_729 + step) % V
    x[ids] += rng.uniform(8.0, 15.0, 5).astype(np.float32)
    if eos_after is not None and step >= eos_after:
        x[eos_id] = np.float32(30.0)
    return x.view(np.uint32)


def run_lockstep(prompts, seeds, limits, eos_after, eos_ids, nan_at, steps, segments=0):
    import torch

    oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
    smp = s.BatchSampler(0, segments=segments)
    dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
    try:
        for step in range(steps):
            rows = []
            for r, d in enumerate(oracle_rows):
                prev = d.working[-1]
                x = stand_in_logits(r, step, prev, eos_after[r], eos_ids[r])
                if nan_at.get(r) == step:
                    x = x.copy()
                    x[4321] = 0x7FC00000
                rows.append(x)
            logits = np.stack(rows)
            want = [d.step(logits[r]) for r, d in enumerate(oracle_rows)]
            got = dec.step(torch.from_numpy(logits.view(np.int32)).to("cuda:0"))
            for r in range(len(prompts)):
                w = s.NO_TOKEN if want[r] is None else want[r]
                assert got[r] == w, (step, r, got[r], w)
            if not dec.active():
                break
        ctx = dec.contexts()
        states = dec.sampling_states()
        errs = dec.errors()
        for r, d in enumerate(oracle_rows):
            assert ctx[r].tolist() == d.working, r
            assert (states[r].state(), states[r].draws()) == (d.state.state(), d.state.draws())
            if d.reason is None:
                assert dec.row_state_host[r] == s.ROW_ACTIVE
            else:
                assert REASON[int(dec.row_state_host[r])] == d.reason, r
            if d.reason == "ERROR":
                rec = errs[r]
                got_t = [int(rec[k]) for k in ("status", "domain", "layer", "position",
                                               "tensor_id", "needed", "available", "detail")]
                assert got_t == d.error
        return oracle_rows
    finally:
        dec.close()


@pytest.mark.parametrize("segments", [0, 1, 3])
def test_decode_steps_match_the_oracle_loop(segments):
    rng = np.random.default_rng(11)
    lens = [30, 5, 300, 17, 64, 1, 9, 120]
    prompts = [workloads.zipf_ids(rng, n) for n in lens]
    prompts[6] = np.concatenate([prompts[6], [V + 3]])       # bad id in the prompt
    seeds = [0x0123_4567_89AB_CDEF, 42, 43, 0, 2**64 - 1, 7, 8, 9]
    limits = [24, 6, 24, 24, 24, 0, 24, 24]                  # row 5: no room at all
    eos_after = [9, None, 14, None, 3, None, None, 20]
    eos_ids = [s.IM_END, s.IM_END, s.END_OF_TEXT, s.IM_END, s.END_OF_TEXT, s.IM_END,
               s.IM_END, s.IM_END]
    nan_at = {3: 7}
    rows = run_lockstep(prompts, seeds, limits, eos_after, eos_ids, nan_at, 26, segments)
    reasons = [d.reason for d in rows]
    assert reasons[:7] == ["EOS", "LIMIT", "EOS", "ERROR", "EOS", "LIMIT", "ERROR"]
    assert rows[0].tokens[-1] == s.IM_END and rows[2].tokens[-1] == s.END_OF_TEXT
    assert rows[2].working[-1] == s.IM_END
    assert rows[3].state.draws() == 7 and rows[6].state.draws() == 0


def test_hello_turn_first_step_on_device():
    """The exact host oracle's first step (fixtures/inference/exact-host-oracle.txt:14-16)
    through the batched decode step: 9707, one draw, context grown by it."""
    import pathlib

    import torch

    golden = pathlib.Path(__file__).resolve().parent / "golden"
    logits = np.fromfile(golden / "qwen_hello_logits.f32le", dtype="<u4")
    prompt = np.fromfile(golden / "qwen_hello_prompt.u32le", dtype="<u4")
    dec = s.DecodeBatch([prompt], [0x0123_4567_89AB_CDEF], [128])
    try:
        tok = dec.step(torch.from_numpy(logits.view(np.int32)[None, :].copy()).to("cuda:0"))
        assert tok.tolist() == [9707]
        assert dec.contexts()[0].tolist() == prompt.tolist() + [9707]
        assert dec.sampling_states()[0].draws() == 1
        assert dec.row_state_host.tolist() == [s.ROW_ACTIVE]
    finally:
        dec.close()


def test_lmhead_decode_steps_match_the_oracle_loop():
    import torch

    w = workloads.make_lmhead(rows=4)
    q4 = w["q4"]
    smp = s.BatchSampler(0)
    packed = smp.pack_lmhead(torch.from_numpy(q4).to("cuda:0"))
    rng = np.random.default_rng(5)
    prompts = [workloads.zipf_ids(rng, n) for n in (12, 40, 3)]
    seeds, limits = [1, 2, 3], [6, 6, 4]
    oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
    dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
    try:
        for step in range(7):
            hidden = np.stack([
                np.random.default_rng([r, step, d.working[-1]]).normal(0, 1, workloads.HIDDEN)
                for r, d in enumerate(oracle_rows)]).astype(np.float32)
            logits = o.lmhead_logits(hidden, q4, V, workloads.HIDDEN, threads=8)
            want = [d.step(logits[r]) for r, d in enumerate(oracle_rows)]
            got = dec.lmhead_step(packed, torch.from_numpy(hidden.view(np.int32)).to("cuda:0"))
            assert got.tolist() == [s.NO_TOKEN if t is None else t for t in want], step
            if not dec.active():
                break
        for r, d in enumerate(oracle_rows):
            assert dec.contexts()[r].tolist() == d.working
            assert dec.sampling_states()[r].draws() == d.state.draws()
        assert [d.reason for d in oracle_rows] == ["LIMIT", "LIMIT", "LIMIT"]
    finally:
        dec.close()
        smp.close()


def test_lmhead_decode_steps_in_one_pass():
    """Above 64 rows the head runs in one pass (no logits kept; the selection
    recomputes the tiles it reads): 70 sequences in lockstep with the oracle's
    loop, rows with limits of 2 to 5 tokens, the last rows starting with a bad
    prompt id (an error on the first step, no draw)."""
    import torch

    w = workloads.make_lmhead(rows=4)
    q4 = w["q4"]
    smp = s.BatchSampler(0)
    packed = smp.pack_lmhead(torch.from_numpy(q4).to("cuda:0"))
    rng = np.random.default_rng(9)
    n = 70
    prompts = [workloads.zipf_ids(rng, int(k)) for k in rng.integers(1, 60, n)]
    prompts[-1] = np.append(prompts[-1], np.uint32(V + 3))
    seeds, limits = list(range(100, 100 + n)), [int(x) for x in rng.integers(2, 6, n)]
    oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
    dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
    try:
        for step in range(6):
            hidden = np.stack([
                np.random.default_rng([r, step, d.working[-1]]).normal(0, 1, workloads.HIDDEN)
                for r, d in enumerate(oracle_rows)]).astype(np.float32)
            logits = o.lmhead_logits(hidden, q4, V, workloads.HIDDEN, threads=16)
            want = [d.step(logits[r]) for r, d in enumerate(oracle_rows)]
            got = dec.lmhead_step(packed, torch.from_numpy(hidden.view(np.int32)).to("cuda:0"))
            assert got.tolist() == [s.NO_TOKEN if t is None else t for t in want], step
            if not dec.active():
                break
        assert not dec.active()
        states = dec.sampling_states()
        for r, d in enumerate(oracle_rows):
            assert dec.contexts()[r].tolist() == d.working
            assert (states[r].state(), states[r].draws()) == (d.state.state(), d.state.draws())
        assert oracle_rows[-1].reason == "ERROR" and states[-1].draws() == 0
    finally:
        dec.close()
        smp.close()


def test_active_row_at_its_cap_is_not_sampled():
    """A row still marked active whose context is already at its cap is not
    sampled (the REPL stops before sampling when there is no room): it ends
    with ROW_LIMIT, no token, no draw, an unchanged context; its neighbour is
    sampled as usual.  Both slice plans."""
    from promptboot_amd import hip

    rng = np.random.default_rng(5)
    prompts = [workloads.zipf_ids(rng, 12), workloads.zipf_ids(rng, 40)]
    seeds, limits = [3, 4], [0, 8]
    logits = np.stack([stand_in_logits(r, 0, int(p[-1]), None) for r, p in enumerate(prompts)])
    for segments in (0, 1):
        oracle_rows = [o.DecodeRow(p, sd, lim) for p, sd, lim in zip(prompts, seeds, limits)]
        want = [d.step(logits[r]) for r, d in enumerate(oracle_rows)]
        assert want[0] is None and oracle_rows[0].reason == "LIMIT"
        smp = s.BatchSampler(0, segments=segments)
        dec = s.DecodeBatch(prompts, seeds, limits, sampler=smp)
        try:
            assert dec.row_state_host[0] == s.ROW_LIMIT
            # mark the full row active on both sides, as a caller might
            dec.row_state_host[0] = s.ROW_ACTIVE
            dec.row_state.upload(dec.row_state_host)
            got = dec.step(hip.DeviceArray.from_numpy(logits))
            assert got[0] == s.NO_TOKEN and got[1] == want[1]
            assert dec.row_state_host[0] == s.ROW_LIMIT
            states = dec.sampling_states()
            for r, d in enumerate(oracle_rows):
                assert (states[r].state(), states[r].draws()) == (d.state.state(), d.state.draws())
                assert dec.contexts()[r].tolist() == d.working
        finally:
            dec.close()
            smp.close()


@pytest.mark.parametrize("seed,n", [(0, 3), (1, 40), (2, 193), (3, 230)])
def test_random_decode_loops_match_the_oracle(seed, n):
    """Seeded random decode batches in lockstep with the oracle's loop: batch
    sizes either side of the tile selection's 192 rows, prompt lengths of 1 to
    2,000 ids (a bad id in some), limits of 0 to 12 tokens, end of sequence
    on either id after a random step, a non-finite logit at a random step,
    and the automatic or a forced slice plan."""
    rng = np.random.default_rng([seed, 31])
    prompts = [workloads.zipf_ids(rng, int(k)) for k in rng.integers(1, 2001, n)]
    for r in rng.choice(n, max(1, n // 20), replace=False):
        prompts[r] = np.append(prompts[r], np.uint32(V + int(rng.integers(0, 99))))
    seeds = [int(x) for x in rng.integers(0, 2**63, n)]
    limits = [int(x) for x in rng.integers(0, 13, n)]
    eos_after = [int(x) if x < 12 else None for x in rng.integers(0, 24, n)]
    eos_ids = [s.IM_END if x else s.END_OF_TEXT for x in rng.integers(0, 2, n)]
    nan_at = {int(r): int(rng.integers(0, 8)) for r in rng.choice(n, max(1, n // 25), replace=False)}
    segments = int(rng.choice([0, 0, 1, 3]))
    run_lockstep(prompts, seeds, limits, eos_after, eos_ids, nan_at, 14, segments)
