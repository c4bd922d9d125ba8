"""The single-row drop-ins and the batched entry point called from a plain C
process (tests/c_host/drop_in.c; no Python or PyTorch in it), checked against
the oracle: the transactional error of a short row, the reference's known
answer on the real Qwen "hello" row (token 9707 after one draw) with the
penalised row bit for bit, greedy and top-8, and a batch of the three real
rows with their prompts as histories."""
import pathlib
import subprocess

import numpy as np
import pytest

from oracle import oracle as o
from tests.c_host_build import build_drop_in
from tests.conftest import GOLDEN, load_case

pytestmark = pytest.mark.gpu


def run_host(tmp_path: pathlib.Path) -> dict:
    exe = build_drop_in(tmp_path)
    print(f"running {exe}", flush=True)
    out = subprocess.run([str(exe), str(GOLDEN), str(tmp_path)], check=True, capture_output=True,
                         text=True, timeout=120)
    lines = {}
    for line in out.stdout.splitlines():
        key, *rest = line.split()
        lines[key] = rest
    assert "done" in lines, out.stdout + out.stderr
    return lines


def test_c_host_matches_the_oracle(tmp_path):
    got = run_host(tmp_path)
    logits, prompt = load_case("hello")

    # 1. one word short: the reference's error tuple, nothing mutated, no draw
    ref_state = o.SamplingState(0x0123456789ABCDEF)
    short = logits[:-1].copy()
    st, _, err = o.sample_token_with_repetition(short, prompt, np.zeros(o.SEEN_BYTES, np.uint8),
                                                ref_state)
    assert [int(x) for x in got["short_error"]] == err.tuple()
    assert got["short_status"] == [str(st), "unchanged", "1", "seen_zero", "1", "draws", "0"]

    # 2. the whole row: token, state and the penalised row
    row = logits.copy()
    st, token, _ = o.sample_token_with_repetition(row, prompt, np.zeros(o.SEEN_BYTES, np.uint8),
                                                  ref_state)
    assert st == 0 and token == 9707
    assert got["sample_status"] == ["0", "token", str(token), "state", str(ref_state.state()),
                                    "draws", "1", "seen_zero", "1"]
    penalised = np.fromfile(tmp_path / "hello_penalised.u32le", dtype="<u4")
    assert (penalised == row).all()

    # 3. greedy and top-8 of the original row
    _, greedy, _ = o.greedy_token(logits)
    assert got["greedy_status"] == ["0", "token", str(greedy)]
    _, top8, _ = o.top_logits_8(logits)
    assert [int(x) for x in got["top8_status"]] == [0] + top8.tolist()

    # 4. the batched entry point on the three real rows
    names = ("hello", "arithmetic", "color")
    rows = [load_case(n) for n in names]
    lg = np.stack([r[0] for r in rows])
    hist = np.zeros((3, 64), np.uint32)
    hl = np.zeros(3, np.uint32)
    for i, (_, p) in enumerate(rows):
        hist[i, :len(p)] = p
        hl[i] = len(p)
    r24 = np.array([o.SamplingState(42 + i).next_24() for i in range(3)], np.uint32)
    tok, _, _, _ = o.sample_batch(lg, hist, hl, r24)
    b = got["batch_status"]
    assert b[0] == "0" and [int(x) for x in b[2:5]] == tok.tolist()
    assert [int(x) for x in b[6:9]] == r24.tolist()
