import json
import pathlib
import sys

import numpy as np
import pytest

# Some GPU tests build their inputs with torch.  torch bundles its own HIP
# runtime, so it is imported before libpbsample.so opens one: the library and
# promptboot_amd.hip then share torch's copy (one runtime per process).
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = pathlib.Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def known():
    return json.loads((GOLDEN / "known_answers.json").read_text())


def load_case(name: str):
    logits = np.fromfile(GOLDEN / f"qwen_{name}_logits.f32le", dtype="<u4").copy()
    prompt = np.fromfile(GOLDEN / f"qwen_{name}_prompt.u32le", dtype="<u4").copy()
    return logits, prompt


@pytest.fixture(scope="session")
def qwen_cases():
    return {n: load_case(n) for n in ("hello", "arithmetic", "color")}


def to_dev(a, device="cuda:0"):
    """numpy words (uint32/float32/int) -> torch int32 CUDA tensor (plumbing)."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype in (np.float32, np.uint32):
        a = a.view(np.int32)
    return torch.from_numpy(a.astype(np.int32, copy=False)).to(device)


def assert_rows_equal(tok, det, err, rtok, rdet, rerr):
    """GPU batch results vs oracle batch results: every field bit-exact."""
    assert (err["status"] == rerr["status"]).all(), (err["status"], rerr["status"])
    for field in ("status", "domain", "layer", "position", "tensor_id", "needed",
                  "available", "detail"):
        bad = np.flatnonzero(err[field] != rerr[field])
        assert bad.size == 0, (field, bad[:5], err[bad[:5]], rerr[bad[:5]])
    bad = np.flatnonzero(tok != rtok)
    assert bad.size == 0, ("token", bad[:8], tok[bad[:8]], rtok[bad[:8]])
    if det is not None:
        for field in ("ids", "value_bits", "weight_bits", "kept", "rank", "flags", "token"):
            a, b = det[field], rdet[field]
            rows = np.flatnonzero((a != b).reshape(len(a), -1).any(axis=1))
            assert rows.size == 0, (field, rows[:5], a[rows[:5]], b[rows[:5]])
        pa = det["probs"].view(np.uint32)
        pb = rdet["probs"].view(np.uint32)
        rows = np.flatnonzero((pa != pb).any(axis=1))
        assert rows.size == 0, ("probs", rows[:5], det["probs"][rows[:5]], rdet["probs"][rows[:5]])
