import json
import pathlib
import sys

import numpy as np
import pytest

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
