"""Device binary32 routines vs the oracle, bit for bit (GPU).

The sampler's softmax weights come from a step-by-step restatement of libm's
expf (fp32_sse2.rs:404-469) and its penalty from one correctly rounded
multiply or divide (fp32_sse2.rs:1860-1866).  Both must agree with the oracle
on every input, including subnormal results, the overflow/underflow
thresholds and the special values.
"""
import numpy as np
import pytest

from oracle import oracle as o
from tests.conftest import GOLDEN, to_dev

pytestmark = pytest.mark.gpu


def run_probe(fn, words: np.ndarray) -> np.ndarray:
    import torch

    from promptboot_amd import sampler as s

    inp = to_dev(words.astype(np.uint32))
    out = torch.empty_like(inp)
    getattr(s, fn)(inp, out)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32)


def test_wave_lane_exchange_and_reductions():
    """The selection's lane exchanges (DPP quad_perm / row_ror, gfx950
    permlane16/32 swaps) must read exactly lane ^ j, and the wave max, sort
    and min built on them must agree with numpy."""
    import ctypes

    import torch

    from promptboot_amd import sampler as s

    out = torch.zeros(11 * 64, dtype=torch.int32, device="cuda:0")
    st = s.lib().pb_device_wave_selftest(ctypes.c_void_p(out.data_ptr()),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    o_ = out.cpu().numpy().view(np.uint32).reshape(11, 64).astype(np.uint64)
    lane = np.arange(64, dtype=np.uint64)
    for row, j in enumerate((1, 2, 4, 8, 16, 32)):
        assert (o_[row] == ((lane ^ j) * 7 + 3)).all(), (j, o_[row][:20])
    keys = ((lane * 2654435761) % 2**32 << 32) | (lane ^ 0x55)
    got_max = o_[6] | (o_[7] << 32)
    assert (got_max == keys.max()).all()
    got_sorted = o_[8] | (o_[9] << 32)
    assert (got_sorted == np.sort(keys)[::-1]).all()
    assert (o_[10] == ((lane * 13) % 64 + 5).min()).all()


def test_device_expf_on_softmax_domain():
    # Every (v - max) / 0.7 the sampler can form is <= 0: sweep all non-positive
    # binary32 values down to the underflow threshold at a prime stride, plus
    # the positive range up to overflow and the special values.
    neg = np.arange(0x80000000, 0xC2D00000, 61, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0x00000000, 0x42B20000, 977, dtype=np.uint64).astype(np.uint32)
    edge = np.fromfile(GOLDEN / "expf_edge.u32le", dtype="<u4").reshape(-1, 2)[:, 0]
    special = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x80000001,
                        0x42AEAC4F, 0x42AEAC50, 0xC2CFF1B4, 0xC2CFF1B5, 0x42B17217,
                        0x42B17218, 0x3EB17218, 0x3EB17219, 0x3F851592, 0x3F851593,
                        0x39000000, 0x39000001, 0xB9000000, 0xB9000001], np.uint32)
    words = np.concatenate([neg, pos, edge, special])
    got = run_probe("device_expf_bits", words)
    want = o.expf_array(words)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(words[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    assert words.size > 17_000_000


def test_device_penalty_on_every_class():
    rng = np.random.default_rng(5)
    rand = rng.integers(0, 2**32, 4_000_000, dtype=np.uint64).astype(np.uint32)
    finite = rand[(rand & 0x7F800000) != 0x7F800000]
    sub = rng.integers(0, 0x00800000, 200_000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007FFFFF,
                        0x807FFFFF, 0x00800000, 0x80800000, 0x7F7FFFFF, 0xFF7FFFFF,
                        0x3F800000, 0xBF800000, 0x41300000, 0xC0000000], np.uint32)
    words = np.concatenate([finite, sub, sub | 0x80000000, special])
    got = run_probe("device_penalize_bits", words)
    want = o.penalize_array(words)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(words[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    # -FLT_MAX * 1.1 overflows to -inf; -0 and +0 stay put (tests.rs:468-481)
    idx = {int(w): i for i, w in enumerate(words[-len(special):])}
    tail = got[-len(special):]
    assert tail[idx[0xFF7FFFFF]] == 0xFF800000
    assert tail[idx[0x80000000]] == 0x80000000 and tail[idx[0x00000000]] == 0
