"""Pins the oracle's Q8_0 activation quantizer and Q4_0 x Q8_0 head.

Known answers: fixtures/inference/kernels/q8.bin and dots.bin (asserted by
the reference in crates/promptboot-core/src/tests.rs:4108-4198, produced by
the pinned llama.cpp helper), and the nibble-order / extrema block-dot tests
of tests.rs:3962-4023.  The fp16 conversions are checked against numpy's
IEEE binary16 on every bit pattern, and the head against a float64
computation.
"""
import numpy as np

from oracle import oracle as o
from tests.conftest import GOLDEN


def f32w(x) -> int:
    return int(np.array([x], np.float32).view(np.uint32)[0])


def test_q8_quantizer_matches_pinned_llama_blocks():
    quant = np.zeros(32 * 6, np.uint32)
    quant[32:36] = [f32w(1.0), f32w(-1.0), f32w(1.0), f32w(-1.0)]
    quant[64:69] = [f32w(127.0), f32w(0.5), f32w(-0.5), f32w(1.5), f32w(-1.5)]
    quant[96:99] = [0x34000000, 0x33800000, 0x33000000]
    quant[128:131] = [f32w(126.5), f32w(-126.5), f32w(63.25)]
    quant[160:162] = [f32w(-0.0), f32w(0.0)]
    staging = np.full(o.Q8_STAGING_BYTES, 0xA5, np.uint8)
    o.prepare_q8(quant, staging)
    expected = np.fromfile(GOLDEN / "q8_block_quant.bin", dtype=np.uint8)
    assert expected.size == 204
    assert (staging[:204] == expected).all()
    assert not staging[204:].any()


def reference_matvec_input():
    x = np.array([float((i % 31) - 15) for i in range(64)], np.float32)
    x[31], x[63] = 127.0, -127.0
    q4 = np.zeros(36, np.uint8)
    for block in range(2):
        q4[block * 18:block * 18 + 2] = [0x00, 0x3C]  # fp16 1.0, little endian
        for i in range(16):
            q4[block * 18 + 2 + i] = ((15 - i) << 4) | i
    return x, q4


def test_q4_matvec_matches_pinned_dot():
    x, q4 = reference_matvec_input()
    staging = o.prepare_q8(x)
    assert not staging[68:].any()
    out = o.q4_matvec(q4, staging, rows=1, columns=64)
    dots = np.fromfile(GOLDEN / "q4_q8_dots.bin", dtype="<u4")
    assert int(out[0]) == int(dots[0]) == 0x43E08000


def numpy_q4_dot(weights16, act32):
    w = np.asarray(weights16, np.uint8).astype(np.int64)
    a = np.asarray(act32, np.int8).astype(np.int64)
    return int(((w & 15) - 8) @ a[:16] + ((w >> 4) - 8) @ a[16:])


def test_q4_block_dot_nibble_order_and_extrema():
    ordered_w = np.array([((15 - i) << 4) | i for i in range(16)], np.uint8)
    ordered_a = np.array([i + 1 if i < 16 else -(i - 15) for i in range(32)], np.int8)
    swapped = int(((ordered_w.astype(np.int64) >> 4) - 8) @ ordered_a[:16].astype(np.int64)
                  + ((ordered_w.astype(np.int64) & 15) - 8) @ ordered_a[16:].astype(np.int64))
    assert o.q4_block_dot(ordered_w, ordered_a) == numpy_q4_dot(ordered_w, ordered_a) != swapped
    ext_w = np.array([0x0F if i % 2 == 0 else 0xF0 for i in range(16)], np.uint8)
    ext_a = np.array([-128 if (i < 16) == (i % 2 == 0) else 127 for i in range(32)], np.int8)
    assert o.q4_block_dot(ext_w, ext_a) == numpy_q4_dot(ext_w, ext_a)
    rng = np.random.default_rng(0)
    for _ in range(200):
        w = rng.integers(0, 256, 16).astype(np.uint8)
        a = rng.integers(-128, 128, 32).astype(np.int8)
        assert o.q4_block_dot(w, a) == numpy_q4_dot(w, a)


def test_half_to_f32_on_every_binary16():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = np.array([o.half_to_f32_bits(int(v)) for v in h], np.uint32)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    finite = (h & 0x7C00) != 0x7C00
    assert (got[finite] == want[finite]).all()
    inf = (h & 0x7FFF) == 0x7C00
    assert (got[inf] == want[inf]).all()
    nan = ~finite & ~inf  # payload kept, quiet bit not forced
    assert (got[nan] == ((h[nan].astype(np.uint32) & 0x8000) << 16 | 0x7F800000
                         | (h[nan].astype(np.uint32) & 0x3FF) << 13)).all()


def test_f32_to_half_rounds_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3),
        rng.uniform(-1e-4, 1e-4, 5000).astype(np.float32),        # fp16 subnormals
        rng.uniform(6e4, 7e4, 2000).astype(np.float32),           # around fp16 overflow
        np.float32([0.0, -0.0, 65504.0, 65520.0, 6e-8, 3e-8, 2.98e-8, np.inf, -np.inf]),
    ]).astype(np.float32)
    got = np.array([o.f32_to_half_bits(int(b)) for b in vals.view(np.uint32)], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert (got == want).all(), vals[got != want][:5]


def test_q8_dequantization_error_and_half_away_ties():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(896).astype(np.float32)
    st = o.prepare_q8(x)
    for b in range(28):
        blk = st[b * 34:(b + 1) * 34]
        scale = np.uint16(int(blk[0]) | int(blk[1]) << 8).view(np.float16).astype(np.float64)
        q = blk[2:].view(np.int8).astype(np.float64)
        xb = x[b * 32:(b + 1) * 32].astype(np.float64)
        amax = np.abs(xb).max()
        assert np.abs(q).max() == 127
        assert np.abs(xb - q * amax / 127).max() <= amax / 127 * 0.5 + 1e-6
        assert abs(scale - amax / 127) <= amax / 127 * 2**-11
    # round half away from zero: 0.5 * 127/127 scale -> +-1 (q8.bin block 2)
    blk = o.prepare_q8(np.float32([127.0, 0.5, -0.5, 1.5, -1.5] + [0.0] * 27))[:34]
    assert blk[2:7].view(np.int8).tolist() == [127, 1, -1, 2, -2]


def test_lmhead_logits_against_float64():
    rng = np.random.default_rng(3)
    vocab, cols, rows = 96, 896, 3
    hidden = rng.standard_normal((rows, cols)).astype(np.float32)
    blocks = cols // 32
    w = np.zeros((vocab, blocks, 18), np.uint8)
    scales = rng.uniform(0.001, 0.02, (vocab, blocks)).astype(np.float16)
    w[:, :, 0:2] = scales.view(np.uint8).reshape(vocab, blocks, 2)
    w[:, :, 2:] = rng.integers(0, 256, (vocab, blocks, 16))
    logits = o.lmhead_logits(hidden, w.reshape(-1), vocab, cols, threads=2)
    # float64 with the same quantised operands
    nib = w[:, :, 2:].astype(np.int64)
    wq = np.concatenate([(nib & 15) - 8, (nib >> 4) - 8], axis=2)  # [vocab, blocks, 32]
    for r in range(rows):
        st = o.prepare_q8(hidden[r])
        sb = st[:blocks * 34].reshape(blocks, 34)
        a_scale = sb[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(blocks)
        a = sb[:, 2:].view(np.int8).astype(np.int64)
        dots = np.einsum("vbk,bk->vb", wq, a)
        want = (dots * scales.astype(np.float64) * a_scale).sum(axis=1)
        got = logits[r].view(np.float32).astype(np.float64)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
        # and the single-row matvec agrees bit for bit
        assert (o.q4_matvec(w.reshape(-1), st, vocab, cols) == logits[r]).all()


def test_q4_head_scale_order_and_block_order_are_the_references():
    """fp32_sse2.rs:1241-1244 scales as mul(mul(f32(dot), w_scale), a_scale)
    and accumulates the blocks left to right in binary32; the Q8 head
    (:1271-1274) uses mul(f32(dot), mul(w_scale, a_scale)).  Random rows where
    the two orders round differently must follow the Q4 order bit for bit."""
    # The orders only round differently when f32(dot) * w_scale needs more than
    # 24 bits, i.e. |dot| >~ 2^13: saturate the activations (|q| = 127) and
    # align the nibbles with their signs so |dot| is near 32 * 7.5 * 127.
    rng = np.random.default_rng(4)
    vocab, cols = 64, 896
    blocks = cols // 32
    signs = np.where(rng.random(cols) < 0.5, -1.0, 1.0).astype(np.float32)
    hidden = signs * rng.uniform(0.5, 1.5, blocks).astype(np.float32).repeat(32)
    st = o.prepare_q8(hidden)
    sb = st[:blocks * 34].reshape(blocks, 34)
    a_scale = sb[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(blocks)
    a = sb[:, 2:].view(np.int8).astype(np.int64)
    w = np.zeros((vocab, blocks, 18), np.uint8)
    scales = rng.uniform(0.001, 0.02, (vocab, blocks)).astype(np.float16)
    w[:, :, 0:2] = scales.view(np.uint8).reshape(vocab, blocks, 2)
    nib = np.where(signs.reshape(blocks, 32) > 0, 15, 0)
    flip = rng.random((vocab, blocks, 32)) < 0.1
    nib = np.where(flip, 15 - nib[None], nib[None])
    w[:, :, 2:] = (nib[:, :, :16] | (nib[:, :, 16:] << 4)).astype(np.uint8)
    got = o.q4_matvec(w.reshape(-1), st, vocab, cols)
    nib = w[:, :, 2:].astype(np.int64)
    wq = np.concatenate([(nib & 15) - 8, (nib >> 4) - 8], axis=2)
    differs = 0
    for v in range(vocab):
        t4 = np.float32(0)
        t8 = np.float32(0)
        for b in range(blocks):
            d = np.float32(int(wq[v, b] @ a[b]))
            ws = np.float32(scales[v, b])
            t4 = np.float32(t4 + np.float32(np.float32(d * ws) * a_scale[b]))
            t8 = np.float32(t8 + np.float32(d * np.float32(ws * a_scale[b])))
        assert got[v] == t4.view(np.uint32), v
        differs += t4 != t8
    assert differs > 0


# ---- the Q8_0 head (fp32_sse2.rs:1251-1280) ----

def reference_q8_weights():
    """The Q8_0 rows of tests.rs:4152-4158: two blocks with fp16 scale 1.0 and
    weight i = (i % 17) - 8."""
    q8 = np.zeros(68, np.uint8)
    for block in range(2):
        q8[block * 34:block * 34 + 2] = [0x00, 0x3C]
        q8[block * 34 + 2:block * 34 + 34] = (np.arange(32) % 17 - 8).astype(np.int8).view(np.uint8)
    return q8


def test_q8_matvec_matches_pinned_dot():
    x, _ = reference_matvec_input()
    staging = o.prepare_q8(x)
    out = o.q8_matvec(reference_q8_weights(), staging, rows=1, columns=64)
    dots = np.fromfile(GOLDEN / "q4_q8_dots.bin", dtype="<u4")
    assert int(out[0]) == int(dots[1]) == 0x44388000


def test_q8_block_dot_extrema_and_the_references_deterministic_cases():
    """tests.rs:4026-4050 (signed extrema, dot 8) and tests.rs:4053-4100: the
    reference's 256 generated cases, against an integer dot product."""
    w = np.array([-128 if (i & 3) in (0, 1) else 127 for i in range(32)], np.int8)
    a = np.array([-128 if (i & 3) in (0, 2) else 127 for i in range(32)], np.int8)
    assert o.q8_block_dot(w, a) == 8
    state = 0x243F6A88

    def nxt():
        nonlocal state
        state = (state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
        return state >> 24

    for _ in range(256):
        q4w = np.array([nxt() for _ in range(16)], np.uint8)
        q8w = np.array([nxt() for _ in range(32)], np.uint8).view(np.int8)
        act = np.array([nxt() for _ in range(32)], np.uint8).view(np.int8)
        assert o.q8_block_dot(q8w, act) == int(q8w.astype(np.int64) @ act.astype(np.int64))
        assert o.q4_block_dot(q4w, act) == numpy_q4_dot(q4w, act)


def test_q8_lmhead_logits_against_float64():
    rng = np.random.default_rng(5)
    vocab, cols, rows = 96, 896, 3
    hidden = rng.standard_normal((rows, cols)).astype(np.float32)
    blocks = cols // 32
    w = np.zeros((vocab, blocks, 34), np.uint8)
    scales = rng.uniform(0.001, 0.02, (vocab, blocks)).astype(np.float16)
    w[:, :, 0:2] = scales.view(np.uint8).reshape(vocab, blocks, 2)
    w[:, :, 2:] = rng.integers(0, 256, (vocab, blocks, 32))
    logits = o.lmhead_logits(hidden, w.reshape(-1), vocab, cols, threads=2, q8=True)
    wq = w[:, :, 2:].view(np.int8).astype(np.int64)
    for r in range(rows):
        st = o.prepare_q8(hidden[r])
        sb = st[:blocks * 34].reshape(blocks, 34)
        a_scale = sb[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(blocks)
        a = sb[:, 2:].view(np.int8).astype(np.int64)
        dots = np.einsum("vbk,bk->vb", wq, a)
        want = (dots * scales.astype(np.float64) * a_scale).sum(axis=1)
        got = logits[r].view(np.float32).astype(np.float64)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
        assert (o.q8_matvec(w.reshape(-1), st, vocab, cols) == logits[r]).all()


def test_q8_head_scale_order_is_the_references():
    """fp32_sse2.rs:1271-1274 multiplies the two scales first:
    mul(f32(dot), mul(w_scale, a_scale)).  (Both are fp16 values, so their
    product is exact and each term is rounded once.)  Rows where the Q4_0
    head's order would round differently must follow the Q8_0 order."""
    rng = np.random.default_rng(6)
    vocab, cols = 64, 896
    blocks = cols // 32
    hidden = rng.standard_normal(cols).astype(np.float32) * np.float32(3)
    st = o.prepare_q8(hidden)
    sb = st[:blocks * 34].reshape(blocks, 34)
    a_scale = sb[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(blocks)
    a = sb[:, 2:].view(np.int8).astype(np.int64)
    w = np.zeros((vocab, blocks, 34), np.uint8)
    scales = rng.uniform(0.001, 0.02, (vocab, blocks)).astype(np.float16)
    w[:, :, 0:2] = scales.view(np.uint8).reshape(vocab, blocks, 2)
    # weights aligned with the activations' signs: |dot| large, so f32(dot) * ws needs
    # more than 24 bits and the two orders can round differently
    sign = np.sign(a).astype(np.int64)
    mag = rng.integers(64, 128, (vocab, blocks, 32))
    w[:, :, 2:] = (sign[None] * mag).astype(np.int8).view(np.uint8)
    got = o.q8_matvec(w.reshape(-1), st, vocab, cols)
    wq = w[:, :, 2:].view(np.int8).astype(np.int64)
    differs = 0
    for v in range(vocab):
        t8 = np.float32(0)
        t4 = np.float32(0)
        for b in range(blocks):
            d = np.float32(int(wq[v, b] @ a[b]))
            ws = np.float32(scales[v, b])
            t8 = np.float32(t8 + np.float32(d * np.float32(ws * a_scale[b])))
            t4 = np.float32(t4 + np.float32(np.float32(d * ws) * a_scale[b]))
        assert got[v] == t8.view(np.uint32), v
        differs += t4 != t8
    assert differs > 0
