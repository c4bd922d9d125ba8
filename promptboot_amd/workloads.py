"""Seeded synthetic sampler workloads (the shapes promptboot's sampler sees).

Every workload is a batch of independent decode-step rows over the Qwen2.5
vocabulary (151,936 logits): fp32 logits, a padded uint32 history matrix
with per-row lengths, and one 24-bit uniform per row drawn with the
reference's own xorshift64* generator (SamplingState::new(seed_r), one
next_24; inference.rs:779-810).  Row r uses seed_r = base_seed + r.

    single    B=1: logits N(0, 2.5^2) with 5 distinct ids boosted by +U(8, 15);
              300 history ids ~ truncated Zipf(s=1.1) on [0, V); seed 42.
    small     B=64: same logits; history length ~ U[16, 1024], Zipf ids.
    large     B=4096: same logits; history length ~ U[16, 32768] (full
              context), stored as a [4096, 32768] padded matrix.
    flat      B=1024: logits N(0, 0.1^2) (top-p mass spread over all 20).
    ties      B=1024: the `small` logits rounded to multiples of 0.25, so many
              values tie at the rank-20 boundary.
    dominant  B=1024: N(0, 2.5^2) with one id at +40.
    half      B=1024: the `small` logits; each history is a shuffled set of
              V/2 distinct ids (penalty on half the vocabulary).
    boundary  B=1024: the `small` logits and histories, with rows whose draw
              lands exactly on, or one 2^-24 step of the uniform beside, a
              step of the cumulative distribution (the strict `>` of
              fp32_sse2.rs:1838-1844 decides them), cycling over four kinds:
              24 ids tied at +40 (kept 16, steps at the integers, the top-p
              cutoff exactly on the 16th prefix) with a uniform k/16; the
              same with k/16 +- 2^-24; two ids tied at +40 with a uniform of
              1/2 (or 1/2 +- 2^-24); an ordinary `small` row.  The uniform of
              a constructed row is the first next_24 of a seed chosen for it
              (seed_for_draw), so every row still draws from the repo PRNG.

Generation is numpy with a fixed PCG64 seed, so every machine builds the
same bytes.
"""
from __future__ import annotations

import numpy as np

VOCAB = 151_936
ZIPF_S = 1.1
_ZIPF_CDF = None


def next_24_stream(seeds: np.ndarray) -> np.ndarray:
    """One next_24 per seed (vectorised xorshift64*, inference.rs:779-810)."""
    s = np.asarray(seeds, dtype=np.uint64).copy()
    s[s == 0] = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        s ^= s >> np.uint64(12)
        s ^= s << np.uint64(25)
        s ^= s >> np.uint64(27)
        out = (s * np.uint64(0x2545F4914F6CDD1D)) >> np.uint64(40)
    return out.astype(np.uint32)


_MUL = 0x2545F4914F6CDD1D
_MASK64 = (1 << 64) - 1


def _undo_xorshift(v: int) -> int:
    """Inverse of next_24's state step (v ^= v >> 12; v ^= v << 25; v ^= v >> 27)."""
    v ^= (v >> 27) ^ (v >> 54)
    v = (v ^ (v << 25) ^ (v << 50)) & _MASK64
    v ^= (v >> 12) ^ (v >> 24) ^ (v >> 36) ^ (v >> 48) ^ (v >> 60)
    return v


def seed_for_draw(value_24: int, salt: int = 0) -> int:
    """A seed whose SamplingState's first next_24 is value_24: the scrambled
    state (s * 0x2545F4914F6CDD1D mod 2^64) must have value_24 in its top 24
    bits; the multiplier is odd, so s follows, and the state step is undone."""
    scrambled = ((value_24 & 0xFFFFFF) << 40) | (0x5DEECE66D * (salt + 1) & ((1 << 40) - 1))
    stepped = scrambled * pow(_MUL, -1, 1 << 64) & _MASK64
    seed = _undo_xorshift(stepped)
    assert seed != 0 and seed != 0x9E3779B97F4A7C15
    return seed


def zipf_ids(rng: np.random.Generator, n: int) -> np.ndarray:
    """n ids from P(k) proportional to (k+1)^-1.1 on [0, VOCAB)."""
    global _ZIPF_CDF
    if _ZIPF_CDF is None:
        w = np.arange(1, VOCAB + 1, dtype=np.float64) ** -ZIPF_S
        c = np.cumsum(w)
        _ZIPF_CDF = c / c[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(_ZIPF_CDF, u, side="right"), VOCAB - 1).astype(np.uint32)


def boosted_normal(rng: np.random.Generator, rows: int, sigma: float = 2.5,
                   boosts: int = 5) -> np.ndarray:
    x = rng.standard_normal((rows, VOCAB), dtype=np.float32)
    x *= np.float32(sigma)
    for r in range(rows):
        ids = rng.choice(VOCAB, boosts, replace=False)
        x[r, ids] += rng.uniform(8.0, 15.0, boosts).astype(np.float32)
    return x


def zipf_history(rng: np.random.Generator, lengths: np.ndarray, hist_ld: int) -> np.ndarray:
    rows = len(lengths)
    hist = np.zeros((rows, hist_ld), np.uint32)
    total = int(lengths.sum())
    ids = zipf_ids(rng, total)
    pos = 0
    for r, L in enumerate(lengths):
        hist[r, :L] = ids[pos:pos + L]
        pos += L
    return hist


CONFIGS = {
    "single": dict(rows=1),
    "small": dict(rows=64),
    "large": dict(rows=4096),
    "flat": dict(rows=1024),
    "ties": dict(rows=1024),
    "dominant": dict(rows=1024),
    "half": dict(rows=1024),
    "boundary": dict(rows=1024),
}


def make(name: str, rows: int | None = None, seed: int = 20240601, base_seed: int = 42) -> dict:
    """Returns dict(logits float32 [B, V], hist uint32 [B, hist_ld],
    hist_len uint32 [B], random_24 uint32 [B], seeds uint64 [B], name)."""
    if name not in CONFIGS:
        raise KeyError(name)
    B = rows if rows is not None else CONFIGS[name]["rows"]
    rng = np.random.default_rng([seed, list(CONFIGS).index(name)])
    if name == "single":
        logits = boosted_normal(rng, B)
        lengths = np.full(B, 300, np.uint32)
        hist = zipf_history(rng, lengths, 300)
    elif name in ("small", "ties", "half"):
        logits = boosted_normal(rng, B)
        if name == "ties":
            logits = (np.round(logits * np.float32(4.0)) / np.float32(4.0)).astype(np.float32)
        if name == "half":
            half = VOCAB // 2
            lengths = np.full(B, half, np.uint32)
            hist = np.empty((B, half), np.uint32)
            for r in range(B):
                hist[r] = rng.permutation(VOCAB)[:half].astype(np.uint32)
        else:
            lengths = rng.integers(16, 1025, B).astype(np.uint32)
            hist = zipf_history(rng, lengths, 1024)
    elif name == "large":
        logits = boosted_normal(rng, B)
        lengths = rng.integers(16, 32769, B).astype(np.uint32)
        hist = zipf_history(rng, lengths, 32768)
    elif name == "flat":
        logits = rng.standard_normal((B, VOCAB), dtype=np.float32) * np.float32(0.1)
        lengths = rng.integers(16, 1025, B).astype(np.uint32)
        hist = zipf_history(rng, lengths, 1024)
    elif name == "dominant":
        logits = rng.standard_normal((B, VOCAB), dtype=np.float32) * np.float32(2.5)
        logits[np.arange(B), rng.integers(0, VOCAB, B)] = np.float32(40.0)
        lengths = rng.integers(16, 1025, B).astype(np.uint32)
        hist = zipf_history(rng, lengths, 1024)
    seeds = np.uint64(base_seed) + np.arange(B, dtype=np.uint64)
    if name == "boundary":
        logits = boosted_normal(rng, B)
        lengths = rng.integers(16, 1025, B).astype(np.uint32)
        hist = zipf_history(rng, lengths, 1024)
        for r in range(B):
            kind, k = r % 4, (r // 4) % 16
            if kind == 3:
                continue
            tied = rng.choice(np.arange(VOCAB // 2, VOCAB), 24 if kind < 2 else 2, replace=False)
            logits[r, tied] = np.float32(40.0)
            hist[r][np.isin(hist[r], tied)] = 1  # the tied ids stay unpenalised
            if kind == 0:
                value = k << 20
            elif kind == 1:
                value = (k << 20) + (1 if k == 0 or (r // 64) % 2 == 0 else -1)
            else:
                value = (1 << 23) + (0, 1, -1)[(r // 4) % 3]
            seeds[r] = np.uint64(seed_for_draw(value, r))
    return dict(name=name, logits=logits, hist=hist, hist_len=lengths.astype(np.uint32),
                random_24=next_24_stream(seeds), seeds=seeds)


HIDDEN = 896


def make_lmhead(rows: int = 256, seed: int = 20240601, base_seed: int = 42) -> dict:
    """Fused LM head workload: hidden states [rows, 896] ~ N(0, 1); a Q4_0 head
    of 151,936 x 896 in promptboot's layout (vocab rows of 28 blocks of 18
    bytes: fp16 scale ~ U(0.001, 0.02), 16 random nibble bytes); histories as
    in `small` (length ~ U[16, 1024], Zipf ids); one uniform per row."""
    rng = np.random.default_rng([seed, 99])
    blocks = HIDDEN // 32
    hidden = rng.standard_normal((rows, HIDDEN), dtype=np.float32)
    q4 = np.empty((VOCAB, blocks, 18), np.uint8)
    scales = rng.uniform(0.001, 0.02, (VOCAB, blocks)).astype(np.float16)
    q4[:, :, 0:2] = scales.view(np.uint8).reshape(VOCAB, blocks, 2)
    q4[:, :, 2:] = rng.integers(0, 256, (VOCAB, blocks, 16), dtype=np.uint8)
    lengths = rng.integers(16, 1025, rows).astype(np.uint32)
    hist = zipf_history(rng, lengths, 1024)
    seeds = np.uint64(base_seed) + np.arange(rows, dtype=np.uint64)
    return dict(name="lmhead", hidden=hidden, q4=q4.reshape(-1), hist=hist, hist_len=lengths,
                random_24=next_24_stream(seeds), seeds=seeds)


def make_q8_head(seed: int = 20240601, cols: int = HIDDEN) -> np.ndarray:
    """A Q8_0 head of 151,936 x cols in promptboot's layout (the model's output
    tensor, model.rs:817-818): vocab rows of cols/32 blocks of 34 bytes, fp16
    scale ~ U(0.0005, 0.004) and 32 signed weights over the whole int8 range."""
    rng = np.random.default_rng([seed, 88])
    blocks = cols // 32
    q8 = np.empty((VOCAB, blocks, 34), np.uint8)
    scales = rng.uniform(0.0005, 0.004, (VOCAB, blocks)).astype(np.float16)
    q8[:, :, 0:2] = scales.view(np.uint8).reshape(VOCAB, blocks, 2)
    q8[:, :, 2:] = rng.integers(0, 256, (VOCAB, blocks, 32), dtype=np.uint8)
    return q8.reshape(-1)


def lmhead_algorithmic_bytes(rows: int, hist_len: np.ndarray, q8: bool = False) -> int:
    """HBM bytes of one fused step: the head once (18 B per 32 Q4_0 weights, 34
    B per 32 Q8_0 weights), the hidden states, the valid history ids, and
    per-row length, uniform and token words."""
    return (VOCAB * HIDDEN // 32 * (34 if q8 else 18) + rows * HIDDEN * 4 + 12 * rows
            + 4 * int(np.asarray(hist_len, np.int64).sum()))


def algorithmic_bytes(hist_len: np.ndarray) -> int:
    """HBM bytes the path must move per batch: every logit once, every valid
    history id once, plus the per-row length, uniform and token words."""
    rows = len(hist_len)
    return rows * (4 * VOCAB + 12) + 4 * int(np.asarray(hist_len, np.int64).sum())
