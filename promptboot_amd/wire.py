"""Interchange formats of promptboot's sampler evidence.

* Word files: raw little-endian 32-bit words with no header.  `*.f32le`
  holds binary32 logits rows (151,936 words per row) and `*.u32le` holds
  token id lists.  The reference reads both as u32 words; the length must be
  a multiple of 4 bytes (crates/promptboot-core/examples/validate_inference.rs:74-81).
* Logits checkpoints are identified by the SHA-256 of the row's words as
  little-endian bytes (`words_sha256`, validate_inference.rs:597-609).
* The exact host oracle is a key=value text file
  (fixtures/inference/exact-host-oracle.txt, written by ExactOracle::encode,
  validate_inference.rs:611-649):

      schema=1
      logit_words=151936
      seed=0123456789abcdef
      sampling_policy=<policy string>
      checkpoint=<name> sha256=<64 hex>        (zero or more, in order)
      sampled_tokens=<id>,<id>,...
      sampler_state=<16 hex>
      sampler_draws=<decimal>

  The harness compares the whole text byte for byte (validate_inference.rs:1233-1243),
  so `encode` reproduces the exact layout and `parse` rejects anything else.
"""
from __future__ import annotations

import dataclasses
import hashlib
import os
import re

import numpy as np

LOGIT_WORDS = 151_936
SAMPLING_POLICY = "temperature_0p7_top_k_20_top_p_0p8_repetition_penalty_1p1"


def read_words(path: str | os.PathLike) -> np.ndarray:
    """A .u32le / .f32le file as uint32 words (binary32 bit patterns for logits)."""
    data = open(path, "rb").read()
    if len(data) % 4 != 0:
        raise ValueError(f"{path}: {len(data)} bytes is not a whole number of words")
    return np.frombuffer(data, dtype="<u4").astype(np.uint32)


def write_words(path: str | os.PathLike, words) -> None:
    a = np.asarray(words)
    if a.dtype == np.float32:
        a = a.view(np.uint32)
    if a.dtype != np.uint32:
        raise TypeError("words must be uint32 (or float32 bit patterns)")
    with open(path, "wb") as f:
        f.write(np.ascontiguousarray(a, dtype="<u4").tobytes())


def read_logits_rows(path: str | os.PathLike, vocab: int = LOGIT_WORDS) -> np.ndarray:
    """An .f32le file of whole rows as a [rows, vocab] uint32 matrix."""
    w = read_words(path)
    if w.size % vocab != 0:
        raise ValueError(f"{path}: {w.size} words is not a whole number of {vocab}-word rows")
    return w.reshape(-1, vocab)


def words_sha256(words) -> str:
    """SHA-256 of the words as little-endian bytes, lowercase hex."""
    a = np.asarray(words)
    if a.dtype == np.float32:
        a = a.view(np.uint32)
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<u4").tobytes()).hexdigest()


@dataclasses.dataclass
class ExactOracle:
    """The exact host oracle record (validate_inference.rs:611-617)."""

    seed: int = 0x0123_4567_89AB_CDEF
    checkpoints: list[tuple[str, str]] = dataclasses.field(default_factory=list)
    sampled_tokens: list[int] = dataclasses.field(default_factory=list)
    sampler_state: int = 0
    sampler_draws: int = 0
    logit_words: int = LOGIT_WORDS
    sampling_policy: str = SAMPLING_POLICY

    def checkpoint(self, name: str, logits) -> None:
        """Records a logits row by its hash (ExactOracle::checkpoint, :620-624)."""
        a = np.asarray(logits)
        if a.size != self.logit_words:
            raise ValueError(f"{name}: {a.size} logits, expected {self.logit_words}")
        self.checkpoints.append((name, words_sha256(a)))

    def encode(self) -> str:
        """The text ExactOracle::encode writes (:626-649)."""
        lines = ["schema=1", f"logit_words={self.logit_words}", f"seed={self.seed:016x}",
                 f"sampling_policy={self.sampling_policy}"]
        lines += [f"checkpoint={n} sha256={h}" for n, h in self.checkpoints]
        lines.append("sampled_tokens=" + ",".join(str(int(t)) for t in self.sampled_tokens))
        lines.append(f"sampler_state={self.sampler_state:016x}")
        lines.append(f"sampler_draws={self.sampler_draws}")
        return "\n".join(lines) + "\n"

    _CHECKPOINT = re.compile(r"checkpoint=(\S+) sha256=([0-9a-f]{64})")

    @classmethod
    def parse(cls, text: str) -> "ExactOracle":
        """Strict inverse of `encode`: the same fields, in the same order."""
        lines = text.split("\n")
        if not lines or lines[-1] != "":
            raise ValueError("oracle text must end with a newline")
        lines = lines[:-1]

        def field(i: int, key: str) -> str:
            if i >= len(lines) or not lines[i].startswith(key + "="):
                raise ValueError(f"line {i + 1}: expected {key}=")
            return lines[i][len(key) + 1:]

        if field(0, "schema") != "1":
            raise ValueError("unsupported schema")
        out = cls(logit_words=int(field(1, "logit_words")))
        seed = field(2, "seed")
        if not re.fullmatch(r"[0-9a-f]{16}", seed):
            raise ValueError("seed must be 16 lowercase hex digits")
        out.seed = int(seed, 16)
        out.sampling_policy = field(3, "sampling_policy")
        i = 4
        while i < len(lines) and lines[i].startswith("checkpoint="):
            m = cls._CHECKPOINT.fullmatch(lines[i])
            if m is None:
                raise ValueError(f"line {i + 1}: malformed checkpoint")
            out.checkpoints.append((m.group(1), m.group(2)))
            i += 1
        toks = field(i, "sampled_tokens")
        out.sampled_tokens = [int(t) for t in toks.split(",")] if toks else []
        state = field(i + 1, "sampler_state")
        if not re.fullmatch(r"[0-9a-f]{16}", state):
            raise ValueError("sampler_state must be 16 lowercase hex digits")
        out.sampler_state = int(state, 16)
        out.sampler_draws = int(field(i + 2, "sampler_draws"))
        if len(lines) != i + 3:
            raise ValueError("trailing lines after sampler_draws")
        if out.encode() != text:
            raise ValueError("oracle text is not in canonical form")
        return out
