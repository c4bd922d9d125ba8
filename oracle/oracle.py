"""ctypes bindings for the CPU oracle (oracle/pb_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py use this module as the checker (or as the
reported single-core CPU baseline).  The product (promptboot_amd) never
imports it.

Every function mirrors one reference function; the C file carries the
reference file:line citations.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# PB_ORACLE_LIB lets a mutation check load a deliberately broken build.
LIB_PATH = pathlib.Path(os.environ.get("PB_ORACLE_LIB", HERE / "_build" / "libpboracle.so"))

VOCAB = 151_936
TOP_K = 20
SEEN_BYTES = (VOCAB + 7) // 8

FLAG_DRAW_BOUNDARY = 1
FLAG_CUTOFF_BOUNDARY = 2

u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
size_t = ctypes.c_size_t
vp = ctypes.c_void_p


class State(ctypes.Structure):
    _fields_ = [("state", u64), ("draws", u64)]


class Error(ctypes.Structure):
    _fields_ = [
        ("status", u32), ("domain", u32), ("layer", u32), ("position", u32),
        ("tensor_id", u32), ("reserved", u32),
        ("needed", u64), ("available", u64), ("detail", u64),
    ]

    def tuple(self) -> list[int]:
        """Same 8-tuple as the reference's inference_error_tuple (tests.rs:185-196)."""
        return [self.status, self.domain, self.layer, self.position, self.tensor_id,
                self.needed, self.available, self.detail]


class TopLogit(ctypes.Structure):
    _fields_ = [("token", u32), ("logit_bits", u32)]


DETAIL_DTYPE = np.dtype([
    ("ids", "<u4", (TOP_K,)),
    ("value_bits", "<u4", (TOP_K,)),
    ("weight_bits", "<u4", (TOP_K,)),
    ("probs", "<f4", (TOP_K,)),
    ("kept", "<u4"),
    ("rank", "<u4"),
    ("flags", "<u4"),
    ("token", "<u4"),
])

ERROR_DTYPE = np.dtype([
    ("status", "<u4"), ("domain", "<u4"), ("layer", "<u4"), ("position", "<u4"),
    ("tensor_id", "<u4"), ("reserved", "<u4"),
    ("needed", "<u8"), ("available", "<u8"), ("detail", "<u8"),
])

_lib = None


def build() -> None:
    """Compile the oracle with its own Makefile (gcc, scalar SSE, no FMA)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.pbo_state_new.argtypes = [ctypes.POINTER(State), u64]
        L.pbo_next_24.argtypes = [ctypes.POINTER(State)]
        L.pbo_next_24.restype = u32
        L.pbo_expf_bits.argtypes = [u32]
        L.pbo_expf_bits.restype = u32
        L.pbo_apply_repetition_penalty.argtypes = [vp, vp, size_t, vp]
        L.pbo_sample_top_k_top_p.argtypes = [vp, size_t, u32, vp]
        L.pbo_sample_top_k_top_p.restype = u32
        L.pbo_sample_token.argtypes = [vp, size_t, ctypes.POINTER(State), vp,
                                       ctypes.POINTER(Error)]
        L.pbo_sample_token_with_repetition.argtypes = [
            vp, size_t, vp, size_t, vp, size_t, ctypes.POINTER(State), vp,
            ctypes.POINTER(Error), vp]
        L.pbo_greedy_token.argtypes = [vp, size_t, vp, ctypes.POINTER(Error)]
        L.pbo_top_logits_8.argtypes = [vp, size_t, vp, ctypes.POINTER(Error)]
        L.pbo_sample_batch.argtypes = [vp, size_t, size_t, u32, vp, size_t, vp, vp,
                                       vp, vp, vp, vp, ctypes.c_int]
        L.pbo_time_batch.argtypes = [vp, size_t, u32, vp, size_t, vp, vp, vp]
        L.pbo_time_batch.restype = u64
        L.pbo_half_to_f32_bits.argtypes = [ctypes.c_uint16]
        L.pbo_half_to_f32_bits.restype = u32
        L.pbo_f32_to_half_bits.argtypes = [u32]
        L.pbo_f32_to_half_bits.restype = ctypes.c_uint16
        L.pbo_prepare_q8.argtypes = [vp, vp, size_t]
        L.pbo_q4_block_dot.argtypes = [vp, vp]
        L.pbo_q4_block_dot.restype = ctypes.c_int32
        L.pbo_q4_matvec_rows.argtypes = [vp, vp, vp, size_t, size_t]
        L.pbo_lmhead_logits.argtypes = [vp, u32, vp, size_t, size_t, vp, ctypes.c_int]
        L.pbo_q8_block_dot.argtypes = [vp, vp]
        L.pbo_q8_block_dot.restype = ctypes.c_int32
        L.pbo_q8_matvec_rows.argtypes = [vp, vp, vp, size_t, size_t]
        L.pbo_lmhead_q8_logits.argtypes = [vp, u32, vp, size_t, size_t, vp, ctypes.c_int]
        L.pbo_expf_array.argtypes = [vp, vp, size_t]
        L.pbo_penalize_array.argtypes = [vp, vp, size_t]
        for name in ("pbo_sizeof_detail", "pbo_sizeof_error", "pbo_sizeof_state"):
            getattr(L, name).restype = size_t
        assert L.pbo_sizeof_detail() == DETAIL_DTYPE.itemsize
        assert L.pbo_sizeof_error() == ERROR_DTYPE.itemsize == 48
        assert L.pbo_sizeof_state() == 16
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(vp)


def _u32(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float32:
        a = a.view(np.uint32)
    return np.ascontiguousarray(a, dtype=np.uint32)


class SamplingState:
    """xorshift64* generator with a draw counter (inference.rs:772-810)."""

    def __init__(self, seed: int = 0, *, state: int | None = None, draws: int = 0):
        self._s = State()
        if state is None:
            lib().pbo_state_new(ctypes.byref(self._s), seed & (2**64 - 1))
        else:
            self._s.state, self._s.draws = state, draws

    def state(self) -> int:
        return self._s.state

    def draws(self) -> int:
        return self._s.draws

    def next_24(self) -> int:
        return lib().pbo_next_24(ctypes.byref(self._s))

    def copy(self) -> "SamplingState":
        return SamplingState(state=self._s.state, draws=self._s.draws)

    def __eq__(self, other) -> bool:
        return (self.state(), self.draws()) == (other.state(), other.draws())


def expf_bits(x: int) -> int:
    return lib().pbo_expf_bits(x & 0xFFFFFFFF)


def time_batch(logits, hist, hist_len, seeds) -> tuple[float, np.ndarray]:
    """Single-threaded timing of sample_token_with_repetition per row (seconds
    summed over rows, timer boundary of validate_inference.rs:780-794)."""
    lg = _u32(logits)
    h = _u32(hist)
    hl = _u32(hist_len)
    sd = np.ascontiguousarray(seeds, dtype=np.uint64)
    tok = np.zeros(lg.shape[0], np.uint32)
    ns = lib().pbo_time_batch(_ptr(lg), lg.shape[1], lg.shape[0], _ptr(h), h.shape[1],
                              _ptr(hl), _ptr(sd), _ptr(tok))
    return ns * 1e-9, tok


Q8_STAGING_BYTES = 5184


def half_to_f32_bits(h: int) -> int:
    return lib().pbo_half_to_f32_bits(h & 0xFFFF)


def f32_to_half_bits(bits: int) -> int:
    return lib().pbo_f32_to_half_bits(bits & 0xFFFFFFFF)


def prepare_q8(words, staging: np.ndarray | None = None) -> np.ndarray:
    """inference_prepare_q8: returns the 5,184-byte staging area."""
    x = _u32(words)
    if staging is None:
        staging = np.zeros(Q8_STAGING_BYTES, np.uint8)
    lib().pbo_prepare_q8(_ptr(x), _ptr(staging), x.size)
    return staging


def q4_block_dot(weights16, activation32) -> int:
    w = np.ascontiguousarray(weights16, dtype=np.uint8)
    a = np.ascontiguousarray(activation32, dtype=np.int8)
    return lib().pbo_q4_block_dot(_ptr(w), _ptr(a))


def q4_matvec(weights: np.ndarray, staging: np.ndarray, rows: int, columns: int) -> np.ndarray:
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    out = np.zeros(rows, np.uint32)
    lib().pbo_q4_matvec_rows(_ptr(w), _ptr(out), _ptr(staging), rows, columns)
    return out


def q8_block_dot(weights32, activation32) -> int:
    w = np.ascontiguousarray(weights32, dtype=np.int8)
    a = np.ascontiguousarray(activation32, dtype=np.int8)
    return lib().pbo_q8_block_dot(_ptr(w), _ptr(a))


def q8_matvec(weights: np.ndarray, staging: np.ndarray, rows: int, columns: int) -> np.ndarray:
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    out = np.zeros(rows, np.uint32)
    lib().pbo_q8_matvec_rows(_ptr(w), _ptr(out), _ptr(staging), rows, columns)
    return out


def lmhead_logits(hidden, weights: np.ndarray, vocab: int, columns: int,
                  threads: int = 1, q8: bool = False) -> np.ndarray:
    """Logits [rows, vocab] (uint32 words) of each hidden row through a Q4_0
    head (vocab rows of columns/32 blocks of 18 bytes) or, with q8, a Q8_0 head
    (blocks of 34 bytes), both in the reference layout."""
    h = _u32(hidden)
    rows = h.shape[0]
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    assert w.size == vocab * columns // 32 * (34 if q8 else 18)
    out = np.zeros((rows, vocab), np.uint32)
    fn = lib().pbo_lmhead_q8_logits if q8 else lib().pbo_lmhead_logits
    fn(_ptr(h), rows, _ptr(w), vocab, columns, _ptr(out), threads)
    return out


def expf_array(words) -> np.ndarray:
    a = _u32(words)
    out = np.empty_like(a)
    lib().pbo_expf_array(_ptr(a), _ptr(out), a.size)
    return out


def penalize_array(words) -> np.ndarray:
    """Repetition penalty of each word as a lone history id."""
    a = _u32(words)
    out = np.empty_like(a)
    lib().pbo_penalize_array(_ptr(a), _ptr(out), a.size)
    return out


def apply_repetition_penalty(logits: np.ndarray, tokens, seen: np.ndarray) -> None:
    t = _u32(tokens)
    lib().pbo_apply_repetition_penalty(_ptr(logits), _ptr(t), t.size, _ptr(seen))


def sample_top_k_top_p(logits, random_24: int):
    """Returns (token, detail record) for one already-penalised row."""
    row = _u32(logits)
    det = np.zeros(1, DETAIL_DTYPE)
    tok = lib().pbo_sample_top_k_top_p(_ptr(row), row.size, random_24 & 0xFFFFFFFF, _ptr(det))
    return tok, det[0]


def sample_token(logits, state: SamplingState):
    row = _u32(logits)
    out = np.zeros(1, np.uint32)
    err = Error()
    st = lib().pbo_sample_token(_ptr(row), row.size, ctypes.byref(state._s), _ptr(out),
                                ctypes.byref(err))
    return st, int(out[0]), err


def sample_token_with_repetition(logits: np.ndarray, tokens, seen: np.ndarray,
                                 state: SamplingState, want_detail: bool = False):
    """Mutates `logits` (uint32 array) in place like the reference on success."""
    assert logits.dtype == np.uint32 and logits.flags.c_contiguous
    t = _u32(tokens)
    out = np.zeros(1, np.uint32)
    err = Error()
    det = np.zeros(1, DETAIL_DTYPE) if want_detail else None
    st = lib().pbo_sample_token_with_repetition(
        _ptr(logits), logits.size, _ptr(t), t.size, _ptr(seen), seen.size,
        ctypes.byref(state._s), _ptr(out), ctypes.byref(err), _ptr(det))
    if want_detail:
        return st, int(out[0]), err, (det[0] if st == 0 else None)
    return st, int(out[0]), err


def greedy_token(logits):
    row = _u32(logits)
    out = np.zeros(1, np.uint32)
    err = Error()
    st = lib().pbo_greedy_token(_ptr(row), row.size, _ptr(out), ctypes.byref(err))
    return st, int(out[0]), err


def top_logits_8(logits, output: np.ndarray | None = None):
    """output: uint32 array of 16 words (token, bits) x 8, untouched on error."""
    row = _u32(logits)
    if output is None:
        output = np.zeros(16, np.uint32)
    err = Error()
    st = lib().pbo_top_logits_8(_ptr(row), row.size, _ptr(output), ctypes.byref(err))
    return st, output, err


def sample_batch(logits: np.ndarray, hist: np.ndarray | None, hist_len: np.ndarray | None,
                 random_24: np.ndarray, threads: int = 1, want_penalized: bool = False):
    """Rows of a [B, ld] uint32/float32 matrix; history [B, hist_ld] + lengths.

    Returns (tokens[B], detail[B], errors[B], penalized or None)."""
    lg = _u32(logits)
    B, ld = lg.shape
    vocab = VOCAB if ld >= VOCAB else ld
    if hist is None:
        h, hl, hld = None, None, 0
    else:
        h = _u32(hist)
        hl = _u32(hist_len)
        hld = h.shape[1]
    r = _u32(random_24)
    tok = np.zeros(B, np.uint32)
    det = np.zeros(B, DETAIL_DTYPE)
    err = np.zeros(B, ERROR_DTYPE)
    pen = np.empty_like(lg) if want_penalized else None
    lib().pbo_sample_batch(_ptr(lg), ld, vocab, B, _ptr(h), hld, _ptr(hl), _ptr(r),
                           _ptr(tok), _ptr(det), _ptr(err), _ptr(pen), threads)
    return tok, det, err, pen


IM_END = 151_645       # src/repl_contract.rs:26
END_OF_TEXT = 151_643  # crates/promptboot-core/src/tokenizer.rs:39


class DecodeRow:
    """One sequence through the REPL's generation loop, restated from
    src/model_repl.rs:928-1150 with the model replaced by the caller's logits:

    * the sampler sees the whole working context, working[..prompt_count +
      generated] (:961-968), with the session's `seen` scratch and the boot's
      SamplingState;
    * a sampler error ends the turn; nothing is appended (:989-996);
    * the context receives the token, or IM_END when the piece is an
      end-of-sequence one (:1099-1103; tokenizer.rs:1047 classes IM_END and
      END_OF_TEXT as EOS), then generated += 1 (:1114);
    * the turn ends on end-of-sequence (:1119-1150) or once generated reaches
      the generation limit (the `while generated < generation_limit` of :928).
    """

    def __init__(self, prompt, seed: int, limit: int, state: SamplingState | None = None):
        self.working = [int(t) for t in prompt]
        self.prompt_count = len(self.working)
        self.generated = 0
        self.limit = int(limit)
        # one SamplingState per boot, kept across turns (model_repl.rs:333-334)
        self.state = state if state is not None else SamplingState(seed)
        self.seen = np.zeros(SEEN_BYTES, np.uint8)
        self.reason = None if self.limit > 0 else "LIMIT"
        self.error: list[int] | None = None
        self.tokens: list[int] = []

    def active(self) -> bool:
        return self.reason is None

    def step(self, logits) -> int | None:
        """Samples one token from `logits` (not modified); None once ended."""
        if not self.active():
            return None
        row = _u32(logits).copy()
        st, tok, err = sample_token_with_repetition(
            row, self.working[:self.prompt_count + self.generated], self.seen, self.state)
        if st != 0:
            self.reason = "ERROR"
            self.error = err.tuple()
            return None
        eos = tok in (IM_END, END_OF_TEXT)
        self.working.append(IM_END if eos else tok)
        self.tokens.append(tok)
        self.generated += 1
        if eos:
            self.reason = "EOS"
        elif self.generated >= self.limit:
            self.reason = "LIMIT"
        return tok
