"""Host-side mirror of promptboot's sampler API over libpbsample.so.

Same names, argument meaning and error behaviour as the reference
(crates/promptboot-core/src/inference.rs:737-965):

    SamplingState(seed)                     inference.rs:779-799
    sample_token_with_repetition(...)       inference.rs:919-965
    sample_token(logits, state)             inference.rs:914-917
    greedy_token(logits)                    inference.rs:861-881
    top_logits_8(logits)                    inference.rs:814-859

Rust's `Result<T, InferenceError>` becomes a return value or a raised
`InferenceError` carrying the 48-byte record.  Logits are numpy uint32 words
(binary32 bit patterns) as in the reference; float32 arrays are accepted and
viewed as words.

`BatchSampler` drives the batched device entry points on torch device
tensors (torch is used for device memory and streams only).

All selection arithmetic runs in the HIP kernels; if the library is missing
the import fails.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

VOCAB = 151_936
TOP_K = 20
SEEN_BYTES = (VOCAB + 7) // 8
NO_TOKEN = 0xFFFF_FFFF
SAMPLING_TEMPERATURE_MILLI = 700
SAMPLING_TOP_K = 20
SAMPLING_TOP_P_MILLI = 800
SAMPLING_REPETITION_PENALTY_MILLI = 1_100
SAMPLING_POLICY = b"temperature_0p7_top_k_20_top_p_0p8_repetition_penalty_1p1"

# InferenceStatus (inference.rs:155-169) plus the device-failure code.
OK, STATE, CONTEXT, TOKEN_ID, CAPACITY, ALIGNMENT = 0, 1, 2, 3, 4, 5
NONFINITE_INPUT, NONFINITE_OUTPUT, MODEL, ARITHMETIC, FAULTED = 6, 7, 8, 9, 10
DEVICE = 0x100

FLAG_DRAW_BOUNDARY = 1
FLAG_CUTOFF_BOUNDARY = 2

# Decode-loop row states (pb_row_state) and end-of-sequence ids
# (src/repl_contract.rs:26, crates/promptboot-core/src/tokenizer.rs:38-39).
ROW_ACTIVE, ROW_EOS, ROW_LIMIT, ROW_ERROR = 0, 1, 2, 3
IM_END = 151_645
END_OF_TEXT = 151_643

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libpbsample.so"

u32, u64, size_t, vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_void_p


class _State(ctypes.Structure):
    _fields_ = [("state", u64), ("draws", u64)]


class _Error(ctypes.Structure):
    _fields_ = [
        ("status", u32), ("domain", u32), ("layer", u32), ("position", u32),
        ("tensor_id", u32), ("reserved", u32),
        ("needed", u64), ("available", u64), ("detail", u64),
    ]


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

# name -> (restype, argtypes); every symbol include/pbsample.h declares.
EXPORTS = {
    "pb_sampling_state_new": (None, [ctypes.POINTER(_State), u64]),
    "pb_next_24": (u32, [ctypes.POINTER(_State)]),
    "pb_fill_random_24": (None, [vp, u32, vp]),
    "pb_sample_token_with_repetition": (
        u32, [vp, size_t, vp, size_t, vp, size_t, ctypes.POINTER(_State), vp,
              ctypes.POINTER(_Error)]),
    "pb_sample_token": (u32, [vp, size_t, ctypes.POINTER(_State), vp, ctypes.POINTER(_Error)]),
    "pb_greedy_token": (u32, [vp, size_t, vp, ctypes.POINTER(_Error)]),
    "pb_top_logits_8": (u32, [vp, size_t, vp, ctypes.POINTER(_Error)]),
    "pb_context_create": (u32, [ctypes.c_int, ctypes.POINTER(vp)]),
    "pb_context_destroy": (None, [vp]),
    "pb_sample_batch": (
        u32, [vp, vp, size_t, size_t, u32, vp, size_t, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_sample_batch_inplace": (
        u32, [vp, vp, size_t, size_t, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_segments_for_rows": (u32, [u32]),
    "pb_context_set_segments": (None, [vp, u32]),
    "pb_device_expf_bits": (u32, [vp, vp, size_t, vp]),
    "pb_device_penalize_bits": (u32, [vp, vp, size_t, vp]),
    "pb_device_wave_selftest": (u32, [vp, vp]),
    "pb_device_mfma_selftest": (u32, [vp, vp]),
    "pb_lmhead_packed_bytes": (size_t, [size_t, size_t]),
    "pb_lmhead_pack_q4_0": (u32, [vp, size_t, size_t, vp, vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_sample_batch": (
        u32, [vp, vp, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_decode_step": (
        u32, [vp, vp, size_t, size_t, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_lmhead_decode_step": (
        u32, [vp, vp, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp, vp,
              vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_packed_bytes": (size_t, [size_t, size_t]),
    "pb_lmhead_pack_q8_0": (u32, [vp, size_t, size_t, vp, vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_sample_batch": (
        u32, [vp, vp, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_decode_step": (
        u32, [vp, vp, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp, vp,
              vp, ctypes.POINTER(_Error)]),
    "pb_decode_draw": (None, [vp, vp, u32, vp, vp]),
    "pb_decode_settle": (u32, [vp, vp, vp, vp, u32]),
    "pb_version": (ctypes.c_char_p, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libpbsample.so; raises if it was not built (no fallback path)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`make -C promptboot_amd/csrc` (hipcc, gfx950)")
        # One HIP runtime per process: torch wheels bundle their own
        # libamdhip64 (SONAME libamdhip64.so.7, but requested by torch as
        # "libamdhip64.so").  Loaded first, it satisfies this library's
        # libamdhip64.so.7 dependency as well; loaded after /opt/rocm's copy,
        # torch would map a second runtime that finds no GPU.  So torch, when
        # installed, is imported before the library is opened; torch stream
        # handles are then valid for the sampler's launches.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class InferenceError(Exception):
    """The reference's 48-byte InferenceError (inference.rs:226-264)."""

    def __init__(self, rec):
        self.status = int(rec.status if hasattr(rec, "status") else rec["status"])
        get = (lambda k: int(getattr(rec, k))) if hasattr(rec, "status") else (lambda k: int(rec[k]))
        self.domain, self.layer, self.position = get("domain"), get("layer"), get("position")
        self.tensor_id, self.needed = get("tensor_id"), get("needed")
        self.available, self.detail = get("available"), get("detail")
        super().__init__(f"InferenceError{self.tuple()}")

    def tuple(self) -> list[int]:
        """Same order as the reference tests' inference_error_tuple (tests.rs:185-196)."""
        return [self.status, self.domain, self.layer, self.position, self.tensor_id,
                self.needed, self.available, self.detail]


class SamplingState:
    """xorshift64* with a draw counter (inference.rs:772-810), kept on the host."""

    def __init__(self, seed: int = 0):
        self._s = _State()
        lib().pb_sampling_state_new(ctypes.byref(self._s), seed & (2**64 - 1))

    @classmethod
    def from_parts(cls, state: int, draws: int) -> "SamplingState":
        s = cls.__new__(cls)
        s._s = _State(state, draws)
        return s

    def state(self) -> int:
        return self._s.state

    def draws(self) -> int:
        return self._s.draws

    def next_24(self) -> int:
        return lib().pb_next_24(ctypes.byref(self._s))

    def copy(self) -> "SamplingState":
        return SamplingState.from_parts(self._s.state, self._s.draws)

    def __eq__(self, other) -> bool:
        return (self.state(), self.draws()) == (other.state(), other.draws())

    def __repr__(self) -> str:
        return f"SamplingState(state={self.state():#018x}, draws={self.draws()})"


def _words(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float32:
        a = a.view(np.uint32)
    return np.ascontiguousarray(a, dtype=np.uint32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(vp)


def _check(status: int, err: _Error):
    if status != OK:
        raise InferenceError(err)


def sample_token_with_repetition(logits: np.ndarray, tokens, seen: np.ndarray,
                                 state: SamplingState) -> int:
    """Penalises `logits` in place once per unique history id, then draws.

    `logits` must be a writable C-contiguous uint32 (or float32) array; `seen`
    a writable uint8 scratch of at least SEEN_BYTES that is zero on entry."""
    if logits.dtype == np.float32:
        logits = logits.view(np.uint32)
    assert logits.dtype == np.uint32 and logits.flags.c_contiguous and logits.flags.writeable
    assert seen.dtype == np.uint8 and seen.flags.c_contiguous
    t = _words(tokens)
    out = np.zeros(1, np.uint32)
    err = _Error()
    st = lib().pb_sample_token_with_repetition(
        _ptr(logits), logits.size, _ptr(t), t.size, _ptr(seen), seen.size,
        ctypes.byref(state._s), _ptr(out), ctypes.byref(err))
    _check(st, err)
    return int(out[0])


def sample_token(logits, state: SamplingState) -> int:
    row = _words(logits)
    out = np.zeros(1, np.uint32)
    err = _Error()
    st = lib().pb_sample_token(_ptr(row), row.size, ctypes.byref(state._s), _ptr(out),
                               ctypes.byref(err))
    _check(st, err)
    return int(out[0])


def greedy_token(logits) -> int:
    row = _words(logits)
    out = np.zeros(1, np.uint32)
    err = _Error()
    st = lib().pb_greedy_token(_ptr(row), row.size, _ptr(out), ctypes.byref(err))
    _check(st, err)
    return int(out[0])


def top_logits_8(logits, output: np.ndarray | None = None) -> np.ndarray:
    """Returns (and fills) a uint32 [8, 2] array of (token, logit_bits);
    `output` is left untouched on error, as in the reference."""
    row = _words(logits)
    if output is None:
        output = np.zeros((8, 2), np.uint32)
    assert output.dtype == np.uint32 and output.size == 16 and output.flags.c_contiguous
    err = _Error()
    st = lib().pb_top_logits_8(_ptr(row), row.size, _ptr(output), ctypes.byref(err))
    _check(st, err)
    return output


def fill_random_24(states: list[SamplingState]) -> np.ndarray:
    """One next_24 per row from the rows' own generators (host)."""
    return np.array([s.next_24() for s in states], np.uint32)


class BatchSampler:
    """Batched device sampling on one GPU (pb_context).

    Tensors are torch CUDA tensors (int32/uint32-compatible words):
    logits [B, ld] (float32 or int32 view), history [B, hist_ld] int32,
    history lengths [B] int32, uniforms [B] int32."""

    def __init__(self, device: int = -1, segments: int = 0):
        self._ctx = vp()
        st = lib().pb_context_create(device, ctypes.byref(self._ctx))
        if st != OK:
            raise InferenceError(_Error(status=st))
        self.segments = segments
        if segments:
            lib().pb_context_set_segments(self._ctx, segments)

    def close(self):
        if self._ctx:
            lib().pb_context_destroy(self._ctx)
            self._ctx = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_segments(self, segments: int) -> None:
        self.segments = segments
        lib().pb_context_set_segments(self._ctx, segments)

    def sample(self, logits, random_24, history=None, history_len=None, *, token=None,
               detail=None, err=None, inplace=False, seen=None, stream=None) -> None:
        """Enqueues one batched sample; outputs are preallocated torch tensors:
        token [B] int32, detail [B, 84] int32 (DETAIL_DTYPE), err [B, 12] int32."""
        import torch

        rows, ld = logits.shape
        hist_ld = history.shape[1] if history is not None else 0
        s = stream if stream is not None else torch.cuda.current_stream(logits.device)
        e = _Error()

        def p(t):
            return None if t is None else ctypes.c_void_p(t.data_ptr())

        if inplace:
            st = lib().pb_sample_batch_inplace(
                self._ctx, p(logits), VOCAB, ld, rows, p(history), hist_ld, p(history_len),
                p(random_24), p(seen), p(token), p(detail), p(err),
                ctypes.c_void_p(s.cuda_stream), ctypes.byref(e))
        else:
            st = lib().pb_sample_batch(
                self._ctx, p(logits), VOCAB, ld, rows, p(history), hist_ld, p(history_len),
                p(random_24), p(token), p(detail), p(err), ctypes.c_void_p(s.cuda_stream),
                ctypes.byref(e))
        _check(st, e)

    def pack_lmhead(self, weights, vocab: int = VOCAB, cols: int = 896, stream=None,
                    q8: bool = False):
        """Repacks a Q4_0 head (or, with q8, a Q8_0 head) given as a torch uint8
        device tensor in promptboot's layout into the device layout; returns
        the packed uint8 tensor."""
        import torch

        nbytes = (lib().pb_lmhead_q8_packed_bytes if q8 else lib().pb_lmhead_packed_bytes)(
            vocab, cols)
        packed = torch.empty(nbytes, dtype=torch.uint8, device=weights.device)
        s = stream if stream is not None else torch.cuda.current_stream(weights.device)
        e = _Error()
        pack = lib().pb_lmhead_pack_q8_0 if q8 else lib().pb_lmhead_pack_q4_0
        st = pack(ctypes.c_void_p(weights.data_ptr()), vocab, cols,
                  ctypes.c_void_p(packed.data_ptr()), ctypes.c_void_p(s.cuda_stream),
                  ctypes.byref(e))
        _check(st, e)
        return packed

    def lmhead_sample(self, packed, hidden, random_24, history=None, history_len=None, *,
                      token, detail=None, err=None, logits=None, cols: int = 896,
                      stream=None, q8: bool = False) -> None:
        """Enqueues the fused Q4_0 (or, with q8, Q8_0) LM head + sampler for
        hidden [B, cols]; `packed` comes from pack_lmhead with the same q8."""
        import torch

        rows = hidden.shape[0]
        hist_ld = history.shape[1] if history is not None else 0
        s = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        e = _Error()

        def p(t):
            return None if t is None else ctypes.c_void_p(t.data_ptr())

        fn = lib().pb_lmhead_q8_sample_batch if q8 else lib().pb_lmhead_sample_batch
        st = fn(
            self._ctx, p(packed), VOCAB, cols, p(hidden), rows, p(history), hist_ld,
            p(history_len), p(random_24), p(token), p(detail), p(err), p(logits),
            ctypes.c_void_p(s.cuda_stream), ctypes.byref(e))
        _check(st, e)

    def sample_rows(self, logits, history, history_len, states: list[SamplingState],
                    want_detail: bool = True):
        """Host-driven batch like calling sample_token_with_repetition per row
        without the in-place write-back: one draw per row from that row's own
        state; failing rows keep their state (transactional).  Returns numpy
        (tokens, detail or None, errors)."""
        import torch

        rows = logits.shape[0]
        before = [s.copy() for s in states]
        r24 = torch.from_numpy(fill_random_24(states).view(np.int32)).to(logits.device)
        token = torch.empty(rows, dtype=torch.int32, device=logits.device)
        det = (torch.empty((rows, DETAIL_DTYPE.itemsize // 4), dtype=torch.int32,
                           device=logits.device) if want_detail else None)
        err = torch.empty((rows, ERROR_DTYPE.itemsize // 4), dtype=torch.int32,
                          device=logits.device)
        self.sample(logits, r24, history, history_len, token=token, detail=det, err=err)
        torch.cuda.synchronize(logits.device)
        tok = token.cpu().numpy().view(np.uint32)
        errs = err.cpu().numpy().view(ERROR_DTYPE).reshape(rows)
        for r in np.flatnonzero(errs["status"] != OK):
            states[r]._s = before[r]._s
        dets = det.cpu().numpy().view(DETAIL_DTYPE).reshape(rows) if want_detail else None
        return tok, dets, errs


class DecodeBatch:
    """Many sequences through the REPL's decode loop (src/model_repl.rs:928-1150),
    one device launch per step.

    Each row owns a working context (prompt, then every generated token; an
    end-of-sequence piece is stored as IM_END), a length cap (prompt length +
    generation limit) and its own SamplingState, advanced once per sampled
    token and never for a failed sample.  The contexts, lengths and row states
    stay on the device; the host keeps the generators (pb_decode_draw /
    pb_decode_settle)."""

    def __init__(self, prompts, seeds, limits, capacity: int | None = None, device: int = 0,
                 sampler: "BatchSampler | None" = None):
        import torch

        self.rows = len(prompts)
        self.dev = torch.device(f"cuda:{device}")
        cap = max(len(p) + int(g) for p, g in zip(prompts, limits))
        self.hist_ld = int(capacity) if capacity is not None else (cap + 3) // 4 * 4
        hist = np.zeros((self.rows, self.hist_ld), np.uint32)
        for r, p in enumerate(prompts):
            hist[r, :len(p)] = np.asarray(p, np.uint32)
        lens = np.array([len(p) for p in prompts], np.uint32)
        max_len = np.minimum(lens + np.asarray(limits, np.uint32), self.hist_ld).astype(np.uint32)

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(self.dev)

        self.hist, self.hist_len, self.max_len = dev(hist), dev(lens), dev(max_len)
        self.row_state_host = np.where(lens < max_len, ROW_ACTIVE, ROW_LIMIT).astype(np.uint32)
        self.row_state = dev(self.row_state_host)
        self.states = (_State * self.rows)()
        for r, seed in enumerate(seeds):
            lib().pb_sampling_state_new(ctypes.byref(self.states[r]), int(seed) & (2**64 - 1))
        self._saved = (_State * self.rows)()
        self.token = torch.empty(self.rows, dtype=torch.int32, device=self.dev)
        self.err = torch.empty((self.rows, ERROR_DTYPE.itemsize // 4), dtype=torch.int32,
                               device=self.dev)
        self._own = sampler is None
        self.sampler = sampler if sampler is not None else BatchSampler(device)

    def close(self):
        if self._own and self.sampler is not None:
            self.sampler.close()
        self.sampler = None

    def active(self) -> bool:
        return bool((self.row_state_host == ROW_ACTIVE).any())

    def _draw(self):
        import torch

        r24 = np.zeros(self.rows, np.uint32)
        before = self.row_state_host.copy()
        lib().pb_decode_draw(self.states, before.ctypes.data_as(vp), self.rows,
                             r24.ctypes.data_as(vp), self._saved)
        return before, torch.from_numpy(r24.view(np.int32)).to(self.dev)

    def _settle(self, before):
        import torch

        torch.cuda.synchronize(self.dev)
        after = self.row_state.cpu().numpy().view(np.uint32).copy()
        lib().pb_decode_settle(self.states, self._saved, before.ctypes.data_as(vp),
                               after.ctypes.data_as(vp), self.rows)
        self.row_state_host = after
        return self.token.cpu().numpy().view(np.uint32).copy()

    def step(self, logits, stream=None) -> np.ndarray:
        """One step on logits [rows, ld] (rows that have ended are ignored).
        Returns the tokens (NO_TOKEN for rows not sampled)."""
        import torch

        before, r24 = self._draw()
        s = stream if stream is not None else torch.cuda.current_stream(self.dev)
        e = _Error()
        st = lib().pb_decode_step(
            self.sampler._ctx, ctypes.c_void_p(logits.data_ptr()), VOCAB, logits.shape[1],
            self.rows, ctypes.c_void_p(self.hist.data_ptr()), self.hist_ld,
            ctypes.c_void_p(self.hist_len.data_ptr()), ctypes.c_void_p(self.max_len.data_ptr()),
            ctypes.c_void_p(self.row_state.data_ptr()), ctypes.c_void_p(r24.data_ptr()),
            ctypes.c_void_p(self.token.data_ptr()), None, ctypes.c_void_p(self.err.data_ptr()),
            ctypes.c_void_p(s.cuda_stream), ctypes.byref(e))
        _check(st, e)
        return self._settle(before)

    def lmhead_step(self, packed, hidden, cols: int = 896, stream=None,
                    q8: bool = False) -> np.ndarray:
        """One step through the fused Q4_0 (or, with q8, Q8_0) LM head on
        hidden [rows, cols]."""
        import torch

        before, r24 = self._draw()
        s = stream if stream is not None else torch.cuda.current_stream(self.dev)
        e = _Error()
        fn = lib().pb_lmhead_q8_decode_step if q8 else lib().pb_lmhead_decode_step
        st = fn(
            self.sampler._ctx, ctypes.c_void_p(packed.data_ptr()), VOCAB, cols,
            ctypes.c_void_p(hidden.data_ptr()), self.rows,
            ctypes.c_void_p(self.hist.data_ptr()), self.hist_ld,
            ctypes.c_void_p(self.hist_len.data_ptr()), ctypes.c_void_p(self.max_len.data_ptr()),
            ctypes.c_void_p(self.row_state.data_ptr()), ctypes.c_void_p(r24.data_ptr()),
            ctypes.c_void_p(self.token.data_ptr()), None, ctypes.c_void_p(self.err.data_ptr()),
            None, ctypes.c_void_p(s.cuda_stream), ctypes.byref(e))
        _check(st, e)
        return self._settle(before)

    def contexts(self) -> list[np.ndarray]:
        h = self.hist.cpu().numpy().view(np.uint32)
        n = self.hist_len.cpu().numpy().view(np.uint32)
        return [h[r, :n[r]].copy() for r in range(self.rows)]

    def errors(self) -> np.ndarray:
        return self.err.cpu().numpy().view(ERROR_DTYPE).reshape(self.rows)

    def sampling_states(self) -> list[SamplingState]:
        return [SamplingState.from_parts(s.state, s.draws) for s in self.states]


def device_expf_bits(inp, out, stream=None) -> None:
    """Runs the sampler's device expf on a torch CUDA int32 tensor (verification hook)."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream(inp.device)
    st = lib().pb_device_expf_bits(ctypes.c_void_p(inp.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                   inp.numel(), ctypes.c_void_p(s.cuda_stream))
    if st != OK:
        raise RuntimeError("pb_device_expf_bits failed")


def device_penalize_bits(inp, out, stream=None) -> None:
    """Runs the sampler's device repetition penalty of single logits (verification hook)."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream(inp.device)
    st = lib().pb_device_penalize_bits(ctypes.c_void_p(inp.data_ptr()),
                                       ctypes.c_void_p(out.data_ptr()), inp.numel(),
                                       ctypes.c_void_p(s.cuda_stream))
    if st != OK:
        raise RuntimeError("pb_device_penalize_bits failed")
