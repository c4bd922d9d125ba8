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

`BatchSampler` and `DecodeBatch` drive the batched device entry points on
device buffers: `promptboot_amd.hip.DeviceArray`, raw device pointers, or any
array object with `data_ptr()` and a shape (tensors of another framework
that shares this process's HIP runtime).  Streams are hipStream_t handles
(`hip.Stream`, an int, or an object with `cuda_stream`); None is the null
stream.

All selection arithmetic runs in the HIP kernels; if the library is missing
the import fails.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

from . import hip

VOCAB = 151_936
TILE_SELECT_ROWS = 192  # PB_TILE_SELECT_ROWS: batches up to it take the tile selection
LMHEAD_MAX_ROWS = 262_144  # PB_LMHEAD_MAX_ROWS: largest batch of one LM-head call
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
    "pb_context_reserve": (u32, [vp, u32, size_t, ctypes.POINTER(_Error)]),
    "pb_sample_batch": (
        u32, [vp, vp, size_t, size_t, u32, vp, size_t, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_sample_batch_noalloc": (
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
    "pb_device_read_probe": (u32, [vp, size_t, vp, u32, vp]),
    "pb_device_read_probe_grid_stride": (u32, [vp, size_t, vp, u32, vp]),
    "pb_device_mfma_selftest": (u32, [vp, vp]),
    "pb_lmhead_packed_bytes": (size_t, [size_t, size_t]),
    "pb_lmhead_pack_q4_0": (u32, [vp, size_t, size_t, vp, vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_sample_batch": (
        u32, [vp, vp, size_t, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_decode_step": (
        u32, [vp, vp, size_t, size_t, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_lmhead_decode_step": (
        u32, [vp, vp, size_t, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              vp, vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_packed_bytes": (size_t, [size_t, size_t]),
    "pb_lmhead_pack_q8_0": (u32, [vp, size_t, size_t, vp, vp, ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_sample_batch": (
        u32, [vp, vp, size_t, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              ctypes.POINTER(_Error)]),
    "pb_lmhead_q8_decode_step": (
        u32, [vp, vp, size_t, size_t, size_t, vp, u32, vp, size_t, vp, vp, vp, vp, vp, vp, vp,
              vp, vp, ctypes.POINTER(_Error)]),
    "pb_decode_draw": (None, [vp, vp, u32, vp, vp]),
    "pb_decode_settle": (u32, [vp, vp, vp, vp, u32]),
    "pb_version": (ctypes.c_char_p, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libpbsample.so; raises if it was not built (no fallback path).

    The library links the HIP runtime by SONAME (libamdhip64.so.7); when the
    process already mapped a runtime of that name, the library shares it."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`make -C promptboot_amd/csrc` (hipcc, gfx950)")
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
    # the address as an int (the void* parameters take it): the cheapest of
    # numpy's routes, about 1 us against 2 us for ctypes.data_as
    return None if a is None else a.ctypes.data


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
    out = u32()
    err = _Error()
    st = lib().pb_sample_token_with_repetition(
        _ptr(logits), logits.size, _ptr(t), t.size, _ptr(seen), seen.size,
        ctypes.byref(state._s), ctypes.byref(out), ctypes.byref(err))
    _check(st, err)
    return out.value


def sample_token(logits, state: SamplingState) -> int:
    row = _words(logits)
    out = u32()
    err = _Error()
    st = lib().pb_sample_token(_ptr(row), row.size, ctypes.byref(state._s), ctypes.byref(out),
                               ctypes.byref(err))
    _check(st, err)
    return out.value


def greedy_token(logits) -> int:
    row = _words(logits)
    out = u32()
    err = _Error()
    st = lib().pb_greedy_token(_ptr(row), row.size, ctypes.byref(out), ctypes.byref(err))
    _check(st, err)
    return out.value


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
    return np.array([st.next_24() for st in states], np.uint32)


# ---- device buffers handed to the batched entry points ----

def _shape(x) -> tuple:
    return tuple(int(d) for d in x.shape)


def _itemsize(x) -> int:
    return int(x.element_size()) if hasattr(x, "element_size") else int(x.dtype.itemsize)


def _dev(x, name: str, *, itemsize: int = 4, rows: int | None = None,
         row_elems: int | None = None, ndim: int | None = None):
    """The device pointer of `x` (None stays None).  Array objects are checked:
    C-contiguous, `itemsize`-byte elements, `ndim` dimensions when given, and
    at least rows x row_elems elements.  A raw int pointer is taken as is."""
    if x is None:
        return None
    if isinstance(x, int):
        return vp(x)
    if hasattr(x, "is_contiguous") and not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if _itemsize(x) != itemsize:
        raise ValueError(f"{name} must have {itemsize}-byte elements, not {_itemsize(x)}")
    shape = _shape(x)
    if ndim is not None and len(shape) != ndim:
        raise ValueError(f"{name} must have {ndim} dimensions, has shape {shape}")
    if rows is not None:
        need = rows * (row_elems if row_elems is not None else 1)
        have = int(np.prod(shape, dtype=np.int64))
        if have < need:
            raise ValueError(f"{name} holds {have} elements, {need} needed for {rows} rows")
    return vp(x.data_ptr())


def _nbytes(x) -> int:
    return int(np.prod(_shape(x), dtype=np.int64)) * _itemsize(x)


class BatchSampler:
    """Batched device sampling on one GPU (pb_context).

    Device buffers hold 32-bit words: logits [B, ld] (binary32 bit patterns),
    history [B, hist_ld], history lengths [B], uniforms [B]; outputs token
    [B], detail [B, 84] (DETAIL_DTYPE), err [B, 12] (ERROR_DTYPE).  The
    context's workspace is reserved (pb_context_reserve) before any call
    that needs more, so the enqueue calls themselves never allocate."""

    def __init__(self, device: int = -1, segments: int = 0):
        self._ctx = vp()
        st = lib().pb_context_create(device, ctypes.byref(self._ctx))
        if st != OK:
            raise InferenceError(_Error(status=st))
        self.segments = 0
        self._rows = 0          # rows reserved under the current slice plan
        self._lm = (0, 0)       # (rows, cols) reserved for the LM head
        if segments:
            self.set_segments(segments)

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
        self._rows = 0

    def reserve(self, rows: int, cols: int = 0) -> None:
        """Sizes the context for batches of up to `rows` rows (and the LM head
        for up to `cols` columns); a set-up call, it may allocate."""
        e = _Error()
        _check(lib().pb_context_reserve(self._ctx, rows, cols, ctypes.byref(e)), e)
        self._rows = max(self._rows, rows)
        if cols:
            self._lm = (max(self._lm[0], rows), max(self._lm[1], cols))

    def _ensure(self, rows: int, cols: int = 0) -> None:
        if self.segments and rows > self._rows:
            self.reserve(rows)
        if cols and (rows > self._lm[0] or cols > self._lm[1]):
            self.reserve(max(rows, self._lm[0]), max(cols, self._lm[1]))

    def sample(self, logits, random_24, history=None, history_len=None, *, token=None,
               detail=None, err=None, inplace=False, seen=None, stream=None) -> None:
        """Enqueues one batched sample on `stream`."""
        rows, ld = _shape(logits)
        hist_ld = _shape(history)[1] if history is not None else 0
        self._ensure(rows)
        args = dict(rows=rows)
        ptrs = [_dev(logits, "logits", ndim=2), _dev(history, "history", ndim=2, **args),
                _dev(history_len, "history_len", **args), _dev(random_24, "random_24", **args)]
        outs = [_dev(token, "token", **args), _dev(detail, "detail", row_elems=84, **args),
                _dev(err, "err", row_elems=12, **args)]
        e = _Error()
        s = vp(hip.stream_handle(stream))
        if inplace:
            st = lib().pb_sample_batch_inplace(
                self._ctx, ptrs[0], VOCAB, ld, rows, ptrs[1], hist_ld, ptrs[2], ptrs[3],
                _dev(seen, "seen", itemsize=1, rows=rows, row_elems=SEEN_BYTES), *outs, s,
                ctypes.byref(e))
        else:
            st = lib().pb_sample_batch(self._ctx, ptrs[0], VOCAB, ld, rows, ptrs[1], hist_ld,
                                       ptrs[2], ptrs[3], *outs, s, ctypes.byref(e))
        _check(st, e)

    def bind_sample(self, logits, random_24, history=None, history_len=None, *, token=None,
                    detail=None, err=None, stream=None):
        """A zero-argument callable that enqueues this exact pb_sample_batch
        call: the arguments are checked and converted once, so each call
        costs one foreign call, as it does a C caller (for timing loops)."""
        rows, ld = _shape(logits)
        hist_ld = _shape(history)[1] if history is not None else 0
        self._ensure(rows)
        args = dict(rows=rows)
        argv = (self._ctx, _dev(logits, "logits", ndim=2), VOCAB, ld, rows,
                _dev(history, "history", ndim=2, **args), hist_ld,
                _dev(history_len, "history_len", **args), _dev(random_24, "random_24", **args),
                _dev(token, "token", **args), _dev(detail, "detail", row_elems=84, **args),
                _dev(err, "err", row_elems=12, **args), vp(hip.stream_handle(stream)))
        fn = lib().pb_sample_batch

        def call():
            e = _Error()
            st = fn(*argv, ctypes.byref(e))
            if st != OK:
                raise InferenceError(e)

        return call

    def bind_lmhead(self, packed, hidden, random_24, history=None, history_len=None, *,
                    token, detail=None, err=None, logits=None, stream=None, q8: bool = False):
        """bind_sample for the fused LM head + sampler (lmhead_sample)."""
        rows, width, nbytes = self._head_args(packed, hidden, None, q8)
        self._ensure(rows, width)
        hist_ld = _shape(history)[1] if history is not None else 0
        args = dict(rows=rows)
        argv = (self._ctx, _dev(packed, "packed", itemsize=1), nbytes, VOCAB, width,
                _dev(hidden, "hidden", ndim=2), rows, _dev(history, "history", ndim=2, **args),
                hist_ld, _dev(history_len, "history_len", **args),
                _dev(random_24, "random_24", **args), _dev(token, "token", **args),
                _dev(detail, "detail", row_elems=84, **args),
                _dev(err, "err", row_elems=12, **args),
                _dev(logits, "logits", row_elems=VOCAB, **args), vp(hip.stream_handle(stream)))
        fn = lib().pb_lmhead_q8_sample_batch if q8 else lib().pb_lmhead_sample_batch

        def call():
            e = _Error()
            st = fn(*argv, ctypes.byref(e))
            if st != OK:
                raise InferenceError(e)

        return call

    def pack_lmhead(self, weights, vocab: int = VOCAB, cols: int = 896, stream=None,
                    q8: bool = False) -> hip.DeviceArray:
        """Repacks a Q4_0 head (or, with q8, a Q8_0 head) held on the device in
        promptboot's layout into the device layout; returns the packed bytes."""
        src = vocab * (cols // 32) * (34 if q8 else 18)
        if _nbytes(weights) != src:
            raise ValueError(f"a {'Q8_0' if q8 else 'Q4_0'} head of {vocab} x {cols} is "
                             f"{src} bytes, not {_nbytes(weights)}")
        nbytes = (lib().pb_lmhead_q8_packed_bytes if q8 else lib().pb_lmhead_packed_bytes)(
            vocab, cols)
        packed = hip.DeviceArray(nbytes, np.uint8)
        e = _Error()
        pack = lib().pb_lmhead_pack_q8_0 if q8 else lib().pb_lmhead_pack_q4_0
        st = pack(_dev(weights, "weights", itemsize=_itemsize(weights)), vocab, cols,
                  vp(packed.data_ptr()), vp(hip.stream_handle(stream)), ctypes.byref(e))
        _check(st, e)
        return packed

    @staticmethod
    def _head_args(packed, hidden, cols, q8):
        rows, width = _shape(hidden)
        if cols is not None and cols != width:
            raise ValueError(f"cols={cols} but the hidden states have {width} columns")
        nbytes = (lib().pb_lmhead_q8_packed_bytes if q8 else lib().pb_lmhead_packed_bytes)(
            VOCAB, width)
        if _nbytes(packed) != nbytes:
            raise ValueError(f"the packed head holds {_nbytes(packed)} bytes; a "
                             f"{'Q8_0' if q8 else 'Q4_0'} head of width {width} holds {nbytes}")
        return rows, width, nbytes

    def lmhead_sample(self, packed, hidden, random_24, history=None, history_len=None, *,
                      token, detail=None, err=None, logits=None, cols: int | None = None,
                      stream=None, q8: bool = False) -> None:
        """Enqueues the fused Q4_0 (or, with q8, Q8_0) LM head + sampler for
        hidden [B, cols]; `packed` comes from pack_lmhead with the same q8."""
        rows, width, nbytes = self._head_args(packed, hidden, cols, q8)
        self._ensure(rows, width)
        hist_ld = _shape(history)[1] if history is not None else 0
        args = dict(rows=rows)
        fn = lib().pb_lmhead_q8_sample_batch if q8 else lib().pb_lmhead_sample_batch
        e = _Error()
        st = fn(self._ctx, _dev(packed, "packed", itemsize=1), nbytes, VOCAB, width,
                _dev(hidden, "hidden", ndim=2), rows, _dev(history, "history", ndim=2, **args),
                hist_ld, _dev(history_len, "history_len", **args),
                _dev(random_24, "random_24", **args), _dev(token, "token", **args),
                _dev(detail, "detail", row_elems=84, **args),
                _dev(err, "err", row_elems=12, **args),
                _dev(logits, "logits", row_elems=VOCAB, **args), vp(hip.stream_handle(stream)),
                ctypes.byref(e))
        _check(st, e)

    def sample_rows(self, logits, history, history_len, states: list[SamplingState],
                    want_detail: bool = True):
        """Host-driven batch like calling sample_token_with_repetition per row
        without the in-place write-back: one draw per row from that row's own
        state; failing rows keep their state (transactional).  Returns numpy
        (tokens, detail or None, errors)."""
        rows = _shape(logits)[0]
        before = [st.copy() for st in states]
        r24 = hip.DeviceArray.from_numpy(fill_random_24(states))
        token = hip.DeviceArray(rows, np.uint32)
        det = hip.DeviceArray((rows, DETAIL_DTYPE.itemsize // 4), np.uint32) if want_detail else None
        err = hip.DeviceArray((rows, ERROR_DTYPE.itemsize // 4), np.uint32)
        try:
            self.sample(logits, r24, history, history_len, token=token, detail=det, err=err)
        except Exception:
            for r in range(rows):
                states[r]._s = before[r]._s
            raise
        tok = token.numpy()
        errs = err.numpy().view(ERROR_DTYPE).reshape(rows)
        for r in np.flatnonzero(errs["status"] != OK):
            states[r]._s = before[r]._s
        dets = det.numpy().view(DETAIL_DTYPE).reshape(rows) if want_detail else None
        return tok, dets, errs


class DecodeBatch:
    """Many sequences through the REPL's decode loop (src/model_repl.rs:928-1150),
    one device launch per step.

    Each row owns a working context (prompt, then every generated token; an
    end-of-sequence piece is stored as IM_END), a length cap (prompt length +
    generation limit) and its own SamplingState, advanced once per sampled
    token and never for a failed sample or a row already at its cap.  The
    contexts, lengths and row states stay on the device; the host keeps the
    generators (pb_decode_draw / pb_decode_settle)."""

    def __init__(self, prompts, seeds, limits, capacity: int | None = None, device: int = 0,
                 sampler: "BatchSampler | None" = None):
        self.rows = len(prompts)
        cap = max(len(p) + int(g) for p, g in zip(prompts, limits))
        self.hist_ld = int(capacity) if capacity is not None else (cap + 3) // 4 * 4
        hist = np.zeros((self.rows, self.hist_ld), np.uint32)
        for r, p in enumerate(prompts):
            hist[r, :len(p)] = np.asarray(p, np.uint32)
        lens = np.array([len(p) for p in prompts], np.uint32)
        max_len = np.minimum(lens + np.asarray(limits, np.uint32), self.hist_ld).astype(np.uint32)
        self._own = sampler is None
        self.sampler = sampler if sampler is not None else BatchSampler(device)
        dev = hip.DeviceArray.from_numpy
        self.hist, self.hist_len, self.max_len = dev(hist), dev(lens), dev(max_len)
        self.row_state_host = np.where(lens < max_len, ROW_ACTIVE, ROW_LIMIT).astype(np.uint32)
        self.row_state = dev(self.row_state_host)
        self.states = (_State * self.rows)()
        for r, seed in enumerate(seeds):
            lib().pb_sampling_state_new(ctypes.byref(self.states[r]), int(seed) & (2**64 - 1))
        self._saved = (_State * self.rows)()
        self.r24 = hip.DeviceArray(self.rows, np.uint32)
        self.token = hip.DeviceArray(self.rows, np.uint32)
        self.err = hip.DeviceArray((self.rows, ERROR_DTYPE.itemsize // 4), np.uint32)

    def close(self):
        if self._own and self.sampler is not None:
            self.sampler.close()
        self.sampler = None

    def active(self) -> bool:
        return bool((self.row_state_host == ROW_ACTIVE).any())

    def _draw(self):
        r24 = np.zeros(self.rows, np.uint32)
        before = self.row_state_host.copy()
        lib().pb_decode_draw(self.states, before.ctypes.data_as(vp), self.rows,
                             r24.ctypes.data_as(vp), self._saved)
        self.r24.upload(r24)
        return before

    def _undraw(self):
        for r in range(self.rows):
            self.states[r] = self._saved[r]

    def _settle(self, before):
        after = self.row_state.numpy()
        tokens = self.token.numpy()
        lib().pb_decode_settle(self.states, self._saved, before.ctypes.data_as(vp),
                               tokens.ctypes.data_as(vp), self.rows)
        self.row_state_host = after
        return tokens.copy()

    def _ptrs(self):
        return (vp(self.hist.data_ptr()), self.hist_ld, vp(self.hist_len.data_ptr()),
                vp(self.max_len.data_ptr()), vp(self.row_state.data_ptr()),
                vp(self.r24.data_ptr()), vp(self.token.data_ptr()), None,
                vp(self.err.data_ptr()))

    def step(self, logits, stream=None) -> np.ndarray:
        """One step on logits [rows, ld] (rows that have ended are ignored).
        Returns the tokens (NO_TOKEN for rows not sampled).  A refused step
        leaves every SamplingState as it was."""
        rows, ld = _shape(logits)
        if rows != self.rows:
            raise ValueError(f"logits have {rows} rows, the batch has {self.rows}")
        lp = _dev(logits, "logits", ndim=2)
        before = self._draw()
        e = _Error()
        try:
            st = lib().pb_decode_step(self.sampler._ctx, lp, VOCAB, ld, self.rows, *self._ptrs(),
                                      vp(hip.stream_handle(stream)), ctypes.byref(e))
            _check(st, e)
        except Exception:
            self._undraw()
            raise
        return self._settle(before)

    def lmhead_step(self, packed, hidden, cols: int | None = None, stream=None,
                    q8: bool = False) -> np.ndarray:
        """One step through the fused Q4_0 (or, with q8, Q8_0) LM head on
        hidden [rows, cols]."""
        rows, width, nbytes = BatchSampler._head_args(packed, hidden, cols, q8)
        if rows != self.rows:
            raise ValueError(f"hidden has {rows} rows, the batch has {self.rows}")
        self.sampler._ensure(rows, width)
        pp, hp = _dev(packed, "packed", itemsize=1), _dev(hidden, "hidden", ndim=2)
        before = self._draw()
        fn = lib().pb_lmhead_q8_decode_step if q8 else lib().pb_lmhead_decode_step
        e = _Error()
        try:
            p = self._ptrs()
            st = fn(self.sampler._ctx, pp, nbytes, VOCAB, width, hp, self.rows, *p, None,
                    vp(hip.stream_handle(stream)), ctypes.byref(e))
            _check(st, e)
        except Exception:
            self._undraw()
            raise
        return self._settle(before)

    def contexts(self) -> list[np.ndarray]:
        h = self.hist.numpy()
        n = self.hist_len.numpy()
        return [h[r, :n[r]].copy() for r in range(self.rows)]

    def errors(self) -> np.ndarray:
        return self.err.numpy().view(ERROR_DTYPE).reshape(self.rows)

    def sampling_states(self) -> list[SamplingState]:
        return [SamplingState.from_parts(st.state, st.draws) for st in self.states]


def device_expf_bits(inp, out, stream=None) -> None:
    """Runs the sampler's device expf on device words (verification hook)."""
    n = int(np.prod(_shape(inp), dtype=np.int64))
    st = lib().pb_device_expf_bits(_dev(inp, "inp"), _dev(out, "out", rows=n), n,
                                   vp(hip.stream_handle(stream)))
    if st != OK:
        raise RuntimeError("pb_device_expf_bits failed")


def device_penalize_bits(inp, out, stream=None) -> None:
    """Runs the sampler's device repetition penalty of single logits (verification hook)."""
    n = int(np.prod(_shape(inp), dtype=np.int64))
    st = lib().pb_device_penalize_bits(_dev(inp, "inp"), _dev(out, "out", rows=n), n,
                                       vp(hip.stream_handle(stream)))
    if st != OK:
        raise RuntimeError("pb_device_penalize_bits failed")
