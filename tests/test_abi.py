"""C ABI checks that need no GPU: the library loads, exports every function
include/pbsample.h declares, the Python binding covers exactly those, the
structs have the reference's repr(C) layouts (inference.rs:226-291), and the
host-only parts (PRNG, length validation) behave like the reference."""
import pathlib
import re
import subprocess

import numpy as np
import pytest

from promptboot_amd import sampler as s
from tests.conftest import ROOT

HEADER = ROOT / "include" / "pbsample.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(pb_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 16
    out = subprocess.run(["nm", "-D", "--defined-only", str(s.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (pb_[a-z0-9_]+)$", out, flags=re.M))
    assert names <= exported, names - exported
    assert exported <= names, exported - names
    assert set(s.EXPORTS) == names
    lib = s.lib()
    for n in names:
        assert getattr(lib, n) is not None


def test_header_constants_match_the_binding():
    """Every numeric #define of the header that the binding mirrors has the
    same value there."""
    defines = {m[0]: int(m[1], 0) for m in
               re.findall(r"^#define PB_([A-Z0-9_]+) (0x[0-9a-fA-F]+|[0-9]+)u", HEADER.read_text(),
                          flags=re.M)}
    mirrored = {k: getattr(s, k) for k in defines if hasattr(s, k)}
    assert {"VOCAB", "TOP_K", "TILE_SELECT_ROWS", "LMHEAD_MAX_ROWS", "IM_END",
            "END_OF_TEXT"} <= set(mirrored)
    assert mirrored == {k: defines[k] for k in mirrored}


def test_one_hip_runtime_is_mapped():
    """The binding opens the library after torch, so torch's bundled
    libamdhip64 serves both and the process holds a single HIP runtime."""
    s.lib()
    maps = pathlib.Path("/proc/self/maps").read_text().splitlines()
    paths = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(paths) == 1, paths


def test_struct_layouts_match_the_reference(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text("""
#include <stddef.h>
#include <stdio.h>
#include "pbsample.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(pb_inference_error),
         _Alignof(pb_inference_error), offsetof(pb_inference_error, needed),
         offsetof(pb_inference_error, detail), sizeof(pb_sampling_state),
         sizeof(pb_top_logit), sizeof(pb_sample_detail),
         offsetof(pb_sample_detail, kept), offsetof(pb_sample_detail, probs));
  return 0;
}
""")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{HEADER.parent}", str(src), "-o",
                    str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                           text=True).stdout.split()]
    # InferenceError: 48 bytes, align 8, needed at 24 (inference.rs:226-237, 287-288)
    assert vals[:4] == [48, 8, 24, 40]
    assert vals[4:6] == [16, 8]
    assert vals[6:] == [s.DETAIL_DTYPE.itemsize, s.DETAIL_DTYPE.fields["kept"][1],
                        s.DETAIL_DTYPE.fields["probs"][1]]


def test_host_prng_matches_reference_states(known):
    p = known["unit"]["prng"]
    st = s.SamplingState(p["seed"])
    for _ in range(8):
        st.next_24()
    assert (st.state(), st.draws()) == (p["state_after"], 8)
    e = known["exact_host_oracle"]
    st = s.SamplingState(e["seed"])
    for _ in range(e["final_draws"]):
        st.next_24()
    assert st.state() == e["final_state"]
    assert s.SamplingState(0).state() == p["zero_seed_state"]


def test_fill_random_24_is_one_draw_per_row():
    import ctypes

    states = (s._State * 3)()
    for i, seed in enumerate((42, 43, 0)):
        s.lib().pb_sampling_state_new(ctypes.byref(states[i]), seed)
    out = np.zeros(3, np.uint32)
    s.lib().pb_fill_random_24(states, 3, out.ctypes.data_as(ctypes.c_void_p))
    expect = [s.SamplingState(seed).next_24() for seed in (42, 43, 0)]
    assert out.tolist() == expect
    assert out[0] == 5_688_906
    assert [st.draws for st in states] == [1, 1, 1]


def test_length_errors_need_no_device(known):
    t = known["unit"]["error_tuples"]
    short = np.zeros(s.VOCAB - 1, np.uint32)
    state = s.SamplingState(1)
    for call in (lambda: s.sample_token(short, state), lambda: s.greedy_token(short),
                 lambda: s.top_logits_8(short),
                 lambda: s.sample_token_with_repetition(short.copy(), [], np.zeros(10, np.uint8),
                                                        state)):
        with pytest.raises(s.InferenceError) as ex:
            call()
        assert ex.value.tuple() == t["short"]
    assert state.draws() == 0


def test_version_and_segment_plan():
    assert s.lib().pb_version().endswith(b"gfx950")
    assert s.lib().pb_segments_for_rows(4096) == 1
    assert 1 < s.lib().pb_segments_for_rows(64) <= 64
    assert s.lib().pb_segments_for_rows(1) <= 64


def _state_after_one(seed: int) -> int:
    st = s.SamplingState(seed)
    st.next_24()
    return st.state()


def test_decode_draw_and_settle_keep_one_draw_per_sampled_token():
    """Host side of the decode step: one next_24 per active row; a row that
    was active and got no token -- it failed, or its context was already
    full -- gets its state back (inference.rs:954-963: no draw on error; the
    REPL does not sample without room)."""
    import ctypes

    rows = 5
    states = (s._State * rows)()
    for r in range(rows):
        s.lib().pb_sampling_state_new(ctypes.byref(states[r]), 42 + r)
    saved = (s._State * rows)()
    before = np.array([s.ROW_ACTIVE, s.ROW_EOS, s.ROW_ACTIVE, s.ROW_LIMIT, s.ROW_ACTIVE],
                      np.uint32)
    r24 = np.full(rows, 7, np.uint32)
    s.lib().pb_decode_draw(states, before.ctypes.data_as(ctypes.c_void_p), rows,
                           r24.ctypes.data_as(ctypes.c_void_p), saved)
    for r in range(rows):
        ref = s.SamplingState(42 + r)
        if before[r] == s.ROW_ACTIVE:
            assert r24[r] == ref.next_24()
        else:
            assert r24[r] == 0
        assert (states[r].state, states[r].draws) == (ref.state(), ref.draws())
        assert (saved[r].state, saved[r].draws) == (s.SamplingState(42 + r).state(), 0)
    # row 0 failed, row 2 sampled, row 4 was full; rows 1 and 3 were not active
    tokens = np.array([s.NO_TOKEN, s.NO_TOKEN, 123, s.NO_TOKEN, s.NO_TOKEN], np.uint32)
    n = s.lib().pb_decode_settle(states, saved, before.ctypes.data_as(ctypes.c_void_p),
                                 tokens.ctypes.data_as(ctypes.c_void_p), rows)
    assert n == 2  # rows 1 and 3 drew nothing and have nothing to restore
    assert [states[r].draws for r in range(rows)] == [0, 0, 1, 0, 0]
    assert states[2].state == _state_after_one(44)


def test_decode_step_argument_errors_need_no_device():
    """Missing context pointers are rejected before any device work."""
    import ctypes

    e = s._Error()
    st = s.lib().pb_decode_step(None, None, s.VOCAB, s.VOCAB, 4, None, 0, None, None, None,
                                None, None, None, None, None, ctypes.byref(e))
    assert st == s.CAPACITY and e.status == s.CAPACITY and e.detail == (4 << 32) | 5
    st = s.lib().pb_decode_step(None, None, s.VOCAB + 1, s.VOCAB, 0, None, 0, None, None, None,
                                None, None, None, None, None, ctypes.byref(e))
    assert st == s.CAPACITY and e.needed == s.VOCAB and e.available == s.VOCAB + 1


def test_lmhead_pack_argument_errors_need_no_device():
    """The packed heads group the vocabulary in 64-id tiles; other sizes,
    hidden widths that are not whole blocks and unaligned outputs are rejected
    before any device work, by the Q4_0 and the Q8_0 repack alike."""
    import ctypes

    e = s._Error()
    for pack in (s.lib().pb_lmhead_pack_q4_0, s.lib().pb_lmhead_pack_q8_0):
        st = pack(None, s.VOCAB + 32, 896, None, None, ctypes.byref(e))
        assert st == s.CAPACITY and e.needed == 64 and e.available == s.VOCAB + 32
        st = pack(None, s.VOCAB, 900, None, None, ctypes.byref(e))
        assert st == s.CAPACITY and e.needed == 32 and e.available == 900
        st = pack(None, s.VOCAB, 896, ctypes.c_void_p(8), None, ctypes.byref(e))
        assert st == s.ALIGNMENT and e.needed == 16 and e.available == 8
    # the source matrices, plus the Q4_0 layout's flag word per 64-id tile
    assert s.lib().pb_lmhead_packed_bytes(s.VOCAB, 896) == s.VOCAB * 28 * 18 + s.VOCAB // 64 * 4
    assert s.lib().pb_lmhead_q8_packed_bytes(s.VOCAB, 896) == s.VOCAB * 28 * 34


def test_lmhead_and_reserve_argument_errors_need_no_device():
    """A head packed for another width or format is refused by its size
    before any device work (the C calls take the packed length), and so are a
    reservation for a width the head cannot take and a batch or reservation
    above PB_LMHEAD_MAX_ROWS rows."""
    import ctypes

    e = s._Error()
    q4 = s.lib().pb_lmhead_packed_bytes(s.VOCAB, 896)
    q8 = s.lib().pb_lmhead_q8_packed_bytes(s.VOCAB, 896)
    cases = [(s.lib().pb_lmhead_sample_batch, q8, q4), (s.lib().pb_lmhead_q8_sample_batch, q4, q8),
             (s.lib().pb_lmhead_sample_batch, s.lib().pb_lmhead_packed_bytes(s.VOCAB, 1024), q4)]
    for fn, given, want in cases:
        st = fn(None, None, given, s.VOCAB, 896, None, 4, None, 0, None, None, None, None, None,
                None, None, ctypes.byref(e))
        assert st == s.CAPACITY and (e.needed, e.available, e.detail) == (want, given, (4 << 32) | 7)
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check comes first
    for fn, want in ((s.lib().pb_lmhead_decode_step, q4), (s.lib().pb_lmhead_q8_decode_step, q8)):
        st = fn(None, None, want + 1, s.VOCAB, 896, None, 4, fake, 4, fake, None, fake, None,
                None, None, None, None, None, ctypes.byref(e))
        assert st == s.CAPACITY and (e.needed, e.available) == (want, want + 1)
    st = s.lib().pb_context_reserve(None, 256, 900, ctypes.byref(e))
    assert st == s.CAPACITY and (e.needed, e.available) == (32, 900)
    st = s.lib().pb_context_reserve(None, 256, 4096, ctypes.byref(e))
    assert st == s.CAPACITY and e.available == 4096
    # more rows than the LM head's 32-bit activation offsets allow
    over = s.LMHEAD_MAX_ROWS + 1
    want_err = (s.LMHEAD_MAX_ROWS, over, (4 << 32) | 8)
    for fn, size in ((s.lib().pb_lmhead_sample_batch, q4), (s.lib().pb_lmhead_q8_sample_batch, q8)):
        st = fn(None, fake, size, s.VOCAB, 896, fake, over, None, 0, None, fake, fake, None, None,
                None, None, ctypes.byref(e))
        assert st == s.CAPACITY and (e.needed, e.available, e.detail) == want_err
    st = s.lib().pb_context_reserve(None, over, 896, ctypes.byref(e))
    assert st == s.CAPACITY and (e.needed, e.available, e.detail) == want_err
