"""The C ABI without a GPU: the library loads, exports every symbol the
headers declare, and lays its table out as the reference core reads it."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import turboembed_amd as T
from turboembed_amd import seam as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("turbo_rocm.h",):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(turbo_rocm_\w+)\s*\(", text))
        names |= set(re.findall(r"extern const turbo_backend (\w+);", text))
    return names


def test_the_library_exports_every_declared_symbol():
    lib = T.library()
    names = declared_symbols()
    assert "turbo_rocm_backend" in names and len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n


def test_the_seam_layout_is_the_reference_core_s():
    S.check_layout()


def test_the_table_is_one_the_core_accepts():
    t = T.table()
    # core/src/backend/mod.rs:363-374: struct_size is one of the known sizes.
    sizes = {S.turbo_backend.context_create.offset, S.turbo_backend.model_load.offset,
             S.turbo_backend.session_create.offset, S.turbo_backend.buffer_read.offset,
             S.turbo_backend.formats.offset, S.turbo_backend.session_create_tuned.offset,
             S.turbo_backend.session_open.offset, S.turbo_backend.token_head.offset,
             S.turbo_backend.buffer_quantize.offset, C.sizeof(S.turbo_backend)}
    assert t.struct_size in sizes and t.struct_size == C.sizeof(S.turbo_backend)
    assert t.name == b"rocm"
    assert t.runtime_version.startswith(b"HIP ")
    assert t.formats == 1 << (S.TURBO_FORMAT_SAFETENSORS - 1)
    has = lambda f: bool(C.cast(getattr(t, f), C.c_void_p).value)  # noqa: E731
    # The pairing rules of core/src/backend/mod.rs:397-409.
    pairs = [("context_create", "context_release"), ("buffer_alloc", "buffer_release"),
             ("buffer_import", "buffer_release"), ("model_load", "model_release"),
             ("session_create", "session_release"), ("session_create", "session_run"),
             ("session_create_tuned", "session_release"), ("session_create_tuned", "session_run"),
             ("session_open", "session_release"), ("session_open", "session_run"),
             ("embed_write_ranges", "session_open")]
    for f, g in pairs:
        assert not has(f) or has(g), (f, g)
    for f in ("device_count", "device_info", "capability", "embed_write", "buffer_read", "session_open",
              "embed_write_ranges"):
        assert has(f), f
    # token_head is 1: a QA model's span head runs on the device, which only
    # a backend offering embed_write_ranges may claim.
    assert t.token_head == 1 and has("embed_write_ranges")


def test_device_count_answers_without_a_device():
    # Listing is not a compute call: with no GPU it lists nothing, not an error.
    n = T.Runtime().device_count()
    assert n >= 0


# ---- The core's checks (core/src/session/tokens.rs:274-384) -------------------------

def _check_tokens(ids, mask, types=None, max_batch=8, max_seq=16, vocab=100, token_types=2, max_tokens=0):
    ids = np.ascontiguousarray(ids, np.int32)
    mask = np.ascontiguousarray(mask, np.int32)
    tt = None if types is None else np.ascontiguousarray(types, np.int32)
    err = S.new_error()
    b, s = ids.shape
    p = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))  # noqa: E731
    rc = T.library().turbo_rocm_check_tokens(b, s, s, p(ids), p(mask), None if tt is None else p(tt), max_batch,
                                             max_seq, vocab, token_types, max_tokens, C.byref(err))
    return rc, err.message.decode()


def test_checks_accept_good_rows():
    assert _check_tokens([[1, 2, 3]], [[1, 1, 0]])[0] == S.TURBO_OK


@pytest.mark.parametrize("ids,mask,types,kw,code,text", [
    ([[1, 2]], [[0, 0]], None, {}, S.TURBO_E_INVALID_ARGUMENT, "has no 1"),
    ([[1, 200]], [[1, 1]], None, {}, S.TURBO_E_INVALID_ARGUMENT, "outside the model's vocabulary"),
    ([[1, -1]], [[1, 0]], None, {}, S.TURBO_E_INVALID_ARGUMENT, "outside the model's vocabulary"),
    ([[1, 2]], [[1, 2]], None, {}, S.TURBO_E_INVALID_ARGUMENT, "not 0 or 1"),
    ([[1, 2]], [[1, 1]], [[0, 2]], {}, S.TURBO_E_INVALID_ARGUMENT, "token types"),
    ([[1] * 20], [[1] * 20], None, {}, S.TURBO_E_CAPACITY, "max_seq"),
    ([[1]] * 9, [[1]] * 9, None, {}, S.TURBO_E_CAPACITY, "max_batch"),
    ([[1, 2, 3]], [[1, 1, 1]], None, {"max_tokens": 2}, S.TURBO_E_CAPACITY, "max_tokens"),
])
def test_checks_refuse_what_the_core_refuses(ids, mask, types, kw, code, text):
    rc, msg = _check_tokens(ids, mask, types, **kw)
    assert rc == code and text in msg, (rc, msg)


def _check_ranges(mask, ranges, max_ranges=8):
    mask = np.ascontiguousarray(mask, np.int32)
    arr = (S.turbo_token_range * max(1, len(ranges)))()
    for i, (r, a, b) in enumerate(ranges):
        arr[i].row, arr[i].start, arr[i].end = r, a, b
    err = S.new_error()
    b, s = mask.shape
    rc = T.library().turbo_rocm_check_ranges(b, s, s, mask.ctypes.data_as(C.POINTER(C.c_int32)), arr, len(ranges),
                                             max_ranges, C.byref(err))
    return rc, err.message.decode()


@pytest.mark.parametrize("ranges,code,text", [
    ([(0, 0, 2)], S.TURBO_OK, ""),
    ([], S.TURBO_E_INVALID_ARGUMENT, "count is 0"),
    ([(2, 0, 1)], S.TURBO_E_INVALID_ARGUMENT, "not under batch"),
    ([(0, 2, 2)], S.TURBO_E_INVALID_ARGUMENT, "not under end"),
    ([(0, 0, 5)], S.TURBO_E_INVALID_ARGUMENT, "over seq"),
    ([(0, 2, 4)], S.TURBO_E_UNSUPPORTED_OPTION, "mask-0 columns"),
    ([(0, 0, 1)] * 9, S.TURBO_E_CAPACITY, "max_ranges"),
])
def test_range_checks(ranges, code, text):
    rc, msg = _check_ranges([[1, 1, 0, 0], [1, 1, 1, 1]], ranges)
    assert rc == code and text in msg, (rc, msg)


def test_the_library_leaves_none_of_its_own_symbols_undefined():
    import subprocess
    out = subprocess.run(["nm", "-u", "--demangle", T.LIB_PATH], capture_output=True, text=True).stdout
    assert "rocm::" not in out, [l for l in out.splitlines() if "rocm::" in l]
