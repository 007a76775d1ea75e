"""The no-allocation buffer_quantize (turbo_rocm_buffer_quantize_static)
against the table's buffer_quantize, through the C ABI on the device: the
same codes byte for byte (and the oracle's), on two calls in a row, the
second smaller, so the fixed staging area still holds the first call's
bytes; no device allocation counted; a call past the area refused before
any device work."""
import ctypes as C

import numpy as np
import pytest

import oracle
import turboembed_amd as T
from turboembed_amd import seam as S

pytestmark = pytest.mark.gpu

INT8, UBINARY = S.TURBO_QUANTIZE_INT8, S.TURBO_QUANTIZE_UBINARY
AREA = 16 << 20   # the staging area's bytes


def _run():
    r = S.turbo_backend_run()
    r.struct_size = C.sizeof(r)
    return r


def _codes(context, x, mode, ranges, static):
    rows, dim = x.shape
    buf = context.buffer(x.nbytes, S.TURBO_PLACE_SHARED)
    buf.view(np.float32)[:] = x.ravel()
    run = _run()
    call = buf.quantize_static if static else buf.quantize
    call(mode, rows, dim, ranges if mode == INT8 else None, run=run)
    width = dim if mode == INT8 else (dim + 7) // 8
    codes = buf.read(rows * width).reshape(rows, width)
    buf.close()
    return codes, run


def _inputs(seed, rows, dim):
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal((rows, dim)).astype(np.float32)
    lo = (g.standard_normal(dim) * 0.1 - 1.0).astype(np.float32)
    ranges = np.stack([lo, lo + np.abs(g.standard_normal(dim)).astype(np.float32) + 1.0]).astype(np.float32)
    ranges[:, 3] = 0.25   # a dimension whose step is 0
    return x, ranges


@pytest.mark.parametrize("mode", [INT8, UBINARY])
def test_static_codes_are_the_allocating_call_s(context, mode):
    cases = [_inputs(71, 600, 1024), _inputs(72, 37, 77)]   # the second call smaller
    want = []
    for x, ranges in cases:
        codes, run = _codes(context, x, mode, ranges, static=False)
        assert run.device_allocs == (2 if mode == INT8 else 1)
        assert np.array_equal(codes, oracle.quantize(x, mode, ranges))
        want.append(codes)
    for (x, ranges), w in zip(cases, want):
        got, run = _codes(context, x, mode, ranges, static=True)
        assert np.array_equal(got, w)
        assert run.device_allocs == 0
        assert run.h2d_bytes == (2 * x.shape[1] * 4 if mode == INT8 else 0)


def test_static_codes_past_the_area_are_refused(context):
    # 4097 x 4096 int8 codes are past the 16 MiB area: refused on the host,
    # the buffer untouched.
    rows, dim = 4097, 4096
    assert rows * dim > AREA
    buf = context.buffer(rows * dim * 4, S.TURBO_PLACE_SHARED)
    v = buf.view(np.float32)
    v[:16] = np.arange(16, dtype=np.float32)
    ranges = np.stack([np.full(dim, -1.0, np.float32), np.full(dim, 1.0, np.float32)])
    with pytest.raises(T.TurboError) as e:
        buf.quantize_static(INT8, rows, dim, ranges)
    assert e.value.code == S.TURBO_E_INVALID_ARGUMENT and "at most 16777216 bytes" in e.value.message
    assert np.array_equal(v[:16], np.arange(16, dtype=np.float32))
    # The table's own call takes it (it allocates).
    buf.quantize(INT8, 1, dim, ranges)
    buf.close()


def test_static_calls_through_two_contexts_on_two_threads_keep_their_codes(runtime):
    # Both contexts' calls stage in the GPU's one area; the lock per GPU
    # holds each call's codes until it has copied them out, so every call
    # gets its own codes whichever thread's call runs beside it.
    import threading
    ctxs = [runtime.context(0), runtime.context(0)]
    cases = [_inputs(80, 300, 512), _inputs(81, 450, 384)]
    want = [_codes(ctxs[i], x, INT8, r, static=False)[0] for i, (x, r) in enumerate(cases)]
    bad = []

    def calls(i):
        try:
            for _ in range(40):
                got, run = _codes(ctxs[i], cases[i][0], INT8, cases[i][1], static=True)
                if not np.array_equal(got, want[i]) or run.device_allocs != 0:
                    bad.append(i)
                    return
        except Exception as e:   # noqa: BLE001 (reported below)
            bad.append(repr(e))

    threads = [threading.Thread(target=calls, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for c in ctxs:
        c.close()
    assert not bad, bad
