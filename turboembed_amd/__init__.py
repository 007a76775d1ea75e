"""turboembed_amd: TurboEmbed's encoder forward pass as an MI355X-native `rocm` backend.

The product is libturbo_rocm.so (built from csrc/ by build.py): the
`turbo_rocm_backend` function table behind the reference's backend seam, and
its gfx950 kernels. This module is the host side above that C ABI, playing
the TurboEmbed core's part for this path: it loads a model description,
opens sessions, checks rows and ranges as the core does before it calls a
backend, and reads results back. It mirrors the core's session flow
(reference core/src/session/create.rs:56-281, tokens.rs:9-152,
result.rs:8-63) and raises `TurboError` with the status the core would
return.

There is no fallback: without the built library every call raises.
"""
import ctypes as C
import os

import numpy as np

from . import seam as S
from .model import ModelDesc  # noqa: F401  (re-exported)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libturbo_rocm.so")

_lib = None


class TurboError(RuntimeError):
    def __init__(self, code, field, message):
        self.code, self.field, self.message = code, field, message
        super().__init__(f"{S.STATUS_NAMES.get(code, code)}"
                         f"{' (field ' + str(field) + ')' if field else ''}: {message}")


def library():
    """The loaded libturbo_rocm.so, with the hook prototypes set. Raises when
    it has not been built: this package has no other path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run turboembed_amd/build.py (or __graft_entry__.build())")
    lib = C.CDLL(LIB_PATH)
    E = C.POINTER(S.turbo_error)
    P = C.c_void_p
    u32 = C.c_uint32
    i32p = C.POINTER(C.c_int32)
    protos = {
        "turbo_rocm_check_tokens": [u32, u32, u32, i32p, i32p, i32p, u32, u32, u32, u32, u32, E],
        "turbo_rocm_check_ranges": [u32, u32, u32, i32p, C.POINTER(S.turbo_token_range), u32, u32, E],
        "turbo_rocm_session_packing": [P, P, P, P, C.POINTER(u32), E],
        "turbo_rocm_session_hidden": [P, P, C.c_uint64, E],
        "turbo_rocm_session_timing": [P, u32, E],
        "turbo_rocm_session_times": [P, C.c_char_p, u32, E],
        "turbo_rocm_session_intervals": [P, C.c_char_p, u32, E],
        "turbo_rocm_host_allocs": [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), E],
        "turbo_rocm_session_choices": [P, C.c_char_p, u32, E],
        "turbo_rocm_session_replay": [P, u32, E],
        "turbo_rocm_session_graphs": [P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), E],
        "turbo_rocm_gemm_check": [u32, u32, u32, u32, u32, P, P, P, P, u32, E],
        "turbo_rocm_gemm_time": [u32, u32, u32, u32, u32, u32, u32, C.POINTER(C.c_float), E],
        "turbo_rocm_copy_probe": [u32, C.c_uint64, u32, C.POINTER(C.c_float), E],
        "turbo_rocm_mfma_probe": [u32, u32, u32, C.POINTER(C.c_float), C.POINTER(C.c_float), E],
        "turbo_rocm_pair_windows": [P, u32, P, u32, C.c_int32, C.c_int32, u32, u32, u32, u32, P, P, P, u32,
                                    C.POINTER(u32), E],
        "turbo_rocm_rerank_scores": [P, u32, u32, P, P, P, C.c_float, P, E],
        "turbo_rocm_rerank_run": [P, P, P, P, u32, u32, P, u32, P, P, P, C.c_float, P, E],
        "turbo_rocm_fail_variant": [C.c_char_p, E],
        "turbo_rocm_buffer_quantize_static": [P, u32, C.POINTER(C.c_float), u32, u32, C.POINTER(S.turbo_backend_run),
                                              E],
    }
    for name, args in protos.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = C.c_int32
    _lib = lib
    return lib


def table():
    """The backend's turbo_backend table."""
    return S.turbo_backend.in_dll(library(), "turbo_rocm_backend")


def _ok(rc, err):
    if rc != S.TURBO_OK:
        raise TurboError(rc, err.field, err.message.decode(errors="replace"))


def _i32(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


class Runtime:
    """The backend's devices (the core's runtime, restricted to this backend)."""

    def __init__(self):
        self.t = table()
        self._log = S.turbo_log_fn(lambda ud, level, text: None)

    def device_count(self):
        n = C.c_uint32()
        err = S.new_error()
        _ok(self.t.device_count(C.byref(n), C.byref(err)), err)
        return n.value

    def device_info(self, ordinal=0):
        info = S.turbo_device_info()
        info.struct_size = C.sizeof(info)
        err = S.new_error()
        _ok(self.t.device_info(ordinal, C.byref(info), C.byref(err)), err)
        return info

    def capability(self, ordinal, task, precision):
        st, dt, hon = C.c_uint32(), C.c_uint32(), C.c_uint32()
        reason = C.create_string_buffer(160)
        err = S.new_error()
        _ok(self.t.capability(ordinal, task, precision, C.byref(st), C.byref(dt), C.byref(hon), reason, 160,
                              C.byref(err)), err)
        return st.value, dt.value, hon.value, reason.value.decode()

    def context(self, ordinal=0):
        return Context(self, ordinal)


class Context:
    def __init__(self, rt, ordinal):
        self.rt, self.t, self.ordinal = rt, rt.t, ordinal
        h = C.c_void_p()
        err = S.new_error()
        _ok(self.t.context_create(ordinal, rt._log, None, C.byref(h), C.byref(err)), err)
        self.h = h

    def load(self, desc: ModelDesc):
        return Model(self, desc)

    def load_bundle(self, path, artifact=0):
        """turbo_model_load of a bundle directory: the manifest's artifact
        read and verified (bundle.Bundle), then model_load. The model keeps
        the bundle as .bundle."""
        from .bundle import Bundle
        b = Bundle(path)
        m = Model(self, b.model_desc(artifact))
        m.bundle = b
        return m

    def buffer(self, nbytes, placement=S.TURBO_PLACE_SHARED):
        """A buffer of the context's device (buffer_alloc): DEVICE, PINNED,
        SHARED or HOST; the last three have a host pointer."""
        return Buffer(self, nbytes, placement)

    def close(self):
        if self.h:
            self.t.context_release(self.h)
            self.h = None


class Buffer:
    """A buffer the core allocates through the table (core/src/buffer_api.rs:83-211)."""

    def __init__(self, ctx, nbytes, placement):
        self.ctx, self.t, self.nbytes, self.placement = ctx, ctx.t, nbytes, placement
        d = S.turbo_buffer_desc()
        d.struct_size = C.sizeof(d)
        d.placement, d.dtype, d.ndim, d.bytes = placement, S.TURBO_DTYPE_U8, 1, nbytes
        d.shape[0] = nbytes
        h, host = C.c_void_p(), C.c_void_p()
        err = S.new_error()
        _ok(self.t.buffer_alloc(ctx.h, C.byref(d), C.byref(h), C.byref(host), C.byref(err)), err)
        self.h, self.host = h, host.value

    def view(self, dtype=np.uint8):
        """The host view of a buffer that has one."""
        if not self.host:
            raise TurboError(S.TURBO_E_UNSUPPORTED, 0, "a device buffer has no host view")
        return np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(self.host)).view(dtype)

    def read(self, nbytes=None):
        out = np.empty(self.nbytes if nbytes is None else nbytes, np.uint8)
        err = S.new_error()
        _ok(self.t.buffer_read(self.h, out.ctypes.data, out.nbytes, C.byref(err)), err)
        return out

    def quantize(self, quantization, rows, dim, int8_ranges=None, run=None):
        """buffer_quantize: the first rows x dim F32 values as codes, over
        the buffer's leading bytes."""
        rr = None
        if int8_ranges is not None:
            rr = np.ascontiguousarray(int8_ranges, np.float32)
        err = S.new_error()
        _ok(self.t.buffer_quantize(self.h, quantization,
                                   None if rr is None else rr.ctypes.data_as(C.POINTER(C.c_float)), rows, dim,
                                   None if run is None else C.byref(run), C.byref(err)), err)

    def quantize_static(self, quantization, rows, dim, int8_ranges=None, run=None):
        """turbo_rocm_buffer_quantize_static: the same codes as quantize,
        staged in the device's fixed area instead of allocated memory."""
        rr = None
        if int8_ranges is not None:
            rr = np.ascontiguousarray(int8_ranges, np.float32)
        err = S.new_error()
        _ok(library().turbo_rocm_buffer_quantize_static(
            self.h, quantization, None if rr is None else rr.ctypes.data_as(C.POINTER(C.c_float)), rows, dim,
            None if run is None else C.byref(run), C.byref(err)), err)

    def close(self):
        if self.h:
            self.t.buffer_release(self.h)
            self.h = None


class Model:
    def __init__(self, ctx, desc):
        self.ctx, self.t, self.desc = ctx, ctx.t, desc
        h = C.c_void_p()
        err = S.new_error()
        _ok(self.t.model_load(ctx.h, C.byref(desc.struct()), C.byref(h), C.byref(err)), err)
        self.h = h

    def session(self, max_batch, max_seq, precision=S.TURBO_PRECISION_MODEL, max_ranges=0, task=S.TURBO_TASK_EMBED,
                numerics_allowed=0, autotune=S.TURBO_AUTOTUNE_OFF, cache=None, budget_ms=None):
        return Session(self, max_batch, max_seq, precision, max_ranges, task, numerics_allowed, autotune, cache,
                       budget_ms)

    def close(self):
        if self.h:
            self.t.model_release(self.h)
            self.h = None


class Session:
    """A session opened through session_open, as the core opens one
    (core/src/session/create.rs:151-180)."""

    def __init__(self, model, max_batch, max_seq, precision, max_ranges, task, numerics_allowed,
                 autotune=S.TURBO_AUTOTUNE_OFF, cache=None, budget_ms=None):
        """autotune: TURBO_AUTOTUNE_OFF (the backend's rule and what the
        environment forces), ON (the cached choice for the session's key,
        else measured now and cached) or RETUNE (measured now against the
        cached one, which it replaces); cache: a tuning.TuneCache, the
        process's own by default; budget_ms: the measuring budget, else the
        cache's (core/src/session/create.rs:82-180, core/src/tuning.rs)."""
        from . import tuning as TU
        self.model, self.t, self.lib = model, model.t, library()
        d = S.turbo_backend_session_desc()
        d.struct_size = C.sizeof(d)
        # A QA session's encoder is the embedding encoder, with a range for
        # every token a run may hold (core/src/session/create.rs:61-62,
        # core/src/qa/session.rs:138-140).
        self.task = task
        # The core asks the backend about the model's own task first and
        # refuses the session when the backend cannot run it
        # (core/src/session/create.rs:93-111).
        ctx = model.ctx
        st, _, _, reason = ctx.rt.capability(ctx.ordinal, task, precision)
        if st == S.TURBO_CAP_UNSUPPORTED:
            raise TurboError(S.TURBO_E_UNSUPPORTED_TASK, 0,
                             f"the rocm backend does not run task {task}: {reason}")
        if task == S.TURBO_TASK_EXTRACTIVE_QA:
            task, max_ranges = S.TURBO_TASK_EMBED, max_ranges or max_batch * max_seq
        d.task, d.max_batch, d.max_seq, d.precision = task, max_batch, max_seq, precision
        d.max_ranges = max_ranges or max_batch
        self.max_batch, self.max_seq, self.max_ranges = max_batch, max_seq, d.max_ranges
        tun = S.turbo_backend_tuning()
        tun.struct_size = C.sizeof(tun)
        tun.mode = autotune
        tun.numerics_allowed = numerics_allowed
        tuned = autotune in (S.TURBO_AUTOTUNE_ON, S.TURBO_AUTOTUNE_RETUNE)
        self.key, self.cache = None, None
        if tuned:
            self.cache = cache if cache is not None else _process_cache()
            tun.budget_ms = budget_ms if budget_ms is not None else self.cache.budget_ms()
            self.key = self._tune_key(model, precision, numerics_allowed, max_batch * max_seq, max_seq)
            entry = self.cache.get(self.key)
            self._cached = C.create_string_buffer(entry["choices"].encode()) if entry else None
            tun.cached = C.cast(self._cached, C.c_char_p) if entry else None
        self._timings = C.create_string_buffer(16384)
        tun.timings = C.cast(self._timings, C.c_char_p)
        tun.timings_len = len(self._timings)
        self.tuning = tun
        cd = C.c_uint32()
        h = C.c_void_p()
        err = S.new_error()
        _ok(self.t.session_open(model.h, C.byref(d), C.byref(tun), C.byref(cd), C.byref(h), C.byref(err)), err)
        self.h, self.compute_dtype = h, cd.value
        self.tuned = tun.tuned
        self.timings = TU.parse_timings(self._timings.value.decode())
        # A measured choice goes into the cache, unless the backend widened
        # the numeric classes (tuning.rs: such a session is never cached).
        if tuned and tun.tuned == S.TURBO_TUNED_MEASURED and tun.numerics_used == tun.numerics_allowed:
            self.cache.put(self.key, tun.choices.decode(), self.timings)
        self.run_info = None
        self.n_out, self.headed = 0, False
        self.od = 0

    def _tune_key(self, model, precision, numerics_allowed, tcap, max_seq):
        from . import tuning as TU
        ctx = model.ctx
        info = ctx.rt.device_info(ctx.ordinal)
        st, dt, _, _ = ctx.rt.capability(ctx.ordinal, S.TURBO_TASK_EMBED, precision)
        return TU.TuneKey(backend=info.backend.decode(), device_name=info.name.decode(), arch=info.arch.decode(),
                          runtime_version=info.runtime_version.decode(), library_build=TU.library_build(LIB_PATH),
                          model=TU.model_fingerprint(model.desc), precision=precision, compute_dtype=dt,
                          numerics_allowed=numerics_allowed, tcap_bin=TU.tcap_bin(tcap),
                          max_seq_bin=TU.max_seq_bin(max_seq))

    # -- writes ---------------------------------------------------------------
    def _rows(self, ids, mask, types, pooling, normalize, output_dim):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        mask = np.ascontiguousarray(mask, dtype=np.int32)
        types = None if types is None else np.ascontiguousarray(types, dtype=np.int32)
        desc = self.model.desc
        err = S.new_error()
        b, s = ids.shape
        _ok(self.lib.turbo_rocm_check_tokens(b, s, s, _i32(ids), _i32(mask), None if types is None else _i32(types),
                                             self.max_batch, self.max_seq, desc.vocab_size, desc.token_types, 0,
                                             C.byref(err)), err)
        od = output_dim or desc.hidden
        if not 1 <= od <= desc.hidden:
            raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 6, f"output_dim {od} is not 1 to {desc.hidden}")
        r = S.turbo_backend_embed_rows()
        r.struct_size = C.sizeof(r)
        r.batch, r.seq, r.row_stride = b, s, s
        r.ids, r.mask = _i32(ids), _i32(mask)
        r.types = None if types is None else _i32(types)
        r.pooling, r.normalize, r.output_dim = pooling, normalize, od
        r.head, r.taps, r.tap_alone = 0, 1, 0
        self._keep = (ids, mask, types)
        return r

    def write_tokens(self, ids, mask, types=None, pooling=S.TURBO_POOLING_MEAN, normalize=S.TURBO_NORMALIZE_L2,
                     output_dim=0):
        r = self._rows(ids, mask, types, pooling, normalize, output_dim)
        err = S.new_error()
        _ok(self.t.embed_write(self.h, C.byref(r), C.byref(err)), err)
        self.n_out, self.od, self.headed = r.batch, r.output_dim, False

    def write_ranges(self, ids, mask, ranges, types=None, normalize=S.TURBO_NORMALIZE_L2, output_dim=0, layers=1,
                     layer_alone=False):
        """Ranges are (row, start, end) triples; pooled by the mean, as the
        core forces for a range write (core/src/session/tokens.rs:132-146).

        On a model loaded with a span head each range's row is the head's
        logits, [count, head_out]: normalize must be NONE (else
        TURBO_E_UNSUPPORTED_OPTION naming field 4) and output_dim 0 or the
        hidden width (field 6), as the core holds them
        (tokens.rs:140-143, 217-235).

        layers > 1 reads each range from each of the model's last `layers`
        layers, rows [layers, count, output_dim] block by block, the last
        the final layer's; with layer_alone the first of them alone,
        [count, output_dim] (turbo_embed_write_layer_ranges; the core's
        checks, tokens.rs:99-130, 153-215)."""
        head = self.model.desc.span_head
        ranges = list(ranges)
        if not ranges:
            raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 0, "count is 0: a run needs at least one range")
        if layers == 0:
            raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 9, "layers 0: a range write needs at least 1 layer")
        if layers > 1:
            if layers > self.model.desc.layers:
                raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 9,
                                 f"layers {layers}: the model has 1 to {self.model.desc.layers} to read")
            if head is not None:
                raise TurboError(S.TURBO_E_UNSUPPORTED_OPTION, 9, f"layers {layers}: the span head reads the final layer")
        alone = bool(layer_alone) and layers > 1
        blocks = 1 if alone else layers
        if len(ranges) * blocks > self.max_ranges:
            raise TurboError(S.TURBO_E_CAPACITY, 0, f"{len(ranges)} ranges from {blocks} layers is "
                                                    f"{len(ranges) * blocks} vectors, over max_ranges {self.max_ranges}")
        if head is not None:
            if normalize != S.TURBO_NORMALIZE_NONE:
                raise TurboError(S.TURBO_E_UNSUPPORTED_OPTION, 4, "normalize: the span head's logits are not normalized")
            if output_dim not in (0, self.model.desc.hidden):
                raise TurboError(S.TURBO_E_UNSUPPORTED_OPTION, 6, f"output_dim {output_dim}: the span head reads all "
                                                                  f"{self.model.desc.hidden} values of a range's vector")
        r = self._rows(ids, mask, types, S.TURBO_POOLING_MEAN, normalize, output_dim)
        if head is not None:
            r.head, r.output_dim = 1, head[0].shape[0]
        r.taps, r.tap_alone = layers, 1 if alone else 0
        arr = (S.turbo_token_range * max(1, len(ranges)))()
        for i, (row, start, end) in enumerate(ranges):
            arr[i].row, arr[i].start, arr[i].end = row, start, end
        err = S.new_error()
        mask = self._keep[1]
        _ok(self.lib.turbo_rocm_check_ranges(r.batch, r.seq, r.seq, _i32(mask), arr, len(ranges), self.max_ranges,
                                             C.byref(err)), err)
        _ok(self.t.embed_write_ranges(self.h, C.byref(r), arr, len(ranges), C.byref(err)), err)
        self.n_out, self.od, self.headed = len(ranges) * blocks, r.output_dim, head is not None

    def write_layer_ranges(self, ids, mask, ranges, layers, types=None, normalize=S.TURBO_NORMALIZE_L2,
                           output_dim=0, layer_alone=False):
        """turbo_embed_write_layer_ranges: write_ranges with `layers` layer reads."""
        self.write_ranges(ids, mask, ranges, types, normalize, output_dim, layers, layer_alone)

    # -- run and read -----------------------------------------------------------
    def run(self):
        out = S.turbo_backend_run()
        out.struct_size = C.sizeof(out)
        err = S.new_error()
        _ok(self.t.session_run(self.h, C.byref(out), C.byref(err)), err)
        self.run_info = out
        return out

    def read(self):
        """The last run's vectors, [n, output_dim] F32, via buffer_read."""
        v = np.empty((self.n_out, self.od), dtype=np.float32)
        err = S.new_error()
        _ok(self.t.buffer_read(self.run_info.output, v.ctypes.data, v.nbytes, C.byref(err)), err)
        return v

    def read_quantized(self, quantization, int8_ranges=None):
        """The last run's vectors as codes made on the device, as the core
        reads a quantized write (core/src/session/result.rs:84-102):
        buffer_quantize over the session's output, then buffer_read of the
        codes alone. int8: [n, output_dim] int8 with ranges [2, output_dim];
        ubinary: [n, ceil(output_dim / 8)] uint8. The output holds codes,
        not vectors, afterwards."""
        if getattr(self, "headed", False):
            raise TurboError(S.TURBO_E_UNSUPPORTED_OPTION, 7, "quantization: the span head's rows are logits, not vectors")
        rr = None
        if quantization == S.TURBO_QUANTIZE_INT8:
            rr = np.ascontiguousarray(int8_ranges, np.float32)
            if rr.shape != (2, self.od):
                raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 8, f"int8 ranges must be [2, {self.od}]")
        err = S.new_error()
        _ok(self.t.buffer_quantize(self.run_info.output, quantization,
                                   None if rr is None else rr.ctypes.data_as(C.POINTER(C.c_float)), self.n_out,
                                   self.od, C.byref(self.run_info), C.byref(err)), err)
        width = self.od if quantization == S.TURBO_QUANTIZE_INT8 else (self.od + 7) // 8
        v = np.empty((self.n_out, width), np.uint8)
        _ok(self.t.buffer_read(self.run_info.output, v.ctypes.data, v.nbytes, C.byref(err)), err)
        return v.view(np.int8) if quantization == S.TURBO_QUANTIZE_INT8 else v

    def embed(self, ids, mask, types=None, **kw):
        self.write_tokens(ids, mask, types, **kw)
        self.run()
        return self.read()

    def rerank(self, pairs, head, start_id, end_id, **kw):
        """Scores of (query ids, passage ids) pairs; see rerank.rerank."""
        from .rerank import rerank
        return rerank(self, pairs, head, start_id, end_id, **kw)

    def span_logits(self, windows, fill_id=0):
        """Start and end logits of QA windows; see qa.span_logits."""
        from .qa import span_logits
        return span_logits(self, windows, fill_id)

    # -- hooks ---------------------------------------------------------------------
    def graphs(self):
        """(graphs captured, runs that replayed one) of this session."""
        c, l = C.c_uint64(), C.c_uint64()
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_graphs(self.h, C.byref(c), C.byref(l), C.byref(err)), err)
        return c.value, l.value

    def packing(self):
        b = self._keep[0].shape[0]
        start = np.zeros(b, np.int32)
        ln = np.zeros(b, np.int32)
        at = np.zeros(self._keep[0].size, np.int32)
        t = C.c_uint32()
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_packing(self.h, start.ctypes.data, ln.ctypes.data, at.ctypes.data,
                                                C.byref(t), C.byref(err)), err)
        return start, ln, at[: t.value]

    def hidden(self):
        _, ln, _ = self.packing()
        n = int(ln.sum())
        out = np.empty((n, self.model.desc.hidden), np.float32)
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_hidden(self.h, out.ctypes.data, out.size, C.byref(err)), err)
        return out

    def set_timing(self, on=True):
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_timing(self.h, 1 if on else 0, C.byref(err)), err)

    def times(self):
        buf = C.create_string_buffer(8192)
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_times(self.h, buf, 8192, C.byref(err)), err)
        out = {}
        for line in buf.value.decode().splitlines():
            name, ms, _ = line.split()
            out[name] = float(ms)
        return out

    def launches(self):
        """The last timed run's launch count of each kernel, by name."""
        buf = C.create_string_buffer(8192)
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_times(self.h, buf, 8192, C.byref(err)), err)
        return {name: int(n) for name, _, n in (line.split() for line in buf.value.decode().splitlines())}

    def intervals(self):
        """The last timed run's launches: (kernel, start ms, end ms) from the
        run's start, in launch order."""
        buf = C.create_string_buffer(1 << 16)
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_intervals(self.h, buf, 1 << 16, C.byref(err)), err)
        out = []
        for line in buf.value.decode().splitlines():
            name, a, b = line.split()
            out.append((name, float(a), float(b)))
        return out

    def replay(self, runs):
        """Run the written rows `runs` more times on the device, then wait."""
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_replay(self.h, runs, C.byref(err)), err)

    def choices(self):
        buf = C.create_string_buffer(1024)
        err = S.new_error()
        _ok(self.lib.turbo_rocm_session_choices(self.h, buf, 1024, C.byref(err)), err)
        return buf.value.decode()

    def close(self):
        if self.h:
            self.t.session_release(self.h)
            self.h = None


_cache = None


def _process_cache():
    """The process's tune cache (TURBO_AUTOTUNE_CACHE names its directory)."""
    global _cache
    if _cache is None:
        from .tuning import TuneCache
        _cache = TuneCache()
    return _cache


def gemm_check(a, w, bias=None, dtype=S.TURBO_DTYPE_F32, tile=0, ordinal=0):
    """out = a w^T + bias on the device, through the GEMM kernel alone."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = a.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    err = S.new_error()
    _ok(library().turbo_rocm_gemm_check(ordinal, dtype, m, n, k, a.ctypes.data, w.ctypes.data,
                                        None if b is None else b.ctypes.data, out.ctypes.data, tile, C.byref(err)),
        err)
    return out


def gemm_time(m, n, k, dtype=S.TURBO_DTYPE_F16, tile=0, iters=20, ordinal=0):
    """Average milliseconds of one GEMM launch on device-resident operands."""
    ms = C.c_float()
    err = S.new_error()
    _ok(library().turbo_rocm_gemm_time(ordinal, dtype, m, n, k, tile, iters, C.byref(ms), C.byref(err)), err)
    return ms.value


def mfma_probe(random=True, iters=20000, ordinal=0):
    """(TFLOP/s, MHz): the matrix cores' sustained F16 rate on every compute
    unit, with random operands changing every product (as a GEMM's) or
    fixed ones, and the clock under that load."""
    tf, mhz = C.c_float(), C.c_float()
    err = S.new_error()
    _ok(library().turbo_rocm_mfma_probe(ordinal, 1 if random else 0, iters, C.byref(tf), C.byref(mhz), C.byref(err)),
        err)
    return tf.value, mhz.value


def copy_probe(nbytes, iters=5, ordinal=0):
    """Average milliseconds of a plain device copy of nbytes (read and
    write nbytes each): the reference for the profiler's traffic counters."""
    ms = C.c_float()
    err = S.new_error()
    _ok(library().turbo_rocm_copy_probe(ordinal, nbytes, iters, C.byref(ms), C.byref(err)), err)
    return ms.value


def host_allocs():
    """(process, calling thread): the backend's heap allocations so far, every
    malloc-family and operator new call its own code has made."""
    p, t = C.c_uint64(), C.c_uint64()
    err = S.new_error()
    _ok(library().turbo_rocm_host_allocs(C.byref(p), C.byref(t), C.byref(err)), err)
    return p.value, t.value


def fail_variant(name=None):
    """Makes the GEMM block shape `name` fail to launch from now on, as on
    a device that cannot take it (None for none); a test hook."""
    err = S.new_error()
    _ok(library().turbo_rocm_fail_variant(name.encode() if name else None, C.byref(err)), err)
