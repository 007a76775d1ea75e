"""Model descriptions as the seam hands them to model_load.

`ModelDesc` holds a model's tensors (numpy arrays, row-major, little-endian)
in the family's TURBO_* order and builds the `turbo_backend_model` struct the
reference core builds in core/src/model/mod.rs:379-438 (rotary fields
core/src/model/rotary.rs:121-155). The arrays stay referenced for as long as
the description lives, as the seam requires of tensor data until
model_release (reference include/turbo/turbo_backend.h:505-513).
"""
import ctypes as C

import numpy as np

from . import seam as S

_DTYPES = {np.dtype(np.float32): S.TURBO_DTYPE_F32, np.dtype(np.float16): S.TURBO_DTYPE_F16}


def rope_table(global_theta, local_theta, positions, pairs):
    """The core's cos/sin table, [2 (global, local)][2 (cos, sin)][positions][pairs] F32.

    As core/src/rope.rs:20-38: the exponent 2i/width divided in F32, theta
    rounded to F32, the power taken in F64 and rounded to F32, the inverse
    frequency 1/power divided in F32, the angle p * inv multiplied in F32,
    then cos and sin of that angle taken in F64 and rounded once.
    """
    width = np.float32(2 * pairs)
    out = np.empty((2, 2, positions, pairs), dtype=np.float32)
    p = np.arange(positions, dtype=np.float32)[:, None]
    for b, theta in enumerate((global_theta, local_theta)):
        expo = (np.arange(pairs, dtype=np.float32) * np.float32(2)) / width          # F32 exponent
        power = np.power(np.float64(np.float32(theta)), expo.astype(np.float64)).astype(np.float32)
        inv = np.float32(1.0) / power                                                  # F32 division
        angle = (p * inv[None, :]).astype(np.float32).astype(np.float64)           # F32 angle
        out[b, 0] = np.cos(angle).astype(np.float32)
        out[b, 1] = np.sin(angle).astype(np.float32)
    return out


class ModelDesc:
    """A model's architecture and tensors, and its turbo_backend_model.

    `tensors` is the list of arrays in the family's TURBO_* order; an entry
    may be None (ModernBERT's layer-0 attention norm, whose data is NULL and
    bytes 0).
    """

    def __init__(self, family, layers, hidden, heads, intermediate, vocab_size, max_positions, token_types,
                 layer_norm_eps, tensors, position_offset=0, rope=None, attention_window=0, global_every=0,
                 mlp=S.TURBO_MLP_DENSE, activation=S.TURBO_ACTIVATION_GELU_ERF, norm=S.TURBO_NORM_LAYER,
                 names=None, compute_dtype=0, span_head=None, relative=None):
        self.family, self.layers, self.hidden, self.heads = family, layers, hidden, heads
        self.intermediate, self.vocab_size, self.max_positions = intermediate, vocab_size, max_positions
        self.token_types, self.layer_norm_eps, self.position_offset = token_types, layer_norm_eps, position_offset
        self.tensors = [None if t is None else np.ascontiguousarray(t) for t in tensors]
        dts = {t.dtype for t in self.tensors if t is not None}
        assert len(dts) == 1, f"every tensor has the model's dtype, not {dts}"
        self.np_dtype = dts.pop()
        if self.np_dtype == np.dtype(np.uint16):
            self.dtype = S.TURBO_DTYPE_BF16       # bfloat16 bits
        else:
            self.dtype = _DTYPES[self.np_dtype]
        self.rope = rope          # (global_theta, local_theta) or None
        self.attention_window, self.global_every = attention_window, global_every
        self.mlp, self.activation, self.norm = mlp, activation, norm
        self.names = names or [f"tensor{i}" for i in range(len(self.tensors))]
        # TURBO_DTYPE_I8 asks for int8 GEMMs below EXACT; 0 leaves it to the precision.
        self.compute_dtype = compute_dtype
        # A DeBERTa-v2 model's (position_buckets, max_relative_positions).
        self.relative = relative
        # An extractive QA model's span head, (weight [head_out, hidden],
        # bias [head_out]) in F32, for a backend that applies it
        # (turbo_backend.h:332-337); None on every other model.
        self.span_head = None
        if span_head is not None:
            w, b = (np.ascontiguousarray(a, np.float32) for a in span_head)
            assert w.ndim == 2 and w.shape[1] == hidden and b.shape == (w.shape[0],), "head is [out, hidden], [out]"
            self.span_head = (w, b)
        self._struct = None

    @property
    def head_dim(self):
        return self.hidden // self.heads

    @property
    def rotary(self):
        return self.family in (S.TURBO_FAMILY_MODERNBERT, S.TURBO_FAMILY_NOMIC_BERT)

    def struct(self):
        """The turbo_backend_model, built once; valid while self lives."""
        if self._struct is not None:
            return self._struct
        n = len(self.tensors)
        arr = (S.turbo_backend_tensor * n)()
        self._names_b = [s.encode() for s in self.names]
        for i, t in enumerate(self.tensors):
            e = arr[i]
            e.name = self._names_b[i]
            if t is None:
                e.data, e.ndim, e.dtype, e.bytes = None, 1, self.dtype, 0
                continue
            e.data = t.ctypes.data
            e.ndim = t.ndim
            e.shape[0] = t.shape[0]
            e.shape[1] = t.shape[1] if t.ndim == 2 else 0
            e.dtype = self.dtype
            e.bytes = t.nbytes
        m = S.turbo_backend_model()
        m.struct_size = C.sizeof(S.turbo_backend_model)
        m.family, m.dtype, m.layers, m.hidden, m.heads = self.family, self.dtype, self.layers, self.hidden, self.heads
        m.intermediate, m.vocab_size, m.max_positions = self.intermediate, self.vocab_size, self.max_positions
        m.token_types, m.layer_norm_eps = self.token_types, self.layer_norm_eps
        m.tensor_count, m.position_offset = n, self.position_offset
        m.compute_dtype = self.compute_dtype
        if self.relative is not None:
            m.position_buckets, m.max_relative_positions = self.relative
        m.tensors = C.cast(arr, C.POINTER(S.turbo_backend_tensor))
        m.format, m.graph_input, m.graph_output = S.TURBO_FORMAT_SAFETENSORS, S.TURBO_INPUT_TOKEN_IDS, \
            S.TURBO_OUTPUT_HIDDEN_STATES
        if self.rotary:
            g, loc = self.rope
            pairs = self.head_dim // 2
            self._rope = np.ascontiguousarray(rope_table(g, loc, self.max_positions, pairs))
            m.rope_global_theta, m.rope_local_theta = g, loc
            m.rope_table = self._rope.ctypes.data_as(C.POINTER(C.c_float))
            m.rope_pairs = pairs
            m.mlp, m.activation, m.norm = self.mlp, self.activation, self.norm
            m.attention_window, m.global_every = self.attention_window, self.global_every
        if self.span_head is not None:
            harr = (S.turbo_backend_tensor * 2)()
            self._head_names = [b"head.weight", b"head.bias"]
            for e, t, name in zip(harr, self.span_head, self._head_names):
                e.name, e.data, e.ndim, e.dtype, e.bytes = name, t.ctypes.data, t.ndim, S.TURBO_DTYPE_F32, t.nbytes
                e.shape[0] = t.shape[0]
                e.shape[1] = t.shape[1] if t.ndim == 2 else 0
            m.head = C.cast(harr, C.POINTER(S.turbo_backend_tensor))
            m.head_out = self.span_head[0].shape[0]
            self._harr = harr
        self._arr = arr
        self._struct = m
        return m


def to_bf16_bits(a):
    """F32 array -> bfloat16 bits (uint16), rounded to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def with_dtype(desc, dtype):
    """The same model with every tensor stored as `dtype` ("f32", "f16" or "bf16")."""
    conv = {"f32": lambda t: t.astype(np.float32), "f16": lambda t: t.astype(np.float16), "bf16": to_bf16_bits}[dtype]
    out = ModelDesc(desc.family, desc.layers, desc.hidden, desc.heads, desc.intermediate, desc.vocab_size,
                    desc.max_positions, desc.token_types, desc.layer_norm_eps,
                    [None if t is None else conv(t) for t in desc.tensors], desc.position_offset, desc.rope,
                    desc.attention_window, desc.global_every, desc.mlp, desc.activation, desc.norm, desc.names,
                    desc.compute_dtype, desc.span_head, desc.relative)
    return out
