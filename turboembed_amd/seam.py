"""ctypes mirrors of the seam structs in include/turbo/turbo_seam.h.

The layouts are the reference's (include/turbo/turbo_backend.h:234-627 and
include/turbo/turbo.h:263-390, 644-648); `check_layout()` holds them to the
offsets the reference core checks (core/src/backend/tests.rs:99-101).
"""
import ctypes as C

# Status codes (turbo.h:99-127).
TURBO_OK = 0
TURBO_E_INVALID_ARGUMENT = 256
TURBO_E_INVALID_STRUCT_SIZE = 257
TURBO_E_INVALID_SHAPE = 260
TURBO_E_INVALID_STATE = 261
TURBO_E_INVALID_ENUM = 262
TURBO_E_UNSUPPORTED = 512
TURBO_E_UNSUPPORTED_OPTION = 513
TURBO_E_UNSUPPORTED_TASK = 514
TURBO_E_OUT_OF_MEMORY = 768
TURBO_E_BUSY = 769
TURBO_E_CAPACITY = 771
TURBO_E_DEVICE_NOT_FOUND = 1024
TURBO_E_RUNTIME = 1026
TURBO_E_INTERNAL = 1536

STATUS_NAMES = {v: k for k, v in dict(globals()).items() if k.startswith("TURBO_E_") or k == "TURBO_OK"}

TURBO_TASK_EMBED = 1
TURBO_TASK_RERANK = 2
TURBO_TASK_EXTRACTIVE_QA = 3

TURBO_CAP_UNSUPPORTED = 0
TURBO_CAP_EXPERIMENTAL = 1

TURBO_DTYPE_I8 = 6
TURBO_DTYPE_U8 = 7
TURBO_DTYPE_I32 = 8
TURBO_DTYPE_F16 = 10
TURBO_DTYPE_BF16 = 11
TURBO_DTYPE_F32 = 12

TURBO_PLACE_HOST = 1
TURBO_PLACE_PINNED = 2
TURBO_PLACE_DEVICE = 3
TURBO_PLACE_SHARED = 4

TURBO_STAGE_MAX = 16
TURBO_STAGE_UNUSED, TURBO_STAGE_HOST, TURBO_STAGE_DEVICE, TURBO_STAGE_FUSED = 0, 1, 2, 3

TURBO_NORMALIZE_NONE = 1
TURBO_NORMALIZE_L2 = 2
TURBO_POOLING_MEAN = 1
TURBO_POOLING_CLS = 2
TURBO_POOLING_LAST = 3

TURBO_PRECISION_MODEL = 0
TURBO_PRECISION_FASTEST = 1
TURBO_PRECISION_EXACT = 2

TURBO_QUANTIZE_MODEL = 0
TURBO_QUANTIZE_NONE = 1
TURBO_QUANTIZE_INT8 = 2
TURBO_QUANTIZE_UBINARY = 3

TURBO_HANDLE_HOST_PTR = 1
TURBO_HANDLE_CUDA_PTR = 2

TURBO_AUTOTUNE_OFF = 1
TURBO_AUTOTUNE_ON = 2
TURBO_AUTOTUNE_RETUNE = 3
TURBO_TUNED_DEFAULT, TURBO_TUNED_FORCED, TURBO_TUNED_MEASURED, TURBO_TUNED_CACHE = 0, 1, 2, 3
TURBO_CHOICES_LEN = 1024

TURBO_FAMILY_BERT = 1
TURBO_FAMILY_ROBERTA = 2
TURBO_FAMILY_DEBERTA_V2 = 4
TURBO_FAMILY_MODERNBERT = 5
TURBO_FAMILY_NOMIC_BERT = 6
TURBO_FORMAT_SAFETENSORS = 1
TURBO_INPUT_TOKEN_IDS = 1
TURBO_OUTPUT_HIDDEN_STATES = 1
TURBO_MLP_DENSE = 1
TURBO_MLP_GATED = 2
TURBO_ACTIVATION_GELU_ERF = 1
TURBO_ACTIVATION_SILU = 2
TURBO_NORM_LAYER = 1
TURBO_NORM_LAYER_NO_BIAS = 2

TURBO_NUMERIC_F32_FMA = 1
TURBO_NUMERIC_TF32 = 2
TURBO_NUMERIC_F16_F32ACC = 4
TURBO_NUMERIC_F16_CHUNKACC = 8

BERT_EMBEDDING_TENSORS = 5
BERT_LAYER_TENSORS = 16
MODERNBERT_EMBEDDING_TENSORS = 3
MODERNBERT_LAYER_TENSORS = 6
NOMIC_EMBEDDING_TENSORS = 4
NOMIC_LAYER_TENSORS = 9
DEBERTA_EMBEDDING_TENSORS = 6


class turbo_text(C.Structure):
    _fields_ = [("ptr", C.c_char_p), ("len", C.c_uint64)]


class turbo_error(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("code", C.c_int32), ("field", C.c_uint32),
                ("message", C.c_char * 496)]


turbo_log_fn = C.CFUNCTYPE(None, C.c_void_p, C.c_uint32, turbo_text)


class turbo_device_info(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("kind", C.c_uint32), ("ordinal", C.c_uint32),
                ("unified_memory", C.c_uint32), ("memory_total", C.c_uint64), ("memory_free", C.c_uint64),
                ("arch", C.c_char * 32), ("name", C.c_char * 128), ("vendor", C.c_char * 64),
                ("backend", C.c_char * 32), ("runtime_version", C.c_char * 64), ("driver_version", C.c_char * 64)]


class turbo_native_handle(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("kind", C.c_uint32), ("handle", C.c_uint64), ("aux", C.c_uint64),
                ("offset", C.c_uint64)]


class turbo_buffer_desc(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("placement", C.c_uint32), ("dtype", C.c_uint32), ("ndim", C.c_uint32),
                ("shape", C.c_uint64 * 2), ("bytes", C.c_uint64)]


class turbo_token_range(C.Structure):
    _fields_ = [("row", C.c_uint32), ("start", C.c_uint32), ("end", C.c_uint32)]


class turbo_backend_tuning(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("mode", C.c_uint32), ("budget_ms", C.c_uint32),
                ("numerics_allowed", C.c_uint32), ("cached", C.c_char_p), ("tuned", C.c_uint32),
                ("tune_ms", C.c_uint32), ("choices", C.c_char * TURBO_CHOICES_LEN), ("timings", C.c_char_p),
                ("timings_len", C.c_uint32), ("numerics_used", C.c_uint32)]


class turbo_backend_tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("shape", C.c_uint64 * 2), ("ndim", C.c_uint32),
                ("dtype", C.c_uint32), ("bytes", C.c_uint64)]


class turbo_backend_model(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("family", C.c_uint32), ("dtype", C.c_uint32), ("layers", C.c_uint32),
                ("hidden", C.c_uint32), ("heads", C.c_uint32), ("intermediate", C.c_uint32),
                ("vocab_size", C.c_uint32), ("max_positions", C.c_uint32), ("token_types", C.c_uint32),
                ("layer_norm_eps", C.c_double), ("tensor_count", C.c_uint32), ("position_offset", C.c_uint32),
                ("tensors", C.POINTER(turbo_backend_tensor)), ("format", C.c_uint32), ("graph_input", C.c_uint32),
                ("graph_output", C.c_uint32), ("compute_dtype", C.c_uint32), ("fixed_seq", C.c_uint32),
                ("fixed_batch", C.c_uint32), ("artifact", C.c_void_p), ("artifact_bytes", C.c_uint64),
                ("artifact2", C.c_void_p), ("artifact2_bytes", C.c_uint64),
                ("head", C.POINTER(turbo_backend_tensor)), ("head_out", C.c_uint32), ("lookahead", C.c_uint32),
                ("position_buckets", C.c_uint32), ("max_relative_positions", C.c_uint32),
                ("artifact_sha256", C.c_uint8 * 32), ("artifact2_sha256", C.c_uint8 * 32),
                ("rope_global_theta", C.c_double), ("rope_local_theta", C.c_double),
                ("rope_table", C.POINTER(C.c_float)), ("rope_pairs", C.c_uint32), ("mlp", C.c_uint32),
                ("activation", C.c_uint32), ("norm", C.c_uint32), ("attention_window", C.c_uint32),
                ("global_every", C.c_uint32)]


class turbo_backend_session_desc(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("task", C.c_uint32), ("max_batch", C.c_uint32),
                ("max_seq", C.c_uint32), ("precision", C.c_uint32), ("cpu_threads", C.c_uint32),
                ("max_ranges", C.c_uint32), ("reserved", C.c_uint32)]


class turbo_backend_embed_rows(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("batch", C.c_uint32), ("seq", C.c_uint32),
                ("row_stride", C.c_uint32), ("ids", C.POINTER(C.c_int32)), ("mask", C.POINTER(C.c_int32)),
                ("types", C.POINTER(C.c_int32)), ("pooling", C.c_uint32), ("normalize", C.c_uint32),
                ("output_dim", C.c_uint32), ("head", C.c_uint32), ("taps", C.c_uint32), ("tap_alone", C.c_uint32)]


class turbo_backend_run(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("placement", C.c_uint32), ("output", C.c_void_p),
                ("host", C.c_void_p), ("h2d_bytes", C.c_uint64), ("d2h_bytes", C.c_uint64),
                ("host_allocs", C.c_uint64), ("device_allocs", C.c_uint64),
                ("stage", C.c_uint32 * TURBO_STAGE_MAX)]


_P = C.c_void_p
_u32 = C.c_uint32
_err = C.POINTER(turbo_error)


class turbo_backend(C.Structure):
    _fields_ = [
        ("struct_size", _u32), ("reserved", _u32), ("name", C.c_char_p), ("runtime_version", C.c_char_p),
        ("device_count", C.CFUNCTYPE(C.c_int32, C.POINTER(_u32), _err)),
        ("device_info", C.CFUNCTYPE(C.c_int32, _u32, C.POINTER(turbo_device_info), _err)),
        ("capability", C.CFUNCTYPE(C.c_int32, _u32, _u32, _u32, C.POINTER(_u32), C.POINTER(_u32),
                                   C.POINTER(_u32), C.c_char_p, _u32, _err)),
        ("context_create", C.CFUNCTYPE(C.c_int32, _u32, turbo_log_fn, _P, C.POINTER(_P), _err)),
        ("context_release", C.CFUNCTYPE(None, _P)),
        ("buffer_alloc", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_buffer_desc), C.POINTER(_P), C.POINTER(_P),
                                     _err)),
        ("buffer_import", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_buffer_desc), C.POINTER(turbo_native_handle),
                                      C.POINTER(_P), C.POINTER(_P), _err)),
        ("buffer_release", C.CFUNCTYPE(None, _P)),
        ("buffer_export", C.CFUNCTYPE(C.c_int32, _P, _u32, C.POINTER(turbo_native_handle), _err)),
        ("model_load", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_backend_model), C.POINTER(_P), _err)),
        ("model_release", C.CFUNCTYPE(None, _P)),
        ("session_create", C.CFUNCTYPE(C.c_int32, _P, _u32, _u32, _u32, _u32, C.POINTER(_u32), C.POINTER(_P),
                                       _err)),
        ("session_release", C.CFUNCTYPE(None, _P)),
        ("embed_write", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_backend_embed_rows), _err)),
        ("session_run", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_backend_run), _err)),
        ("buffer_read", C.CFUNCTYPE(C.c_int32, _P, _P, C.c_uint64, _err)),
        ("formats", _u32), ("reserved2", _u32),
        ("session_create_tuned", C.CFUNCTYPE(C.c_int32, _P, _u32, _u32, _u32, _u32,
                                             C.POINTER(turbo_backend_tuning), C.POINTER(_u32), C.POINTER(_P), _err)),
        ("session_open", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_backend_session_desc),
                                     C.POINTER(turbo_backend_tuning), C.POINTER(_u32), C.POINTER(_P), _err)),
        ("embed_write_ranges", C.CFUNCTYPE(C.c_int32, _P, C.POINTER(turbo_backend_embed_rows),
                                           C.POINTER(turbo_token_range), _u32, _err)),
        ("token_head", _u32), ("reserved3", _u32),
        ("buffer_quantize", C.CFUNCTYPE(C.c_int32, _P, _u32, C.POINTER(C.c_float), _u32, _u32,
                                        C.POINTER(turbo_backend_run), _err)),
    ]


def check_layout():
    """The offsets the reference core's Rust mirror holds the table to."""
    b = turbo_backend
    want = {"context_create": 48, "model_load": 96, "session_create": 112, "buffer_read": 144, "formats": 152,
            "session_create_tuned": 160, "session_open": 168, "token_head": 184, "buffer_quantize": 192}
    for name, off in want.items():
        got = getattr(b, name).offset
        assert got == off, f"turbo_backend.{name} at {got}, not {off}"
    assert C.sizeof(b) == 200
    assert C.sizeof(turbo_backend_model) == 256
    assert C.sizeof(turbo_backend_embed_rows) == 64
    assert C.sizeof(turbo_backend_run) == 120
    assert C.sizeof(turbo_backend_tuning) == 1072
    assert C.sizeof(turbo_error) == 508
    assert C.sizeof(turbo_device_info) == 416
    assert C.sizeof(turbo_token_range) == 12


def new_error():
    e = turbo_error()
    e.struct_size = C.sizeof(turbo_error)
    return e
