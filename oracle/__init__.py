"""The oracle: the CPU restatement of TurboEmbed's CPU encoder (oracle.cpp).

Test infrastructure only. Tests, the smoke check and the benchmark's CPU
baseline call it as the checker; no product code imports it.
"""
import ctypes as C
import json
import os
import subprocess

import numpy as np

from turboembed_amd import seam as S
from turboembed_amd.model import ModelDesc

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
GOLDEN = os.path.join(os.path.dirname(HERE), "tests", "golden")

_lib = None


def build():
    """Compile oracle.cpp into liboracle.so (a few seconds)."""
    subprocess.check_call(["make", "-s", "-C", HERE, "-B"])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = C.CDLL(LIB)
        _lib.oracle_encode.restype = C.c_int32
        _lib.oracle_encode.argtypes = [C.POINTER(S.turbo_backend_model), C.POINTER(S.turbo_backend_embed_rows),
                                       C.POINTER(S.turbo_token_range), C.c_uint32, C.c_uint32, C.c_void_p,
                                       C.c_void_p, C.c_char_p, C.c_uint32]
        _lib.oracle_pack.restype = C.c_uint32
        _lib.oracle_pack.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(S.turbo_token_range),
                                     C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]
        for f in ("oracle_exp", "oracle_gelu", "oracle_silu"):
            getattr(_lib, f).restype = C.c_float
            getattr(_lib, f).argtypes = [C.c_float]
        _lib.oracle_layer_norm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_float]
        _lib.oracle_quantize.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        _lib.oracle_quantize.restype = None
        _lib.oracle_deberta_bucket.argtypes = [C.c_int64, C.c_uint32, C.c_uint32]
        _lib.oracle_deberta_bucket.restype = C.c_uint32
        _lib.oracle_set_gated_limit.argtypes = [C.c_float]
        _lib.oracle_set_gated_limit.restype = None
        _lib.oracle_set_pinning.argtypes = [C.c_int32]
        _lib.oracle_set_pinning.restype = None
        _lib.oracle_last_encode_seconds.argtypes = []
        _lib.oracle_last_encode_seconds.restype = C.c_double
    return _lib


def rows_struct(ids, mask, types, pooling, normalize, output_dim):
    r = S.turbo_backend_embed_rows()
    r.struct_size = C.sizeof(S.turbo_backend_embed_rows)
    r.batch, r.seq = ids.shape
    r.row_stride = ids.shape[1]
    r.ids = ids.ctypes.data_as(C.POINTER(C.c_int32))
    r.mask = mask.ctypes.data_as(C.POINTER(C.c_int32))
    r.types = types.ctypes.data_as(C.POINTER(C.c_int32)) if types is not None else None
    r.pooling, r.normalize, r.output_dim = pooling, normalize, output_dim
    r.head, r.taps, r.tap_alone = 0, 1, 0
    return r


def ranges_array(ranges):
    arr = (S.turbo_token_range * max(1, len(ranges)))()
    for i, (row, start, end) in enumerate(ranges):
        arr[i].row, arr[i].start, arr[i].end = row, start, end
    return arr


def encode(desc: ModelDesc, ids, mask, types=None, pooling=S.TURBO_POOLING_MEAN, normalize=S.TURBO_NORMALIZE_L2,
           output_dim=None, ranges=None, threads=0, hidden=False, head=False, taps=1, tap_alone=False,
           gated_limit=0.0):
    """The oracle's vectors for the rows (and ranges); with hidden=True also
    the final hidden states of the packed tokens. head=True on a range write
    to a model with a span head: each range's row is the head's logits.
    taps > 1 on a range write: the ranges pooled from each of the last taps
    layers, [taps * count, od] block by block; with tap_alone the first of
    those layers alone, [count, od]. gated_limit > 0 saturates the gated
    MLP's product at that magnitude (an F16 tier's 65504), for this call."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    types = None if types is None else np.ascontiguousarray(types, dtype=np.int32)
    od = desc.span_head[0].shape[0] if head and desc.span_head is not None else output_dim or desc.hidden
    r = rows_struct(ids, mask, types, pooling, normalize, od)
    r.head = 1 if head else 0
    r.taps, r.tap_alone = taps, 1 if tap_alone else 0
    ranges = list(ranges or [])
    rr = ranges_array(ranges)
    n_out = len(ranges) * (1 if tap_alone else max(1, taps)) if ranges else ids.shape[0]
    out = np.zeros((n_out, od), dtype=np.float32)
    hid = np.zeros((ids.shape[0] * ids.shape[1], desc.hidden), dtype=np.float32) if hidden else None
    why = C.create_string_buffer(512)
    if threads == 0:
        # The cores this process may run on (its affinity, not the host's count).
        threads = len(os.sched_getaffinity(0))
    lib().oracle_set_gated_limit(gated_limit)
    try:
        rc = lib().oracle_encode(C.byref(desc.struct()), C.byref(r), rr, len(ranges), threads, out.ctypes.data,
                                 None if hid is None else hid.ctypes.data, why, 512)
    finally:
        lib().oracle_set_gated_limit(0.0)
    if rc != 0:
        raise RuntimeError(f"oracle: {S.STATUS_NAMES.get(rc, rc)}: {why.value.decode()}")
    if hidden:
        _, ln, _ = pack(mask, ranges)
        return out, hid[: int(ln.sum())]
    return out


def quantize(x, mode, ranges=None):
    """Codes of the rows of x (F32, [rows, dim]): mode 2 int8 with ranges
    [2, dim], mode 3 ubinary; as the reference core makes them
    (core/src/quantize.rs:48-80)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, dim = x.shape
    width = dim if mode == 2 else (dim + 7) // 8
    out = np.zeros((rows, width), np.uint8)
    rr = None if ranges is None else np.ascontiguousarray(ranges, np.float32)
    lib().oracle_quantize(C.c_void_p(x.ctypes.data), rows, dim, mode, None if rr is None else C.c_void_p(rr.ctypes.data),
                          C.c_void_p(out.ctypes.data))
    return out


def pack(mask, ranges=()):
    """(start, len, at) of the oracle's packing for `mask` [batch, seq]."""
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    b, s = mask.shape
    start = np.zeros(b, np.uint32)
    ln = np.zeros(b, np.uint32)
    at = np.zeros(b * s, np.uint32)
    rr = ranges_array(list(ranges))
    t = lib().oracle_pack(mask.ctypes.data, b, s, s, rr, len(ranges), start.ctypes.data, ln.ctypes.data, at.ctypes.data)
    return start, ln, at[:t]


# ---- The reference's sealed tiny bundles (tests/golden/) --------------------

_FAMILIES = {"FAMILY_BERT": S.TURBO_FAMILY_BERT, "FAMILY_MODERNBERT": S.TURBO_FAMILY_MODERNBERT,
             "FAMILY_NOMIC_BERT": S.TURBO_FAMILY_NOMIC_BERT, "FAMILY_DEBERTA_V2": S.TURBO_FAMILY_DEBERTA_V2}


def fixture(name):
    """(ModelDesc, ids, lengths, vectors, info) of a golden fixture: the
    reference bundle's weights and its upstream fp32 reference cases."""
    from safetensors.numpy import load_file
    t = load_file(os.path.join(GOLDEN, name + ".safetensors"))
    info = json.load(open(os.path.join(GOLDEN, name + ".json")))
    a = info["architecture"]
    family = _FAMILIES[info["family"]]
    tensors = [t[k] if k else None for k in info["order"]]
    kw = {}
    if family == S.TURBO_FAMILY_MODERNBERT:
        kw = dict(rope=(a["rope"]["global_theta"], a["rope"]["local_theta"]), attention_window=a["attention"]["window"],
                  global_every=a["attention"]["global_every"], mlp=S.TURBO_MLP_GATED,
                  activation=S.TURBO_ACTIVATION_GELU_ERF, norm=S.TURBO_NORM_LAYER_NO_BIAS)
    elif family == S.TURBO_FAMILY_DEBERTA_V2:
        kw = dict(relative=(a["relative"]["position_buckets"], a["relative"]["max_relative_positions"]))
    elif family == S.TURBO_FAMILY_NOMIC_BERT:
        g = a["rope"]["global_theta"]
        kw = dict(rope=(g, g), mlp=S.TURBO_MLP_GATED, activation=S.TURBO_ACTIVATION_SILU, norm=S.TURBO_NORM_LAYER)
    desc = ModelDesc(family, a["layers"], a["hidden"], a["heads"], a["intermediate"], info["vocab_rows_kept"],
                     a["max_positions"], max(1, a["token_types"]), a["layer_norm_eps"], tensors,
                     names=[k or "absent" for k in info["order"]], **kw)
    return desc, t["case.ids"], t["case.lengths"], t["case.vectors"], info


def qa_fixture():
    """(ModelDesc, windows, logits, info) of tests/golden/tiny_qa: the tiny
    BERT encoder with its span head, the reference's QA windows as
    [(ids, types)], and the transformers logits [tokens, 2] (start, end) of
    every window's tokens in order."""
    from safetensors.numpy import load_file
    t = load_file(os.path.join(GOLDEN, "tiny_qa.safetensors"))
    info = json.load(open(os.path.join(GOLDEN, "tiny_qa.json")))
    a = info["architecture"]
    desc = ModelDesc(S.TURBO_FAMILY_BERT, a["layers"], a["hidden"], a["heads"], a["intermediate"],
                     info["vocab_rows_kept"], a["max_positions"], a["token_types"], a["layer_norm_eps"],
                     [t[k] for k in info["order"]], names=info["order"],
                     span_head=(t["head.weight"], t["head.bias"]))
    windows = [(t["case.ids"][i, :n].copy(), t["case.types"][i, :n].copy())
               for i, n in enumerate(t["case.lengths"])]
    return desc, windows, t["case.logits"], info


def qa_logits(desc, windows, pad_id=0):
    """The start and end logits [tokens, 2] of every window's tokens, in
    order, restating core/src/qa/session.rs:196-290: the windows as rows
    padded with pad_id (types 0, mask 0), each live token a range of its
    own, through the span head."""
    seq = max(len(w) for w, _ in windows)
    ids = np.full((len(windows), seq), pad_id, np.int32)
    types = np.zeros_like(ids)
    mask = np.zeros_like(ids)
    ranges = []
    for r, (wi, wt) in enumerate(windows):
        ids[r, :len(wi)], types[r, :len(wt)], mask[r, :len(wi)] = wi, wt, 1
        ranges += [(r, i, i + 1) for i in range(len(wi))]
    return encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges, head=True)


def fixture_rows(ids, lengths):
    """The reference cases as rows: each case's ids, mask 1 through its length."""
    mask = (np.arange(ids.shape[1])[None, :] < lengths[:, None]).astype(np.int32)
    return np.ascontiguousarray(ids, dtype=np.int32), mask


# ---- The rerank caller (pure Python and numpy: a handful of windows) ----------

def pair_windows(query, passage, start_id, end_id, roberta=False, query_tokens=8, max_tokens=512, stride=0):
    """[(ids, types)] of one pair's encoder windows, restating
    core/src/tokenizer/pair.rs:27-99 over token ids."""
    specials = 4 if roberta else 3
    if max_tokens <= specials + 1 or query_tokens >= max_tokens - specials:
        raise ValueError("pair limits leave no passage token")
    q = list(query)[:query_tokens]
    room = max_tokens - specials - len(q)
    step = room if stride == 0 else stride
    if step == 0 or step > room:
        raise ValueError("pair stride must be within passage capacity")
    out, start = [], 0
    while True:
        end = min(start + room, len(passage))
        ids = [start_id] + q + [end_id] + ([end_id] if roberta else [])
        boundary = len(ids)
        ids += list(passage[start:end]) + [end_id]
        types = [0] * len(ids)
        if not roberta:
            types[boundary:] = [1] * (len(ids) - boundary)
        out.append((ids, types))
        if end == len(passage):
            return out
        start += step


def rerank_head(states, classifier_weight, classifier_bias, pooler_weight=None, pooler_bias=None):
    """Logits of CLS states [n, hidden], restating core/src/session/rerank.rs:166-191:
    the pooler's rows summed in F64 from the bias, tanh, rounded to F32, then
    the classifier's row the same way."""
    x = np.asarray(states, np.float32).astype(np.float64)
    if pooler_weight is not None:
        pb = np.zeros(x.shape[1]) if pooler_bias is None else np.asarray(pooler_bias, np.float64)
        x = np.tanh(pb[None, :] + x @ np.asarray(pooler_weight, np.float64).T).astype(np.float32).astype(np.float64)
    w = np.asarray(classifier_weight, np.float64).ravel()
    return (float(classifier_bias) + x @ w).astype(np.float32)


def rerank(desc, pairs, head, start_id, end_id, roberta=False, query_tokens=8, max_tokens=512, stride=0):
    """Each pair's score: its windows through the oracle encoder as CLS rows
    (no normalization, full width), the head, the largest window logit
    (core/src/session/rerank.rs:111-219)."""
    wins, owner = [], []
    for i, (q, p) in enumerate(pairs):
        w = pair_windows(q, p, start_id, end_id, roberta, query_tokens, max_tokens, stride)
        wins += w
        owner += [i] * len(w)
    seq = max(len(ids) for ids, _ in wins)
    ids = np.zeros((len(wins), seq), np.int32)
    types = np.zeros_like(ids)
    mask = np.zeros_like(ids)
    for r, (wi, wt) in enumerate(wins):
        ids[r, :len(wi)] = wi
        types[r, :len(wt)] = wt
        mask[r, :len(wi)] = 1
    states = encode(desc, ids, mask, types, pooling=S.TURBO_POOLING_CLS, normalize=S.TURBO_NORMALIZE_NONE)
    logits = rerank_head(states, **head)
    scores = np.full(len(pairs), -np.inf, np.float32)
    for r, i in enumerate(owner):
        scores[i] = max(scores[i], logits[r])
    return scores


def rerank_fixture():
    """(ModelDesc, pairs, head, info, reference) of tests/golden/tiny_rerank:
    the tiny BERT encoder, its (query ids, passage ids) pairs, the head as
    rerank_head's keywords, and the reference's first windows and
    transformers scores."""
    from safetensors.numpy import load_file
    t = load_file(os.path.join(GOLDEN, "tiny_rerank.safetensors"))
    info = json.load(open(os.path.join(GOLDEN, "tiny_rerank.json")))
    a = info["architecture"]
    desc = ModelDesc(S.TURBO_FAMILY_BERT, a["layers"], a["hidden"], a["heads"], a["intermediate"],
                     info["vocab_rows_kept"], a["max_positions"], a["token_types"], a["layer_norm_eps"],
                     [t[k] for k in info["order"]], names=info["order"])
    pairs = list(zip(info["queries"], info["passages"]))
    head = dict(classifier_weight=t["head.classifier.weight"], classifier_bias=float(t["head.classifier.bias"][0]),
                pooler_weight=t["head.bert.pooler.dense.weight"], pooler_bias=t["head.bert.pooler.dense.bias"])
    ref = dict(first_ids=t["case.first_ids"], first_types=t["case.first_types"],
               first_lengths=t["case.first_lengths"], scores=t["case.scores"])
    return desc, pairs, head, info, ref


def last_encode_seconds():
    """Seconds the last encode spent on its rows (the weights' layout
    before it excluded)."""
    return float(lib().oracle_last_encode_seconds())


def set_pinning(on):
    """Worker threads pin themselves to this process's CPUs, one each."""
    lib().oracle_set_pinning(1 if on else 0)


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None
