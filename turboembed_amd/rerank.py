"""The rerank caller of the encoder: pair windows over token ids, the
backend runs that encode them, and the sequence classification head.

Mirrors the reference core's turbo_rerank_write_pairs and run_pairs
(core/src/session/rerank.rs:47-219) and the pair template
(core/src/tokenizer/pair.rs:27-99) above the already-tokenized query and
passage; the work is done in C++ behind the library's C ABI
(turbo_rocm_pair_windows, turbo_rocm_rerank_run, turbo_rocm_rerank_scores).
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import seam as S

PAIR_BERT, PAIR_ROBERTA = 0, 1


@dataclass
class RerankHead:
    """A cross-encoder's head: BERT's pooler (dense + tanh; None for a model
    without one) and a one-logit classifier."""
    classifier_weight: np.ndarray           # [hidden] (or [1, hidden])
    classifier_bias: float = 0.0
    pooler_weight: np.ndarray = None        # [hidden, hidden]
    pooler_bias: np.ndarray = None          # [hidden]

    def arrays(self):
        cw = np.ascontiguousarray(np.asarray(self.classifier_weight, np.float32).ravel())
        pw = None if self.pooler_weight is None else np.ascontiguousarray(self.pooler_weight, np.float32)
        pb = None if self.pooler_bias is None else np.ascontiguousarray(self.pooler_bias, np.float32)
        return cw, pw, pb


def _p(a):
    return None if a is None else a.ctypes.data


def pair_windows(query, passage, start_id, end_id, template=PAIR_BERT, query_tokens=8, max_tokens=512, stride=0):
    """The encoder windows of one (query, passage) pair of token-id lists:
    (ids [n, max_tokens], types [n, max_tokens], lengths [n])."""
    from . import _ok, library
    lib = library()
    q = np.ascontiguousarray(query, np.int32)
    p = np.ascontiguousarray(passage, np.int32)
    room = max(1, max_tokens - 4)
    cap = len(p) // max(1, stride or 1) + 2 if stride else len(p) // room + 2
    cap = max(cap, 1)
    while True:
        ids = np.zeros((cap, max_tokens), np.int32)
        types = np.zeros((cap, max_tokens), np.int32)
        lengths = np.zeros(cap, np.uint32)
        n = C.c_uint32()
        err = S.new_error()
        rc = lib.turbo_rocm_pair_windows(_p(q), len(q), _p(p), len(p), start_id, end_id,
                                         1 if template == PAIR_ROBERTA else 0, query_tokens, max_tokens, stride,
                                         ids.ctypes.data, types.ctypes.data, lengths.ctypes.data, cap, C.byref(n),
                                         C.byref(err))
        if rc == S.TURBO_E_CAPACITY and n.value > cap:
            cap = n.value
            continue
        _ok(rc, err)
        return ids[: n.value], types[: n.value], lengths[: n.value]


def rerank(session, pairs, head, start_id, end_id, template=PAIR_BERT, query_tokens=8, max_tokens=0, stride=0):
    """One score per (query ids, passage ids) pair through a TURBO_TASK_RERANK
    session: each pair's windows encoded as CLS rows, the head applied in
    F64, the best window's logit kept (core/src/session/rerank.rs:47-219)."""
    from . import TurboError, _ok, library
    if not pairs:
        raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 0, "pairs is NULL or count is zero")
    if len(pairs) > session.max_batch:
        raise TurboError(S.TURBO_E_CAPACITY, 0, "pair count exceeds max_batch")
    if max_tokens > session.max_seq:
        raise TurboError(S.TURBO_E_CAPACITY, 2, "rerank max_tokens exceeds session max_seq")
    max_tokens = max_tokens or session.max_seq
    ids, types, lengths, owner = [], [], [], []
    for i, (q, p) in enumerate(pairs):
        wi, wt, wl = pair_windows(q, p, start_id, end_id, template, query_tokens, max_tokens, stride)
        ids.append(wi)
        types.append(wt)
        lengths.append(wl)
        owner += [i] * len(wl)
    lengths = np.concatenate(lengths).astype(np.uint32)
    seq = int(lengths.max())
    ids = np.ascontiguousarray(np.concatenate(ids)[:, :seq])
    types = np.ascontiguousarray(np.concatenate(types)[:, :seq])
    owner = np.asarray(owner, np.uint32)
    cw, pw, pb = head.arrays()
    scores = np.empty(len(pairs), np.float32)
    err = S.new_error()
    _ok(library().turbo_rocm_rerank_run(session.h, ids.ctypes.data, types.ctypes.data, lengths.ctypes.data,
                                        len(lengths), seq, owner.ctypes.data, len(pairs), _p(pw), _p(pb),
                                        cw.ctypes.data, float(head.classifier_bias), scores.ctypes.data,
                                        C.byref(err)), err)
    return scores


def head_scores(states, head):
    """The head alone over CLS states [n, hidden] (F64 sums, as the core)."""
    from . import _ok, library
    x = np.ascontiguousarray(states, np.float32)
    cw, pw, pb = head.arrays()
    out = np.empty(x.shape[0], np.float32)
    err = S.new_error()
    _ok(library().turbo_rocm_rerank_scores(x.ctypes.data, x.shape[0], x.shape[1], _p(pw), _p(pb), cw.ctypes.data,
                                           float(head.classifier_bias), out.ctypes.data, C.byref(err)), err)
    return out
