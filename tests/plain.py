"""Textbook encoders in float64 numpy, the closed form the oracle is pinned to.

Written from the architectures' definitions, not from the oracle: numpy
matrix products, softmax by np.exp, GELU by math.erf, LayerNorm as
(x - mean) / sqrt(var + eps) * w + b, RoPE as transformers' rotate_half over
the stored column order. The reference holds its CPU and CUDA paths to the
same kind of f64 BERT (core/tests/common/plain_bert.rs:6-171) within
1e-5 * (1 + |w|).
"""
import math

import numpy as np

from turboembed_amd import seam as S

_erf = np.vectorize(math.erf)


def gelu(x):
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def ln(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps) * w
    return y + b if b is not None else y


def attention(q, k, v, live, window=None):
    """q, k, v [n, heads, d]; live [n] bool over keys."""
    n, heads, d = q.shape
    s = np.einsum("ihd,jhd->hij", q, k) / math.sqrt(d)
    allowed = np.broadcast_to(live[None, :], (n, n)).copy()
    if window is not None:
        i = np.arange(n)
        allowed &= np.abs(i[:, None] - i[None, :]) <= window
    s = np.where(allowed[None], s, -np.inf)
    mx = s.max(-1, keepdims=True)
    none = ~np.isfinite(mx)
    p = np.exp(s - np.where(none, 0.0, mx))
    p = np.where(none, 0.0, p)
    tot = p.sum(-1, keepdims=True)
    p = p / np.where(tot == 0, 1.0, tot)
    return np.einsum("hij,jhd->ihd", p, v).reshape(n, heads * d)


def _f64(t):
    if t is None:
        return None
    if t.dtype == np.uint16:
        return (t.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return t.astype(np.float64)


def bert_states(desc, ids, mask, types):
    """Final hidden states of one row, through its last live token."""
    t = [_f64(x) for x in desc.tensors]
    H, heads = desc.hidden, desc.heads
    d = H // heads
    n = int(np.nonzero(mask)[0].max()) + 1
    live = mask[:n] != 0
    pos = np.arange(n) + desc.position_offset
    x = t[0][ids[:n]] + t[1][pos] + t[2][types[:n]]
    x = ln(x, t[3], t[4], desc.layer_norm_eps)
    for l in range(desc.layers):
        w = t[S.BERT_EMBEDDING_TENSORS + l * S.BERT_LAYER_TENSORS:][:S.BERT_LAYER_TENSORS]
        q = (x @ w[0].T + w[1]).reshape(n, heads, d)
        k = (x @ w[2].T + w[3]).reshape(n, heads, d)
        v = (x @ w[4].T + w[5]).reshape(n, heads, d)
        a = attention(q, k, v, live)
        x = ln(x + a @ w[6].T + w[7], w[8], w[9], desc.layer_norm_eps)
        f = gelu(x @ w[10].T + w[11])
        x = ln(x + f @ w[12].T + w[13], w[14], w[15], desc.layer_norm_eps)
    return x, live


def rope(x, theta, pos):
    """rotate_half RoPE over [n, heads, d] in the stored column order."""
    n, heads, d = x.shape
    inv = 1.0 / theta ** (np.arange(0, d, 2) / d)
    ang = pos[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang)] * 2, -1)[:, None, :]
    sin = np.concatenate([np.sin(ang)] * 2, -1)[:, None, :]
    rot = np.concatenate([-x[..., d // 2:], x[..., : d // 2]], -1)
    return x * cos + rot * sin


def rotary_states(desc, ids, mask, types, gated_limit=0.0):
    """ModernBERT (pre-norm, alternating windows) or nomic-bert (post-norm),
    as turbo_backend.h:107-153 describes them; gated_limit > 0 clips the
    gated product act(gate) * up to that magnitude."""
    clip = (lambda g: np.clip(g, -gated_limit, gated_limit)) if gated_limit > 0 else (lambda g: g)  # noqa: E731
    t = [_f64(x) for x in desc.tensors]
    H, heads, I = desc.hidden, desc.heads, desc.intermediate
    d = H // heads
    n = int(np.nonzero(mask)[0].max()) + 1
    live = mask[:n] != 0
    pos = np.arange(n, dtype=np.float64)
    eps = desc.layer_norm_eps
    g_theta, l_theta = desc.rope
    act = silu if desc.activation == S.TURBO_ACTIVATION_SILU else gelu
    if desc.family == S.TURBO_FAMILY_MODERNBERT:
        x = ln(t[0][ids[:n]], t[1], None, eps)
        for l in range(desc.layers):
            w = t[S.MODERNBERT_EMBEDDING_TENSORS + l * S.MODERNBERT_LAYER_TENSORS:][:S.MODERNBERT_LAYER_TENSORS]
            glob = l % desc.global_every == 0
            h = x if l == 0 else ln(x, w[0], None, eps)
            qkv = h @ w[1].T
            q, k, v = (qkv[:, i * H:(i + 1) * H].reshape(n, heads, d) for i in range(3))
            th = g_theta if glob else l_theta
            q, k = rope(q, th, pos), rope(k, th, pos)
            a = attention(q, k, v, live, None if glob else desc.attention_window // 2)
            x = x + a @ w[2].T
            h = ln(x, w[3], None, eps)
            y = h @ w[4].T
            x = x + clip(act(y[:, :I]) * y[:, I:]) @ w[5].T
        return ln(x, t[2], None, eps), live
    x = ln(t[0][ids[:n]] + t[1][types[:n]], t[2], t[3], eps)
    for l in range(desc.layers):
        w = t[S.NOMIC_EMBEDDING_TENSORS + l * S.NOMIC_LAYER_TENSORS:][:S.NOMIC_LAYER_TENSORS]
        qkv = x @ w[0].T
        q, k, v = (qkv[:, i * H:(i + 1) * H].reshape(n, heads, d) for i in range(3))
        q, k = rope(q, g_theta, pos), rope(k, g_theta, pos)
        a = attention(q, k, v, live)
        x = ln(x + a @ w[1].T, w[2], w[3], eps)
        x = ln(x + clip(act(x @ w[4].T) * (x @ w[5].T)) @ w[6].T, w[7], w[8], eps)
    return x, live


def log_bucket(rel, buckets, maximum):
    """transformers' make_log_bucket_position over an array of signed
    distances, its logarithms in float32, offset by the buckets and clamped
    to the table."""
    mid = buckets // 2
    rel = np.asarray(rel, np.int64)
    sign = np.sign(rel)
    a = np.where((rel < mid) & (rel > -mid), mid - 1, np.abs(rel))
    log_pos = np.ceil(np.log(a.astype(np.float32) / np.float32(mid)) /
                      np.log(np.float32(maximum - 1) / np.float32(mid)) * np.float32(mid - 1)).astype(np.int64) + mid
    signed = np.where(np.abs(rel) <= mid, rel, log_pos * sign)
    return np.clip(signed + buckets, 0, 2 * buckets - 1)


def deberta_states(desc, ids, mask, types=None, uniform_masked=True):
    """Final hidden states of one DeBERTa-v2 row (shared keys, c2p and p2c),
    through its last live token: embeddings LayerNorm'd and zeroed where
    masked; scores (q k + q pos_k[b(i - j)] + k pos_q[b(i - j)]) / sqrt(3 d),
    p2c gathered at the negated distance and transposed; masked pairs take
    the most negative finite value, so a masked query attends uniformly."""
    t = [_f64(x) for x in desc.tensors]
    H, heads = desc.hidden, desc.heads
    d = H // heads
    buckets, maximum = desc.relative
    n = int(np.nonzero(mask)[0].max()) + 1
    live = mask[:n] != 0
    x = ln(t[0][ids[:n]], t[1], t[2], desc.layer_norm_eps) * live[:, None]
    rel = ln(t[3][: 2 * buckets], t[4], t[5], desc.layer_norm_eps)
    pos = np.arange(n)
    r = log_bucket(pos[:, None] - pos[None, :], buckets, maximum)            # [i, j]
    # (uniform_masked=False plants a mistake for the tests: masked queries
    # reading the live keys, as a visible query does.)
    allowed = live[:, None] & live[None, :] if uniform_masked else np.broadcast_to(live[None, :], (n, n))
    for l in range(desc.layers):
        w = t[S.DEBERTA_EMBEDDING_TENSORS + l * S.BERT_LAYER_TENSORS:][:S.BERT_LAYER_TENSORS]
        q = (x @ w[0].T + w[1]).reshape(n, heads, d)
        k = (x @ w[2].T + w[3]).reshape(n, heads, d)
        v = (x @ w[4].T + w[5]).reshape(n, heads, d)
        pq = (rel @ w[0].T + w[1]).reshape(-1, heads, d)
        pk = (rel @ w[2].T + w[3]).reshape(-1, heads, d)
        c2c = np.einsum("ihd,jhd->hij", q, k)
        c2p_all = np.einsum("ihd,rhd->hir", q, pk)
        c2p = np.take_along_axis(c2p_all, np.broadcast_to(r[None], c2c.shape), axis=2)
        p2c_all = np.einsum("jhd,rhd->hjr", k, pq)
        # transformers: index with the negated distance's bucket, then transpose.
        r_neg = log_bucket(pos[None, :] - pos[:, None], buckets, maximum)      # [i, j] -> bucket(j - i)
        p2c_idx = 2 * buckets - r_neg                                            # -bucket(j - i) offset back
        p2c_idx = np.clip(p2c_idx, 0, 2 * buckets - 1).T                        # as [j, i]
        p2c = np.take_along_axis(p2c_all, np.broadcast_to(p2c_idx[None], c2c.shape), axis=2).transpose(0, 2, 1)
        s = (c2c + c2p + p2c) / math.sqrt(3 * d)
        s = np.where(allowed[None], s, np.finfo(np.float32).min)
        p = np.exp(s - s.max(-1, keepdims=True))
        p = p / p.sum(-1, keepdims=True)
        a = np.einsum("hij,jhd->ihd", p, v).reshape(n, H)
        x = ln(x + a @ w[6].T + w[7], w[8], w[9], desc.layer_norm_eps)
        f = gelu(x @ w[10].T + w[11])
        x = ln(x + f @ w[12].T + w[13], w[14], w[15], desc.layer_norm_eps)
    return x, live


def embed(desc, ids, mask, types=None, pooling=S.TURBO_POOLING_MEAN, normalize=S.TURBO_NORMALIZE_L2,
          output_dim=None, gated_limit=0.0):
    """Pooled, cut and normalized vectors of each row, float64."""
    types = np.zeros_like(ids) if types is None else types
    states = rotary_states if desc.rotary else deberta_states if desc.family == S.TURBO_FAMILY_DEBERTA_V2 else bert_states
    kw = dict(gated_limit=gated_limit) if desc.rotary else {}
    out = []
    for r in range(ids.shape[0]):
        x, live = states(desc, ids[r], mask[r], types[r], **kw)
        if pooling == S.TURBO_POOLING_CLS:
            v = x[0]
        elif pooling == S.TURBO_POOLING_LAST:
            v = x[len(live) - 1]
        else:
            v = x[live].mean(0)
        v = v[: output_dim or desc.hidden]
        if normalize == S.TURBO_NORMALIZE_L2:
            v = v / max(np.linalg.norm(v), 1e-12)
        out.append(v)
    return np.array(out)
