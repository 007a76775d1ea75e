"""The encoder workloads this backend is measured and checked on.

Six encoder shapes with seeded random weights and seeded synthetic rows:

  minilm       MiniLM-L6-shaped BERT: 6 layers, hidden 384, 12 heads, FFN 1536 GELU,
               vocab 30522, 512 positions; 32 rows of lengths U[16, 128] padded to 128;
               MEAN pooling + L2; EXACT (F32).
  bert-base    BERT-base-shaped: 12 layers, hidden 768, 12 heads, FFN 3072 GELU,
               vocab 30522; 64 rows x 512 all live (or lengths U[64, 512]); CLS + L2;
               weights stored F32, FASTEST (F16).
  xlmr-large   XLM-R-large-shaped (BGE-M3 dims): 24 layers, hidden 1024, 16 heads,
               FFN 4096 GELU, vocab 250002, RoBERTa positions from offset 2 (8194 rows);
               8 rows x 4096, lengths U[1024, 4096]; 64 contiguous ranges per row;
               weights stored BF16 (BF16 tier).
  modernbert   ModernBERT-base-shaped: 22 layers, hidden 768, 12 heads, GeGLU FFN
               (768 -> 2 x 1152, 1152 -> 768), no biases, RoPE theta 160000 global /
               10000 local, every 3rd layer global, 128-token window otherwise, vocab
               50368; 16 rows x 8192, lengths U[2048, 8192]; MEAN; F16.
  rerank       a BERT-base-shaped cross-encoder in the int8 tier (int8 weights per
               output channel, int8 activations per token): 256 (query, passage)
               pairs, queries U[8, 32] tokens, passages U[64, 480] cut so each pair's
               one window [CLS] q [SEP] p [SEP] fits 512; types 0 then 1; CLS ->
               pooler (dense 768 + tanh) -> one logit.
  deberta-v3-base
               DeBERTa-v3-base-shaped DeBERTa-v2 encoder: 12 layers, hidden 768, 12
               heads, FFN 3072 GELU, vocab 128100, relative attention over 256
               log buckets to distance 512 (shared keys); 64 rows x 512 all live;
               MEAN + L2; FASTEST (F16).

Weights are N(0, 0.02) from numpy's PCG64 seeded by (workload seed, tensor
index), so every tensor is reproducible on its own; LayerNorm weights are 1
and biases 0; linear biases N(0, 0.02). Token ids are U[1000, vocab) with
[CLS] = 101 first and [SEP] = 102 last in each row (0 and 2 for the RoBERTa
and ModernBERT shapes), padding id 0 (1 for RoBERTa) under mask 0.
"""
from dataclasses import dataclass, field

import numpy as np

from . import seam as S
from .model import ModelDesc, with_dtype


@dataclass
class Shape:
    name: str
    family: int
    layers: int
    hidden: int
    heads: int
    intermediate: int
    vocab: int
    positions: int
    token_types: int
    eps: float
    position_offset: int = 0
    rope: tuple = None
    window: int = 0
    global_every: int = 0
    seed: int = 0
    cls_id: int = 101
    sep_id: int = 102
    pad_id: int = 0
    store: str = "f32"          # the dtype the weights are stored in
    precision: int = S.TURBO_PRECISION_EXACT
    pooling: int = S.TURBO_POOLING_MEAN
    normalize: int = S.TURBO_NORMALIZE_L2
    batch: int = 1
    seq: int = 128
    lengths: tuple = None       # (lo, hi) uniform, or None for all full
    ranges_per_row: int = 0
    compute_dtype: int = 0      # TURBO_DTYPE_I8 for the int8 tier
    task: int = S.TURBO_TASK_EMBED
    extra: dict = field(default_factory=dict)


SHAPES = {
    "minilm": Shape("minilm", S.TURBO_FAMILY_BERT, 6, 384, 12, 1536, 30522, 512, 2, 1e-12, seed=1,
                    precision=S.TURBO_PRECISION_EXACT, pooling=S.TURBO_POOLING_MEAN, batch=32, seq=128,
                    lengths=(16, 128)),
    "bert-base": Shape("bert-base", S.TURBO_FAMILY_BERT, 12, 768, 12, 3072, 30522, 512, 2, 1e-12, seed=2,
                       precision=S.TURBO_PRECISION_FASTEST, pooling=S.TURBO_POOLING_CLS, batch=64, seq=512,
                       lengths=None),
    "xlmr-large": Shape("xlmr-large", S.TURBO_FAMILY_ROBERTA, 24, 1024, 16, 4096, 250002, 8194, 1, 1e-5,
                        position_offset=2, seed=3, cls_id=0, sep_id=2, pad_id=1, store="bf16",
                        precision=S.TURBO_PRECISION_MODEL, pooling=S.TURBO_POOLING_MEAN, batch=8, seq=4096,
                        lengths=(1024, 4096), ranges_per_row=64),
    "modernbert": Shape("modernbert", S.TURBO_FAMILY_MODERNBERT, 22, 768, 12, 1152, 50368, 8192, 1, 1e-5,
                        rope=(160000.0, 10000.0), window=128, global_every=3, seed=4, cls_id=50281, sep_id=50282,
                        pad_id=50283, precision=S.TURBO_PRECISION_FASTEST, pooling=S.TURBO_POOLING_MEAN,
                        normalize=S.TURBO_NORMALIZE_NONE, batch=16, seq=8192, lengths=(2048, 8192)),
    "deberta-v3-base": Shape("deberta-v3-base", S.TURBO_FAMILY_DEBERTA_V2, 12, 768, 12, 3072, 128100, 512, 1, 1e-7,
                             seed=6, cls_id=1, sep_id=2, pad_id=0, precision=S.TURBO_PRECISION_FASTEST,
                             pooling=S.TURBO_POOLING_MEAN, batch=64, seq=512, lengths=None,
                             extra={"relative": (256, 512)}),
    "rerank": Shape("rerank", S.TURBO_FAMILY_BERT, 12, 768, 12, 3072, 30522, 512, 2, 1e-12, seed=5,
                    precision=S.TURBO_PRECISION_FASTEST, pooling=S.TURBO_POOLING_CLS,
                    normalize=S.TURBO_NORMALIZE_NONE, batch=256, seq=512, compute_dtype=S.TURBO_DTYPE_I8,
                    task=S.TURBO_TASK_RERANK,
                    extra=dict(query=(8, 32), passage=(64, 480), query_tokens=32)),
}


def _normal(seed, index, shape, std=0.02):
    g = np.random.Generator(np.random.PCG64([seed, index]))
    return (g.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def model(shape: Shape, layers=None):
    """The workload's model description; `layers` cuts the encoder's depth
    (for parity tests at full width on a small budget)."""
    L = shape.layers if layers is None else layers
    H, I = shape.hidden, shape.intermediate
    idx = iter(range(1 << 20))
    w = lambda *sh: _normal(shape.seed, next(idx), sh)          # noqa: E731
    ones = lambda n: np.ones(n, np.float32)                      # noqa: E731
    zeros = lambda n: np.zeros(n, np.float32)                    # noqa: E731
    if shape.family in (S.TURBO_FAMILY_BERT, S.TURBO_FAMILY_ROBERTA):
        t = [w(shape.vocab, H), w(shape.positions, H), w(shape.token_types, H), ones(H), zeros(H)]
        for _ in range(L):
            t += [w(H, H), w(H), w(H, H), w(H), w(H, H), w(H), w(H, H), w(H), ones(H), zeros(H),
                  w(I, H), w(I), w(H, I), w(H), ones(H), zeros(H)]
        desc = ModelDesc(shape.family, L, H, shape.heads, I, shape.vocab, shape.positions, shape.token_types,
                         shape.eps, t, position_offset=shape.position_offset)
    elif shape.family == S.TURBO_FAMILY_MODERNBERT:
        t = [w(shape.vocab, H), ones(H), ones(H)]
        for l in range(L):
            t += [None if l == 0 else ones(H), w(3 * H, H), w(H, H), ones(H), w(2 * I, H), w(H, I)]
        desc = ModelDesc(shape.family, L, H, shape.heads, I, shape.vocab, shape.positions, shape.token_types,
                         shape.eps, t, rope=shape.rope, attention_window=shape.window,
                         global_every=shape.global_every, mlp=S.TURBO_MLP_GATED,
                         activation=S.TURBO_ACTIVATION_GELU_ERF, norm=S.TURBO_NORM_LAYER_NO_BIAS)
    elif shape.family == S.TURBO_FAMILY_DEBERTA_V2:
        buckets, maximum = shape.extra["relative"]
        t = [w(shape.vocab, H), ones(H), zeros(H), w(2 * buckets, H), ones(H), zeros(H)]
        for _ in range(L):
            t += [w(H, H), w(H), w(H, H), w(H), w(H, H), w(H), w(H, H), w(H), ones(H), zeros(H),
                  w(I, H), w(I), w(H, I), w(H), ones(H), zeros(H)]
        desc = ModelDesc(shape.family, L, H, shape.heads, I, shape.vocab, shape.positions, shape.token_types,
                         shape.eps, t, relative=(buckets, maximum))
    else:
        raise ValueError(shape.family)
    desc.compute_dtype = shape.compute_dtype
    return with_dtype(desc, shape.store) if shape.store != "f32" else desc


def rerank_pairs(shape: Shape, n=None, seed=0):
    """(query ids, passage ids) pairs: lengths uniform in the shape's
    ranges, ids U[1000, vocab), each passage cut so its pair fits one window."""
    n = shape.batch if n is None else n
    g = np.random.Generator(np.random.PCG64([shape.seed, 3000 + seed]))
    (qlo, qhi), (plo, phi) = shape.extra["query"], shape.extra["passage"]
    out = []
    for _ in range(n):
        q = g.integers(1000, shape.vocab, size=int(g.integers(qlo, qhi + 1))).astype(np.int32)
        p = g.integers(1000, shape.vocab, size=int(g.integers(plo, phi + 1))).astype(np.int32)
        out.append((q, p[: shape.seq - 3 - len(q)]))
    return out


def rerank_head(shape: Shape):
    """The cross-encoder head's tensors, as keywords of RerankHead:
    pooler [H, H] and [H], classifier [H] and its bias, all N(0, 0.02)."""
    H = shape.hidden
    return dict(pooler_weight=_normal(shape.seed, 900001, (H, H)), pooler_bias=_normal(shape.seed, 900002, (H,)),
                classifier_weight=_normal(shape.seed, 900003, (H,)),
                classifier_bias=float(_normal(shape.seed, 900004, (1,))[0]))


def rows(shape: Shape, batch=None, seq=None, lengths="default", seed=0):
    """(ids, mask, types) of a synthetic batch: each row [CLS] ids.. [SEP],
    padded with the pad id under mask 0."""
    b = shape.batch if batch is None else batch
    s = shape.seq if seq is None else seq
    lens = shape.lengths if lengths == "default" else lengths
    g = np.random.Generator(np.random.PCG64([shape.seed, 1000 + seed]))
    if lens is None:
        n = np.full(b, s, np.int64)
    else:
        lo, hi = lens
        n = g.integers(min(lo, s), min(hi, s) + 1, size=b)
    ids = np.full((b, s), shape.pad_id, np.int32)
    mask = np.zeros((b, s), np.int32)
    body = g.integers(1000, min(shape.vocab, 30522), size=(b, s)).astype(np.int32)
    for r in range(b):
        k = int(n[r])
        ids[r, :k] = body[r, :k]
        ids[r, 0] = shape.cls_id
        if k > 1:
            ids[r, k - 1] = shape.sep_id
        mask[r, :k] = 1
    types = np.zeros((b, s), np.int32)
    return ids, mask, types


def ranges(shape: Shape, mask, per_row=None, seed=0):
    """Contiguous ranges covering each row's live tokens: per_row pieces cut
    at distinct points drawn uniformly from (0, len)."""
    k = shape.ranges_per_row if per_row is None else per_row
    g = np.random.Generator(np.random.PCG64([shape.seed, 2000 + seed]))
    out = []
    for r in range(mask.shape[0]):
        n = int(mask[r].nonzero()[0].max()) + 1
        cuts = np.sort(g.choice(np.arange(1, n), size=min(k - 1, n - 1), replace=False)) if n > 1 else []
        edges = [0] + [int(c) for c in cuts] + [n]
        out += [(r, edges[i], edges[i + 1]) for i in range(len(edges) - 1)]
    return out


def gemm_flops_per_token(shape: Shape):
    """Algorithmic GEMM FLOPs per live token over the whole encoder."""
    H, I, L = shape.hidden, shape.intermediate, shape.layers
    if shape.family == S.TURBO_FAMILY_MODERNBERT:
        return 2 * L * H * (3 * H + H + 2 * I) + 2 * L * I * H
    return 2 * L * H * (3 * H + H + 2 * I)


def attention_flops(shape: Shape, lengths):
    """Algorithmic attention FLOPs (QK^T and PV, and DeBERTa-v2's two relative
    terms) over rows of these lengths."""
    H, L = shape.hidden, shape.layers
    total = 0.0
    for n in lengths:
        n = float(n)
        if shape.window and shape.global_every:
            g = sum(1 for l in range(L) if l % shape.global_every == 0)
            loc = L - g
            w = shape.window + 1
            keys = sum(min(n, i + shape.window // 2 + 1) - max(0, i - shape.window // 2) for i in range(int(n)))
            total += 4 * g * H * n * n + 4 * loc * H * keys
            del w
        elif shape.family == S.TURBO_FAMILY_DEBERTA_V2:
            # Each score's three dot products (content, content to position,
            # position to content) and its share of the context.
            total += 8 * L * H * n * n
        else:
            total += 4 * L * H * n * n
    return total
