"""Small seeded models and rows for the tests: every family at shapes the
oracle and the textbook encoders finish in milliseconds, and the
adversarial rows the reference's device tests use (left padding, holes,
single-token rows; core/tests/cuda_support/rows.rs:10-60)."""
import numpy as np

from turboembed_amd import seam as S
from turboembed_amd.model import ModelDesc


def bert(seed=0, layers=2, hidden=64, heads=4, inter=128, vocab=300, positions=96, types=2, std=0.2,
         family=S.TURBO_FAMILY_BERT, position_offset=0):
    g = np.random.Generator(np.random.PCG64(seed))
    w = lambda *sh: (g.standard_normal(sh) * std).astype(np.float32)          # noqa: E731
    lnw = lambda: (1.0 + g.standard_normal(hidden) * 0.1).astype(np.float32)  # noqa: E731
    t = [w(vocab, hidden), w(positions, hidden), w(types, hidden), lnw(), w(hidden)]
    for _ in range(layers):
        t += [w(hidden, hidden), w(hidden), w(hidden, hidden), w(hidden), w(hidden, hidden), w(hidden),
              w(hidden, hidden), w(hidden), lnw(), w(hidden), w(inter, hidden), w(inter), w(hidden, inter),
              w(hidden), lnw(), w(hidden)]
    return ModelDesc(family, layers, hidden, heads, inter, vocab, positions, types, 1e-12, t,
                     position_offset=position_offset)


def modernbert(seed=0, layers=3, hidden=64, heads=2, inter=96, vocab=300, positions=128, window=8, global_every=3,
               std=0.2):
    g = np.random.Generator(np.random.PCG64(seed))
    w = lambda *sh: (g.standard_normal(sh) * std).astype(np.float32)          # noqa: E731
    lnw = lambda: (1.0 + g.standard_normal(hidden) * 0.1).astype(np.float32)  # noqa: E731
    t = [w(vocab, hidden), lnw(), lnw()]
    for l in range(layers):
        t += [None if l == 0 else lnw(), w(3 * hidden, hidden), w(hidden, hidden), lnw(), w(2 * inter, hidden),
              w(hidden, inter)]
    return ModelDesc(S.TURBO_FAMILY_MODERNBERT, layers, hidden, heads, inter, vocab, positions, 1, 1e-5, t,
                     rope=(160000.0, 10000.0), attention_window=window, global_every=global_every,
                     mlp=S.TURBO_MLP_GATED, activation=S.TURBO_ACTIVATION_GELU_ERF, norm=S.TURBO_NORM_LAYER_NO_BIAS)


def nomic(seed=0, layers=2, hidden=64, heads=2, inter=96, vocab=300, positions=128, std=0.2):
    g = np.random.Generator(np.random.PCG64(seed))
    w = lambda *sh: (g.standard_normal(sh) * std).astype(np.float32)          # noqa: E731
    lnw = lambda: (1.0 + g.standard_normal(hidden) * 0.1).astype(np.float32)  # noqa: E731
    t = [w(vocab, hidden), w(2, hidden), lnw(), w(hidden)]
    for _ in range(layers):
        t += [w(3 * hidden, hidden), w(hidden, hidden), lnw(), w(hidden), w(inter, hidden), w(inter, hidden),
              w(hidden, inter), lnw(), w(hidden)]
    return ModelDesc(S.TURBO_FAMILY_NOMIC_BERT, layers, hidden, heads, inter, vocab, positions, 2, 1e-12, t,
                     rope=(1000.0, 1000.0), mlp=S.TURBO_MLP_GATED, activation=S.TURBO_ACTIVATION_SILU,
                     norm=S.TURBO_NORM_LAYER)


def gated_overflow(desc, unit=0, scale=500.0):
    """The gated model with one FFN unit's two input rows (the activation's
    and the multiplier's) scaled by `scale` in its last layer, so that the
    unit's product act(gate) * up passes F16's 65504 on most tokens, and
    its FFN-out column scaled by 1 / (6 scale), so that the product's share
    of the residual stays a few units (the other states still count, and
    the column's weights stay normal F16 numbers)."""
    if desc.family == S.TURBO_FAMILY_MODERNBERT:
        first, per, I = S.MODERNBERT_EMBEDDING_TENSORS, S.MODERNBERT_LAYER_TENSORS, desc.intermediate
        rows, out = [(4, unit), (4, I + unit)], 5
    else:
        first, per = S.NOMIC_EMBEDDING_TENSORS, S.NOMIC_LAYER_TENSORS
        rows, out = [(4, unit), (5, unit)], 6
    base = first + (desc.layers - 1) * per
    for k, r in rows:
        t = desc.tensors[base + k].copy()
        t[r] *= np.float32(scale)
        desc.tensors[base + k] = t
    t = desc.tensors[base + out].copy()
    t[:, unit] *= np.float32(1.0 / (6.0 * scale))
    desc.tensors[base + out] = t
    return desc


def ragged_rows(seed, batch, seq, vocab, types=2):
    """Rows of lengths 1..seq with holes (mask-0 columns before the last
    live one), one left-padded row, ids that are not the pad under mask 0,
    and random types."""
    g = np.random.Generator(np.random.PCG64(seed + 77))
    ids = g.integers(0, vocab, size=(batch, seq)).astype(np.int32)
    mask = np.zeros((batch, seq), np.int32)
    for r in range(batch):
        n = int(g.integers(1, seq + 1)) if r > 0 else seq
        mask[r, :n] = 1
        if n > 3 and r % 3 == 1:
            holes = g.choice(np.arange(1, n - 1), size=min(2, n - 2), replace=False)
            mask[r, holes] = 0
    if batch > 2:
        # A left-padded row: its live tokens at the end.
        k = max(1, seq // 3)
        mask[2] = 0
        mask[2, seq - k:] = 1
    tt = g.integers(0, types, size=(batch, seq)).astype(np.int32)
    return ids, mask, tt


def cosine_rows(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return (a * b).sum(1) / np.maximum(np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1), 1e-300)


def spearman(a, b):
    """Spearman's rank correlation of two score vectors (distinct scores)."""
    ra = np.argsort(np.argsort(np.asarray(a))).astype(np.float64)
    rb = np.argsort(np.argsort(np.asarray(b))).astype(np.float64)
    ra -= ra.mean()
    rb -= rb.mean()
    return float((ra * rb).sum() / np.sqrt((ra * ra).sum() * (rb * rb).sum()))
