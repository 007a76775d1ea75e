"""The oracle's DeBERTa-v2 encoder on the CPU.

Pinned by the sealed tiny bundle's upstream vectors (testdata/tiny-deberta-
bundle: sentence-transformers over transformers' DebertaV2Model, 9 rows up to
128 tokens, every token live, 8 relative buckets so the log buckets are
reached), by hand-computed buckets, and, for rows with masked tokens (which
the upstream cases do not hold), by the float64 textbook encoder in plain.py
and the invariants the reference states (docs/deberta.md): visible rows do
not depend on the masked tokens' ids, and every masked position shares one
state.
"""
import numpy as np
import pytest

import oracle
from turboembed_amd import seam as S
from turboembed_amd.model import ModelDesc

import plain
import small


def test_oracle_meets_the_upstream_vectors():
    desc, ids, lengths, vectors, info = oracle.fixture("tiny_deberta")
    assert desc.family == S.TURBO_FAMILY_DEBERTA_V2 and desc.relative == (8, 512)
    i, m = oracle.fixture_rows(ids, lengths)
    norm = S.TURBO_NORMALIZE_L2 if info["embed"]["normalize"] == "NORMALIZE_L2" else S.TURBO_NORMALIZE_NONE
    got = oracle.encode(desc, i, m, normalize=norm)
    assert small.cosine_rows(got, vectors).min() >= 0.9999
    assert np.abs(got - vectors).max() <= 1e-5


@pytest.mark.parametrize("d,want", [(0, 8), (3, 11), (-4, 4), (4, 12), (5, 13), (-5, 3), (100, 14), (-100, 2),
                                    (511, 15), (600, 15), (-600, 0)])
def test_buckets_are_the_log_formula(d, want):
    # 8 buckets (mid 4), 512 the farthest distance: ceil(ln(|d| / 4) / ln(511 / 4) * 3) + 4 beyond 4,
    # by hand: d = 5 gives 1 + 4, d = 100 gives 2 + 4, d = 511 gives 3 + 4; then offset by 8 and clamped to 15.
    assert oracle.lib().oracle_deberta_bucket(d, 8, 512) == want


def small_deberta(seed=2, layers=2, hidden=32, heads=4, inter=64, vocab=60, buckets=8, maximum=64, std=0.3):
    g = np.random.Generator(np.random.PCG64(seed))
    w = lambda *sh: (g.standard_normal(sh) * std).astype(np.float32)          # noqa: E731
    lnw = lambda: (1.0 + g.standard_normal(hidden) * 0.1).astype(np.float32)  # noqa: E731
    t = [w(vocab, hidden), lnw(), w(hidden), w(2 * buckets, hidden), lnw(), w(hidden)]
    for _ in range(layers):
        t += [w(hidden, hidden), w(hidden), w(hidden, hidden), w(hidden), w(hidden, hidden), w(hidden),
              w(hidden, hidden), w(hidden), lnw(), w(hidden), w(inter, hidden), w(inter), w(hidden, inter),
              w(hidden), lnw(), w(hidden)]
    return ModelDesc(S.TURBO_FAMILY_DEBERTA_V2, layers, hidden, heads, inter, vocab, maximum, 1, 1e-7, t,
                     relative=(buckets, maximum))


def holed_rows(vocab, seed=3):
    g = np.random.Generator(np.random.PCG64(seed))
    ids = g.integers(0, vocab, (4, 40)).astype(np.int32)
    mask = np.zeros((4, 40), np.int32)
    mask[0, :40] = 1
    mask[1, :25] = 1
    mask[1, [3, 10, 11]] = 0          # holes
    mask[2, 5:30] = 1                 # masked column 0: CLS reads the masked row
    mask[3, :1] = 1
    return ids, mask


@pytest.mark.parametrize("pooling", [S.TURBO_POOLING_MEAN, S.TURBO_POOLING_CLS, S.TURBO_POOLING_LAST])
def test_rows_with_masked_tokens_meet_the_textbook(pooling):
    desc = small_deberta()
    ids, mask = holed_rows(desc.vocab_size)
    got = oracle.encode(desc, ids, mask, pooling=pooling, normalize=S.TURBO_NORMALIZE_NONE)
    want = plain.embed(desc, ids, mask, pooling=pooling, normalize=S.TURBO_NORMALIZE_NONE)
    assert np.abs(got - want).max() <= 1e-5 * (1 + np.abs(want).max()), np.abs(got - want).max()


def test_visible_rows_ignore_masked_ids_and_masked_rows_share_one_state():
    desc = small_deberta()
    ids, mask = holed_rows(desc.vocab_size)
    _, h1 = oracle.encode(desc, ids, mask, normalize=S.TURBO_NORMALIZE_NONE, hidden=True)
    other = ids.copy()
    other[mask == 0] = (other[mask == 0] + 7) % desc.vocab_size
    _, h2 = oracle.encode(desc, other, mask, normalize=S.TURBO_NORMALIZE_NONE, hidden=True)
    start, ln, at = oracle.pack(mask)
    live = mask.reshape(-1)[at] != 0
    np.testing.assert_array_equal(h1[live], h2[live])
    # Row 1's holes (columns 3, 10, 11) share one state, the same bits.
    rows = start[1] + np.array([3, 10, 11])
    np.testing.assert_array_equal(h1[rows[0]], h1[rows[1]])
    np.testing.assert_array_equal(h1[rows[0]], h1[rows[2]])
    # A planted change to the masked row's rule (attending to the live keys
    # only, as a visible query does) moves row 2's CLS vector (its column 0
    # is masked) far outside the bound the textbook check holds.
    got = oracle.encode(desc, ids, mask, pooling=S.TURBO_POOLING_CLS, normalize=S.TURBO_NORMALIZE_NONE)
    x, _ = plain.deberta_states(desc, ids[2], mask[2], uniform_masked=False)
    assert np.abs(got[2] - x[0]).max() > 1e-2


def test_the_v3_base_workload_meets_the_textbook_at_full_width():
    # The measured DeBERTa-v3-base shape (hidden 768, 12 heads, 256 buckets to
    # distance 512) on one layer: a 300-token row reaches the log buckets
    # (|i - j| > 128) and a row with a hole; the workload counts its
    # attention at twice a plain encoder's FLOPs (three dot products a score
    # and the context against two).
    from turboembed_amd import workloads as W
    sh = W.SHAPES["deberta-v3-base"]
    desc = W.model(sh, layers=1)
    assert desc.family == S.TURBO_FAMILY_DEBERTA_V2 and desc.relative == (256, 512)
    assert len(desc.tensors) == S.DEBERTA_EMBEDDING_TENSORS + S.BERT_LAYER_TENSORS
    g = np.random.Generator(np.random.PCG64(4))
    ids = g.integers(0, sh.vocab, (2, 300)).astype(np.int32)
    mask = np.ones((2, 300), np.int32)
    mask[1, 200:] = 0
    mask[1, 17] = 0
    got = oracle.encode(desc, ids, mask, pooling=S.TURBO_POOLING_MEAN, normalize=S.TURBO_NORMALIZE_NONE)
    want = plain.embed(desc, ids, mask, pooling=S.TURBO_POOLING_MEAN, normalize=S.TURBO_NORMALIZE_NONE)
    assert np.abs(got - want).max() <= 1e-5 * (1 + np.abs(want).max()), np.abs(got - want).max()
    bert = W.SHAPES["bert-base"]
    assert W.attention_flops(sh, [300]) == 2 * W.attention_flops(bert, [300])
