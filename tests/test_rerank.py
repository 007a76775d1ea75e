"""The rerank caller on the host: pair windows and the classification head
(core/src/tokenizer/pair.rs:27-99, core/src/session/rerank.rs:111-219).

The oracle's windows are held bit for bit to the reference's first windows
(testdata/tiny-rerank-reference), and its scores, over the oracle encoder,
to the transformers scores at the F32 score bound (1e-4 of the scale,
docs/conformance.md "Scores"). The library's C++ windows and head are held
to the oracle's. No device is needed: these entry points run on the host.
"""
import numpy as np
import pytest

import oracle
from turboembed_amd import TurboError
from turboembed_amd import seam as S
from turboembed_amd.rerank import PAIR_BERT, PAIR_ROBERTA, RerankHead, head_scores, pair_windows

import small


@pytest.fixture(scope="module")
def tiny():
    return oracle.rerank_fixture()


def test_oracle_windows_are_the_reference_s(tiny):
    desc, pairs, head, info, ref = tiny
    for i, (q, p) in enumerate(pairs):
        ids, types = oracle.pair_windows(q, p, info["start_id"], info["end_id"], query_tokens=info["query_tokens"],
                                         max_tokens=info["max_tokens"])[0]
        n = int(ref["first_lengths"][i])
        assert len(ids) == n
        np.testing.assert_array_equal(ids, ref["first_ids"][i, :n])
        np.testing.assert_array_equal(types, ref["first_types"][i, :n])


def test_oracle_scores_meet_transformers(tiny):
    desc, pairs, head, info, ref = tiny
    got = oracle.rerank(desc, pairs, head, info["start_id"], info["end_id"], query_tokens=info["query_tokens"],
                        max_tokens=info["max_tokens"])
    scale = np.abs(ref["scores"]).max()
    assert np.abs(got - ref["scores"]).max() <= 1e-4 * scale


def test_a_window_dropped_or_a_type_flipped_misses_transformers(tiny):
    # The bound is tight enough to see a window lost (the long pair scored
    # on its first window alone: its best is the short last one) or a
    # segment type wrong.
    desc, pairs, head, info, ref = tiny
    scale = np.abs(ref["scores"]).max()
    q, p = pairs[3]
    first = oracle.rerank(desc, [(q, p[:21])], head, info["start_id"], info["end_id"], query_tokens=8,
                          max_tokens=32)[0]
    assert abs(first - ref["scores"][3]) > 1e-4 * scale
    ids, types = oracle.pair_windows(*pairs[1], info["start_id"], info["end_id"], query_tokens=8, max_tokens=32)[0]
    ids, types = np.array([ids], np.int32), np.zeros((1, len(ids)), np.int32)
    states = oracle.encode(desc, ids, np.ones_like(ids), types, pooling=S.TURBO_POOLING_CLS,
                           normalize=S.TURBO_NORMALIZE_NONE)
    assert abs(oracle.rerank_head(states, **head)[0] - ref["scores"][1]) > 1e-4 * scale


CASES = [
    dict(q=5, p=40, qt=8, mt=32, stride=0, roberta=False),
    dict(q=30, p=70, qt=8, mt=32, stride=0, roberta=False),
    dict(q=30, p=70, qt=8, mt=32, stride=7, roberta=False),
    dict(q=0, p=0, qt=8, mt=32, stride=0, roberta=False),
    dict(q=3, p=100, qt=4, mt=20, stride=13, roberta=True),
    dict(q=12, p=1, qt=12, mt=17, stride=0, roberta=True),
    dict(q=7, p=21, qt=8, mt=32, stride=0, roberta=False),   # the passage fills its one window exactly
]


@pytest.mark.parametrize("c", CASES)
def test_the_library_s_windows_are_the_oracle_s(c):
    g = np.random.Generator(np.random.PCG64(c["q"] * 100 + c["p"]))
    q = g.integers(5, 1000, size=c["q"]).tolist()
    p = g.integers(5, 1000, size=c["p"]).tolist()
    want = oracle.pair_windows(q, p, 1, 2, c["roberta"], c["qt"], c["mt"], c["stride"])
    ids, types, lengths = pair_windows(q, p, 1, 2, PAIR_ROBERTA if c["roberta"] else PAIR_BERT, c["qt"], c["mt"],
                                       c["stride"])
    assert len(lengths) == len(want)
    for (wi, wt), gi, gt, n in zip(want, ids, types, lengths):
        assert n == len(wi)
        np.testing.assert_array_equal(gi[:n], wi)
        np.testing.assert_array_equal(gt[:n], wt)
        assert not gi[n:].any() and not gt[n:].any()


@pytest.mark.parametrize("kw, field", [(dict(max_tokens=4), 2), (dict(query_tokens=29), 1), (dict(stride=30), 3)])
def test_window_limits_are_refused_as_the_reference_does(kw, field):
    args = dict(query_tokens=8, max_tokens=32, stride=0)
    args.update(kw)
    with pytest.raises(TurboError) as e:
        pair_windows([7] * 5, [9] * 50, 1, 2, PAIR_BERT, **args)
    assert e.value.code == S.TURBO_E_INVALID_ARGUMENT and e.value.field == field


@pytest.mark.parametrize("pooler", [True, False])
def test_the_library_s_head_is_the_oracle_s(pooler):
    g = np.random.Generator(np.random.PCG64(5))
    h = 48
    states = g.standard_normal((9, h)).astype(np.float32)
    kw = dict(classifier_weight=g.standard_normal(h).astype(np.float32) * 0.1, classifier_bias=0.25)
    if pooler:
        kw.update(pooler_weight=g.standard_normal((h, h)).astype(np.float32) * 0.1,
                  pooler_bias=g.standard_normal(h).astype(np.float32))
    got = head_scores(states, RerankHead(**kw))
    want = oracle.rerank_head(states, **kw)
    # Both sum in F64; only the order of the sums differs.
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_the_head_refuses_a_non_finite_state():
    states = np.zeros((2, 8), np.float32)
    states[1, 3] = np.nan
    with pytest.raises(TurboError) as e:
        head_scores(states, RerankHead(classifier_weight=np.ones(8, np.float32)))
    assert e.value.code == S.TURBO_E_INTERNAL


def test_the_rank_statistic_is_spearman_s():
    # The rank agreement the int8 cross-encoder is held to: identical orders
    # give 1, reversed -1, and it is scipy's Spearman rho on distinct values.
    from scipy.stats import spearmanr
    a = np.arange(100, dtype=np.float64)
    assert small.spearman(a, a * 3 + 1) == pytest.approx(1.0)
    assert small.spearman(a, -a) == pytest.approx(-1.0)
    g = np.random.Generator(np.random.PCG64(1))
    x, y = g.standard_normal(64), g.standard_normal(64)
    y = x + 0.5 * y
    assert small.spearman(x, y) == pytest.approx(spearmanr(x, y).statistic, abs=1e-12)
