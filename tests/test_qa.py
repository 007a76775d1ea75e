"""The oracle's span head (extractive QA) against the reference's golden
logits and closed forms, on the CPU.

The golden logits are testdata/tiny-qa-reference's: transformers'
BertForQuestionAnswering over the tiny BERT encoder, for every token of six
windows. The reference holds a backend to 1e-4 of their scale at F32
(core/tests/conformance/scores.rs:18-30). The fixture's head has a zero
bias, so the bias and the range mean under the head are pinned by closed
forms instead: identity head rows read a range's vector back exactly.
"""
import numpy as np
import pytest

import oracle
from turboembed_amd import seam as S
from turboembed_amd.model import ModelDesc

import small


def _with_head(desc, w, b):
    return ModelDesc(desc.family, desc.layers, desc.hidden, desc.heads, desc.intermediate, desc.vocab_size,
                     desc.max_positions, desc.token_types, desc.layer_norm_eps, desc.tensors, desc.position_offset,
                     desc.rope, desc.attention_window, desc.global_every, desc.mlp, desc.activation, desc.norm,
                     desc.names, desc.compute_dtype, span_head=(w, b))


def test_oracle_meets_the_upstream_logits():
    desc, windows, logits, info = oracle.qa_fixture()
    assert logits.shape == (sum(len(w) for w, _ in windows), 2) == (105, 2)
    got = oracle.qa_logits(desc, windows, info["pad_id"])
    scale = np.abs(logits).max()
    d = np.abs(got - logits).max() / scale
    assert d <= 1e-5, d          # the F32 bound is 1e-4; the oracle is F32 throughout


def test_a_swapped_head_fails_the_upstream_logits():
    # Start and end exchanged (head rows in the wrong order) is far outside the bound.
    desc, windows, logits, info = oracle.qa_fixture()
    w, b = desc.span_head
    got = oracle.qa_logits(_with_head(desc, w[::-1].copy(), b[::-1].copy()), windows, info["pad_id"])
    assert np.abs(got - logits).max() / np.abs(logits).max() > 1e-2


@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
def test_identity_rows_read_back_the_range_vectors_and_the_bias(family):
    # Head rows e_k with bias c: each range's logit k is its mean vector's
    # column k plus c, rounded once, so the head's indexing, its bias and the
    # mean it reads (all hidden values, not normalized) are all pinned.
    base = {"bert": small.bert, "modernbert": small.modernbert, "nomic": small.nomic}[family](seed=3)
    ids, mask, types = small.ragged_rows(5, 3, 20, base.vocab_size)
    cols = [0, 7, base.hidden - 1]
    w = np.zeros((len(cols), base.hidden), np.float32)
    w[np.arange(len(cols)), cols] = 1.0
    b = np.array([0.25, -1.5, 3.0], np.float32)
    desc = _with_head(base, w, b)
    # Row 1 holds live columns 0 and 3, row 2 is left-padded (live from 14).
    assert mask[1, :4].tolist() == [1, 0, 0, 1] and mask[2, 13:15].tolist() == [0, 1]
    ranges = [(0, 0, 1), (0, 2, 20), (1, 1, 4), (2, 14, 20), (1, 3, 4)]
    got = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges, head=True)
    vec = oracle.encode(base, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges)
    want = (vec[:, cols].astype(np.float64) + b.astype(np.float64)).astype(np.float32)
    assert got.shape == (len(ranges), len(cols))
    assert np.array_equal(got, want)


def test_head_sums_are_f64_from_the_bias():
    # The last LayerNorm with weight 0 makes every final state its bias, a
    # vector chosen here: v = (1, 2^-20, 1, 0.75, ...). Head row 0,
    # (2^30, 1, -2^30), sums 2^-20 in F64 (core/src/qa/session.rs:268-276
    # folds in F64 from the bias); an F32 sum in any order gives 0 or a
    # multiple of 2^7. Row 1 reads v[3] plus its bias.
    base = small.bert(seed=4)
    t = list(base.tensors)
    v = np.full(base.hidden, 0.5, np.float32)
    v[:4] = [1.0, 2.0 ** -20, 1.0, 0.75]
    t[-2], t[-1] = np.zeros(base.hidden, np.float32), v
    w = np.zeros((2, base.hidden), np.float32)
    w[0, :3] = [2.0 ** 30, 1.0, -(2.0 ** 30)]
    w[1, 3] = 1.0
    b = np.array([0.0, 0.5], np.float32)
    desc = ModelDesc(base.family, base.layers, base.hidden, base.heads, base.intermediate, base.vocab_size,
                     base.max_positions, base.token_types, base.layer_norm_eps, t, span_head=(w, b))
    ids, mask, types = small.ragged_rows(6, 2, 12, base.vocab_size)
    got = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=[(0, 0, 1), (0, 0, 5)],
                        head=True)
    assert got.tolist() == [[2.0 ** -20, 1.25], [2.0 ** -20, 1.25]]


def test_a_head_write_without_a_head_is_refused():
    base = small.bert(seed=4)
    ids, mask, types = small.ragged_rows(6, 2, 12, base.vocab_size)
    with pytest.raises(RuntimeError, match="INVALID_ARGUMENT"):
        oracle.encode(base, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=[(0, 0, 1)], head=True)
