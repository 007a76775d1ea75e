"""The oracle's layer reads (taps, tap_alone) on the CPU.

A range write with taps T > 1 pools each range from each of the last T
layers (include/turbo/turbo_backend.h:423-435). The reference's own checks
(core/tests/ranges/layers.rs:18-49, alone.rs:25-84,
core/src/cpu/encoder/taps_tests.rs) pin it by closed forms that hold here
bit for bit: the last block is the plain range write; block k is the plain
range write of the same model cut after its layer (its tensors truncated,
a ModernBERT's final_norm kept), which runs through the ordinary path; one
layer alone is block 0. An off-by-one layer or a missing final_norm fails
the cut-model check, as the planted cases below show.
"""
import numpy as np
import pytest

import oracle
from turboembed_amd import seam as S
from turboembed_amd.model import ModelDesc

import small

_PARTS = {S.TURBO_FAMILY_BERT: (S.BERT_EMBEDDING_TENSORS, S.BERT_LAYER_TENSORS),
          S.TURBO_FAMILY_ROBERTA: (S.BERT_EMBEDDING_TENSORS, S.BERT_LAYER_TENSORS),
          S.TURBO_FAMILY_MODERNBERT: (S.MODERNBERT_EMBEDDING_TENSORS, S.MODERNBERT_LAYER_TENSORS),
          S.TURBO_FAMILY_NOMIC_BERT: (S.NOMIC_EMBEDDING_TENSORS, S.NOMIC_LAYER_TENSORS)}


def cut(desc, layers):
    """The same model cut after `layers` layers."""
    e, per = _PARTS[desc.family]
    n = e + layers * per
    return ModelDesc(desc.family, layers, desc.hidden, desc.heads, desc.intermediate, desc.vocab_size,
                     desc.max_positions, desc.token_types, desc.layer_norm_eps, desc.tensors[:n], desc.position_offset,
                     desc.rope, desc.attention_window, desc.global_every, desc.mlp, desc.activation, desc.norm,
                     desc.names[:n], desc.compute_dtype)


def models():
    out = {"bert": small.bert(seed=7, layers=3), "modernbert": small.modernbert(seed=7, layers=4),
           "nomic": small.nomic(seed=7, layers=3),
           "roberta": small.bert(seed=8, layers=2, family=S.TURBO_FAMILY_ROBERTA, position_offset=2)}
    for name in ("tiny_bert", "tiny_modernbert", "tiny_nomic"):
        out[name] = oracle.fixture(name)[0]
    return out


MODELS = models()


def rows_for(desc):
    ids, mask, types = small.ragged_rows(9, 3, 20, desc.vocab_size, types=max(1, desc.token_types))
    live = [np.flatnonzero(m) for m in mask]
    ranges = [(0, 0, 20), (1, int(live[1][0]), int(live[1][-1]) + 1), (2, int(live[2][0]), int(live[2][0]) + 2),
              (0, 3, 9)]
    return ids, mask, types, ranges


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", list(MODELS))
@pytest.mark.parametrize("normalize", [S.TURBO_NORMALIZE_L2, S.TURBO_NORMALIZE_NONE])
def test_every_block_is_the_model_cut_after_its_layer(name, normalize):
    desc = MODELS[name]
    ids, mask, types, ranges = rows_for(desc)
    n = len(ranges)
    L = desc.layers
    plain = oracle.encode(desc, ids, mask, types, normalize=normalize, ranges=ranges)
    for T in range(2, L + 1):
        got = oracle.encode(desc, ids, mask, types, normalize=normalize, ranges=ranges, taps=T)
        assert got.shape == (T * n, desc.hidden)
        assert np.array_equal(bits(got[(T - 1) * n:]), bits(plain)), f"{name}: last block of {T}"
        for k in range(T - 1):
            layers = L - T + k + 1
            want = oracle.encode(cut(desc, layers), ids, mask, types, normalize=normalize, ranges=ranges)
            assert np.array_equal(bits(got[k * n:(k + 1) * n]), bits(want)), f"{name}: block {k} of {T}"
            assert not np.array_equal(got[k * n:(k + 1) * n], plain), f"{name}: block {k} is an earlier layer's"
        alone = oracle.encode(desc, ids, mask, types, normalize=normalize, ranges=ranges, taps=T, tap_alone=True)
        assert np.array_equal(bits(alone), bits(got[:n])), f"{name}: {T} alone"


def test_the_cut_model_check_tells_layers_and_norms_apart():
    # Block 0 of 3 on a 4-layer ModernBERT is the model cut after layer 2:
    # the cut after layer 1 or 3, or the cut with final_norm's weight left
    # out, are each outside any bound.
    desc = MODELS["modernbert"]
    ids, mask, types, ranges = rows_for(desc)
    n = len(ranges)
    block0 = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges, taps=3)[:n]
    for layers in (1, 3):
        other = oracle.encode(cut(desc, layers), ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges)
        assert small.cosine_rows(block0, other).min() < 0.999
    c = cut(desc, 2)
    t = list(c.tensors)
    t[2] = np.ones_like(t[2])      # final_norm's weight: 1, so only the normalization itself remains
    no_final = ModelDesc(c.family, c.layers, c.hidden, c.heads, c.intermediate, c.vocab_size, c.max_positions,
                         c.token_types, c.layer_norm_eps, t, c.position_offset, c.rope, c.attention_window,
                         c.global_every, c.mlp, c.activation, c.norm, c.names, c.compute_dtype)
    other = oracle.encode(no_final, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges)
    assert np.abs(block0 - other).max() > 1e-2


def test_a_modernbert_read_is_on_the_final_norm_scale():
    # A one-token range read from an earlier layer is that token's state
    # through final_norm (no bias): divided by its weight, mean 0 and
    # variance 1 within eps, whatever the layer.
    desc = MODELS["modernbert"]
    ids, mask, types, _ = rows_for(desc)
    t0 = int(np.flatnonzero(mask[1])[0])
    got = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=[(1, t0, t0 + 1)], taps=4)
    w = desc.tensors[2].astype(np.float64)
    for v in got.astype(np.float64) / w:
        assert abs(v.mean()) < 1e-5 and abs(v.var() - 1.0) < 1e-3, (v.mean(), v.var())


def test_layer_reads_are_refused_where_they_cannot_be():
    desc = MODELS["bert"]
    ids, mask, types, ranges = rows_for(desc)
    for kw in (dict(taps=4), dict(taps=2, ranges=None), dict(taps=1, tap_alone=True)):
        args = dict(ranges=ranges, **kw) if "ranges" not in kw else kw
        with pytest.raises(RuntimeError, match="INVALID_ARGUMENT"):
            oracle.encode(desc, ids, mask, types, **args)
