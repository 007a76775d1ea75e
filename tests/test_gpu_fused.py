"""The out and FFN-out products with the residual add and LayerNorm in their
epilogue (the whole-row 128 x 768 shape) against the same session run with
the separate add_layer_norm, and against the oracle, on an MI355X.

The fused epilogue rounds each product to the operand type as the separate
product stores it and norms each row with the row kernels' own arithmetic,
so the two paths agree bit for bit: the final F32 states, the pooled
vectors and range means alike. Against the oracle the bound is the F16
floor (core/src/record/mod.rs:341-348).
"""
import numpy as np
import pytest

import oracle
import turboembed_amd as T
from turboembed_amd import seam as S
from turboembed_amd import workloads as W

import small

pytestmark = pytest.mark.gpu

SHAPES = ["128x768ln"]
UNFUSED = "all:out=256x384,ffn2=256x384"


def fused(shape):
    return f"all:out={shape},ffn2={shape}"


def _session(model, monkeypatch, choices, *a, split=None, **kw):
    monkeypatch.setenv("TURBO_ROCM_CHOICES", choices)
    if split is not None:
        monkeypatch.setenv("TURBO_ROCM_SPLIT", split)
    s = model.session(*a, **kw)
    monkeypatch.delenv("TURBO_ROCM_CHOICES")
    if split is not None:
        monkeypatch.delenv("TURBO_ROCM_SPLIT")
    return s


def _rows(seed, batch, seq, vocab, lo):
    g = np.random.Generator(np.random.PCG64(seed))
    lengths = g.integers(lo, seq + 1, batch)
    ids = g.integers(1000, vocab, (batch, seq)).astype(np.int32)
    ids[:, 0] = 101
    mask = (np.arange(seq)[None, :] < lengths[:, None]).astype(np.int32)
    mask[1, 3] = 0                                    # a hole
    types = (np.arange(seq)[None, :] >= lengths[:, None] // 2).astype(np.int32)
    return ids, mask, types


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("split", ["0", "2"])
@pytest.mark.parametrize("lo", [1, 200])
def test_fused_norms_are_the_separate_norms_bits(context, monkeypatch, shape, split, lo):
    # BERT-base width (hidden 768, FFN 3072) at 2 layers; ragged rows whose
    # packed tokens are no multiple of the 128-row tile, one row of a
    # single token when lo is 1.
    sh = W.SHAPES["bert-base"]
    desc = W.model(sh, layers=2)
    ids, mask, types = _rows(11 + int(split) + lo, 12, 512, desc.vocab_size, lo)
    if lo == 1:
        mask[4] = 0
        mask[4, 0] = 1
    model = context.load(desc)
    f = _session(model, monkeypatch, fused(shape), 12, 512, sh.precision, max_ranges=64, split=split)
    u = _session(model, monkeypatch, UNFUSED, 12, 512, sh.precision, max_ranges=64, split=split)
    assert f"out={shape}," in f.choices() and f"ffn2={shape}," in f.choices()
    assert f.compute_dtype == S.TURBO_DTYPE_F16
    got = f.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    want = u.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    np.testing.assert_array_equal(f.hidden(), u.hidden())
    np.testing.assert_array_equal(got, want)
    # The fused path's launches: no separate norm.
    f.set_timing(True)
    f.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    n = f.launches()
    f.set_timing(False)
    packed = sum(int(r.nonzero()[0].max()) + 1 for r in mask)
    parts = 2 if split == "2" and packed > 4096 else 1
    assert "add_layer_norm" not in n
    assert n["gemm_out_ln"] == 2 * parts and n["gemm_ffn_out_ln"] == 2 * parts
    # Range means over the fused states: the same bits, whole rows included.
    ranges = [(r, 0, int(mask[r].nonzero()[0].max()) + 1) for r in range(12)] + [(3, 5, 77), (11, 0, 1)]
    for s in (f, u):
        s.write_ranges(ids, mask, ranges, types)
        s.run()
    rf, ru = f.read(), u.read()
    np.testing.assert_array_equal(rf, ru)
    ref = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    assert small.cosine_rows(got, ref).min() >= 0.999
    f.close()
    u.close()
    model.close()


@pytest.mark.parametrize("shape", SHAPES)
def test_fused_bert_base_meets_the_oracle_at_full_depth(context, monkeypatch, shape):
    # All 12 layers of BERT-base F16 on two rows of 512 and 300 tokens.
    sh = W.SHAPES["bert-base"]
    desc = W.model(sh)
    ids, mask, types = W.rows(sh, batch=2, lengths=(300, 512), seed=3)
    model = context.load(desc)
    f = _session(model, monkeypatch, fused(shape), 64, 512, sh.precision)
    got = f.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    want = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    cos = small.cosine_rows(got, want)
    assert cos.min() >= 0.999, cos
    f.close()
    model.close()


@pytest.mark.parametrize("choice, precision", [("qkv=128x768ln", S.TURBO_PRECISION_FASTEST),
                                               ("ffn1=128x768ln", S.TURBO_PRECISION_FASTEST),
                                               ("out=128x768ln", S.TURBO_PRECISION_EXACT),
                                               ("ffn2=128x768ln", S.TURBO_PRECISION_EXACT)])
def test_the_fused_shape_is_refused_where_it_cannot_run(context, monkeypatch, choice, precision):
    sh = W.SHAPES["bert-base"]
    model = context.load(W.model(sh, layers=1))
    monkeypatch.setenv("TURBO_ROCM_CHOICES", choice)
    with pytest.raises(T.TurboError) as e:
        model.session(4, 128, precision)
    assert e.value.code == S.TURBO_E_UNSUPPORTED_OPTION
    model.close()
