"""Split K (the residual products of small bins in 4 or 2 slices of K, their
F32 sums added in slice order by a second pass) against the oracle at each
tier's bound, and its refusals, on an MI355X through the C ABI.

Bounds are the reference's conformance floors (core/src/record/mod.rs:
341-348): F32 cosine >= 0.9999 and max abs <= 1e-4, F16 and BF16 0.999.
"""
import numpy as np
import pytest

import oracle
import turboembed_amd as T
from turboembed_amd import seam as S

import small
from test_gpu_parity import MODELS, assert_close, int8_model

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("family", ["bert", "modernbert"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
@pytest.mark.parametrize("split", ["r128x128sk4", "r64x64sk2"])
def test_split_k_meets_the_oracle(context, monkeypatch, family, precision, split):
    # Rows of up to 300 tokens in a session of 8 x 320 (bins to le4k, none
    # splits into parts): both residual products on the split shape; the
    # FFN-out product's K (the intermediate size) splits unevenly by 4.
    desc = MODELS[family](seed=61, hidden=128, inter=320, positions=640 if family == "modernbert" else 320)
    ids, mask, types = small.ragged_rows(61, 8, 300, desc.vocab_size)
    if family == "modernbert":
        types = None
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_CHOICES", f"all:out={split},ffn2={split}")
    s = model.session(8, 320, precision)
    assert f"out={split}," in s.choices() and f"ffn2={split}," in s.choices()
    got = s.embed(ids, mask, types)
    assert_close(got, want, s.compute_dtype)
    # The same rows again: the same bits (the slices are added in order).
    assert np.array_equal(s.embed(ids, mask, types), got)
    s.close()
    model.close()


@pytest.mark.parametrize("choice, shape, precision", [
    ("qkv=r128x128sk4", (8, 320), S.TURBO_PRECISION_FASTEST),       # not a residual product
    ("ffn1=r64x64sk2", (8, 320), S.TURBO_PRECISION_EXACT),
    ("all:out=r128x128sk4", (16, 512), S.TURBO_PRECISION_FASTEST),   # le16k's runs split into parts
    ("out=r128x128sk4", (8, 320), "int8"),                           # not on the int8 tier
])
def test_split_k_is_refused_where_it_cannot_run(context, monkeypatch, choice, shape, precision):
    desc = small.bert(seed=62, hidden=128, inter=256, positions=640)
    if precision == "int8":
        desc, precision = int8_model(desc), S.TURBO_PRECISION_FASTEST
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_CHOICES", choice)
    with pytest.raises(T.TurboError) as e:
        model.session(shape[0], shape[1], precision)
    assert e.value.code == S.TURBO_E_UNSUPPORTED_OPTION, e.value
    model.close()
