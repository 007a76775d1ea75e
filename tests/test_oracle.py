"""The oracle pinned before it is trusted: against the reference's sealed
upstream vectors, the f64 textbook encoders, the mathematics of its scalar
functions, and the invariants the reference's own tests hold."""
import math

import numpy as np
import pytest

import oracle
from turboembed_amd import seam as S
from turboembed_amd.model import rope_table

import plain
import small

# The reference's conformance floors (core/src/record/mod.rs:341-348).
F32_COS, F32_ABS = 0.9999, 1e-4


@pytest.mark.parametrize("name", ["tiny_bert", "tiny_modernbert", "tiny_nomic"])
def test_oracle_meets_the_sealed_upstream_vectors(name):
    desc, ids, lengths, vectors, info = oracle.fixture(name)
    ids, mask = oracle.fixture_rows(ids, lengths)
    norm = S.TURBO_NORMALIZE_L2 if info["embed"]["normalize"] == "NORMALIZE_L2" else S.TURBO_NORMALIZE_NONE
    got = oracle.encode(desc, ids, mask, normalize=norm)
    cos = small.cosine_rows(got, vectors)
    assert cos.min() >= F32_COS, cos
    assert np.abs(got - vectors).max() <= F32_ABS


@pytest.mark.parametrize("name", ["tiny_bert", "tiny_modernbert"])
def test_oracle_one_row_at_a_time_matches_the_batch(name):
    desc, ids, lengths, vectors, info = oracle.fixture(name)
    ids, mask = oracle.fixture_rows(ids, lengths)
    batch = oracle.encode(desc, ids, mask)
    for r in range(ids.shape[0]):
        one = oracle.encode(desc, ids[r:r + 1], mask[r:r + 1])
        assert np.array_equal(one[0], batch[r])


def _plain_close(got, want):
    got = np.asarray(got, np.float64)
    assert np.all(np.abs(got - want) <= 1e-5 * (1 + np.abs(want))), np.abs(got - want).max()


@pytest.mark.parametrize("pooling", [S.TURBO_POOLING_MEAN, S.TURBO_POOLING_CLS, S.TURBO_POOLING_LAST])
def test_oracle_bert_meets_the_f64_textbook(pooling):
    desc = small.bert(seed=3)
    ids, mask, types = small.ragged_rows(3, 6, 40, desc.vocab_size)
    got = oracle.encode(desc, ids, mask, types, pooling=pooling)
    _plain_close(got, plain.embed(desc, ids, mask, types, pooling=pooling))


def test_oracle_roberta_offset_and_output_dim():
    desc = small.bert(seed=4, family=S.TURBO_FAMILY_ROBERTA, position_offset=2)
    ids, mask, types = small.ragged_rows(4, 4, 30, desc.vocab_size)
    got = oracle.encode(desc, ids, mask, types, output_dim=24)
    _plain_close(got, plain.embed(desc, ids, mask, types, output_dim=24))


def test_oracle_modernbert_meets_the_f64_textbook():
    desc = small.modernbert(seed=5)
    ids, mask, _ = small.ragged_rows(5, 6, 50, desc.vocab_size)
    got = oracle.encode(desc, ids, mask, normalize=S.TURBO_NORMALIZE_NONE)
    want = plain.embed(desc, ids, mask, normalize=S.TURBO_NORMALIZE_NONE)
    # The table's F32 angles move RoPE by ~1e-7 relative; the bound holds.
    _plain_close(got, want)


def test_oracle_nomic_meets_the_f64_textbook():
    desc = small.nomic(seed=6)
    ids, mask, types = small.ragged_rows(6, 5, 40, desc.vocab_size)
    got = oracle.encode(desc, ids, mask, types)
    _plain_close(got, plain.embed(desc, ids, mask, types))


def test_a_planted_mistake_fails_the_textbook_check():
    # The check has teeth: an oracle reading the wrong LayerNorm bias misses it.
    desc = small.bert(seed=7)
    ids, mask, types = small.ragged_rows(7, 3, 20, desc.vocab_size)
    want = plain.embed(desc, ids, mask, types)
    broken = small.bert(seed=7)
    broken.tensors[4] = broken.tensors[4] * 0.5
    got = oracle.encode(broken, ids, mask, types)
    assert np.abs(got - want).max() > 1e-4


def test_whole_row_ranges_are_the_rows_bit_for_bit():
    # The reference's rule (core/tests/ranges/whole_row.rs:8-28).
    desc = small.bert(seed=8)
    ids, mask, types = small.ragged_rows(8, 5, 32, desc.vocab_size)
    rows = oracle.encode(desc, ids, mask, types)
    ranges = [(r, 0, 32) for r in range(5)]
    got = oracle.encode(desc, ids, mask, types, ranges=ranges)
    assert np.array_equal(got, rows)


def test_ranges_meet_the_f64_textbook():
    desc = small.bert(seed=9)
    ids, mask, types = small.ragged_rows(9, 4, 32, desc.vocab_size)
    ranges = [(0, 0, 5), (0, 5, 32), (1, 1, 3), (3, 0, 32), (2, 25, 32), (0, 0, 5)]
    ranges = [g for g in ranges if mask[g[0], g[1]:g[2]].any()]
    got = oracle.encode(desc, ids, mask, types, ranges=ranges)
    want = []
    for r, a, b in ranges:
        x, live = plain.bert_states(desc, ids[r], mask[r], types[r])
        sel = [p for p in range(a, min(b, len(live))) if live[p]]
        v = x[sel].mean(0)
        want.append(v / np.linalg.norm(v))
    _plain_close(got, np.array(want))


def test_bits_do_not_depend_on_the_thread_count():
    desc = small.bert(seed=10, hidden=128, inter=256)
    ids, mask, types = small.ragged_rows(10, 8, 64, desc.vocab_size)
    a = oracle.encode(desc, ids, mask, types, threads=1)
    b = oracle.encode(desc, ids, mask, types, threads=5)
    assert np.array_equal(a, b)


def test_packing_follows_the_rows():
    mask = np.array([[1, 1, 0, 0], [0, 1, 0, 1], [1, 0, 0, 0]], np.int32)
    start, ln, at = oracle.pack(mask)
    assert list(ln) == [2, 4, 1] and list(start) == [0, 2, 6]
    assert list(at) == [0, 1, 4, 5, 6, 7, 8]
    # A range past the last live token extends the row (CPU BERT only).
    start, ln, at = oracle.pack(mask, [(2, 0, 3)])
    assert list(ln) == [2, 4, 3]


# ---- Scalar functions against the mathematics -----------------------------------

def _f(name):
    return getattr(oracle.lib(), name)


def test_exp_is_within_two_ulps():
    f = _f("oracle_exp")
    xs = np.linspace(-79.9, 87.9, 20001).astype(np.float32)
    worst = max(abs(f(float(x)) - math.exp(float(x))) / math.exp(float(x)) for x in xs)
    assert worst < 2 * np.finfo(np.float32).eps
    assert f(-80.01) == 0.0 and f(float("-inf")) == 0.0


def test_gelu_is_within_5e7_of_erf():
    f = _f("oracle_gelu")
    worst = 0.0
    for i in range(-5000, 6001, 7):
        x = float(np.float32(i / 1000.0))
        want = 0.5 * x * (1 + math.erf(x / math.sqrt(2)))
        got = f(x)
        assert abs(got - want) <= 1e-6 * max(abs(want), 1e-3)
        if abs(want) > 1e-3:
            worst = max(worst, abs(got - want) / abs(want))
    assert worst < 5e-7
    assert f(0.0) == 0.0 and f(1e30) == float(np.float32(1e30)) and f(-1e30) == 0.0


def test_silu_matches_its_definition():
    f = _f("oracle_silu")
    for i in range(-12000, 12001, 37):
        x = float(np.float32(i) / np.float32(1000.0))
        want = x / (1 + math.exp(-x))
        assert abs(f(x) - want) <= 4e-7 * max(abs(want), 1e-6)


def test_layer_norm_matches_the_f64_formula():
    import ctypes as C
    g = np.random.Generator(np.random.PCG64(1))
    y = (g.standard_normal(768) * 3 + 1).astype(np.float32)
    w = g.standard_normal(768).astype(np.float32)
    b = g.standard_normal(768).astype(np.float32)
    want = plain.ln(y.astype(np.float64), w, b, 1e-12)
    got = y.copy()
    oracle.lib().oracle_layer_norm(got.ctypes.data, w.ctypes.data, b.ctypes.data, 768, C.c_float(1e-12))
    assert np.abs(got - want).max() < 1e-5


def test_rope_table_follows_the_rope_formula():
    # As core/src/rope.rs:40-80: position 0 is no rotation, pair 0 turns at
    # frequency 1, and every entry is within F32 rounding of the angle.
    t = rope_table(160000.0, 10000.0, 8192, 32)
    assert t.shape == (2, 2, 8192, 32)
    assert np.all(t[:, 0, 0] == 1) and np.all(t[:, 1, 0] == 0)
    assert t[0, 0, 3, 0] == np.float32(math.cos(3.0)) and t[1, 1, 3, 0] == np.float32(math.sin(3.0))
    for p in (1, 63, 2047, 4096, 8191):
        for i in (0, 1, 15, 31):
            ang = p * 160000.0 ** (-(2 * i) / 64)
            tol = 4 * p * np.finfo(np.float32).eps + 1e-7
            assert abs(t[0, 0, p, i] - math.cos(ang)) <= tol
            assert abs(t[0, 1, p, i] - math.sin(ang)) <= tol
    # The pairs past 0 turn slower under the larger base.
    small_t = rope_table(160000.0, 10000.0, 5, 3)
    assert small_t[0, 1, 4, 2] < small_t[1, 1, 4, 2]


@pytest.mark.parametrize("family", ["modernbert", "nomic"])
def test_the_gated_limit_meets_the_textbook_and_bites(family):
    # The F16 tier's saturation of the gated product (65504), restated in the
    # oracle as a limit: the oracle with it meets the f64 textbook with the
    # same clip, the oracle without it meets the textbook without, and on a
    # model whose unit passes 65504 the two differ.
    make = small.modernbert if family == "modernbert" else small.nomic
    desc = small.gated_overflow(make(seed=41))
    ids, mask, types = small.ragged_rows(41, 4, 40, desc.vocab_size)
    types = None if family == "modernbert" else types
    kw = dict(normalize=S.TURBO_NORMALIZE_NONE)
    lim = oracle.encode(desc, ids, mask, types, gated_limit=65504.0, **kw)
    free = oracle.encode(desc, ids, mask, types, **kw)
    _plain_close(lim, plain.embed(desc, ids, mask, types, gated_limit=65504.0, **kw))
    _plain_close(free, plain.embed(desc, ids, mask, types, **kw))
    assert np.abs(lim - free).max() > 1e-3
    # A limit no product reaches changes no bit.
    assert np.array_equal(oracle.encode(desc, ids, mask, types, gated_limit=3e38, **kw), free)
