"""The HIP path against the oracle and the reference's sealed vectors, on an
MI355X, through the C ABI.

Tolerances are the reference's conformance floors
(core/src/record/mod.rs:341-348): F32 cosine >= 0.9999 and max abs diff
<= 1e-4; F16 and BF16 cosine >= 0.999. Bookkeeping (packing) is held bit
for bit, and so is the reference's whole-row range rule.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
import turboembed_amd as T
from turboembed_amd import seam as S
from turboembed_amd import workloads as W

import small

pytestmark = pytest.mark.gpu

FLOOR = {S.TURBO_DTYPE_F32: 0.9999, S.TURBO_DTYPE_F16: 0.999, S.TURBO_DTYPE_BF16: 0.999}


def assert_close(got, want, compute_dtype):
    cos = small.cosine_rows(got, want)
    assert cos.min() >= FLOOR[compute_dtype], f"min cosine {cos.min()} (dtype {compute_dtype})"
    if compute_dtype == S.TURBO_DTYPE_F32:
        assert np.abs(got - want).max() <= 1e-4, np.abs(got - want).max()


# ---- The GEMM kernel alone ------------------------------------------------------

@pytest.mark.parametrize("dtype", [S.TURBO_DTYPE_F32, S.TURBO_DTYPE_F16, S.TURBO_DTYPE_BF16])
@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16])
@pytest.mark.parametrize("mnk", [(256, 256, 64), (300, 200, 96), (33, 96, 32), (1000, 768, 768), (517, 2304, 1152),
                                 (70, 100, 64)])
def test_gemm_matches_numpy(runtime, dtype, tile, mnk):
    m, n, k = mnk
    g = np.random.Generator(np.random.PCG64(m * 7 + n + k))
    a = g.standard_normal((m, k)).astype(np.float32)
    w = g.standard_normal((n, k)).astype(np.float32)
    b = g.standard_normal(n).astype(np.float32)
    got = T.gemm_check(a, w, b, dtype=dtype, tile=tile)
    if dtype == S.TURBO_DTYPE_F16:
        a, w = a.astype(np.float16).astype(np.float64), w.astype(np.float16).astype(np.float64)
    elif dtype == S.TURBO_DTYPE_BF16:
        from turboembed_amd.model import to_bf16_bits
        f = lambda x: (to_bf16_bits(x).astype(np.uint32) << 16).view(np.float32).astype(np.float64)  # noqa: E731
        a, w = f(a), f(w)
    want = a.astype(np.float64) @ w.astype(np.float64).T + b
    err = np.abs(got - want).max() / np.sqrt(k)
    assert err < 1e-4, err


def test_the_mfma_probe_reports_a_rate_and_a_clock(runtime):
    # Random operands never run the matrix cores faster than fixed ones, and
    # the clock under the load is a shader clock (MHz, not a count).
    rnd, rnd_mhz = T.mfma_probe(random=True, iters=2000)
    fix, fix_mhz = T.mfma_probe(random=False, iters=2000)
    assert 50 < rnd <= 1.1 * fix < 3000, (rnd, fix)
    assert 500 < rnd_mhz < 3000 and 500 < fix_mhz < 3000, (rnd_mhz, fix_mhz)


# ---- The sealed tiny bundles ---------------------------------------------------------

@pytest.mark.parametrize("name", ["tiny_bert", "tiny_modernbert", "tiny_nomic", "tiny_deberta"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_tiny_bundles_meet_the_upstream_vectors(context, name, precision):
    desc, ids, lengths, vectors, info = oracle.fixture(name)
    ids, mask = oracle.fixture_rows(ids, lengths)
    norm = S.TURBO_NORMALIZE_L2 if info["embed"]["normalize"] == "NORMALIZE_L2" else S.TURBO_NORMALIZE_NONE
    model = context.load(desc)
    s = model.session(ids.shape[0], ids.shape[1], precision)
    got = s.embed(ids, mask, normalize=norm)
    assert_close(got, vectors, s.compute_dtype)
    want = oracle.encode(desc, ids, mask, normalize=norm)
    assert_close(got, want, s.compute_dtype)
    # One row at a time gives the batch's vectors within the bound.
    for r in (0, 7):
        one = s.embed(ids[r:r + 1], mask[r:r + 1], normalize=norm)
        assert_close(one, got[r:r + 1], s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_a_sealed_bundle_loads_and_meets_its_vectors(context, precision):
    # The tiny ModernBERT bundle as it is sealed, through load_bundle: its
    # files verified, its description built from the manifest, its
    # reference rows at the manifest's pooling, normalization and width.
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny-modernbert-bundle")
    model = context.load_bundle(path)
    ref = model.bundle.reference()
    pooling, normalize, dim, max_seq, max_batch = model.bundle.embed_defaults()
    ids = ref["ids"].astype(np.int32)
    mask = (np.arange(ids.shape[1])[None, :] < ref["lengths"][:, None]).astype(np.int32)
    s = model.session(max_batch, max_seq, precision)
    for at in range(0, ids.shape[0], max_batch):
        got = s.embed(ids[at:at + max_batch], mask[at:at + max_batch], pooling=pooling, normalize=normalize,
                      output_dim=dim)
        assert_close(got, ref["embeddings"][at:at + max_batch], s.compute_dtype)
    s.close()
    model.close()


# ---- Small models of every family, ragged rows ------------------------------------------

MODELS = {"bert": small.bert, "modernbert": small.modernbert, "nomic": small.nomic}


@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_ragged_rows_meet_the_oracle(context, family, precision):
    desc = MODELS[family](seed=11)
    ids, mask, types = small.ragged_rows(11, 7, 48, desc.vocab_size)
    if family == "modernbert":
        types = None
    model = context.load(desc)
    s = model.session(8, 64, precision)
    for pooling in (S.TURBO_POOLING_MEAN, S.TURBO_POOLING_CLS, S.TURBO_POOLING_LAST):
        got = s.embed(ids, mask, types, pooling=pooling, output_dim=40)
        want = oracle.encode(desc, ids, mask, types, pooling=pooling, output_dim=40)
        assert_close(got, want, s.compute_dtype)
    s.close()
    model.close()


def test_a_weight_past_f16_keeps_the_products_in_f32(context):
    # One GEMM weight beyond F16's 65504 (layer 0's FFN-out, [0, 0]) keeps a
    # FASTEST session's products in F32, as the reference's CUDA backend
    # does (core/cuda/backend.cpp:1168-1225): the session reports F32 and its
    # vectors meet the oracle at F32's bound.
    desc = small.bert(seed=51)
    w2 = 5 + 12   # [word, pos, type, ln w, ln b] + layer 0's [Wq, bq, Wk, bk, Wv, bv, Wo, bo, ln1, ln1b, W1, b1, W2]
    desc.tensors[w2] = desc.tensors[w2].copy()
    desc.tensors[w2][0, 0] = 70000.0
    ids, mask, types = small.ragged_rows(51, 4, 40, desc.vocab_size)
    model = context.load(desc)
    s = model.session(4, 40, S.TURBO_PRECISION_FASTEST)
    assert s.compute_dtype == S.TURBO_DTYPE_F32
    got = s.embed(ids, mask, types)
    assert_close(got, oracle.encode(desc, ids, mask, types), s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("family", ["modernbert", "nomic"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_FASTEST, "bf16", S.TURBO_PRECISION_EXACT])
def test_a_gated_product_past_f16_saturates(context, family, precision):
    # One FFN unit's act(gate) * up passes 65504 on most tokens. An F16
    # product saturates there instead of rounding to infinity (the
    # reference's CUDA backend, core/cuda/rotary.cuh:31-45), so the vectors
    # are finite and meet the oracle with the same limit; BF16 and F32 hold
    # the product as it is and meet the plain oracle.
    desc = small.gated_overflow(MODELS[family](seed=41))
    if precision == "bf16":
        from turboembed_amd.model import with_dtype
        desc, precision = with_dtype(desc, "bf16"), S.TURBO_PRECISION_MODEL
    ids, mask, types = small.ragged_rows(41, 4, 40, desc.vocab_size)
    types = None if family == "modernbert" else types
    model = context.load(desc)
    s = model.session(4, 40, precision)
    got = s.embed(ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE)
    assert np.isfinite(got).all()
    f16 = s.compute_dtype == S.TURBO_DTYPE_F16
    want = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, gated_limit=65504.0 if f16 else 0.0)
    assert_close(got, want, s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("batch,width", [(9, 40), (9, 37), (9, 600), (480, 600)])
def test_packing_is_the_oracle_s_bit_for_bit(context, batch, width):
    # Row widths a multiple of 4 (the mask read 16 bytes a lane; 600 takes
    # three steps of 256 columns) and one that is not (a column a lane); 480
    # rows of 600 columns pass the placement grid's 1024 x 256 threads.
    desc = small.bert(seed=12, positions=640)
    ids, mask, types = small.ragged_rows(12, batch, width, desc.vocab_size)
    model = context.load(desc)
    s = model.session(max(batch, 16), 640 if width > 64 else 64, S.TURBO_PRECISION_EXACT)
    s.embed(ids, mask, types)
    start, ln, at = s.packing()
    o_start, o_len, o_at = oracle.pack(mask)
    assert np.array_equal(start, o_start.astype(np.int32))
    assert np.array_equal(ln, o_len.astype(np.int32))
    assert np.array_equal(at, o_at.astype(np.int32))
    s.close()
    model.close()


def test_packing_on_planes_of_an_odd_capacity(context):
    # A session of 3 x 5 token slots keeps its mask plane 16-byte aligned,
    # so rows of 4 columns (read 16 bytes a lane) pack as the oracle does.
    desc = small.bert(seed=13, positions=64)
    ids, mask, types = small.ragged_rows(13, 3, 4, desc.vocab_size)
    model = context.load(desc)
    s = model.session(3, 5, S.TURBO_PRECISION_EXACT)
    got = s.embed(ids, mask, types)
    start, ln, at = s.packing()
    o_start, o_len, o_at = oracle.pack(mask)
    assert np.array_equal(start, o_start.astype(np.int32))
    assert np.array_equal(ln, o_len.astype(np.int32))
    assert np.array_equal(at, o_at.astype(np.int32))
    assert_close(got, oracle.encode(desc, ids, mask, types), s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_ranges(context, precision):
    desc = small.bert(seed=13)
    ids, mask, types = small.ragged_rows(13, 6, 48, desc.vocab_size)
    model = context.load(desc)
    s = model.session(8, 64, precision, max_ranges=64)
    rows = s.embed(ids, mask, types)
    # Whole-row ranges give the rows' vectors bit for bit
    # (core/tests/ranges/whole_row.rs:8-28).
    s.write_ranges(ids, mask, [(r, 0, 48) for r in range(6)], types)
    s.run()
    assert np.array_equal(s.read(), rows)
    g = np.random.Generator(np.random.PCG64(5))
    ranges = []
    while len(ranges) < 40:
        r = int(g.integers(0, 6))
        a = int(g.integers(0, 47))
        b = int(g.integers(a + 1, 49))
        if mask[r, a:b].any():
            ranges.append((r, a, b))
    s.write_ranges(ids, mask, ranges, types)
    s.run()
    got = s.read()
    want = oracle.encode(desc, ids, mask, types, ranges=ranges)
    assert_close(got, want, s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_means_over_many_chunks(context, precision):
    # Rows of up to 1100 tokens with holes: a mean sums 256-token chunks on
    # their own, then the chunk sums in order. Rows and ranges that cross
    # chunk boundaries (or hold a whole chunk of masked tokens) meet the
    # oracle; a whole-row range is the row bit for bit.
    desc = small.bert(seed=17, positions=1200)
    ids, mask, types = small.ragged_rows(17, 4, 1100, desc.vocab_size)
    mask[1] = 0
    mask[1, :1000] = 1
    mask[1, 300:600] = 0
    model = context.load(desc)
    s = model.session(4, 1100, precision, max_ranges=16)
    rows = s.embed(ids, mask, types, pooling=S.TURBO_POOLING_MEAN)
    assert_close(rows, oracle.encode(desc, ids, mask, types, pooling=S.TURBO_POOLING_MEAN), s.compute_dtype)
    lens = [int(np.flatnonzero(m)[-1]) + 1 for m in mask]
    s.write_ranges(ids, mask, [(r, 0, lens[r]) for r in range(4)], types)
    s.run()
    assert np.array_equal(s.read(), rows)
    ranges = [(0, 10, 1000), (1, 250, 650), (1, 290, 610), (1, 255, 257), (3, 0, lens[3]), (0, 511, 513)]
    s.write_ranges(ids, mask, ranges, types)
    s.run()
    assert_close(s.read(), oracle.encode(desc, ids, mask, types, ranges=ranges), s.compute_dtype)
    s.close()
    model.close()


def test_same_rows_same_bits(context):
    desc = small.bert(seed=14)
    ids, mask, types = small.ragged_rows(14, 8, 64, desc.vocab_size)
    model = context.load(desc)
    s = model.session(8, 64, S.TURBO_PRECISION_FASTEST)
    a = s.embed(ids, mask, types)
    b = s.embed(ids, mask, types)
    assert np.array_equal(a, b)
    info = s.run_info
    assert info.device_allocs == 0 and info.host_allocs == 0
    assert info.stage[S.TURBO_STAGE_MAX - 16 + 3] == S.TURBO_STAGE_DEVICE
    s.close()
    model.close()


def test_run_before_write_is_invalid_state(context):
    desc = small.bert(seed=15)
    model = context.load(desc)
    s = model.session(2, 16, S.TURBO_PRECISION_EXACT)
    with pytest.raises(T.TurboError) as e:
        s.run()
    assert e.value.code == S.TURBO_E_INVALID_STATE
    s.close()
    model.close()


# ---- The workloads at their real widths -------------------------------------------------

def test_minilm_exact_meets_the_oracle(context):
    sh = W.SHAPES["minilm"]
    desc = W.model(sh)
    ids, mask, types = W.rows(sh)
    model = context.load(desc)
    s = model.session(sh.batch, sh.seq, sh.precision)
    assert s.compute_dtype == S.TURBO_DTYPE_F32
    got = s.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    want = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    assert_close(got, want, s.compute_dtype)
    s.close()
    model.close()


@pytest.mark.parametrize("lengths", [None, (64, 512)])
def test_bert_base_fastest_meets_the_oracle(context, lengths):
    # Full width and sequence; 2 of the 12 layers and 6 of the 64 rows keep
    # the oracle's share to seconds. The full model runs in the benchmark.
    sh = W.SHAPES["bert-base"]
    desc = W.model(sh, layers=2)
    ids, mask, types = W.rows(sh, batch=6, lengths=lengths)
    model = context.load(desc)
    s = model.session(64, 512, sh.precision)
    assert s.compute_dtype == S.TURBO_DTYPE_F16
    got = s.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    want = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    assert_close(got, want, s.compute_dtype)
    s.close()
    model.close()


# ---- Attention paths ------------------------------------------------------------------

@pytest.mark.parametrize("family", ["bert", "modernbert"])
@pytest.mark.parametrize("heads", [2, 4])
def test_matrix_core_attention_meets_the_oracle(context, family, heads, monkeypatch):
    # Head widths 64 and 32 on long ragged rows (several 128-query blocks and
    # 64-key blocks), and ModernBERT's sliding windows across block edges.
    if family == "bert":
        desc = small.bert(seed=21, hidden=128, heads=heads, inter=256, positions=320, std=0.1)
    else:
        desc = small.modernbert(seed=21, hidden=128, heads=heads, inter=192, positions=320, window=32, std=0.1)
    ids, mask, types = small.ragged_rows(21, 5, 300, desc.vocab_size)
    if family == "modernbert":
        types = None
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    got = {}
    for path in ("mfma", "simple"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", f"attention={path}")
        s = model.session(8, 320, S.TURBO_PRECISION_FASTEST)
        # The string names the path that runs: the matrix-core kernel takes
        # heads of 64 alone.
        runs = path if desc.hidden // desc.heads == 64 else "simple"
        assert f"attn={runs}" in s.choices() and "forced=attn" in s.choices()
        got[path] = s.embed(ids, mask, types)
        assert_close(got[path], want, s.compute_dtype)
        s.close()
    model.close()


@pytest.mark.parametrize("family", ["bert", "modernbert"])
def test_matrix_core_attention_on_long_rows_with_holes(context, family, monkeypatch):
    # Rows past 64 key blocks, where each wave reads its blocks' mask words in
    # more than one batch of eight (4,700 and 2,300 tokens, eight waves of the
    # 256-query path and four of the 128-query one), with masked keys through
    # them: on block edges (63, 64, 4095, 4096), in runs, and a whole 64-key
    # block; ModernBERT's local layers on 16-key windows across those rows.
    # Both query-block sizes against the oracle and against each other (the
    # same per-wave arithmetic over the same blocks).
    seq = 4800
    if family == "bert":
        desc = small.bert(seed=41, layers=2, hidden=128, heads=2, inter=256, positions=seq, std=0.2)
    else:
        desc = small.modernbert(seed=41, layers=2, hidden=128, heads=2, inter=192, positions=seq, window=16,
                                global_every=2, std=0.2)
    g = np.random.Generator(np.random.PCG64(41))
    ids = g.integers(0, desc.vocab_size, size=(3, seq)).astype(np.int32)
    mask = np.zeros((3, seq), np.int32)
    mask[0, :4700] = 1
    mask[0, g.choice(np.arange(1, 4699), size=40, replace=False)] = 0
    mask[0, [63, 64, 4095, 4096]] = 0
    mask[0, 1024:1088] = 0
    mask[1, :2300] = 1
    mask[1, 500:530] = 0
    mask[1, [127, 128, 2047]] = 0
    mask[2, :100] = 1
    types = g.integers(0, 2, size=(3, seq)).astype(np.int32) if family == "bert" else None
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    got = {}
    for path in ("mfma", "mfma128"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", f"attention={path}")
        s = model.session(3, seq, S.TURBO_PRECISION_FASTEST)
        assert f"attn={path}" in s.choices()
        got[path] = s.embed(ids, mask, types)
        assert_close(got[path], want, s.compute_dtype)
        s.close()
    model.close()
    assert small.cosine_rows(got["mfma"], got["mfma128"]).min() >= 0.999999


@pytest.mark.parametrize("tier", ["f16", "bf16"])
@pytest.mark.parametrize("family", ["bert", "modernbert"])
def test_matrix_core_attention_rescales_as_the_scalar_path_does(context, family, tier, monkeypatch):
    # Weights N(0, 0.3) spread a head's scores over tens of units, so in many
    # rows a later 32-key sub-block's max passes the running max by more than
    # 2^8 (log2 units) and the matrix-core kernel rescales the context so far
    # and moves its bias tile. The scalar F32 path over the same 16-bit Q, K and
    # V is the check, with the oracle at the dtype's floor beside it.
    if family == "bert":
        desc = small.bert(seed=31, hidden=128, heads=2, inter=256, positions=320, std=0.3)
    else:
        desc = small.modernbert(seed=31, hidden=128, heads=2, inter=192, positions=320, window=48, std=0.3)
    precision = S.TURBO_PRECISION_FASTEST
    if tier == "bf16":
        # (BF16 operands: the bias tile and the pre-scaled Q in BF16.)
        from turboembed_amd.model import with_dtype
        desc, precision = with_dtype(desc, "bf16"), S.TURBO_PRECISION_MODEL
    ids, mask, types = small.ragged_rows(31, 6, 300, desc.vocab_size)
    if family == "modernbert":
        types = None
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    got = {}
    for path in ("mfma", "simple"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", f"attention={path}")
        s = model.session(8, 320, precision)
        assert f"attn={path}" in s.choices()
        got[path] = s.embed(ids, mask, types)
        assert_close(got[path], want, s.compute_dtype)
        dtype = s.compute_dtype
        s.close()
    model.close()
    # (BF16's 8-bit mantissa: its p values and Q carry 2^-9 rounding.)
    bound = 0.9999 if dtype == S.TURBO_DTYPE_F16 else 0.999
    assert small.cosine_rows(got["mfma"], got["simple"]).min() >= bound


# ---- The int8 tier ---------------------------------------------------------------------
#
# No reference kernel exists for it (the reference's one I8 encoder is a
# compiled Hailo graph); its bound is the conformance floor for I8, cosine
# >= 0.93 against the F32 oracle (core/tests/common/conformance.rs:15).

I8_FLOOR = 0.93


def quantize_rows(x):
    """Symmetric int8 rows as the kernels make them: scale = max|x| / 127,
    q = round-half-even(x * (127 / max|x|)), all in F32."""
    x = np.asarray(x, np.float32)
    mx = np.abs(x).max(1).astype(np.float32)
    inv = np.where(mx > 0, np.float32(127) / np.where(mx > 0, mx, 1), 0).astype(np.float32)
    q = np.clip(np.rint(x * inv[:, None]), -127, 127).astype(np.int64)
    return q, (mx / np.float32(127)).astype(np.float32)


@pytest.mark.parametrize("tile", [0, 7, 9, 15])
@pytest.mark.parametrize("mnk", [(256, 256, 128), (300, 200, 64), (1000, 768, 768), (517, 2304, 3072), (33, 96, 192)])
def test_int8_gemm_is_the_integer_product(runtime, tile, mnk):
    # The int32 sums are exact; the dequantized F32 result differs from
    # (sum * a_scale * w_scale + bias), computed the same way, by F32
    # rounding of a sum past 2^24 at most.
    m, n, k = mnk
    g = np.random.Generator(np.random.PCG64(m * 5 + n + k))
    a = g.standard_normal((m, k)).astype(np.float32)
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    a[3] = 0.0   # a zero row: scale 0, output the bias
    b = g.standard_normal(n).astype(np.float32)
    got = T.gemm_check(a, w, b, dtype=S.TURBO_DTYPE_I8, tile=tile)
    qa, sa = quantize_rows(a)
    qw, sw = quantize_rows(w)
    acc = (qa @ qw.T).astype(np.float64)
    want = acc * sa[:, None].astype(np.float64) * sw[None, :].astype(np.float64) + b
    scale = np.abs(acc).max() * sa.max() * sw.max() + 1
    assert np.abs(got - want).max() <= 1e-6 * scale, np.abs(got - want).max()
    np.testing.assert_array_equal(got[3], b)


def int8_model(desc):
    desc.compute_dtype = S.TURBO_DTYPE_I8
    return desc


@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
def test_int8_ragged_rows_meet_the_oracle(context, family):
    kw = dict(seed=31, hidden=128, inter=256)
    desc = int8_model(MODELS[family](**kw))
    ids, mask, types = small.ragged_rows(31, 7, 48, desc.vocab_size)
    if family == "modernbert":
        types = None
    model = context.load(desc)
    s = model.session(8, 64, S.TURBO_PRECISION_FASTEST)
    assert s.compute_dtype == S.TURBO_DTYPE_I8
    for pooling in (S.TURBO_POOLING_MEAN, S.TURBO_POOLING_CLS):
        got = s.embed(ids, mask, types, pooling=pooling)
        want = oracle.encode(desc, ids, mask, types, pooling=pooling)
        cos = small.cosine_rows(got, want)
        assert cos.min() >= I8_FLOOR, cos.min()
    s.close()
    # EXACT on the same model computes in F32.
    s = model.session(8, 64, S.TURBO_PRECISION_EXACT)
    assert s.compute_dtype == S.TURBO_DTYPE_F32
    assert_close(s.embed(ids, mask, types), oracle.encode(desc, ids, mask, types), s.compute_dtype)
    s.close()
    model.close()


def test_int8_bert_base_meets_the_oracle(context):
    sh = W.SHAPES["bert-base"]
    desc = int8_model(W.model(sh, layers=2))
    ids, mask, types = W.rows(sh, batch=6, lengths=(64, 512))
    model = context.load(desc)
    s = model.session(64, 512, S.TURBO_PRECISION_FASTEST)
    assert s.compute_dtype == S.TURBO_DTYPE_I8
    got = s.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    want = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    cos = small.cosine_rows(got, want)
    assert cos.min() >= I8_FLOOR, cos.min()
    s.close()
    model.close()


@pytest.mark.parametrize("split", ["0", "2"])
def test_int8_block_shapes_give_the_same_bits(context, monkeypatch, split):
    # The int32 sums are exact and each output is dequantized by the same
    # steps in every block shape, so 256 x 384 tiles (their scales and
    # biases read from LDS) and 256 x 256 tiles give the same states bit for
    # bit: BERT-base width at 2 layers, ragged rows, the Q/K/V scatter, GELU
    # and bias epilogues, split into two parts or not.
    sh = W.SHAPES["bert-base"]
    desc = int8_model(W.model(sh, layers=2))
    ids, mask, types = W.rows(sh, batch=24, lengths=(64, 512))
    model = context.load(desc)
    out = {}
    for tile in ("256x256", "256x384"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", f"all:qkv={tile},out={tile},ffn1={tile},ffn2={tile}")
        monkeypatch.setenv("TURBO_ROCM_SPLIT", split)
        s = model.session(24, 512, S.TURBO_PRECISION_FASTEST)
        assert s.compute_dtype == S.TURBO_DTYPE_I8 and f"qkv={tile}," in s.choices()
        out[tile] = (s.embed(ids, mask, types, pooling=sh.pooling, normalize=sh.normalize), s.hidden())
        s.close()
    np.testing.assert_array_equal(out["256x256"][1], out["256x384"][1])
    np.testing.assert_array_equal(out["256x256"][0], out["256x384"][0])
    want = oracle.encode(desc, ids, mask, types, pooling=sh.pooling, normalize=sh.normalize)
    assert small.cosine_rows(out["256x384"][0], want).min() >= I8_FLOOR
    model.close()


# ---- Rerank ------------------------------------------------------------------------------
#
# Scores are bounded one by one, as a fraction of the run's scale (the largest
# reference score in magnitude): F32 1e-4, F16 1e-2, BF16 4e-2, I8 0.15
# (docs/conformance.md "Scores"; core/tests/conformance/scores.rs).

SCORE_BOUND = {S.TURBO_DTYPE_F32: 1e-4, S.TURBO_DTYPE_F16: 1e-2, S.TURBO_DTYPE_BF16: 4e-2, S.TURBO_DTYPE_I8: 0.15}


@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_rerank_scores_meet_transformers(context, precision):
    from turboembed_amd.rerank import RerankHead
    desc, pairs, head, info, ref = oracle.rerank_fixture()
    model = context.load(desc)
    s = model.session(info["max_batch"], info["max_tokens"], precision, task=S.TURBO_TASK_RERANK)
    h = RerankHead(**head)
    kw = dict(query_tokens=info["query_tokens"], max_tokens=info["max_tokens"])
    scale = np.abs(ref["scores"]).max()
    bound = SCORE_BOUND[s.compute_dtype] * scale
    # All pairs in one write (their 7 windows in two runs of max_batch), then one pair a write.
    got = s.rerank(pairs, h, info["start_id"], info["end_id"], **kw)
    assert np.abs(got - ref["scores"]).max() <= bound, (got, ref["scores"])
    for i, pair in enumerate(pairs):
        one = s.rerank([pair], h, info["start_id"], info["end_id"], **kw)
        assert abs(one[0] - ref["scores"][i]) <= bound
    s.close()
    model.close()


def test_rerank_refuses_what_the_core_refuses(context):
    from turboembed_amd.rerank import RerankHead
    desc, pairs, head, info, ref = oracle.rerank_fixture()
    model = context.load(desc)
    h = RerankHead(**head)
    s = model.session(2, 32, S.TURBO_PRECISION_EXACT, task=S.TURBO_TASK_RERANK)
    with pytest.raises(T.TurboError) as e:
        s.rerank(pairs, h, info["start_id"], info["end_id"], query_tokens=8)
    assert e.value.code == S.TURBO_E_CAPACITY
    s.close()
    s = model.session(4, 32, S.TURBO_PRECISION_EXACT)
    with pytest.raises(T.TurboError) as e:
        s.rerank(pairs, h, info["start_id"], info["end_id"], query_tokens=8)
    assert e.value.code == S.TURBO_E_UNSUPPORTED_TASK
    s.close()
    model.close()


# ---- DeBERTa-v2: disentangled attention over relative buckets ----------------------------
#
# Rows with holes and a masked column 0 (a masked token is zero after the
# embedding, and every one shares one uniform-attention state), every pooling,
# ranges and layer reads, against the oracle; and a run long enough to split.

def _close_or_floor(got, want, dtype):
    if dtype == S.TURBO_DTYPE_I8:
        assert small.cosine_rows(got, want).min() >= I8_FLOOR
    else:
        assert_close(got, want, dtype)


@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST, "bf16", "int8"])
def test_deberta_rows_with_masked_tokens_meet_the_oracle(context, precision):
    from test_deberta import holed_rows, small_deberta
    from turboembed_amd.model import with_dtype
    desc = small_deberta()
    tier = {"bf16": S.TURBO_DTYPE_BF16, "int8": S.TURBO_DTYPE_I8}.get(precision)
    if precision == "bf16":
        desc, precision = with_dtype(desc, "bf16"), S.TURBO_PRECISION_FASTEST
    elif precision == "int8":         # int8 products need widths in multiples of 64
        desc, precision = int8_model(small_deberta(hidden=64, inter=128)), S.TURBO_PRECISION_FASTEST
    ids, mask = holed_rows(desc.vocab_size)
    model = context.load(desc)
    s = model.session(4, 40, precision, max_ranges=12)
    assert tier is None or s.compute_dtype == tier
    for pooling in (S.TURBO_POOLING_MEAN, S.TURBO_POOLING_CLS, S.TURBO_POOLING_LAST):
        got = s.embed(ids, mask, pooling=pooling)
        _close_or_floor(got, oracle.encode(desc, ids, mask, pooling=pooling), s.compute_dtype)
    ranges = [(0, 0, 40), (1, 2, 13), (2, 5, 6), (1, 12, 25)]
    s.write_layer_ranges(ids, mask, ranges, 2, normalize=S.TURBO_NORMALIZE_NONE)
    s.run()
    want = oracle.encode(desc, ids, mask, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges, taps=2)
    _close_or_floor(s.read(), want, s.compute_dtype)
    s.close()
    model.close()


def test_deberta_split_runs_meet_the_oracle(context, monkeypatch):
    from test_deberta import small_deberta
    desc = small_deberta(seed=5, hidden=64, heads=4, inter=128, buckets=16, maximum=64)
    g = np.random.Generator(np.random.PCG64(6))
    ids = g.integers(0, desc.vocab_size, (80, 64)).astype(np.int32)
    lengths = g.integers(48, 65, 80)
    mask = (np.arange(64)[None, :] < lengths[:, None]).astype(np.int32)
    mask[7, 3] = 0
    assert mask.sum() >= 4096
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_SPLIT", "4")
    s = model.session(80, 64, S.TURBO_PRECISION_FASTEST)
    got = s.embed(ids, mask)
    assert_close(got, oracle.encode(desc, ids, mask), s.compute_dtype)
    s.close()
    model.close()


def _deberta_rows(seed, batch, seq, vocab):
    g = np.random.Generator(np.random.PCG64(seed))
    lengths = np.concatenate([[seq, 131, 64, 33, 1], g.integers(1, seq + 1, batch - 5)])[:batch]
    ids = g.integers(0, vocab, (batch, seq)).astype(np.int32)
    mask = (np.arange(seq)[None, :] < lengths[:, None]).astype(np.int32)
    mask[0, [5, 6, 100]] = 0          # holes
    mask[1, 0] = 0                    # a masked first column
    return ids, mask


@pytest.mark.parametrize("tier", ["f16", "bf16"])
def test_deberta_matrix_core_path_meets_the_oracle(context, monkeypatch, tier):
    # Heads of 64 on F16 and BF16 take the matrix-core form: rows past one
    # 128-query block, tiles of distances wholly in the buckets' linear half
    # (|i - j| <= 64 of 128 buckets, 256 positions) and tiles past it, holes
    # and a masked first column; the same rows through the scalar form, and a
    # run long enough to split into two parts.
    from test_deberta import small_deberta
    from turboembed_amd.model import with_dtype
    desc = small_deberta(seed=7, hidden=128, heads=2, inter=256, buckets=128, maximum=256, std=0.1)
    if tier == "bf16":
        desc = with_dtype(desc, "bf16")
    ids, mask = _deberta_rows(8, 5, 200, desc.vocab_size)
    want = oracle.encode(desc, ids, mask)
    model = context.load(desc)
    got = {}
    for path in ("mfma", "simple"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", f"attention={path}")
        s = model.session(5, 200, S.TURBO_PRECISION_FASTEST)
        assert f"attn={path}" in s.choices()
        got[path] = s.embed(ids, mask)
        assert_close(got[path], want, s.compute_dtype)
        s.close()
    assert small.cosine_rows(got["mfma"], got["simple"]).min() >= FLOOR[S.TURBO_DTYPE_F16]
    monkeypatch.delenv("TURBO_ROCM_CHOICES")
    ids, mask = _deberta_rows(9, 40, 200, desc.vocab_size)
    assert mask.sum() >= 4096
    monkeypatch.setenv("TURBO_ROCM_SPLIT", "2")
    s = model.session(40, 200, S.TURBO_PRECISION_FASTEST)
    assert_close(s.embed(ids, mask), oracle.encode(desc, ids, mask), s.compute_dtype)
    s.close()
    model.close()


def test_deberta_projections_past_f16_run_the_scalar_form(context):
    # Layer 0's query projections of the relative rows pass F16's range: a
    # weight of 3e4 (within F16) on a hidden column that every LayerNorm
    # zeroes in the states but the relative rows' norm carries at 10, in head
    # dimensions whose keys are zero, so every score stays moderate. The F16
    # session keeps those projections in F32 on the scalar form, its choices
    # say so, and its vectors meet the oracle.
    from test_deberta import small_deberta
    from turboembed_amd.model import with_dtype
    desc = with_dtype(small_deberta(seed=7, hidden=128, heads=2, inter=256, buckets=128, maximum=256, std=0.1),
                      "f32")
    t, col, dims = desc.tensors, 5, [0, 1, 2, 3]
    t[1][col] = t[2][col] = 0.0                   # the embedding norm zeroes the column
    t[4][col] = 10.0                              # the relative rows' norm carries it
    for layer in range(desc.layers):
        for i in (8, 9, 14, 15):                  # the layers' norms zero it too
            t[6 + 16 * layer + i][col] = 0.0
    t[6 + 2][dims, :] = 0.0                       # layer 0's keys are zero in these dimensions
    t[6 + 3][dims] = 0.0
    t[6 + 0][dims, col] = 3.0e4                   # its queries weigh the column
    ids, mask = _deberta_rows(10, 5, 200, desc.vocab_size)
    want = oracle.encode(desc, ids, mask)
    model = context.load(desc)
    s = model.session(5, 200, S.TURBO_PRECISION_FASTEST)
    assert s.compute_dtype == S.TURBO_DTYPE_F16
    assert "attn=simple" in s.choices() and "attn=mfma" not in s.choices(), s.choices()
    assert_close(s.embed(ids, mask), want, s.compute_dtype)
    s.close()
    model.close()


# ---- Split runs: two parts of the rows on two streams -------------------------------------
#
# A run of at least 4096 packed tokens and two rows or more runs its rows in
# two parts on the context's two streams. Each part's products, norms and
# attention read and write its own tokens alone, so the vectors are the
# oracle's at the tier's bound and, token for token, the unsplit run's.

def _long_rows(seed, batch, seq, vocab, types):
    g = np.random.Generator(np.random.PCG64(seed))
    lengths = g.integers(300, seq + 1, batch)
    ids = g.integers(0, vocab, (batch, seq)).astype(np.int32)
    mask = (np.arange(seq)[None, :] < lengths[:, None]).astype(np.int32)
    mask[3, 5] = 0                                   # a hole
    ty = g.integers(0, types, (batch, seq)).astype(np.int32) if types > 1 else None
    assert mask.sum() >= 4096
    return ids, mask, ty


def _unsplit(model, monkeypatch, *a, **kw):
    monkeypatch.setenv("TURBO_ROCM_SPLIT", "0")
    s = model.session(*a, **kw)
    monkeypatch.delenv("TURBO_ROCM_SPLIT")
    return s


@pytest.mark.parametrize("parts", ["2", "4"])
@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST, "int8"])
def test_split_runs_meet_the_oracle_and_the_unsplit_run(context, monkeypatch, parts, family, precision):
    kw = dict(seed=41, hidden=128, inter=256, positions=512 if family == "bert" else 1024)
    desc = MODELS[family](**kw)
    if precision == "int8":
        desc, precision = int8_model(desc), S.TURBO_PRECISION_FASTEST
    ids, mask, types = _long_rows(5, 16, 512, desc.vocab_size, max(1, desc.token_types))
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_SPLIT", parts)      # at most 3 parts of these rows' tokens
    s = model.session(16, 512, precision, max_ranges=64)
    u = _unsplit(model, monkeypatch, 16, 512, precision, max_ranges=64)
    got = s.embed(ids, mask, types)
    want = oracle.encode(desc, ids, mask, types)
    if s.compute_dtype == S.TURBO_DTYPE_I8:
        assert small.cosine_rows(got, want).min() >= I8_FLOOR
    else:
        assert_close(got, want, s.compute_dtype)
    assert small.cosine_rows(got, u.embed(ids, mask, types)).min() >= 0.99999
    # The same shape again (a graph replay), then ranges across both parts.
    np.testing.assert_array_equal(s.embed(ids, mask, types), got)
    ranges = [(r, 0, 40) for r in range(16)] + [(7, 100, 299), (15, 1, 2)]
    s.write_ranges(ids, mask, ranges, types)
    s.run()
    rg = s.read()
    u.write_ranges(ids, mask, ranges, types)
    u.run()
    assert small.cosine_rows(rg, u.read()).min() >= 0.99999
    s.close()
    u.close()
    model.close()


# ---- Extractive QA: the span head on the device ------------------------------------------
#
# testdata/tiny-qa-reference's transformers logits for every token of six
# windows, through headed range writes (include/turbo/turbo.h:699-710), at
# the reference's score bounds; and the head on multi-token ranges of every
# family against the oracle.

@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
@pytest.mark.parametrize("max_batch", [1, 2, 6])
def test_span_head_meets_the_upstream_logits(context, precision, max_batch):
    desc, windows, logits, info = oracle.qa_fixture()
    model = context.load(desc)
    s = model.session(max_batch, info["qa"]["max_seq"], precision, task=S.TURBO_TASK_EXTRACTIVE_QA)
    got = s.span_logits(windows, info["pad_id"])
    assert [len(a) for a, _ in got] == [len(w) for w, _ in windows]
    flat = np.stack([np.concatenate([a for a, _ in got]), np.concatenate([e for _, e in got])], 1)
    scale = np.abs(logits).max()
    d = np.abs(flat - logits).max() / scale
    assert d <= SCORE_BOUND[s.compute_dtype], d
    want = oracle.qa_logits(desc, windows, info["pad_id"])
    dw = np.abs(flat - want).max() / scale
    assert dw <= SCORE_BOUND[s.compute_dtype], dw
    print(f"QA max_batch {max_batch} dtype {s.compute_dtype}: {d:.2e} of the scale from transformers, "
          f"{dw:.2e} from the oracle")
    s.close()
    model.close()


@pytest.mark.parametrize("task", [S.TURBO_TASK_EMBED, S.TURBO_TASK_RERANK, S.TURBO_TASK_EXTRACTIVE_QA])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_MODEL, S.TURBO_PRECISION_FASTEST, S.TURBO_PRECISION_EXACT])
def test_capability_answers_every_task_the_core_maps_to_embed(runtime, task, precision):
    # The core asks with the model's own task (QA and rerank included) and
    # refuses the session on UNSUPPORTED (core/src/session/create.rs:93-111).
    st, dt, honored, reason = runtime.capability(0, task, precision)
    assert st == S.TURBO_CAP_EXPERIMENTAL, reason
    assert dt == (S.TURBO_DTYPE_F16 if precision == S.TURBO_PRECISION_FASTEST else S.TURBO_DTYPE_F32)
    assert honored == 0x338 and reason == ""
    st, _, _, reason = runtime.capability(0, 99, precision)
    assert st == S.TURBO_CAP_UNSUPPORTED and "task 99" in reason


def test_a_qa_session_opens_as_the_core_opens_it(context):
    # Capability with TURBO_TASK_EXTRACTIVE_QA, then session_open with EMBED
    # and a range per token; the span head's logits come back.
    desc, windows, logits, info = oracle.qa_fixture()
    st, _, _, _ = context.rt.capability(context.ordinal, S.TURBO_TASK_EXTRACTIVE_QA, S.TURBO_PRECISION_EXACT)
    assert st == S.TURBO_CAP_EXPERIMENTAL
    model = context.load(desc)
    s = model.session(2, info["qa"]["max_seq"], S.TURBO_PRECISION_EXACT, task=S.TURBO_TASK_EXTRACTIVE_QA)
    assert s.task == S.TURBO_TASK_EXTRACTIVE_QA and s.max_ranges == 2 * info["qa"]["max_seq"]
    got = s.span_logits(windows[:2], info["pad_id"])
    n = sum(len(w) for w, _ in windows[:2])
    flat = np.stack([np.concatenate([a for a, _ in got]), np.concatenate([e for _, e in got])], 1)
    assert np.abs(flat - logits[:n]).max() <= SCORE_BOUND[s.compute_dtype] * np.abs(logits).max()
    s.close()
    model.close()


@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
def test_span_head_on_ranges_meets_the_oracle(context, family):
    base = MODELS[family](seed=11)
    g = np.random.Generator(np.random.PCG64(12))
    w = (g.standard_normal((3, base.hidden)) * 0.3).astype(np.float32)
    b = g.standard_normal(3).astype(np.float32)
    from turboembed_amd.model import ModelDesc
    desc = ModelDesc(base.family, base.layers, base.hidden, base.heads, base.intermediate, base.vocab_size,
                     base.max_positions, base.token_types, base.layer_norm_eps, base.tensors, base.position_offset,
                     base.rope, base.attention_window, base.global_every, base.mlp, base.activation, base.norm,
                     base.names, base.compute_dtype, span_head=(w, b))
    ids, mask, types = small.ragged_rows(21, 5, 40, base.vocab_size, types=max(1, base.token_types))
    live = [np.flatnonzero(m) for m in mask]
    ranges = [(r, int(c), int(c) + 1) for r in range(5) for c in live[r][:3]]
    ranges += [(r, int(live[r][0]), int(live[r][-1]) + 1) for r in range(5)]
    model = context.load(desc)
    s = model.session(5, 40, S.TURBO_PRECISION_EXACT, max_ranges=len(ranges))
    s.write_ranges(ids, mask, ranges, types, normalize=S.TURBO_NORMALIZE_NONE)
    s.run()
    got = s.read()
    want = oracle.encode(desc, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE, ranges=ranges, head=True)
    assert got.shape == want.shape == (len(ranges), 3)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= SCORE_BOUND[S.TURBO_DTYPE_F32] * scale, np.abs(got - want).max() / scale
    # The same shape again replays the run's graph; a row write on the
    # headed model is a plain embedding write.
    s.write_ranges(ids, mask, ranges, types, normalize=S.TURBO_NORMALIZE_NONE)
    s.run()
    assert np.array_equal(s.read(), got)
    v = s.embed(ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE)
    assert_close(v, oracle.encode(base, ids, mask, types, normalize=S.TURBO_NORMALIZE_NONE), s.compute_dtype)
    s.close()
    model.close()


def test_span_head_refuses_what_the_core_refuses(context):
    desc, windows, logits, info = oracle.qa_fixture()
    model = context.load(desc)
    s = model.session(2, 24, S.TURBO_PRECISION_EXACT, task=S.TURBO_TASK_EXTRACTIVE_QA)
    ids = np.zeros((1, 24), np.int32)
    mask = np.zeros((1, 24), np.int32)
    n = len(windows[0][0])
    ids[0, :n], mask[0, :n] = windows[0][0], 1
    for kw, field in ((dict(normalize=S.TURBO_NORMALIZE_L2), 4), (dict(normalize=S.TURBO_NORMALIZE_NONE, output_dim=8), 6)):
        with pytest.raises(T.TurboError) as e:
            s.write_ranges(ids, mask, [(0, 0, 1)], **kw)
        assert (e.value.code, e.value.field) == (S.TURBO_E_UNSUPPORTED_OPTION, field)
    s.write_ranges(ids, mask, [(0, 0, 1), (0, 1, 3)], normalize=S.TURBO_NORMALIZE_NONE)
    s.run()
    assert s.read().shape == (2, 2)
    with pytest.raises(T.TurboError) as e:
        s.read_quantized(S.TURBO_QUANTIZE_UBINARY)
    assert (e.value.code, e.value.field) == (S.TURBO_E_UNSUPPORTED_OPTION, 7)
    # Through the seam itself: the backend holds the same rules.
    r = S.turbo_backend_embed_rows()
    r.struct_size = C.sizeof(r)
    r.batch, r.seq, r.row_stride = 1, 24, 24
    r.ids, r.mask = ids.ctypes.data_as(C.POINTER(C.c_int32)), mask.ctypes.data_as(C.POINTER(C.c_int32))
    r.pooling, r.normalize, r.output_dim, r.head, r.taps = S.TURBO_POOLING_MEAN, S.TURBO_NORMALIZE_L2, 2, 1, 1
    rg = (S.turbo_token_range * 1)()
    rg[0].row, rg[0].start, rg[0].end = 0, 0, 1
    err = S.new_error()
    assert s.t.embed_write_ranges(s.h, C.byref(r), rg, 1, C.byref(err)) == S.TURBO_E_UNSUPPORTED_OPTION
    r.normalize, r.output_dim = S.TURBO_NORMALIZE_NONE, 32
    assert s.t.embed_write_ranges(s.h, C.byref(r), rg, 1, C.byref(err)) == S.TURBO_E_UNSUPPORTED_OPTION
    r.output_dim = 2
    assert s.t.embed_write(s.h, C.byref(r), C.byref(err)) == S.TURBO_E_INVALID_ARGUMENT   # no ranges
    s.close()
    model.close()
    # A headed write to a model loaded without a head.
    plain = context.load(oracle.fixture("tiny_bert")[0])
    s = plain.session(1, 24, S.TURBO_PRECISION_EXACT, max_ranges=1)
    assert s.t.embed_write_ranges(s.h, C.byref(r), rg, 1, C.byref(err)) == S.TURBO_E_INVALID_ARGUMENT
    with pytest.raises(T.TurboError):
        s.span_logits(windows[:1])
    s.close()
    plain.close()


# ---- Layer reads (taps): ranges from each of the last layers ------------------------------
#
# turbo_embed_write_layer_ranges (include/turbo/turbo.h:712-738): every block
# against the oracle at the tier's bound, and bit for bit the invariants the
# reference's tests hold (core/tests/ranges/layers.rs:18-49, alone.rs:25-84):
# the last block is the plain range write, one layer alone is block 0, and
# block k is the model cut after its layer.

def _cut(desc, layers):
    per = {S.TURBO_FAMILY_BERT: (S.BERT_EMBEDDING_TENSORS, S.BERT_LAYER_TENSORS),
           S.TURBO_FAMILY_MODERNBERT: (S.MODERNBERT_EMBEDDING_TENSORS, S.MODERNBERT_LAYER_TENSORS),
           S.TURBO_FAMILY_NOMIC_BERT: (S.NOMIC_EMBEDDING_TENSORS, S.NOMIC_LAYER_TENSORS)}[desc.family]
    n = per[0] + layers * per[1]
    from turboembed_amd.model import ModelDesc
    return ModelDesc(desc.family, layers, desc.hidden, desc.heads, desc.intermediate, desc.vocab_size,
                     desc.max_positions, desc.token_types, desc.layer_norm_eps, desc.tensors[:n], desc.position_offset,
                     desc.rope, desc.attention_window, desc.global_every, desc.mlp, desc.activation, desc.norm,
                     desc.names[:n], desc.compute_dtype)


@pytest.mark.parametrize("family", ["bert", "modernbert", "nomic"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_layer_reads_meet_the_oracle(context, family, precision):
    desc = MODELS[family](seed=13, layers=3)
    ids, mask, types = small.ragged_rows(31, 4, 48, desc.vocab_size, types=max(1, desc.token_types))
    live = [np.flatnonzero(m) for m in mask]
    ranges = [(r, int(live[r][0]), int(live[r][-1]) + 1) for r in range(4)]
    ranges += [(r, int(live[r][0]), int(live[r][0]) + 1) for r in range(4)] + [(0, 5, 17)]
    n = len(ranges)
    L = desc.layers
    model = context.load(desc)
    s = model.session(4, 48, precision, max_ranges=L * n)
    s.write_ranges(ids, mask, ranges, types)
    s.run()
    plain = s.read()
    for T in range(1, L + 1):
        s.write_layer_ranges(ids, mask, ranges, T, types)
        s.run()
        got = s.read()
        assert got.shape == (T * n, desc.hidden)
        want = oracle.encode(desc, ids, mask, types, ranges=ranges, taps=T)
        assert_close(got, want, s.compute_dtype)
        assert np.array_equal(got[(T - 1) * n:], plain), f"last block of {T}"
        if T > 1:
            s.write_layer_ranges(ids, mask, ranges, T, types, layer_alone=True)
            s.run()
            assert np.array_equal(s.read(), got[:n]), f"{T} alone"
            # A replay of the same shape gives the same bits.
            s.write_layer_ranges(ids, mask, ranges, T, types)
            s.run()
            assert np.array_equal(s.read(), got)
    # Block 0 of L against the model cut after layer 1, loaded on its own.
    cut = context.load(_cut(desc, 1))
    c = cut.session(4, 48, precision, max_ranges=n)
    c.write_ranges(ids, mask, ranges, types)
    c.run()
    assert np.array_equal(c.read(), got[:n])
    c.close()
    cut.close()
    s.close()
    model.close()


def test_layer_reads_refuse_what_the_core_refuses(context):
    desc = MODELS["bert"](seed=13, layers=3)
    ids, mask, types = small.ragged_rows(31, 2, 16, desc.vocab_size)
    model = context.load(desc)
    s = model.session(2, 16, S.TURBO_PRECISION_EXACT, max_ranges=4)
    rg = [(0, 0, 2), (1, 0, 1)]
    for layers, code, field in ((0, S.TURBO_E_INVALID_ARGUMENT, 9), (4, S.TURBO_E_INVALID_ARGUMENT, 9),
                                (3, S.TURBO_E_CAPACITY, 0)):
        with pytest.raises(T.TurboError) as e:
            s.write_layer_ranges(ids, mask, rg, layers, types)
        assert (e.value.code, e.value.field) == (code, field)
    s.write_layer_ranges(ids, mask, rg, 3, types, layer_alone=True)     # one block: within max_ranges
    s.run()
    assert s.read().shape == (2, desc.hidden)
    # Through the seam: the backend holds the same rules.
    r = S.turbo_backend_embed_rows()
    r.struct_size = C.sizeof(r)
    r.batch, r.seq, r.row_stride = 2, 16, 16
    r.ids, r.mask = ids.ctypes.data_as(C.POINTER(C.c_int32)), mask.ctypes.data_as(C.POINTER(C.c_int32))
    r.pooling, r.normalize, r.output_dim, r.taps = S.TURBO_POOLING_MEAN, S.TURBO_NORMALIZE_L2, desc.hidden, 2
    arr = (S.turbo_token_range * 3)()
    for i, (a, b_, c_) in enumerate([(0, 0, 2), (1, 0, 1), (0, 1, 2)]):
        arr[i].row, arr[i].start, arr[i].end = a, b_, c_
    err = S.new_error()
    assert s.t.embed_write(s.h, C.byref(r), C.byref(err)) == S.TURBO_E_INVALID_ARGUMENT       # no ranges
    assert err.field == 9
    assert s.t.embed_write_ranges(s.h, C.byref(r), arr, 3, C.byref(err)) == S.TURBO_E_CAPACITY  # 6 over 4
    r.taps = 4
    assert s.t.embed_write_ranges(s.h, C.byref(r), arr, 2, C.byref(err)) == S.TURBO_E_INVALID_ARGUMENT
    r.taps, r.tap_alone = 2, 2
    assert s.t.embed_write_ranges(s.h, C.byref(r), arr, 2, C.byref(err)) == S.TURBO_E_INVALID_ARGUMENT
    assert err.field == 10
    s.close()
    model.close()
    # The span head reads the final layer alone.
    qd, windows, _, _ = oracle.qa_fixture()
    qm = context.load(qd)
    q = qm.session(2, 24, S.TURBO_PRECISION_EXACT, task=S.TURBO_TASK_EXTRACTIVE_QA)
    w = np.zeros((1, 24), np.int32)
    m1 = np.zeros((1, 24), np.int32)
    w[0, :6], m1[0, :6] = windows[0][0][:6], 1
    with pytest.raises(T.TurboError) as e:
        q.write_layer_ranges(w, m1, [(0, 0, 1)], 2, normalize=S.TURBO_NORMALIZE_NONE)
    assert (e.value.code, e.value.field) == (S.TURBO_E_UNSUPPORTED_OPTION, 9)
    q.close()
    qm.close()


def test_int8_cross_encoder_meets_the_oracle(context):
    # The int8 rerank workload at full width on 2 of its 12 layers and 12 of
    # its 256 pairs: scores within I8's bound of the F32 oracle's, and the
    # CLS states the head reads within I8's cosine floor.
    from turboembed_amd.rerank import RerankHead, pair_windows
    sh = W.SHAPES["rerank"]
    desc = W.model(sh, layers=2)
    pairs = W.rerank_pairs(sh, n=12)
    head = W.rerank_head(sh)
    qt = sh.extra["query_tokens"]
    model = context.load(desc)
    s = model.session(16, sh.seq, sh.precision, task=S.TURBO_TASK_RERANK)
    assert s.compute_dtype == S.TURBO_DTYPE_I8
    got = s.rerank(pairs, RerankHead(**head), sh.cls_id, sh.sep_id, query_tokens=qt, max_tokens=sh.seq)
    want = oracle.rerank(desc, pairs, head, sh.cls_id, sh.sep_id, query_tokens=qt, max_tokens=sh.seq)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= SCORE_BOUND[S.TURBO_DTYPE_I8] * scale, (got, want)
    wins = [pair_windows(q, p, sh.cls_id, sh.sep_id, query_tokens=qt, max_tokens=sh.seq) for q, p in pairs]
    ids = np.concatenate([w[0] for w in wins])
    types = np.concatenate([w[1] for w in wins])
    lengths = np.concatenate([w[2] for w in wins])
    mask = (np.arange(sh.seq)[None, :] < lengths[:, None]).astype(np.int32)
    kw = dict(pooling=S.TURBO_POOLING_CLS, normalize=S.TURBO_NORMALIZE_NONE)
    cos = small.cosine_rows(s.embed(ids, mask, types, **kw), oracle.encode(desc, ids, mask, types, **kw))
    assert cos.min() >= I8_FLOOR, cos.min()
    print(f"int8 cross-encoder: min CLS cosine {cos.min():.5f}, "
          f"largest score difference {np.abs(got - want).max() / scale:.4f} of the scale")
    s.close()
    model.close()


# ---- Kernel choices and the autotune cache ------------------------------------------------
#
# The seam's tuning protocol (reference include/turbo/turbo_backend.h:231-257,
# 561-586): ON measures when nothing is cached and reuses a cached choice
# unmeasured, RETUNE measures against it, the environment forces choices in
# every mode; the tuned session's vectors meet the oracle as the default's do.

def test_autotune_measures_caches_and_reuses(context, tmp_path):
    from turboembed_amd import tuning as TU
    desc = small.bert(seed=31, hidden=128, heads=2, inter=256, positions=320, std=0.1)
    ids, mask, types = small.ragged_rows(31, 5, 300, desc.vocab_size)
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    cache = TU.TuneCache(str(tmp_path))
    s = model.session(8, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, cache=cache, budget_ms=2000)
    assert s.tuned == S.TURBO_TUNED_MEASURED, s.tuned
    ch = s.choices()
    # Every bin the session reaches (8 x 320 tokens: up to le4k), the four
    # products and attention.
    for b in ("le256", "le1k", "le4k"):
        assert b + ":qkv=" in ch, ch
    assert "le16k" not in ch and "gt16k" not in ch, ch
    assert ch.endswith("forced=none"), ch
    assert any(k.startswith("le1k/ffn1/") for k in s.timings), s.timings
    assert all(v >= 0 for v in s.timings.values())
    assert_close(s.embed(ids, mask, types), want, s.compute_dtype)
    s.close()
    # The same key again: the cached choice, unmeasured; then from disk alone.
    s2 = model.session(8, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, cache=cache)
    assert s2.tuned == S.TURBO_TUNED_CACHE and s2.choices() == ch and not s2.timings
    s2.close()
    s3 = model.session(8, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON,
                       cache=TU.TuneCache(str(tmp_path)))
    assert s3.tuned == S.TURBO_TUNED_CACHE and s3.choices() == ch
    s3.close()
    # RETUNE measures again, with the cached choice as the incumbent.
    s4 = model.session(8, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_RETUNE, cache=cache,
                       budget_ms=2000)
    assert s4.tuned == S.TURBO_TUNED_MEASURED
    s4.close()
    # OFF: the backend's rule, nothing timed.
    s5 = model.session(8, 320, S.TURBO_PRECISION_FASTEST)
    assert s5.tuned == S.TURBO_TUNED_DEFAULT and "qkv=auto" in s5.choices() and not s5.timings
    s5.close()
    model.close()


def test_a_block_shape_that_cannot_launch_is_skipped_and_refused(context, tmp_path, monkeypatch):
    # The fail-variant hook stands in for a device that cannot take a block
    # shape (reference core/src/cuda.rs:461-469, core/cuda/backend.cpp:
    # 2430-2440, 3006-3010): a session forcing it is refused, the tuner
    # never times it, a cached choice naming it is not taken, and the rule
    # runs another shape whose vectors meet the oracle.
    from turboembed_amd import tuning as TU
    desc = small.bert(seed=33, hidden=128, heads=2, inter=256, positions=320, std=0.1)
    ids, mask, types = small.ragged_rows(33, 16, 300, desc.vocab_size)
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    cache = TU.TuneCache(str(tmp_path))
    with pytest.raises(T.TurboError):
        T.fail_variant("no-such-shape")
    T.fail_variant("256x256")
    try:
        monkeypatch.setenv("TURBO_ROCM_CHOICES", "le16k:qkv=256x256")
        with pytest.raises(T.TurboError) as e:
            model.session(16, 320, S.TURBO_PRECISION_FASTEST)
        assert e.value.code == S.TURBO_E_UNSUPPORTED and "le16k:qkv=256x256" in e.value.message, e.value
        monkeypatch.delenv("TURBO_ROCM_CHOICES")
        s = model.session(16, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, cache=cache,
                          budget_ms=3000)
        assert s.tuned == S.TURBO_TUNED_MEASURED
        assert s.timings and not any(k.endswith("/256x256") for k in s.timings), s.timings
        assert "=256x256" not in s.choices()
        assert_close(s.embed(ids, mask, types), want, s.compute_dtype)
        s.close()
        # The rule's own shape for these products is 256x256; it runs another.
        s = model.session(16, 320, S.TURBO_PRECISION_FASTEST)
        assert_close(s.embed(ids, mask, types), want, s.compute_dtype)
        s.close()
        # A cached choice that names it is measured again, not taken.
        key_cache = TU.TuneCache(str(tmp_path / "named"))
        s = model.session(16, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, cache=key_cache,
                          budget_ms=100)
        key = s.key
        s.close()
        key_cache.put(key, "all:qkv=256x256,out=auto,ffn1=auto,ffn2=auto,attn=mfma;forced=none", {"x": 1.0})
        s = model.session(16, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, cache=key_cache,
                          budget_ms=100)
        assert s.tuned != S.TURBO_TUNED_CACHE and "=256x256" not in s.choices()
        s.close()
    finally:
        T.fail_variant(None)
    # Launchable again once the hook is cleared.
    monkeypatch.setenv("TURBO_ROCM_CHOICES", "le16k:qkv=256x256")
    s = model.session(16, 320, S.TURBO_PRECISION_FASTEST)
    assert_close(s.embed(ids, mask, types), want, s.compute_dtype)
    s.close()
    model.close()


# hidden 192: Q, K and V start inside the 128-column waves of 128x256 and
# 128x256k32, which must then run 64-column waves for the QKV product.
@pytest.mark.parametrize("tile", ["256x256", "256x192", "256x384", "128x128", "256x128k32", "r128x128", "r64x64",
                                  "128x256", "128x256k32", "256x384k32s4"])
def test_forced_tiles_meet_the_oracle(context, tile, monkeypatch):
    desc = small.bert(seed=32, hidden=192, heads=3, inter=384, positions=320, std=0.1)
    ids, mask, types = small.ragged_rows(32, 6, 300, desc.vocab_size)
    want = oracle.encode(desc, ids, mask, types)
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_CHOICES", f"all:qkv={tile},out={tile},ffn1={tile},ffn2={tile},attn=mfma")
    s = model.session(8, 320, S.TURBO_PRECISION_FASTEST, autotune=S.TURBO_AUTOTUNE_ON, budget_ms=2000)
    assert s.tuned == S.TURBO_TUNED_FORCED and f"ffn2={tile}" in s.choices() and not s.timings
    assert_close(s.embed(ids, mask, types), want, s.compute_dtype)
    s.close()
    model.close()


def test_a_bad_choices_string_is_refused(context, monkeypatch):
    desc = small.bert(seed=33)
    model = context.load(desc)
    for bad in ("qkv=999", "le9k:qkv=auto", "attn=fast", "tile=7"):
        monkeypatch.setenv("TURBO_ROCM_CHOICES", bad)
        with pytest.raises(T.TurboError) as e:
            model.session(4, 64, S.TURBO_PRECISION_FASTEST)
        assert e.value.code == S.TURBO_E_INVALID_ARGUMENT and "TURBO_ROCM_CHOICES" in e.value.message
    model.close()


# ---- Allocations ----------------------------------------------------------------------------
#
# The backend's heap allocations are counted as they happen (the library is
# linked with malloc and operator new wrapped, so every such call its code
# makes is seen): opening a session moves the count; writing rows, running
# and reading allocate nothing, on this thread or any other, and each run
# reports it (turbo_backend.h:519-530; the reference's counting allocator,
# core/tests/allocations.rs).
def test_an_open_allocates_and_writes_runs_and_reads_do_not(context):
    desc = small.bert(seed=51)
    a = small.ragged_rows(51, 5, 48, desc.vocab_size)
    b = small.ragged_rows(52, 7, 30, desc.vocab_size)
    model = context.load(desc)
    p0, t0 = T.host_allocs()
    s = model.session(8, 64, S.TURBO_PRECISION_FASTEST)
    p1, t1 = T.host_allocs()
    assert t1 > t0 and p1 - p0 >= t1 - t0, (p0, t0, p1, t1)
    s.embed(*a)
    p2, t2 = T.host_allocs()
    for rows in (a, b, a):
        s.write_tokens(*rows)
        s.run()
        assert s.run_info.host_allocs == 0 and s.run_info.device_allocs == 0
        s.read()
    assert T.host_allocs() == (p2, t2)
    s.close()
    model.close()


# ---- Runs replayed from HIP graphs --------------------------------------------------------
#
# Each token bin's launches are captured once, at session_open, and
# replayed for every run of the bin: every replay, with the host's own work
# (the rows' writes and the reads' syncs) between them, gives the eager
# launches' vectors bit for bit, for two shapes alternating in one session.

@pytest.mark.parametrize("family", ["bert", "modernbert"])
@pytest.mark.parametrize("precision", [S.TURBO_PRECISION_EXACT, S.TURBO_PRECISION_FASTEST])
def test_graph_replays_are_the_eager_runs(context, family, precision, monkeypatch):
    desc = MODELS[family](seed=41)
    a = small.ragged_rows(41, 5, 48, desc.vocab_size)
    b = small.ragged_rows(42, 7, 30, desc.vocab_size)
    if family == "modernbert":
        a, b = (a[0], a[1], None), (b[0], b[1], None)
    model = context.load(desc)
    monkeypatch.setenv("TURBO_ROCM_GRAPHS", "0")
    eager = model.session(8, 64, precision)
    want_a, want_b = eager.embed(*a), eager.embed(*b)
    eager.close()
    monkeypatch.delenv("TURBO_ROCM_GRAPHS")
    s = model.session(8, 64, precision)
    for _ in range(3):
        assert np.array_equal(s.embed(*a), want_a)
        assert np.array_equal(s.embed(*b), want_b)
    # A replay of resident rows, then a read: the same vectors again.
    s.replay(2)
    assert np.array_equal(s.read(), want_b)
    s.close()
    model.close()


@pytest.mark.parametrize("family", ["bert", "modernbert"])
def test_fresh_ragged_batches_replay_their_bin_s_graph(context, family, monkeypatch):
    # Every bin's graph is captured at session_open (reference
    # core/cuda/backend.cpp:2366-2417); a run of new rows of any shape in a
    # bin replays that bin's graph with no capture, its kernels reading the
    # run's extent from the device, bit for bit the directly launched
    # kernels, with no host or device allocation. 16 rows of up to 320
    # tokens reach four bins, the largest split into two parts.
    desc = small.bert(seed=43, hidden=128, heads=2, inter=256, positions=320, std=0.1) if family == "bert" else \
        small.modernbert(seed=43, hidden=128, heads=2, inter=192, positions=320, window=32, std=0.1)
    model = context.load(desc)
    batches = []
    g = np.random.Generator(np.random.PCG64(43))
    # (rows, columns, every column live): 5120, 4800 and 4100 live tokens
    # take the split bin (two parts).
    shapes = [(16, 320, True), (3, 40, False), (9, 300, False), (16, 300, True), (2, 256, False), (12, 320, False),
              (1, 5, False), (13, 316, True), (4, 320, True)]
    for k, (rows, seq, full) in enumerate(shapes):
        ids, mask, types = small.ragged_rows(100 + k, rows, seq, desc.vocab_size)
        if full:
            mask[:] = 1
        batches.append((ids, mask, None if family == "modernbert" else types))
    monkeypatch.setenv("TURBO_ROCM_GRAPHS", "0")
    eager = model.session(16, 320, S.TURBO_PRECISION_FASTEST)
    want = [eager.embed(*b) for b in batches]
    assert eager.graphs() == (0, 0)
    eager.close()
    monkeypatch.delenv("TURBO_ROCM_GRAPHS")
    s = model.session(16, 320, S.TURBO_PRECISION_FASTEST)
    captured, launched = s.graphs()
    assert captured == 4 and launched == 0, (captured, launched)
    for i, b in enumerate(batches):
        got = s.embed(*b)
        assert np.array_equal(got, want[i]), i
        assert s.run_info.host_allocs == 0 and s.run_info.device_allocs == 0
        assert_close(got, oracle.encode(desc, *b), s.compute_dtype)
    assert s.graphs() == (4, len(batches))
    # Range writes, and a span-free MEAN/CLS switch, take the same graphs.
    ids, mask, types = batches[3]
    rr = [(r, 0, int(mask[r].nonzero()[0].max()) + 1) for r in range(ids.shape[0])]
    s.write_ranges(ids, mask, rr, types)
    s.run()
    assert np.array_equal(s.read(), want[3])
    cls = s.embed(ids, mask, types, pooling=S.TURBO_POOLING_CLS, output_dim=100)
    assert_close(cls, oracle.encode(desc, ids, mask, types, pooling=S.TURBO_POOLING_CLS, output_dim=100),
                 s.compute_dtype)
    assert s.graphs() == (4, len(batches) + 2)
    s.close()
    model.close()


# ---- Vector codes on the device (buffer_quantize) --------------------------------------------
#
# Byte-exact against the reference's golden codes (testdata/quantize, copied
# as data) and against the oracle's codes of the session's own vectors.

def test_buffer_quantize_makes_the_golden_codes(context):
    import test_quantize as TQ
    for x, r, i8, ub in TQ.golden_rows():
        dim = x.shape[1]
        for mode, want in ((S.TURBO_QUANTIZE_INT8, i8), (S.TURBO_QUANTIZE_UBINARY, ub)):
            buf = context.buffer(4 * dim, S.TURBO_PLACE_SHARED)
            buf.view(np.float32)[:] = x[0]
            buf.quantize(mode, 1, dim, r.reshape(2, dim) if mode == S.TURBO_QUANTIZE_INT8 else None)
            assert buf.read(len(want)).tobytes() == want
            buf.close()


@pytest.mark.parametrize("mode", [S.TURBO_QUANTIZE_INT8, S.TURBO_QUANTIZE_UBINARY])
def test_a_session_s_codes_are_the_oracle_s(context, mode):
    desc = small.bert(seed=51, hidden=96, heads=3, inter=192)
    ids, mask, types = small.ragged_rows(51, 6, 40, desc.vocab_size)
    model = context.load(desc)
    s = model.session(8, 64, S.TURBO_PRECISION_FASTEST)
    vecs = s.embed(ids, mask, types, output_dim=77)
    g = np.random.Generator(np.random.PCG64(51))
    lo = (g.standard_normal(77) * 0.05 - 0.1).astype(np.float32)
    ranges = np.stack([lo, lo + np.abs(g.standard_normal(77)).astype(np.float32) * 0.2]).astype(np.float32)
    ranges[:, 5] = 0.03   # a dimension whose step is 0
    codes = s.read_quantized(mode, ranges)
    want = oracle.quantize(vecs, mode, ranges)
    assert np.array_equal(codes.view(np.uint8), want)
    if mode == S.TURBO_QUANTIZE_INT8:
        assert s.run_info.device_allocs == 2 and s.run_info.h2d_bytes >= 2 * 77 * 4
    s.close()
    model.close()


def test_buffer_quantize_refuses_what_it_cannot_do(context):
    buf = context.buffer(64, S.TURBO_PLACE_SHARED)
    for mode, rows, dim, ranges in ((S.TURBO_QUANTIZE_NONE, 1, 4, None), (S.TURBO_QUANTIZE_INT8, 1, 4, None),
                                    (S.TURBO_QUANTIZE_UBINARY, 5, 4, None),
                                    (S.TURBO_QUANTIZE_INT8, 1, 2, np.array([[1.0, 0.0], [0.0, 1.0]], np.float32))):
        with pytest.raises(T.TurboError) as e:
            buf.quantize(mode, rows, dim, ranges)
        assert e.value.code == S.TURBO_E_INVALID_ARGUMENT
    buf.close()


def test_a_timed_run_times_each_launch_by_its_kernels(context):
    # A timed run binds each launch's event pair to its kernels' dispatch
    # packets: the same bits as the untimed run (which replays the bin's
    # graph), one interval a launch, each inside the run and as long as the
    # launch's own time, and no graph replayed for it (bins to le4k, a split
    # run of two parts at the top).
    desc = MODELS["bert"](seed=83, hidden=128, inter=256, positions=320)
    model = context.load(desc)
    s = model.session(16, 320, S.TURBO_PRECISION_FASTEST)
    for seed, (batch, seq) in enumerate([(3, 60), (16, 300)]):
        ids, mask, types = small.ragged_rows(83 + seed, batch, seq, desc.vocab_size)
        want = s.embed(ids, mask, types)
        s.set_timing(True)
        _, launched = s.graphs()
        got = s.embed(ids, mask, types)
        iv, times = s.intervals(), s.times()
        assert s.graphs()[1] == launched
        s.set_timing(False)
        np.testing.assert_array_equal(got, want)
        assert iv and all(0 <= a <= b for _, a, b in iv), iv[:4]
        assert any(n.startswith("gemm") for n, _, _ in iv)
        for name, ms in times.items():
            spans = sum(b - a for n, a, b in iv if n == name)
            assert abs(spans - ms) <= 1e-3 + 1e-2 * ms, (name, spans, ms)
    s.close()
    model.close()
