"""Vector codes (int8 and ubinary) as the reference core makes them
(core/src/quantize.rs:48-80): the oracle against the byte goldens the
reference's own tests hold (testdata/quantize/sentence-transformers-145ef47d.txt,
copied as data), and the golden rows pin what a plausible mistake would
change: floor against round, the top bit first, the step's zero case."""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize-sentence-transformers-145ef47d.txt")


def golden_rows():
    out = []
    for line in open(GOLDEN):
        if line.startswith("#"):
            continue
        dim, xh, rh, ih, uh = line.split()
        dim = int(dim)
        out.append((np.frombuffer(bytes.fromhex(xh), "<f4").reshape(1, dim), np.frombuffer(bytes.fromhex(rh), "<f4"),
                    bytes.fromhex(ih), bytes.fromhex(uh)))
    return out


def test_the_oracle_s_codes_are_the_golden_bytes():
    rows = golden_rows()
    assert len(rows) == 30
    for x, r, i8, ub in rows:
        assert oracle.quantize(x, 2, r).tobytes() == i8
        assert oracle.quantize(x, 3).tobytes() == ub


def mistaken_int8(x, r, rounding):
    dim = x.shape[1]
    lo, hi = r[:dim], r[dim:]
    step = (hi - lo) / np.float32(255)
    step = np.where(step == 0, np.float32(1), step).astype(np.float32)
    q = rounding(((x[0] - lo) / step).astype(np.float32))
    return (np.clip(q, 0, 255).astype(np.int32) - 128).astype(np.int8).tobytes()


def test_the_goldens_tell_floor_from_round_and_the_bit_order():
    rows = golden_rows()
    # floor is what the oracle does (it passes above); rounding to nearest
    # misses at least one golden row.
    assert any(mistaken_int8(x, r, np.rint) != i8 for x, r, i8, _ in rows)
    assert all(mistaken_int8(x, r, np.floor) == i8 for x, r, i8, _ in rows)
    # The first value in the least significant bit misses too.
    lsb = [np.packbits(x[0] > 0, bitorder="little").tobytes() for x, _, _, _ in rows]
    assert any(b != ub for b, (_, _, _, ub) in zip(lsb, rows))
    # A constant dimension (max == min) takes step 1: code -128 + floor(x - min).
    x = np.array([[0.0, 2.5, -1.0]], np.float32)
    r = np.array([0.0, 0.0, -1.0, 0.0, 5.0, -1.0], np.float32)
    assert oracle.quantize(x, 2, r).view(np.int8).tolist() == [[-128, -128 + 127, -128]]


@pytest.mark.parametrize("dim", [1, 7, 8, 9, 384])
def test_ubinary_pads_the_last_byte_with_zeros(dim):
    x = np.ones((2, dim), np.float32)
    codes = oracle.quantize(x, 3)
    assert codes.shape == (2, (dim + 7) // 8)
    bits = np.unpackbits(codes, axis=1)[:, : (dim + 7) // 8 * 8]
    assert bits[:, :dim].all() and not bits[:, dim:].any()
