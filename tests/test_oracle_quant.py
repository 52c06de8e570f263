"""Pins the oracle's codec (quant.rs) against the reference's own layout
fixture (tests/core.rs:50-151), its shape-rejection test (core.rs:43-48), an
exhaustive f16 check and independent array equations per format."""
import math

import numpy as np
import pytest

import oracle
from helpers import KINDS, LAYOUT, layout_fixture, np_dequant, random_blocks


def test_reject_bad_quant_shapes():  # tests/core.rs:43-48
    with pytest.raises(oracle.OracleError):
        oracle.row_bytes(12, 255)
    with pytest.raises(oracle.OracleError):
        oracle.row_bytes(99, 256)
    with pytest.raises(oracle.OracleError):
        oracle.decode(b"", 14, 256)


@pytest.mark.parametrize("kind", KINDS)
def test_layout_table(kind):  # quant.rs:5-21
    assert oracle.layout(kind) == LAYOUT[kind]
    blk, size = LAYOUT[kind]
    assert oracle.row_bytes(kind, blk * 3) == 3 * size
    if blk > 1:
        with pytest.raises(oracle.OracleError):
            oracle.row_bytes(kind, blk + 1)
    with pytest.raises(oracle.OracleError):
        oracle.row_bytes(kind, 0)


@pytest.mark.parametrize("kind", KINDS)
def test_quantized_blocks_match_known_layouts(kind):  # tests/core.rs:144-151
    b, expected = layout_fixture(kind)
    got = oracle.decode(b.tobytes(), kind, expected.size)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), kind


def test_f16_exhaustive():
    """All 65,536 half patterns: against numpy's IEEE widening and a closed
    form (ldexp) for every finite value; NaNs stay NaN with their sign."""
    got = oracle.f16_all()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    nan = np.isnan(ref)
    assert np.isnan(got[nan]).all()
    assert np.array_equal(np.signbit(got[nan]), np.signbit(ref[nan]))
    for h in range(0, 65536, 7):
        s, e, m = h >> 15, (h >> 10) & 31, h & 1023
        if e == 31:
            continue
        v = math.ldexp(m, -24) if e == 0 else math.ldexp(1024 + m, e - 25)
        v = -v if s else v
        assert np.float32(v).view(np.uint32) == got[h].view(np.uint32) or (v == 0 and got[h] == 0), h


@pytest.mark.parametrize("kind", KINDS)
def test_decode_matches_array_equations(kind):
    rng = np.random.default_rng(1234 + kind)
    blk, size = LAYOUT[kind]
    cols = max(blk, 1) * 4
    rows = 6
    data = random_blocks(kind, rows, cols, rng)
    ref = np_dequant(data, kind, cols)
    rb = oracle.row_bytes(kind, cols)
    for r in range(rows):
        got = oracle.decode(data[r * rb:(r + 1) * rb].tobytes(), kind, cols)
        assert np.array_equal(got.view(np.uint32), ref[r].view(np.uint32)), (kind, r)


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_fold_and_threads(kind):
    """Cpu::matvec (backend.rs:41-48): sequential f32 fold of x[i]*w[i]; the
    threaded block-decode path is bit-identical to the faithful one, and both
    equal a numpy sequential fold (cumsum) and sit near an f64 dot."""
    rng = np.random.default_rng(99 + kind)
    blk, size = LAYOUT[kind]
    cols = 512 if blk > 1 else 96
    rows = 37
    data = random_blocks(kind, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    y0 = oracle.packed_matvec(data, kind, rows, cols, x, threads=0)
    y8 = oracle.packed_matvec(data, kind, rows, cols, x, threads=8)
    assert np.array_equal(y0.view(np.uint32), y8.view(np.uint32))
    w = np_dequant(data, kind, cols)
    seq = np.cumsum(x[None, :] * w, axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(y0, seq)
    f64 = w.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(y0 - f64)) <= 1e-5 * np.max(np.abs(f64)) + 1e-6
