"""GPU parity of the engine's kernel-level surfaces against the oracle, through
the C ABI.  Bars: dequant, top-k ids and argmax bit-exact; matvec and
attention within max|gpu-cpu| / max|cpu| <= 1e-4 (FP32 accumulation)."""
import importlib

import numpy as np
import pytest

import oracle
from helpers import KINDS, LAYOUT, layout_fixture, np_dequant, random_blocks

engine = importlib.import_module("qwen-30brust_amd")
synth = importlib.import_module("qwen-30brust_amd.synth")

pytestmark = pytest.mark.gpu
REL = 1e-4  # matvec / logits tolerance (relative to the largest |value|)


@pytest.fixture(scope="module")
def dev():
    return engine.Device(0)


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


# ------------------------------------------------------------------ dequant --
@pytest.mark.parametrize("kind", KINDS)
def test_dequant_fixture_bit_exact(dev, kind):  # tests/core.rs:144-151 on the device
    b, expected = layout_fixture(kind)
    got = dev.dequant(b, kind, 1, expected.size)[0]
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_random_rows_bit_exact(dev, kind):
    rng = np.random.default_rng(100 + kind)
    blk, _ = LAYOUT[kind]
    cols = 768 if blk > 1 else 100
    rows = 9
    data = random_blocks(kind, rows, cols, rng)
    got = dev.dequant(data, kind, rows, cols)
    rb = oracle.row_bytes(kind, cols)
    for r in range(rows):
        ref = oracle.decode(data[r * rb:(r + 1) * rb].tobytes(), kind, cols)
        assert np.array_equal(got[r].view(np.uint32), ref.view(np.uint32)), (kind, r)


def test_dequant_f16_exhaustive(dev):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = dev.dequant(bits.view(np.uint8), 1, 1, 65536)[0]
    ref = oracle.f16_all()
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_dequant_rejects_bad_shapes(dev):
    with pytest.raises(engine.EngineError):
        dev.dequant(np.zeros(10, np.uint8), 12, 1, 255)
    with pytest.raises(engine.EngineError):
        dev.dequant(np.zeros(10, np.uint8), 99, 1, 256)
    with pytest.raises(engine.EngineError):
        dev.dequant(np.zeros(10, np.uint8), 14, 1, 256)  # truncated row


# ------------------------------------------------------------------- matvec --
@pytest.mark.parametrize("kind", KINDS)
def test_packed_matvec_fixture_three_rows(dev, kind):
    """tests/core.rs:152-185: 3 copies of the fixture blocks, x_i = ((i%13)-6)/7,
    |y - e| < 0.002 + 5e-5|e|, run twice."""
    b, decoded = layout_fixture(kind)
    cols = decoded.size
    x = ((np.arange(cols) % 13) - 6).astype(np.float32) / np.float32(7)
    expected = float(np.sum(x.astype(np.float64) * decoded))
    data = np.tile(b, 3)
    for _ in range(2):
        y = dev.packed_matvec(data, kind, 3, cols, x)
        assert np.all(np.abs(y - expected) < 0.002 + abs(expected) * 5e-5)
    ref = oracle.packed_matvec(data, kind, 3, cols, x, threads=0)
    assert rel_err(y, ref) <= REL


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows,cols", [(37, 512), (5, 256), (130, 2048), (64, 768)])
def test_packed_matvec_vs_oracle(dev, kind, rows, cols):
    blk, _ = LAYOUT[kind]
    if cols % blk:
        pytest.skip("shape not representable in this format")
    rng = np.random.default_rng(rows * 7 + cols + kind)
    data = random_blocks(kind, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    y = dev.packed_matvec(data, kind, rows, cols, x)
    ref = oracle.packed_matvec(data, kind, rows, cols, x, threads=8)
    assert rel_err(y, ref) <= REL


@pytest.mark.parametrize("cols", [1, 3, 33, 100, 1000])
@pytest.mark.parametrize("kind", [0, 1])
def test_packed_matvec_ragged_float_rows(dev, kind, cols):
    rng = np.random.default_rng(cols)
    data = random_blocks(kind, 11, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    y = dev.packed_matvec(data, kind, 11, cols, x)
    ref = oracle.packed_matvec(data, kind, 11, cols, x, threads=0)
    assert rel_err(y, ref) <= REL


@pytest.mark.parametrize("name,kind,rows,cols", [
    ("q_proj", 12, 4096, 2048), ("o_proj", 12, 2048, 4096),
    ("expert_down", 14, 2048, 768), ("vocab", 14, 151936, 2048)])
def test_matvec_30b_shapes(dev, name, kind, rows, cols):
    """The four matvec microbench cases at 30B-A3B shapes: W ~ N(0, 0.02)
    quantized with the project's quantizer, x ~ N(0, 1)."""
    seed = {"q_proj": 1, "o_proj": 2, "expert_down": 3, "vocab": 4}[name]
    w = synth.normal(seed, rows * cols, 0.0, 0.02).reshape(rows, cols)
    data = synth.quantize(kind, w)
    x = synth.normal(17, cols)
    y = dev.packed_matvec(data, kind, rows, cols, x)
    ref = oracle.packed_matvec(data, kind, rows, cols, x, threads=8)
    assert rel_err(y, ref) <= REL


QUANT_KINDS = [2, 8, 12, 13, 14]


@pytest.mark.parametrize("kind", QUANT_KINDS)
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 3072), (40, 4096), (9, 8192), (17, 160), (33, 8448)])
def test_packed_matvec_lane_layouts(dev, kind, rows, cols):
    """Row lengths that select every (chunks per lane, lanes per row) layout
    of the streaming kernel (3,072 columns: 3 chunks on 32 lanes; 8,192: 4 on
    64; 160: 3 on 2) and, past 8,192 columns, the general kernel."""
    blk, _ = LAYOUT[kind]
    if cols % blk:
        pytest.skip("shape not representable in this format")
    rng = np.random.default_rng(rows * 13 + cols + kind)
    data = random_blocks(kind, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    y = dev.packed_matvec(data, kind, rows, cols, x)
    ref = oracle.packed_matvec(data, kind, rows, cols, x, threads=8)
    assert rel_err(y, ref) <= REL


@pytest.mark.parametrize("kind", QUANT_KINDS)
@pytest.mark.parametrize("nvec,rows,cols", [(1, 37, 512), (3, 130, 2048), (8, 64, 768), (2, 7, 4096)])
def test_packed_matvec_batch_vs_oracle(dev, kind, nvec, rows, cols):
    """The batched launch (one matrix and one x per vector) against the
    oracle's matvec of each matrix."""
    blk, _ = LAYOUT[kind]
    if cols % blk:
        pytest.skip("shape not representable in this format")
    rng = np.random.default_rng(nvec * 101 + rows + cols + kind)
    data = random_blocks(kind, nvec * rows, cols, rng)
    x = rng.standard_normal(nvec * cols).astype(np.float32)
    y = dev.packed_matvec_batch(data, kind, rows, cols, x, nvec)
    per = data.size // nvec
    for b in range(nvec):
        ref = oracle.packed_matvec(data[b * per:(b + 1) * per], kind, rows, cols, x[b * cols:(b + 1) * cols],
                                   threads=8)
        assert rel_err(y[b], ref) <= REL, b


def test_packed_matvec_batch_30b_down(dev):
    """The 8 routed experts' down projections of a 30B-A3B layer (768 -> 2048
    Q6_K each) in one launch, against the oracle per expert."""
    rows, cols, nvec = 2048, 768, 8
    w = synth.normal(5, nvec * rows * cols, 0.0, 0.02).reshape(nvec * rows, cols)
    data = synth.quantize(14, w)
    x = synth.normal(18, nvec * cols)
    y = dev.packed_matvec_batch(data, 14, rows, cols, x, nvec)
    per = data.size // nvec
    for b in range(nvec):
        ref = oracle.packed_matvec(data[b * per:(b + 1) * per], 14, rows, cols, x[b * cols:(b + 1) * cols],
                                   threads=8)
        assert rel_err(y[b], ref) <= REL, b


def test_packed_matvec_batch_refusals(dev):
    x = np.zeros(2 * 256, np.float32)
    with pytest.raises(engine.EngineError, match="not covered"):
        dev.packed_matvec_batch(np.zeros(2 * 256 * 4, np.uint8), 0, 1, 256, x, 2)  # F32 rows
    with pytest.raises(engine.EngineError, match="shape mismatch"):
        dev.packed_matvec_batch(np.zeros(9 * 144, np.uint8), 12, 1, 256, np.zeros(9 * 256), 9)
    with pytest.raises(engine.EngineError, match="not covered"):  # 2 x 8,192 x floats
        dev.packed_matvec_batch(np.zeros(2 * 32 * 144, np.uint8), 12, 1, 8192, np.zeros(2 * 8192), 2)


def test_large_grid(dev):  # tests/core.rs:186-209: 70,001 rows x 2 cols F32
    rows = 70001
    x = np.array([1.5, -0.5], np.float32)
    for scale in (1.0, 2.0, 3.0, 1.0):
        data = np.tile(np.array([scale, scale * 2], np.float32), rows).view(np.uint8)
        y = dev.packed_matvec(data, 0, rows, 2, x)
        assert y.size == rows
        assert np.all(np.abs(y - scale * 0.5) < 1e-5)


def test_packed_matvec_shape_errors(dev):
    with pytest.raises(engine.EngineError):
        dev.packed_matvec(np.zeros(144, np.uint8), 12, 2, 256, np.zeros(256))  # len != rows*rb
    with pytest.raises(engine.EngineError):
        dev.packed_matvec(np.zeros(144, np.uint8), 12, 1, 255, np.zeros(255))


# -------------------------------------------------------------------- route --
def test_route_kat(dev):  # tests/core.rs:3-12
    ids, w = dev.route([1.0, 3.0, 2.0, -10.0], 2)
    assert list(ids) == [1, 2]
    assert abs(float(w.sum()) - 1) < 1e-6 and abs(float(w[0]) - 0.7310586) < 1e-6
    with pytest.raises(engine.EngineError):
        dev.route([float("nan")], 1)
    with pytest.raises(engine.EngineError):
        dev.route([1.0], 0)


@pytest.mark.parametrize("n,top", [(128, 8), (8, 2), (1000, 8), (300, 300), (5, 1)])
def test_route_bit_exact_ids(dev, n, top):
    rng = np.random.default_rng(n + top)
    for trial in range(4):
        lg = rng.standard_normal(n).astype(np.float32)
        if trial == 1:
            lg = np.round(lg * 2) / 2  # many exact ties: lower index wins
        if trial == 2:
            lg[: n // 2] = 0.0
            lg[n // 2:] = -0.0  # +0 ranks above -0
        ids, w = dev.route(lg, top)
        rids, rw = oracle.route(lg, top)
        assert np.array_equal(ids, rids)
        assert np.allclose(w, rw, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------- argmax --
def test_argmax_bit_exact(dev):
    rng = np.random.default_rng(4)
    lg = rng.standard_normal(151936).astype(np.float32)
    assert dev.argmax(lg) == oracle.greedy(lg)
    lg2 = lg.copy()
    lg2[[7, 99999, 151935]] = lg.max() + 1  # ties: lowest index
    assert dev.argmax(lg2) == oracle.greedy(lg2) == 7
    assert dev.argmax([-0.0, 0.0, -1.0]) == 1
    assert dev.argmax([0.0, 4.0, 2.0]) == 1  # tests/core.rs:29-30
    with pytest.raises(engine.EngineError):
        dev.argmax([1.0, float("nan")])
    with pytest.raises(engine.EngineError):
        dev.argmax([float("inf")])


# ---------------------------------------------------------------- attention --
def test_gqa_kat(dev):  # tests/core.rs:20-27
    out = dev.attention([0.0] * 8, [0.0] * 8, [2.0, 4.0, 10.0, 20.0, 6.0, 8.0, 30.0, 40.0], 4, 2, 2)
    assert np.allclose(out, [4, 6, 4, 6, 20, 30, 20, 30], rtol=1e-6)


@pytest.mark.parametrize("heads,kvh,d,t", [(4, 2, 4, 1), (8, 2, 16, 7), (32, 4, 128, 1025),
                                           (32, 4, 128, 64), (2, 2, 8, 130), (16, 1, 64, 300),
                                           # several key tiles per chunk (online softmax across tiles)
                                           (32, 4, 128, 2049), (32, 4, 128, 8192), (64, 4, 128, 5000)])
def test_attention_vs_oracle(dev, heads, kvh, d, t):
    rng = np.random.default_rng(heads * t + d)
    q = rng.standard_normal(heads * d).astype(np.float32)
    k = rng.standard_normal(t * kvh * d).astype(np.float32)
    v = rng.standard_normal(t * kvh * d).astype(np.float32)
    got = dev.attention(q, k, v, heads, kvh, d)
    ref = oracle.attention(q, k, v, heads, kvh, d)
    assert rel_err(got, ref) <= REL


def test_attention_errors(dev):
    with pytest.raises(engine.EngineError):
        dev.attention(np.zeros(8), np.zeros(0), np.zeros(0), 4, 2, 2)  # empty KV
    with pytest.raises(engine.EngineError):
        dev.attention(np.zeros(8), np.zeros(8), np.zeros(8), 4, 3, 2)  # heads % kvheads
