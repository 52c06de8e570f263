"""The device sampler (src/sampling.rs:26-63 with the padding-vocab mask of
src/main.rs:262-266) against the oracle's restatement, through the C ABI:
same seed, same logits -> the same id sequence."""
import importlib
import os

import numpy as np
import pytest

import oracle
from helpers import GOLDEN

engine = importlib.import_module("qwen-30brust_amd")

pytestmark = pytest.mark.gpu
FMIN = np.float32(np.finfo(np.float32).min)


@pytest.fixture(scope="module")
def dev():
    return engine.Device(0)


def run_both(dev, logits, seed, t, k, p, steps, valid=None):
    lg = np.ascontiguousarray(logits, np.float32)
    ref_lg = lg if valid is None else np.where(valid.astype(bool), lg, FMIN).astype(np.float32)
    a, b = engine.Sampler(seed, t, k, p), oracle.Sampler(seed, t, k, p)
    got = [a.sample(dev, lg, valid) for _ in range(steps)]
    want = [b.sample(ref_lg) for _ in range(steps)]
    return got, want


CASES = [  # (vocab, scale, temperature, top_k, top_p)
    (151936, 3.0, 0.0, 0, 1.0),
    (151936, 3.0, 0.2, 20, 0.8),   # the reference CLI's defaults (src/main.rs:92-99)
    (151936, 3.0, 0.7, 100, 0.95),
    (151936, 3.0, 1.5, 1, 1.0),
    (151936, 3.0, 1.0, 4096, 1.0),
    (151936, 20.0, 0.05, 0, 0.9),  # no top-k: every id with nonzero probability
    (4000, 1.0, 1.0, 0, 0.5),      # no top-k, every id a candidate
    (257, 0.5, 2.0, 300, 1.0),     # top_k above the vocabulary
    (3, 1.0, 1.0, 0, 1.0),
    # more than 4096 candidates: sorted in HBM (sampling.rs:36-63 over the full support)
    (151936, 1.0, 1.0, 0, 1.0),    # every id has nonzero probability
    (151936, 1.0, 1.0, 0, 0.9),
    (151936, 5.0, 1.0, 0, 1.0),    # part of the vocabulary underflows to probability 0
    (151936, 3.0, 1.0, 10000, 1.0),
    (151936, 0.5, 2.0, 50000, 0.99),
    (9000, 1.0, 1.0, 0, 1.0),
]


@pytest.mark.parametrize("case", CASES)
def test_sampler_matches_oracle(dev, case):
    v, scale, t, k, p = case
    rng = np.random.default_rng(v + k)
    logits = (rng.standard_normal(v) * scale).astype(np.float32)
    got, want = run_both(dev, logits, seed=v * 7 + k, t=t, k=k, p=p, steps=24)
    assert got == want


def test_sampler_ties_and_mask(dev):
    # runs of equal logits: the sort is by index within a run (sampling.rs:31)
    lg = np.zeros(4096 + 100, np.float32)
    lg[::7] = 0.5
    for k in (5, 700, 4096):
        got, want = run_both(dev, lg, 11, 1.0, k, 1.0, 16)
        assert got == want
    # masked ids read as f32::MIN and are never drawn
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(151936).astype(np.float32)
    valid = np.ones(151936, np.uint8)
    valid[np.argsort(-lg)[:50]] = 0
    valid[151669:] = 0  # a padded vocabulary tail
    for t, k, p in ((0.0, 0, 1.0), (0.8, 40, 0.9), (1.0, 4096, 1.0)):
        got, want = run_both(dev, lg, 5, t, k, p, 20, valid)
        assert got == want
        assert all(valid[g] for g in got)


def test_sampler_errors_leave_the_stream(dev):
    s, ref = engine.Sampler(99, 1.0, 0, 1.0), oracle.Sampler(99, 1.0, 0, 1.0)
    bad = np.array([1.0, np.nan, 2.0], np.float32)
    with pytest.raises(engine.EngineError, match="invalid logits"):
        s.sample(dev, bad)
    with pytest.raises(engine.EngineError, match="invalid logits"):
        s.sample(dev, np.array([1.0, np.inf], np.float32))
    with pytest.raises(engine.EngineError, match="at most 1048576 logits"):
        s.sample(dev, np.zeros((1 << 20) + 1, np.float32))
    # a flat support of 10,000 ids (the HBM path) draws like the reference
    flat = np.zeros(10000, np.float32)
    assert [s.sample(dev, flat) for _ in range(5)] == [ref.sample(flat) for _ in range(5)]
    lg = np.array([1.0, 2.0, 3.0], np.float32)
    assert [s.sample(dev, lg) for _ in range(10)] == [ref.sample(lg) for _ in range(10)]


def test_model_sample_after_forward(dev):
    m = engine.Model(os.path.join(GOLDEN, "tiny-qwen3moe.gguf"), 16, device=dev)
    s, ref = engine.Sampler(42, 0.2, 20, 0.8), oracle.Sampler(42, 0.2, 20, 0.8)
    tok = 1
    for _ in range(8):
        lg = m.forward(tok)
        tok = m.sample(s)
        assert tok == ref.sample(lg)
    valid = np.ones(m.config["vocab"], np.uint8)
    valid[tok] = 0
    m.set_valid_tokens(valid)
    lg = m.forward(tok)
    assert m.sample(engine.Sampler(1, 0.0, 0, 1.0)) == oracle.greedy(np.where(valid == 1, lg, FMIN))
    m.set_valid_tokens(None)
