"""Pins the oracle's GGUF reader and full forward against the reference's own
fixture model and NumPy-derived logits (tests/model.rs:48-97)."""
import json
import os

import numpy as np
import pytest

import oracle
from helpers import GOLDEN

FIXTURE = os.path.join(GOLDEN, "tiny-qwen3moe.gguf")


def load_expected():
    with open(os.path.join(GOLDEN, "expected-logits.json")) as f:
        return [np.array(v, np.float32) for v in json.load(f)]


def test_full_forward_matches_independent_reference_and_reset():  # tests/model.rs:48-69
    expected = load_expected()
    g = oracle.Gguf.open(FIXTURE)
    m = oracle.Model(g, 4)
    for tok, exp in zip([1, 5, 2, 9], expected):
        got = m.forward(tok)
        assert np.max(np.abs(got - exp)) < 2e-5
    assert m.position == 4
    with pytest.raises(oracle.OracleError):
        m.forward(1)
    assert m.position == 0
    again = m.forward(1)
    assert np.max(np.abs(again - expected[0])) < 2e-5
    with pytest.raises(oracle.OracleError):
        m.forward(999)
    assert m.position == 0


def test_fixture_errors_equal_reference_cpu_record():
    """validation/parity-cpu.json:9-14 records the Rust CPU backend's max
    |logit - NumPy| per prefix of [1,5,2,9].  A bit-identical restatement
    reproduces those four numbers exactly."""
    expected = load_expected()
    with open(os.path.join(GOLDEN, "parity-cpu.json")) as f:
        record = json.load(f)["max_absolute_error_by_prefix"]
    m = oracle.Model(oracle.Gguf.open(FIXTURE), 4, threads=0)
    errs = [float(np.max(np.abs(m.forward(t) - e))) for t, e in zip([1, 5, 2, 9], expected)]
    assert errs == record


def test_fixture_header_and_config():
    g = oracle.Gguf.open(FIXTURE)
    assert g.tensor_count() == 27
    m = oracle.Model(g, 4)
    c = m.config
    assert (c["hidden"], c["layers"], c["heads"], c["kvheads"], c["head_dim"]) == (8, 2, 4, 2, 4)
    assert (c["experts"], c["top"], c["intermediate"], c["vocab"], c["max_context"]) == (4, 2, 12, 16, 32)
    assert abs(c["theta"] - 10000.0) < 1e-3
    with pytest.raises(oracle.OracleError):
        oracle.Model(g, 33)  # context > context_length
    with pytest.raises(oracle.OracleError):
        oracle.Model(g, 0)


def test_faithful_and_threaded_forward_identical():
    g = oracle.Gguf.open(FIXTURE)
    a = oracle.Model(g, 8, threads=0)
    b = oracle.Model(g, 8, threads=4)
    for t in [3, 1, 4, 1, 5, 9, 2, 6]:
        la, lb = a.forward(t), b.forward(t)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def _reject(image):
    with pytest.raises(oracle.OracleError):
        oracle.Gguf(image)


def test_malformed_headers_and_truncated_data_are_rejected():  # tests/model.rs:83-97
    data = open(FIXTURE, "rb").read()
    _reject(data[:10])
    _reject(data[:-20])
    v = bytearray(data)
    v[:4] = b"NOPE"
    _reject(bytes(v))
    v = bytearray(data)
    v[4:8] = (999).to_bytes(4, "little")
    _reject(bytes(v))
    v = bytearray(data)
    v[8:16] = (2**64 - 1).to_bytes(8, "little")
    _reject(bytes(v))


def test_backend_matvec_surface():
    """Backend::matvec (name, expert) resolution, backend.rs:57-75."""
    g = oracle.Gguf.open(FIXTURE)
    m = oracle.Model(g, 4)
    x = np.arange(8, dtype=np.float32) / 7
    y = m.matvec("blk.0.attn_q.weight", None, x)
    w = np.frombuffer(g.data("blk.0.attn_q.weight").tobytes(), np.float32).reshape(16, 8)
    assert np.allclose(y, w @ x, rtol=1e-6, atol=1e-7)
    ye = m.matvec("blk.1.ffn_down_exps.weight", 3, np.ones(12, np.float32))
    wd = np.frombuffer(g.data("blk.1.ffn_down_exps.weight").tobytes(), np.float32).reshape(4, 8, 12)
    assert np.allclose(ye, wd[3].sum(axis=1), rtol=1e-6, atol=1e-7)
    with pytest.raises(oracle.OracleError):
        m.matvec("blk.1.ffn_down_exps.weight", 4, np.ones(12, np.float32))  # expert out of bounds
    with pytest.raises(oracle.OracleError):
        m.matvec("blk.0.attn_q.weight", 0, x)  # rank mismatch
    with pytest.raises(oracle.OracleError):
        m.matvec("blk.0.attn_q.weight", None, np.ones(7, np.float32))  # shape mismatch
