"""Pins the oracle's vector ops (ops.rs, sampling.rs greedy) against the
reference's known-answer tests (tests/core.rs:3-42) and closed forms."""
import math

import numpy as np
import pytest

import oracle


def test_routing_uses_topk_and_renormalizes():  # tests/core.rs:3-12
    ids, w = oracle.route([1.0, 3.0, 2.0, -10.0], 2)
    assert list(ids) == [1, 2]
    assert abs(float(w.sum()) - 1.0) < 1e-6
    assert abs(float(w[0]) - 0.7310586) < 1e-6
    with pytest.raises(oracle.OracleError):
        oracle.route([float("nan")], 1)
    with pytest.raises(oracle.OracleError):
        oracle.route([1.0], 0)


def test_route_ties_and_total_order():
    ids, _ = oracle.route([2.0, 5.0, 5.0, 5.0, 1.0], 3)
    assert list(ids) == [1, 2, 3]
    ids, _ = oracle.route([-0.0, 0.0, -1.0], 1)  # total order: +0 > -0
    assert list(ids) == [1]
    rng = np.random.default_rng(5)
    for _ in range(20):
        lg = rng.standard_normal(128).astype(np.float32)
        ids, w = oracle.route(lg, 8)
        ref = np.argsort(-lg, kind="stable")[:8]
        assert list(ids) == list(ref)
        e = np.exp(lg[ref].astype(np.float64) - lg[ref].max())
        assert np.allclose(w, e / e.sum(), rtol=1e-6, atol=1e-7)


def test_neox_rotates_split_halves():  # tests/core.rs:13-19
    x = oracle.rope([1.0, 2.0, 3.0, 4.0], 4, 1, 10000.0)
    assert abs(x[0] - (math.cos(1) - 3 * math.sin(1))) < 1e-6
    assert abs(x[1] - (2 * math.cos(0.01) - 4 * math.sin(0.01))) < 1e-6


def test_rope_closed_form():
    rng = np.random.default_rng(3)
    d, heads, pos, theta = 16, 3, 37, 1e6
    x = rng.standard_normal(heads * d).astype(np.float32)
    got = oracle.rope(x, d, pos, theta)
    ref = x.astype(np.float64).reshape(heads, d).copy()
    i = np.arange(d // 2)
    ang = pos * theta ** (-2.0 * i / d)
    a, b = ref[:, : d // 2].copy(), ref[:, d // 2:].copy()
    ref[:, : d // 2] = a * np.cos(ang) - b * np.sin(ang)
    ref[:, d // 2:] = a * np.sin(ang) + b * np.cos(ang)
    assert np.max(np.abs(got - ref.reshape(-1))) < 2e-5


def test_gqa_maps_contiguous_query_heads():  # tests/core.rs:20-27
    out = oracle.attention([0.0] * 8, [0.0] * 8, [2.0, 4.0, 10.0, 20.0, 6.0, 8.0, 30.0, 40.0], 4, 2, 2)
    assert list(out) == [4.0, 6.0, 4.0, 6.0, 20.0, 30.0, 20.0, 30.0]


def test_attention_vs_float64_and_shapes():
    rng = np.random.default_rng(11)
    heads, kvh, d, t = 8, 2, 16, 19
    q = rng.standard_normal(heads * d).astype(np.float32)
    k = rng.standard_normal(t * kvh * d).astype(np.float32)
    v = rng.standard_normal(t * kvh * d).astype(np.float32)
    got = oracle.attention(q, k, v, heads, kvh, d)
    K = k.reshape(t, kvh, d).astype(np.float64)
    V = v.reshape(t, kvh, d).astype(np.float64)
    ref = np.zeros((heads, d))
    for h in range(heads):
        g = h // (heads // kvh)
        s = K[:, g, :] @ q[h * d:(h + 1) * d] / math.sqrt(d)
        p = np.exp(s - s.max())
        ref[h] = (p / p.sum()) @ V[:, g, :]
    assert np.max(np.abs(got - ref.reshape(-1))) < 1e-5
    with pytest.raises(oracle.OracleError):
        oracle.attention(q, k, v, heads, 3, d)  # heads % kvheads != 0
    with pytest.raises(oracle.OracleError):
        oracle.attention(q, np.zeros(0), np.zeros(0), heads, kvh, d)  # empty KV


def test_rms_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2048).astype(np.float32)
    w = (1 + 0.05 * rng.standard_normal(2048)).astype(np.float32)
    got = oracle.rms(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / math.sqrt((x64 * x64).mean() + 1e-6) * w
    assert np.max(np.abs(got - ref) / np.abs(ref).max()) < 1e-6
    with pytest.raises(oracle.OracleError):
        oracle.rms(x, w, 0.0)


def test_softmax_rejects_and_normalises():
    p = oracle.softmax([1.0, 2.0, 3.0])
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)
    with pytest.raises(oracle.OracleError):
        oracle.softmax([1.0, float("inf")])


def test_sampler_greedy():  # tests/core.rs:28-31
    assert oracle.greedy([0.0, 4.0, 2.0]) == 1
    with pytest.raises(oracle.OracleError):
        oracle.greedy([float("nan")])
    assert oracle.greedy([1.0, 3.0, 3.0, 2.0]) == 1  # lowest index on ties
    assert oracle.greedy([-0.0, 0.0]) == 1  # +0 > -0 under total order
    rng = np.random.default_rng(8)
    lg = rng.standard_normal(151936).astype(np.float32)
    assert oracle.greedy(lg) == int(np.argmax(lg))
