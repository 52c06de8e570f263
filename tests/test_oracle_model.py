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


def _mat(g, name):
    """An F32 tensor of the fixture as (rows, cols) or (experts, rows, cols)."""
    t = g.tensor(name)
    return np.frombuffer(g.data(name).tobytes(), np.float32).reshape(t["dims"][::-1])


def _np_forward(g, c, tokens, routes):
    """model.rs:217-302 restated in NumPy (float64) for the F32 fixture, with
    the expert ids of every (token, layer) given: routes[t][l] in rank order,
    weighted by the softmax of the router logits at those ids."""
    H, d, nh, nkv = c["hidden"], c["head_dim"], c["heads"], c["kvheads"]

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v) + c["eps"]) * w

    def rope(v, pos):
        v = v.reshape(-1, d).copy()
        i = np.arange(d // 2)
        ang = pos * float(c["theta"]) ** (-2.0 * i / d)
        a, b = v[:, : d // 2].copy(), v[:, d // 2:].copy()
        v[:, : d // 2] = a * np.cos(ang) - b * np.sin(ang)
        v[:, d // 2:] = a * np.sin(ang) + b * np.cos(ang)
        return v.reshape(-1)

    f = lambda n: _mat(g, n).astype(np.float64)
    K = [[] for _ in range(c["layers"])]
    V = [[] for _ in range(c["layers"])]
    for pos, tok in enumerate(tokens):
        x = f("token_embd.weight")[tok].copy()
        for l in range(c["layers"]):
            p = f"blk.{l}."
            xn = rms(x, f(p + "attn_norm.weight"))
            q = (f(p + "attn_q.weight") @ xn).reshape(nh, d)
            k = (f(p + "attn_k.weight") @ xn).reshape(nkv, d)
            v = f(p + "attn_v.weight") @ xn
            q = np.stack([rms(h, f(p + "attn_q_norm.weight")) for h in q]).reshape(-1)
            k = np.stack([rms(h, f(p + "attn_k_norm.weight")) for h in k]).reshape(-1)
            K[l].append(rope(k, pos).reshape(nkv, d))
            V[l].append(v.reshape(nkv, d))
            q = rope(q, pos).reshape(nh, d)
            a = np.zeros((nh, d))
            for h in range(nh):
                kh = h // (nh // nkv)
                s = np.array([q[h] @ kt[kh] for kt in K[l]]) / np.sqrt(d)
                e = np.exp(s - s.max())
                a[h] = (e / e.sum()) @ np.array([vt[kh] for vt in V[l]])
            x = x + f(p + "attn_output.weight") @ a.reshape(-1)
            xn = rms(x, f(p + "ffn_norm.weight"))
            lg = f(p + "ffn_gate_inp.weight") @ xn
            ids = list(routes[pos][l])
            e = np.exp(lg[ids] - lg[ids].max())
            wts = e / e.sum()
            moe = np.zeros(H)
            for wgt, ex in zip(wts, ids):
                gt = f(p + "ffn_gate_exps.weight")[ex] @ xn
                up = f(p + "ffn_up_exps.weight")[ex] @ xn
                moe += wgt * (f(p + "ffn_down_exps.weight")[ex] @ (gt / (1 + np.exp(-gt)) * up))
            x = x + moe
    return f("output.weight") @ rms(x, f("output_norm.weight"))


def test_forced_routes_hook():
    """The oracle's forced-routing hook (or_model_force_routes).  Forcing the
    oracle's own expert ids reproduces its forward bit for bit; forcing other
    ids matches a float64 NumPy restatement of model.rs:217-302 that takes
    those ids (so the hook uses the given ids, in the given rank order, with
    softmax weights of the path's own router logits at them); bad id lists are
    refused and a forced routing holds for one step only."""
    g = oracle.Gguf.open(FIXTURE)
    m = oracle.Model(g, 4)
    c = m.config
    tokens = [1, 5, 2]
    own, own_routes = [], []
    for t in tokens:
        own.append(m.forward(t))
        own_routes.append(m.routes())
    m.reset()
    for t, r, lg in zip(tokens, own_routes, own):
        assert np.array_equal(m.forward(t, routes=r).view(np.uint32), lg.view(np.uint32))
    # for every (token, layer) the experts the oracle did not choose, in
    # descending id order (4 experts, top 2: the complement)
    other = [np.stack([np.array([e for e in range(c["experts"]) if e not in r[l]][::-1], np.uint32)
                       for l in range(c["layers"])]) for r in own_routes]
    m.reset()
    forced = [m.forward(t, routes=r) for t, r in zip(tokens, other)]
    ref = _np_forward(g, c, tokens, other)
    scale = float(np.max(np.abs(ref)))
    assert np.max(np.abs(forced[-1] - ref)) <= 1e-5 * scale
    assert np.max(np.abs(forced[-1] - own[-1])) > 1e-3 * scale  # the routing mattered
    # the oracle's own routes through the same restatement agree too
    assert np.max(np.abs(own[-1] - _np_forward(g, c, tokens, own_routes))) <= 1e-5 * scale
    # one step only: after a forced step the next one routes by itself
    m.reset()
    m.forward(tokens[0], routes=other[0])
    lg1 = m.forward(tokens[1])
    r1 = m.routes()
    assert any(set(r1[l]) != set(other[1][l]) for l in range(c["layers"]))
    m2 = oracle.Model(g, 4)
    m2.forward(tokens[0], routes=other[0])
    assert np.array_equal(m2.forward(tokens[1], routes=r1).view(np.uint32), lg1.view(np.uint32))
    for bad in (np.zeros(c["layers"] * c["top"] - 1, np.uint32),     # wrong length
                np.full(c["layers"] * c["top"], c["experts"], np.uint32),  # out of range
                np.zeros(c["layers"] * c["top"], np.uint32)):          # repeated expert
        with pytest.raises(oracle.OracleError):
            m.force_routes(bad)
