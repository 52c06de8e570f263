"""GPU parity of the device-resident token step against the oracle and the
reference's own fixture model (tests/model.rs:48-118), through the C ABI."""
import ctypes as C
import importlib
import json
import os

import numpy as np
import pytest

import oracle
from helpers import GOLDEN

engine = importlib.import_module("qwen-30brust_amd")
synth = importlib.import_module("qwen-30brust_amd.synth")

pytestmark = pytest.mark.gpu
REL = 1e-4
FIXTURE = os.path.join(GOLDEN, "tiny-qwen3moe.gguf")


@pytest.fixture(scope="module")
def dev():
    return engine.Device(0)


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def expected_logits():
    with open(os.path.join(GOLDEN, "expected-logits.json")) as f:
        return [np.array(v, np.float32) for v in json.load(f)]


def test_fixture_forward_matches_reference_and_reset(dev):  # tests/model.rs:48-69
    exp = expected_logits()
    m = engine.Model(FIXTURE, 4, device=dev)
    for tok, e in zip([1, 5, 2, 9], exp):
        assert np.max(np.abs(m.forward(tok) - e)) < 2e-5
    assert m.position == 4
    with pytest.raises(engine.EngineError, match="context limit"):
        m.forward(1)
    assert m.position == 0
    assert np.max(np.abs(m.forward(1) - exp[0])) < 2e-5
    with pytest.raises(engine.EngineError, match="vocabulary"):
        m.forward(999)
    assert m.position == 0


def test_fixture_reload_invalidates_previous_model(dev):  # tests/model.rs:112-117
    exp = expected_logits()
    img = open(FIXTURE, "rb").read()
    m = engine.Model(img, 4, device=dev)
    m.forward(1)
    m2 = engine.Model(img, 4, device=dev)  # same context, new model
    assert m2.position == 0
    assert np.max(np.abs(m2.forward(1) - exp[0])) < 2e-5


def test_malformed_images_rejected(dev):  # tests/model.rs:83-97
    data = open(FIXTURE, "rb").read()
    bad = [data[:10], data[:-20], b"NOPE" + data[4:], data[:4] + (999).to_bytes(4, "little") + data[8:],
           data[:8] + (2**64 - 1).to_bytes(8, "little") + data[16:]]
    for b in bad:
        with pytest.raises(engine.EngineError):
            engine.Model(b, 4, device=dev)


def test_backend_matvec_surface_and_stats(dev):
    g = oracle.Gguf.open(FIXTURE)
    om = oracle.Model(g, 4)
    m = engine.Model(FIXTURE, 4, device=dev)
    b = engine.HipBackend(m)
    s0 = b.stats()
    x = np.linspace(-1, 1, 8).astype(np.float32)
    for name, e, n in [("blk.0.attn_q.weight", None, 8), ("blk.1.ffn_up_exps.weight", 3, 8),
                       ("blk.1.ffn_down_exps.weight", 2, 12), ("output.weight", None, 8)]:
        xi = np.linspace(-1, 1, n).astype(np.float32)
        assert rel_err(b.matvec(name, e, xi), om.matvec(name, e, xi)) <= REL
    with pytest.raises(engine.EngineError):
        b.matvec("blk.1.ffn_down_exps.weight", 4, np.ones(12))
    with pytest.raises(engine.EngineError):
        b.matvec("blk.0.attn_q.weight", 0, x)
    with pytest.raises(engine.EngineError):
        b.matvec("nope.weight", None, x)
    s = b.stats()
    assert s["matvecs"] - s0["matvecs"] == 4 and s["cache_hits"] == 0
    assert s["uploaded_bytes"] > s0["uploaded_bytes"]


@pytest.mark.parametrize("make", [synth.tiny_k, synth.tiny_lit])
def test_tiny_quantized_model_logits_and_greedy(dev, make):
    """C1 (both variants): 16-token prompt, then 16 greedy tokens.  Logits
    within 1e-4 of the oracle at every prompt step; greedy ids identical."""
    spec = make()
    img = synth.build_image(spec, threads=8)
    g = oracle.Gguf(img)
    om = oracle.Model(g, spec.context)
    m = engine.Model(img, spec.context, device=dev)
    rng = np.random.default_rng(16)
    prompt = rng.integers(0, spec.vocab, 16).astype(np.uint32)
    for t in prompt:
        ref = om.forward(int(t))
        got = m.forward(int(t))
        assert rel_err(got, ref) <= REL
        assert m.last_argmax == oracle.greedy(ref)
    # greedy continuation: oracle loop vs device-chained generate
    ref_ids = []
    nxt = oracle.greedy(ref)
    for i in range(16):
        ref_ids.append(nxt)
        if i + 1 < 16:
            nxt = oracle.greedy(om.forward(nxt))
    m.reset()
    got_ids = m.generate(prompt, 16)
    assert list(got_ids) == ref_ids


def test_generate_matches_stepwise_forward(dev):
    spec = synth.tiny_k(seed=5)
    img = synth.build_image(spec, threads=8)
    m = engine.Model(img, spec.context, device=dev)
    prompt = [3, 1, 4, 1, 5]
    ids, lg = m.generate(prompt, 6, want_logits=True)
    assert m.position == len(prompt) + 5
    m.reset()
    step = []
    for t in prompt:
        m.forward(t)
    tok = m.last_argmax
    for i in range(6):
        step.append(tok)
        if i + 1 < 6:
            last = m.forward(tok)
            tok = m.last_argmax
    assert list(ids) == step
    assert np.array_equal(lg, last)


@pytest.mark.parametrize("persistent", [True, False])
@pytest.mark.parametrize("more_bits", [True, False])
def test_layer_30b_shapes_at_pos_1024(dev, more_bits, persistent):
    """Config 3: one decoder layer at 30B-A3B shapes, position 1024 with 1024
    pre-filled N(0,1) KV positions; layer 0 types (Q6_K attn_v / down) and a
    plain Q4_K layer; through the persistent step and the per-phase kernels."""
    # a previously loaded model with a different attention tile must not leak
    # its geometry into this one (regression: tile chosen after sizing buffers)
    engine.Model(synth.build_image(synth.tiny_k(), threads=8), 64, device=dev).forward(1)
    spec = synth.layer30b(more_bits=more_bits)
    img = synth.build_image(spec, threads=8)
    g = oracle.Gguf(img)
    om = oracle.Model(g, spec.context)
    m = engine.Model(img, spec.context, device=dev)
    m.persistent = persistent
    assert m.persistent == persistent
    pos, kvd = 1024, spec.kvheads * spec.head_dim
    x = synth.normal(21, spec.hidden)
    kp = synth.normal(22, pos * kvd)
    vp = synth.normal(23, pos * kvd)
    xr, ids_r, w_r = om.layer_forward(0, x, pos, kp, vp)
    xg, ids_g, w_g = m.layer_forward(0, x, pos, kp, vp)
    lg = om.last_router(0)
    s = np.sort(lg)[::-1]
    margin = float(s[spec.top - 1] - s[spec.top])
    print(f"router 8th/9th margin {margin:.3e}")
    assert np.array_equal(ids_g, ids_r), margin
    assert np.allclose(w_g, w_r, rtol=1e-5, atol=1e-6)
    assert rel_err(xg, xr) <= REL


@pytest.fixture(scope="module")
def layer30b_q4k():
    spec = synth.layer30b(more_bits=False, context=4096)
    img = synth.build_image(spec, threads=8)
    return spec, img


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 700, 1100, 2047, 2500, 3000, 3583, 4095])
def test_persistent_layer_attention_chunking(dev, layer30b_q4k, pos):
    """The persistent step at positions that exercise the attention split: one
    key, one chunk, chunk boundaries (64-key tiles, at least 64 keys per
    chunk), 11 and then 16 chunks per XCD of one tile or two (up to 2,048
    keys), then chunks of two tiles, up to 32 per XCD: 2,501 keys in 20
    (the last of 69 keys), 3,001 in 24, 3,584 in 28 and 4,096 in 32;
    against the oracle layer."""
    spec, img = layer30b_q4k
    om = oracle.Model(oracle.Gguf(img), spec.context)
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    kvd = spec.kvheads * spec.head_dim
    x = synth.normal(31 + pos, spec.hidden)
    kp = synth.normal(32 + pos, max(pos, 1) * kvd)[: pos * kvd]
    vp = synth.normal(33 + pos, max(pos, 1) * kvd)[: pos * kvd]
    xr, ids_r, _ = om.layer_forward(0, x, pos, kp, vp)
    xg, ids_g, _ = m.layer_forward(0, x, pos, kp, vp)
    assert np.array_equal(ids_g, ids_r)
    assert rel_err(xg, xr) <= REL


@pytest.fixture(scope="module")
def layer30b_long():
    spec = synth.layer30b(more_bits=False, context=16384)
    img = synth.build_image(spec, threads=8)
    return spec, img


@pytest.mark.parametrize("pos", [8191, 16383])
def test_persistent_layer_long_context(dev, layer30b_long, pos):
    """The persistent step beyond 4,096 positions: 32 chunks per XCD of 256
    and of 512 keys (4 and 8 key tiles each), against the oracle layer."""
    spec, img = layer30b_long
    om = oracle.Model(oracle.Gguf(img), spec.context)
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    kvd = spec.kvheads * spec.head_dim
    x = synth.normal(41 + pos, spec.hidden)
    kp = synth.normal(42 + pos, pos * kvd)
    vp = synth.normal(43 + pos, pos * kvd)
    xr, ids_r, _ = om.layer_forward(0, x, pos, kp, vp)
    xg, ids_g, _ = m.layer_forward(0, x, pos, kp, vp)
    assert np.array_equal(ids_g, ids_r)
    assert rel_err(xg, xr) <= REL


@pytest.mark.parametrize("main,out", [(synth.Q4_0, synth.Q4_0), (synth.Q8_0, synth.Q8_0),
                                      (synth.Q5_K, synth.Q5_K), (synth.Q6_K, synth.Q4_K)])
def test_persistent_step_main_formats(dev, main, out):
    """The persistent step for the other block formats (Q4_0, Q8_0, Q5_K,
    Q6_K as the q/k/o/gate/up format): two 30B-shaped layers, the second with
    Q6_K v/down (llama.cpp's more-bits rule), vocab projection in the given
    format; logits of three tokens and one layer at position 700 against the
    oracle."""
    t = synth._k_types(attn=main, down=main, out=out, embd=main)
    spec = synth.Spec(2048, 2, 32, 4, 128, 128, 8, 768, 512, 1024, types=t,
                      more_bits_type=synth.Q6_K, seed=11)
    img = synth.build_image(spec, threads=8)
    om = oracle.Model(oracle.Gguf(img), spec.context)
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    for tok in (5, 300, 77):
        ref = om.forward(tok)
        got = m.forward(tok)
        assert rel_err(got, ref) <= REL
        assert m.last_argmax == oracle.greedy(ref)
    pos, kvd = 700, spec.kvheads * spec.head_dim
    for layer in (0, 1):
        x = synth.normal(41 + layer, spec.hidden)
        kp = synth.normal(42 + layer, pos * kvd)
        vp = synth.normal(43 + layer, pos * kvd)
        xr, ids_r, w_r = om.layer_forward(layer, x, pos, kp, vp)
        xg, ids_g, w_g = m.layer_forward(layer, x, pos, kp, vp)
        assert np.array_equal(ids_g, ids_r)
        assert np.allclose(w_g, w_r, rtol=1e-5, atol=1e-6)
        assert rel_err(xg, xr) <= REL


@pytest.mark.parametrize("persistent", [True, False])
def test_tied_vocab_projection(dev, persistent):
    """A model without output.weight projects onto the vocabulary with
    token_embd.weight (src/model.rs:290-294): two 30B-shaped layers, Q4_K
    embedding, vocab 4096, through the persistent step and the per-phase
    kernels; logits of five tokens within 1e-4 of the oracle's, the same greedy
    ids, and the routing of every (position, layer) equal to the oracle's."""
    t = synth._k_types(attn=synth.Q4_K, down=synth.Q4_K, out=synth.Q6_K, embd=synth.Q4_K)
    spec = synth.Spec(2048, 2, 32, 4, 128, 128, 8, 768, 4096, 64, types=t, more_bits_type=synth.Q6_K,
                      tied_output=True, seed=21)
    img = synth.build_image(spec, threads=8)
    g = oracle.Gguf(img)
    with pytest.raises(oracle.OracleError):
        g.tensor("output.weight")  # the image really has no output matrix
    om = oracle.Model(g, spec.context)
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    m.persistent = persistent
    toks = [5, 4095, 77, 1024, 3]
    for i, tok in enumerate(toks):
        ref = om.forward(tok)
        got = m.forward(tok)
        assert rel_err(got, ref) <= REL
        assert m.last_argmax == oracle.greedy(ref)
        assert np.array_equal(np.sort(m.route_log(i, 1)[0], axis=1), np.sort(om.routes(), axis=1))


def test_greedy_30b_token_loop_matches_oracle(dev):
    """Config 4 token loop: the random-init 48-layer Qwen3-30B-A3B Q4_K_M
    model, a 32-token uniform random prompt, then 64 greedy tokens chained on
    the device; the ids must equal the oracle's greedy loop.  The oracle's
    top-1/top-2 logit margin per step is printed so a flip can be attributed
    to a near-tie."""
    threads = min(16, os.cpu_count() or 1)
    spec = synth.qwen30b(context=256)
    img = synth.build_image(spec, threads=threads)
    g = oracle.Gguf(img)
    om = oracle.Model(g, spec.context, threads=threads)
    m = engine.Model(img, spec.context, device=dev)
    prompt = np.random.default_rng(4).integers(0, spec.vocab, 32).astype(np.uint32)
    got = m.generate(prompt, 64)
    for t in prompt:
        ref = om.forward(int(t))
    ref_ids, margins = [], []
    for i in range(64):
        s = np.partition(ref, -2)[-2:]
        margins.append(float(s[1] - s[0]))
        ref_ids.append(oracle.greedy(ref))
        if i + 1 < 64:
            ref = om.forward(ref_ids[-1])
        print(f"step {i}: oracle {ref_ids[-1]} device {int(got[i])} margin {margins[-1]:.3e}", flush=True)
    print(f"smallest top-1/top-2 margin {min(margins):.3e}")
    assert list(got) == ref_ids


def test_persistent_profile_decode(dev, layer30b_q4k):
    """qh_profile_decode times the embedding kernel and the k_decode launch of
    each step and advances the position by one per step, like qh_forward."""
    spec, img = layer30b_q4k
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    m.generate(np.array([3, 17, 5], np.uint32), 1)
    pos = m.position
    e, d = m.profile_decode(4)
    assert e > 0 and d > 0
    assert m.position == pos + 4
    m.persistent = False
    with pytest.raises(engine.EngineError):
        m.profile_decode(1)


def test_persistent_step_error_paths_and_rollback(dev):
    """The persistent step's failure paths (src/model.rs:209-224: any error
    resets the KV cache and the position): the context limit, a token outside
    the vocabulary, and an abandoned step (the abort flag raised from the
    host: every wait of the step gives up and the kernels exit normally).
    Each raises, leaves position 0, and a clean re-run afterwards gives the
    first run's logits bit for bit."""
    spec = synth.layer30b(more_bits=False, context=8)
    img = synth.build_image(spec, threads=8)
    m = engine.Model(img, spec.context, device=dev)
    assert m.persistent
    toks = [5, 17, 3, 250, 9, 0, 77, 128]
    first = [m.forward(t) for t in toks]
    assert m.position == 8
    with pytest.raises(engine.EngineError, match="context limit 8 reached"):
        m.forward(1)
    assert m.position == 0
    for t, ref in zip(toks[:3], first):
        assert np.array_equal(m.forward(t), ref)
    with pytest.raises(engine.EngineError, match="token outside vocabulary"):
        m.forward(spec.vocab)
    assert m.position == 0
    m.forward(toks[0])
    m.inject_fault(1)
    with pytest.raises(engine.EngineError, match="synchronisation"):
        m.forward(toks[1])
    assert m.position == 0
    for t, ref in zip(toks, first):
        assert np.array_equal(m.forward(t), ref)
    with pytest.raises(engine.EngineError, match="exceed"):
        m.generate(toks, 4)
    m.reset()
    ids = m.generate(toks[:4], 4)
    m.reset()
    for t in toks[:4]:
        m.forward(t)
    step = [m.last_argmax]
    for _ in range(3):
        m.forward(step[-1])
        step.append(m.last_argmax)
    assert list(ids) == step


def test_model_replaced_by_a_later_load_raises(dev):
    """The context holds one model: a Model whose weights a later load on the
    same Device replaced refuses to run (it would otherwise run the other
    model and size its logits from the old vocabulary); the C ABI refuses a
    logits buffer smaller than the loaded vocabulary."""
    m1 = engine.Model(FIXTURE, 4, device=dev)
    m1.forward(1)
    spec = synth.tiny_k()
    m2 = engine.Model(synth.build_image(spec, threads=8), spec.context, device=dev)
    assert m2.config["vocab"] > m1.config["vocab"]
    with pytest.raises(engine.EngineError, match="replaced by a later load"):
        m1.forward(1)
    with pytest.raises(engine.EngineError, match="replaced by a later load"):
        m1.generate([1, 2], 2)
    m2.forward(3)
    buf = np.zeros(10, np.float32)
    am = C.c_uint32()
    rc = engine.lib().qh_forward(dev.h, 1, buf.ctypes.data, buf.size, C.byref(am))
    assert rc != 0
    assert b"logits buffer holds 10 floats" in engine.lib().qh_last_error(dev.h)
