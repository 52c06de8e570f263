"""GPU parity of the batched prefill (qh_prefill: fp16 matrix-core GEMMs and
flash attention in place of the reference's one-forward-per-token prompt
loop, src/main.rs:250-256) against the FP32 oracle's sequential forward.
fp16 operands cannot meet the decode path's 1e-4, so the bar is the logits
of the last prompt token within 1e-2 (infinity-norm relative) and the same
greedy id unless the top-1/top-2 margin is inside that tolerance; the decode
steps that follow must stay within 2e-2.  The fp16 router may pick another
expert where the oracle's 8th/9th router logits nearly tie: every routing
difference is counted and each token's first one attributed to such a
near-tie, and the logits are compared with the oracle routed to the device's
expert ids, so the bars hold whatever flipped."""
import importlib
import os

import numpy as np
import pytest

import oracle

engine = importlib.import_module("qwen-30brust_amd")
synth = importlib.import_module("qwen-30brust_amd.synth")

pytestmark = pytest.mark.gpu
TOL = 1e-2
NEAR_TIE = 1e-2  # 8th/9th router logit gap, relative to the largest |logit|, that fp16 noise may flip


@pytest.fixture(scope="module")
def dev():
    return engine.Device(0)


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.fixture(scope="module")
def model2():
    """Two 30B-shaped layers (layer 0 with Q6_K attn_v / ffn_down_exps, layer
    1 all Q4_K), vocab 512."""
    t = synth._k_types(attn=12, down=12, out=14, embd=12)
    spec = synth.Spec(2048, 2, 32, 4, 128, 128, 8, 768, 512, 512, types=t, more_bits_type=14, seed=11)
    img = synth.build_image(spec, threads=min(16, os.cpu_count() or 1))
    return spec, img


def router_gap(logits, top):
    """Gap between the top-th and (top+1)-th router logit, relative to the
    largest |logit|: a decision whose gap sits inside the prefill's fp16
    noise may legitimately go the other way."""
    r = np.sort(logits)[::-1]
    return float(r[top - 1] - r[top]) / float(np.max(np.abs(r)))


def oracle_runs(spec, img, tokens, dev_routes, n_prompt):
    """The oracle over `tokens` twice: (1) routing by itself, recording its
    expert ids and router gaps per (token, layer); (2) routed to the device's
    expert ids (dev_routes[t], the reference's arithmetic with the device's
    routing, so no routing difference is left).  Returns the logits of both
    runs after the prompt and after each later token, the oracle's own routes
    and gaps."""
    threads = min(16, os.cpu_count() or 1)
    own = oracle.Model(oracle.Gguf(img), spec.context, threads=threads)
    forced = oracle.Model(oracle.Gguf(img), spec.context, threads=threads)
    lo, lf, routes, gaps = [], [], [], []
    for i, t in enumerate(tokens):
        want = i >= n_prompt - 1
        if want:
            lo.append(own.forward(int(t)))
            lf.append(forced.forward(int(t), routes=dev_routes[i]))
        else:
            own.step(int(t))
            forced.step(int(t), routes=dev_routes[i])
        routes.append(own.routes())
        gaps.append([router_gap(own.last_router(l), spec.top) for l in range(spec.layers)])
    return lo, lf, np.stack(routes), np.array(gaps)


def check_routing(dev_routes, ref_routes, gaps, label):
    """Counts the (token, layer) decisions where the device chose another
    expert set than the oracle and attributes each token's first such
    difference to a near-tie of the oracle's router (later layers of that
    token, and later tokens through the KV cache, inherit a changed input, so
    only the first is attributable).  Returns the number of differences."""
    n, layers = ref_routes.shape[:2]
    dis = np.array([[set(dev_routes[t, l]) != set(ref_routes[t, l]) for l in range(layers)] for t in range(n)])
    first = [(t, int(np.argmax(dis[t]))) for t in range(n) if dis[t].any()]
    worst = max((gaps[t, l] for t, l in first), default=0.0)
    print(f"{label}: {int(dis.sum())} of {dis.size} routing decisions differ from the oracle's, "
          f"{len(first)} tokens; largest oracle gap at a first difference {worst:.2e}")
    assert worst <= NEAR_TIE, f"a routing difference at gap {worst:.2e}, not a near-tie"
    return int(dis.sum())


def check_top1(got_id, ref):
    s = np.sort(ref)
    margin = float(s[-1] - s[-2])
    if margin > TOL * float(np.max(np.abs(ref))):
        assert got_id == int(np.argmax(ref))
    return margin


def run_and_check(m, spec, img, prompt, extra, label, prior=()):
    """The device prefills `prompt` (after `prior` tokens already run through
    the exact step) and decodes `extra`; every routing difference from the
    oracle is attributed to a near-tie, and the logits after the prompt
    (bar TOL) and after each decode step (bar 2 TOL) are compared with the
    oracle routed as the device was, whatever flipped.  The greedy id is
    compared with the same run."""
    am, lg = m.prefill(prompt)
    assert m.position == len(prior) + len(prompt)
    assert m.prefill_reruns == 0  # the batched path's fp16 operands held every activation
    dec = [m.forward(int(t)) for t in extra]
    tokens = list(prior) + list(prompt) + list(extra)
    dev_routes = m.route_log(0, len(tokens))
    n_prompt = len(prior) + len(prompt)
    lo, lf, ref_routes, gaps = oracle_runs(spec, img, tokens, dev_routes, n_prompt)
    check_routing(dev_routes, ref_routes, gaps, label)
    err = rel_err(lg, lf[0])
    margin = check_top1(am, lf[0])
    print(f"{label}: last-token logits rel err {err:.2e} (vs the oracle's own routing {rel_err(lg, lo[0]):.2e}), "
          f"top-1 margin {margin:.3e}")
    assert err <= TOL
    for i, (got, ref) in enumerate(zip(dec, lf[1:])):
        e2 = rel_err(got, ref)
        print(f"  decode step {i} after prefill: rel err {e2:.2e}")
        assert e2 <= 2 * TOL


@pytest.mark.parametrize("n", [1, 31, 32, 33, 64, 65, 100, 257])
def test_prefill_matches_oracle(dev, model2, n):
    """Prompt lengths around the 16-query attention blocks and the 64-key
    blocks; then four decode steps on the prefilled KV cache."""
    spec, img = model2
    prompt = np.random.default_rng(n).integers(0, spec.vocab, n).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched
    run_and_check(m, spec, img, prompt, [7, 300, 11, 499], f"n={n}")


@pytest.mark.parametrize("heads,kvheads", [(20, 4), (12, 2), (4, 1)])
def test_prefill_fewer_query_heads_per_kv_head(dev, heads, kvheads):
    """Batched attention with 5, 6 and 4 query heads per KV head (the
    kernel's waves take two heads each, so some hold one head or none) and
    query widths of 2,560, 1,536 and 512: a 257-token prompt (17 query
    blocks, the long blocks' keys split between two workgroups), then two
    decode steps, against the oracle."""
    t = synth._k_types(attn=12, down=12, out=14, embd=12)
    spec = synth.Spec(2048, 2, heads, kvheads, 128, 128, 8, 768, 512, 512, types=t, more_bits_type=14, seed=heads)
    img = synth.build_image(spec, threads=min(16, os.cpu_count() or 1))
    prompt = np.random.default_rng(heads).integers(0, spec.vocab, 257).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched
    run_and_check(m, spec, img, prompt, [7, 300], f"{heads} query heads over {kvheads} KV heads")


@pytest.mark.parametrize("main,out", [(synth.Q4_0, synth.Q4_0), (synth.Q8_0, synth.Q8_0),
                                      (synth.Q5_K, synth.Q5_K), (synth.Q6_K, synth.Q4_K)])
def test_prefill_main_formats(dev, main, out):
    """The batched path's other weight formats (Q4_0, Q8_0, Q5_K, Q6_K
    projections dequantised in the GEMM tiles): two 30B-shaped layers, the
    second with Q6_K v/down; a 65-token prompt, then two decode steps."""
    t = synth._k_types(attn=main, down=main, out=out, embd=main)
    spec = synth.Spec(2048, 2, 32, 4, 128, 128, 8, 768, 512, 512, types=t, more_bits_type=synth.Q6_K, seed=12)
    img = synth.build_image(spec, threads=min(16, os.cpu_count() or 1))
    prompt = np.random.default_rng(65).integers(0, spec.vocab, 65).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched
    run_and_check(m, spec, img, prompt, [7, 300], f"kind {main}")


def test_prefill_chunks_match_one_pass(dev, model2, monkeypatch):
    """A 150-token prompt in chunks of 64 (attention over the cached earlier
    chunks) against the oracle."""
    spec, img = model2
    prompt = np.random.default_rng(150).integers(0, spec.vocab, 150).astype(np.uint32)
    monkeypatch.setenv("QH_PREFILL_CHUNK", "64")
    m = engine.Model(img, spec.context, device=dev)
    run_and_check(m, spec, img, prompt, [5], "150 tokens in chunks of 64")


def test_prefill_continues_a_sequence(dev, model2):
    """Prefill from a nonzero position: 20 tokens through the exact decode
    path, then 40 more batched."""
    spec, img = model2
    prompt = np.random.default_rng(60).integers(0, spec.vocab, 60).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    m.generate(prompt[:20], 0)
    assert m.position == 20
    run_and_check(m, spec, img, prompt[20:], [9], "20 + 40 tokens", prior=prompt[:20])


def test_prefill_release_rebuilds_the_same_bits(dev, model2):
    """qh_prefill_release frees the tile-layout weight copy and the chunk
    buffers; a prefill after it (from position 0, and continuing a sequence
    whose earlier 65 positions sit only in the KV cache) gives the bits of a
    run that never released, and so does the decode step that follows."""
    spec, img = model2
    prompt = np.random.default_rng(100).integers(0, spec.vocab, 100).astype(np.uint32)
    ref = engine.Model(img, spec.context, device=dev)
    ra0, rl0 = ref.prefill(prompt[:65])
    ra1, rl1 = ref.prefill(prompt[65:])
    rnext = ref.forward(ra1)

    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_bytes == 0
    m.prefill(prompt[:65])
    held = m.prefill_bytes
    assert held > 0
    m.prefill_release()
    assert m.prefill_bytes == 0 and m.position == 65
    m.reset()
    a0, l0 = m.prefill(prompt[:65])
    assert m.prefill_bytes == held
    m.prefill_release()
    m.prefill_release()  # idempotent
    a1, l1 = m.prefill(prompt[65:])
    assert (a0, a1) == (ra0, ra1)
    assert np.array_equal(l0, rl0) and np.array_equal(l1, rl1)
    m.prefill_release()
    assert np.array_equal(m.forward(a1), rnext)
    assert m.position == 101


def test_prefill_uncovered_model_runs_the_exact_step(dev):
    """head_dim 16 with F32 weights (the reference's fixture model) is outside
    the batched path: the prompt then runs through the exact token step on the
    device, so the logits, the greedy id, the position and the decode that
    follows equal a stepwise forward bit for bit."""
    from helpers import GOLDEN
    path = os.path.join(GOLDEN, "tiny-qwen3moe.gguf")
    m = engine.Model(path, 8, device=dev)
    assert not m.prefill_batched
    prompt = np.array([1, 5, 2, 9], np.uint32)
    am, lg = m.prefill(prompt)
    assert m.position == 4
    assert am == int(np.argmax(lg))
    nxt = m.forward(am)
    ref = engine.Model(path, 8, device=dev)
    for t in prompt:
        ref_lg = ref.forward(int(t))
    assert np.array_equal(lg, ref_lg)
    assert np.array_equal(nxt, ref.forward(int(np.argmax(ref_lg))))


def test_prefill_odd_query_width_runs_the_exact_step(dev):
    """Two query heads (query width 256): the o-projection's two column halves
    would not be whole super-blocks, so the batched path leaves the model to
    the exact token step (bit-equal to a stepwise forward) instead of failing."""
    spec = synth.Spec(256, 1, 2, 1, 128, 8, 2, 256, 256, 64, types=synth._k_types(), seed=5)
    img = synth.build_image(spec)
    prompt = np.random.default_rng(3).integers(0, spec.vocab, 9).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    assert not m.prefill_batched
    am, lg = m.prefill(prompt)
    assert m.position == 9
    ref = engine.Model(img, spec.context, device=dev)
    for t in prompt:
        ref_lg = ref.forward(int(t))
    assert np.array_equal(lg, ref_lg)
    assert am == int(np.argmax(ref_lg))


def test_prefill_errors_roll_back_like_forward(dev, model2):
    """qh_prefill fails as the reference's loop of forwards would
    (src/model.rs:209-223): the first prompt token past the context limit
    gives "context limit N reached", a token outside the vocabulary "token
    outside vocabulary" (also when a later token would overflow the context),
    and every failure leaves a clean cache at position 0, so the next prefill
    gives the bits of a first run."""
    spec, img = model2
    m = engine.Model(img, spec.context, device=dev)
    prompt = np.random.default_rng(33).integers(0, spec.vocab, 33).astype(np.uint32)
    am0, lg0 = m.prefill(prompt)
    with pytest.raises(engine.EngineError, match=f"context limit {spec.context} reached"):
        m.prefill(np.zeros(spec.context, np.uint32))  # 33 + 512 tokens
    assert m.position == 0
    bad = prompt.copy()
    bad[5] = spec.vocab
    with pytest.raises(engine.EngineError, match="token outside vocabulary"):
        m.prefill(bad)
    assert m.position == 0
    over = np.zeros(spec.context + 1, np.uint32)
    over[7] = spec.vocab  # the vocabulary check of token 7 comes before the overflow at token 512
    with pytest.raises(engine.EngineError, match="token outside vocabulary"):
        m.prefill(over)
    assert m.position == 0
    am1, lg1 = m.prefill(prompt)
    assert am1 == am0 and np.array_equal(lg1, lg0)
    assert m.position == len(prompt)


def test_prefill_beyond_fp16_range_reruns_exactly(dev):
    """RMSNorm weights of 4e4 put the normalised activations far beyond the
    fp16 range of the batched path's operands (|x| <= 65504): the prefill
    notices (an fp16 range flag at every activation it converts), runs the
    prompt again through the exact FP32 token step and counts it, so the
    logits, the greedy id and the decode step that follows equal a stepwise
    forward bit for bit."""
    t = synth._k_types(attn=12, down=12, out=14, embd=12)
    spec = synth.Spec(2048, 2, 32, 4, 128, 128, 8, 768, 512, 64, types=t, more_bits_type=14, seed=13,
                      norm_mean=4e4)
    img = synth.build_image(spec, threads=min(16, os.cpu_count() or 1))
    prompt = np.random.default_rng(21).integers(0, spec.vocab, 21).astype(np.uint32)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched and m.prefill_reruns == 0
    am, lg = m.prefill(prompt)
    assert m.prefill_reruns == 1
    assert m.position == len(prompt)
    assert np.all(np.isfinite(lg)) and float(np.max(np.abs(lg))) > 0
    nxt = m.forward(am)
    ref = engine.Model(img, spec.context, device=dev)  # replaces m on this device
    for tok in prompt:
        ref_lg = ref.forward(int(tok))
    assert np.array_equal(lg, ref_lg)
    assert am == int(np.argmax(ref_lg))
    assert np.array_equal(nxt, ref.forward(am))
