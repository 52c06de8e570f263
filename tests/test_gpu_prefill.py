"""GPU parity of the batched prefill (qh_prefill: fp16 matrix-core GEMMs and
flash attention in place of the reference's one-forward-per-token prompt
loop, src/main.rs:250-256) against the FP32 oracle's sequential forward.
fp16 operands cannot meet the decode path's 1e-4, so the bar is the logits
of the last prompt token within 1e-2 (infinity-norm relative) and the same
greedy id unless the oracle's top-1/top-2 margin is inside that tolerance;
the decode steps that follow must stay within 2e-2."""
import importlib
import os

import numpy as np
import pytest

import oracle

engine = importlib.import_module("qwen-30brust_amd")
synth = importlib.import_module("qwen-30brust_amd.synth")

pytestmark = pytest.mark.gpu
TOL = 1e-2


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


def router_gap(om, spec):
    """Smallest relative gap between the top-th and (top+1)-th router logit
    over the layers of the oracle's last forward: a gap inside the prefill's
    fp16 noise lets the device pick another expert for that token."""
    gaps = []
    for layer in range(spec.layers):
        r = np.sort(om.last_router(layer))[::-1]
        gaps.append(float(r[spec.top - 1] - r[spec.top]) / float(np.max(np.abs(r))))
    return min(gaps)


def oracle_logits(spec, img, prompt, extra=()):
    """Oracle logits after the prompt (and after each extra token), and the
    last prompt token's smallest router gap."""
    om = oracle.Model(oracle.Gguf(img), spec.context, threads=min(16, os.cpu_count() or 1))
    for t in prompt:
        ref = om.forward(int(t))
    gap = router_gap(om, spec)
    out = [ref]
    for t in extra:
        out.append(om.forward(int(t)))
    return out, gap


def check_logits(err, gap, tol=TOL):
    """err within tol, or the last prompt token sits on a router near-tie
    (relative gap below 2e-3), where a different expert choice is the fp16
    path's legitimate outcome."""
    if err > tol:
        assert gap < 2e-3, f"rel err {err:.2e} without a router near-tie (smallest gap {gap:.2e})"


def check_top1(got_id, ref):
    s = np.sort(ref)
    margin = float(s[-1] - s[-2])
    if margin > TOL * float(np.max(np.abs(ref))):
        assert got_id == int(np.argmax(ref))
    return margin


@pytest.mark.parametrize("n", [1, 31, 32, 33, 64, 65, 100, 257])
def test_prefill_matches_oracle(dev, model2, n):
    """Prompt lengths around the 32-query attention blocks and the 64-key
    blocks; then four decode steps on the prefilled KV cache."""
    spec, img = model2
    prompt = np.random.default_rng(n).integers(0, spec.vocab, n).astype(np.uint32)
    extra = [7, 300, 11, 499]
    refs, gap = oracle_logits(spec, img, prompt, extra)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched
    am, lg = m.prefill(prompt)
    err = rel_err(lg, refs[0])
    margin = check_top1(am, refs[0])
    print(f"n={n}: last-token logits rel err {err:.2e}, oracle top-1 margin {margin:.3e}, router gap {gap:.2e}")
    check_logits(err, gap)
    assert m.position == n
    if err <= TOL:
        for t, ref in zip(extra, refs[1:]):
            e2 = rel_err(m.forward(t), ref)
            print(f"  decode after prefill: rel err {e2:.2e}")
            assert e2 <= 2 * TOL


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
    extra = [7, 300]
    refs, gap = oracle_logits(spec, img, prompt, extra)
    m = engine.Model(img, spec.context, device=dev)
    assert m.prefill_batched
    am, lg = m.prefill(prompt)
    err = rel_err(lg, refs[0])
    margin = check_top1(am, refs[0])
    print(f"kind {main}: last-token logits rel err {err:.2e}, oracle top-1 margin {margin:.3e}, router gap {gap:.2e}")
    check_logits(err, gap)
    assert m.position == len(prompt)
    if err <= TOL:
        for t, ref in zip(extra, refs[1:]):
            assert rel_err(m.forward(t), ref) <= 2 * TOL


def test_prefill_chunks_match_one_pass(dev, model2, monkeypatch):
    """A 150-token prompt in chunks of 64 (attention over the cached earlier
    chunks) against the oracle."""
    spec, img = model2
    prompt = np.random.default_rng(150).integers(0, spec.vocab, 150).astype(np.uint32)
    (ref,), gap = oracle_logits(spec, img, prompt)
    monkeypatch.setenv("QH_PREFILL_CHUNK", "64")
    m = engine.Model(img, spec.context, device=dev)
    am, lg = m.prefill(prompt)
    err = rel_err(lg, ref)
    print(f"150 tokens in chunks of 64: rel err {err:.2e}, router gap {gap:.2e}")
    check_logits(err, gap)
    check_top1(am, ref)


def test_prefill_continues_a_sequence(dev, model2):
    """Prefill from a nonzero position: 20 tokens through the exact decode
    path, then 40 more batched."""
    spec, img = model2
    prompt = np.random.default_rng(60).integers(0, spec.vocab, 60).astype(np.uint32)
    (ref,), gap = oracle_logits(spec, img, prompt)
    m = engine.Model(img, spec.context, device=dev)
    m.generate(prompt[:20], 0)
    assert m.position == 20
    am, lg = m.prefill(prompt[20:])
    assert m.position == 60
    check_logits(rel_err(lg, ref), gap)
    check_top1(am, ref)


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
