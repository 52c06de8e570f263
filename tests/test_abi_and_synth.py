"""CPU checks: the C-ABI library loads and exports every symbol the public
header declares (no compute calls), and the synthetic-model generator emits
GGUF images the reference reader's rules accept, at the shapes and byte
totals of the real Qwen3-30B-A3B Q4_K_M file."""
import ctypes
import importlib
import json
import os
import re

import numpy as np
import pytest

import oracle
from helpers import GOLDEN, ROOT, np_dequant

synth = importlib.import_module("qwen-30brust_amd.synth")
engine = importlib.import_module("qwen-30brust_amd")


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "qwen_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qh_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 20
    lib = ctypes.CDLL(engine.LIB_PATH)
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # the Python mirror binds exactly the declared surface
    assert set(engine._SIGS) == set(syms)


def test_create_fails_loudly_without_gfx950():
    """No silent CPU fallback (src/main.rs:36): without a GPU, creating a
    context must fail with a message, not degrade."""
    if os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"):
        pytest.skip("a GPU may be present")
    with pytest.raises(engine.EngineError):
        engine.Device(0)


def test_qwen30b_layout_reproduces_real_file_bytes():
    with open(os.path.join(GOLDEN, "real-header-inspection.json")) as f:
        real = json.load(f)
    spec = synth.qwen30b()
    assert synth.packed_bytes(spec) == real["packed_weight_bytes"] == 18_550_716_416
    c = real["config"]
    assert (spec.hidden, spec.layers, spec.heads, spec.kvheads, spec.head_dim, spec.experts,
            spec.top, spec.ff, spec.vocab) == (c["hidden"], c["layers"], c["heads"], c["kvheads"],
                                               c["head_dim"], c["experts"], c["top"],
                                               c["intermediate"], c["vocab"])
    # FP32 KV at ctx 4096 (src/model.rs:150-156): ctx*layers*kvheads*d*8
    assert 4096 * spec.layers * spec.kvheads * spec.head_dim * 8 == real["kv_f32_bytes_at_context"]


@pytest.mark.parametrize("make", [synth.tiny_k, synth.tiny_lit])
def test_tiny_images_parse_and_run_on_oracle(make):
    spec = make()
    img = synth.build_image(spec, threads=4)
    g = oracle.Gguf(img)
    assert g.tensor_count() == 12 * spec.layers + 3
    m = oracle.Model(g, 16)
    c = m.config
    assert (c["hidden"], c["heads"], c["kvheads"], c["head_dim"], c["experts"], c["top"],
            c["intermediate"], c["vocab"]) == (spec.hidden, spec.heads, spec.kvheads,
                                               spec.head_dim, spec.experts, spec.top, spec.ff,
                                               spec.vocab)
    lg = m.forward(3)
    assert np.isfinite(lg).all() and lg.std() > 0
    assert g.packed_bytes() == synth.packed_bytes(spec)


def test_image_is_deterministic_across_thread_counts():
    spec = synth.tiny_k(seed=11)
    a = synth.build_image(spec, threads=1)
    b = synth.build_image(spec, threads=7)
    assert np.array_equal(a, b)
    c = synth.build_image(synth.tiny_k(seed=12), threads=3)
    assert not np.array_equal(a, c)


def test_more_bits_rule_types():
    """llama.cpp's Q4_K_M upgrade of attn_v / ffn_down_exps: layers < L/8,
    >= 7L/8, or (i - L/8) % 3 == 2 (24 of 48 layers)."""
    spec = synth.qwen30b(layers=48)
    spec.hidden, spec.heads, spec.kvheads, spec.head_dim = 256, 2, 1, 128
    spec.experts, spec.top, spec.ff, spec.vocab, spec.context = 2, 1, 256, 32, 8
    g = oracle.Gguf(synth.build_image(spec, threads=8))
    upgraded = [i for i in range(48) if g.tensor(f"blk.{i}.attn_v.weight")["kind"] == 14]
    assert upgraded == [i for i in range(48) if i < 6 or i >= 42 or (i - 6) % 3 == 2]
    assert len(upgraded) == 24
    for i in range(48):
        assert g.tensor(f"blk.{i}.ffn_down_exps.weight")["kind"] == (14 if i in upgraded else 12)
    assert g.tensor("output.weight")["kind"] == 14
    assert g.tensor("blk.0.ffn_gate_inp.weight")["kind"] == 0


@pytest.mark.parametrize("kind,tol", [(2, 0.2), (8, 0.01), (12, 0.12), (13, 0.06), (14, 0.04)])
def test_quantizer_round_trip(kind, tol):
    x = synth.normal(5, 8 * 512).reshape(8, 512) * 0.02
    q = synth.quantize(kind, x)
    back = np_dequant(q, kind, 512)
    rel = np.sqrt(np.mean((back - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel < tol, rel
    # every field is exercised: high scale bits, Q5_K qh, negative Q6_K scales
    if kind in (12, 13):
        assert (q.reshape(8, 2, -1)[:, :, 4:8] >> 6).any()
    if kind == 14:
        assert (q.reshape(8, 2, 210)[:, :, 192:208].view(np.int8) < 0).any()
