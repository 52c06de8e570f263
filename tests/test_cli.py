"""The qwen-hip command-line driver: the `inspect` / `logits` commands and JSON
outputs of the reference binary (src/main.rs:112-153), driven the way
tools/reference_fixture.py:123-131 drives the reference."""
import decimal
import importlib
import json
import math
import os
import struct
import subprocess

import numpy as np
import pytest

from helpers import GOLDEN, ROOT

synth = importlib.import_module("qwen-30brust_amd.synth")
PKG = os.path.join(ROOT, "qwen-30brust_amd")
CLI = os.path.join(PKG, "qwen-hip")
FIXTURE = os.path.join(GOLDEN, "tiny-qwen3moe.gguf")

needs_cli = pytest.mark.skipif(not os.path.exists(CLI), reason="qwen-hip not built (run __graft_entry__.build())")


def run(*args):
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=300)


@pytest.fixture(scope="module")
def header_30b(tmp_path_factory):
    """Header of the Qwen3-30B-A3B Q4_K_M layout at the real file's metadata
    (context_length 262144, rope theta 1e7), extended to the full 18.55 GB
    as a sparse file."""
    spec = synth.qwen30b(context=262144)
    spec.theta = 1e7
    path = tmp_path_factory.mktemp("h30b") / "qwen30b-header.gguf"
    synth.write_header_only(spec, str(path))
    return path


@needs_cli
def test_inspect_matches_reference_output_for_30b_header(header_30b):
    # validation/real-header-inspection.json is the reference binary's stdout
    # for the real model file at the default --ctx 4096
    r = run("inspect", "--model", header_30b)
    assert r.returncode == 0, r.stderr
    with open(os.path.join(GOLDEN, "real-header-inspection.json")) as f:
        assert r.stdout == f.read()


@needs_cli
def test_inspect_context_and_file_errors(header_30b, tmp_path):
    r = run("inspect", "--model", header_30b, "--ctx", 262145)
    assert r.returncode == 1 and r.stderr.strip() == "Error: invalid context"
    r = run("inspect", "--model", header_30b, "--ctx", 0)
    assert r.returncode == 1 and "invalid context" in r.stderr
    r = run("inspect", "--model", FIXTURE, "--ctx=16")
    assert r.returncode == 0
    out = json.loads(r.stdout)
    assert out["kv_f32_bytes_at_context"] == 16 * 2 * 2 * 4 * 8
    assert out["tensor_count"] == 27 and out["config"]["vocab"] == 16
    # a truncated file fails with the reference's message (src/gguf.rs:183)
    bad = tmp_path / "cut.gguf"
    bad.write_bytes(open(FIXTURE, "rb").read()[:-64])
    r = run("inspect", "--model", bad)
    assert r.returncode == 1 and "truncated tensor" in r.stderr
    r = run("inspect", "--model", tmp_path / "missing.gguf")
    assert r.returncode == 1 and r.stderr.startswith("Error: open ")


@needs_cli
def test_argument_errors():
    assert run().returncode == 2
    assert run("bogus").returncode == 2
    assert run("inspect").returncode == 2  # --model is required
    assert run("logits", "--model", FIXTURE).returncode == 2  # --tokens is required
    assert run("logits", "--model", FIXTURE, "--tokens", "1,x").returncode == 2
    assert run("logits", "--model", FIXTURE, "--tokens", "1", "--device", "tpu").returncode == 2
    assert run("inspect", "--model", FIXTURE, "--tokens", "1").returncode == 2
    r = run("logits", "--model", FIXTURE, "--tokens", "1,2,3", "--ctx", "2")
    assert r.returncode == 1 and r.stderr.strip() == "Error: tokens exceed context"
    # no CPU fallback: the cpu device is refused before any work
    r = run("logits", "--model", FIXTURE, "--tokens", "1", "--device", "cpu")
    assert r.returncode == 1 and "cpu device is not part of this engine" in r.stderr
    assert run("--version").stdout.startswith("qwen-hip ")


# ------------------------------------------------------------ JSON numbers --

def serde_layout(v):
    """serde_json's f64 text from Python's shortest round-trip digits (repr,
    David Gay's algorithm: an implementation independent of the engine's)."""
    if not math.isfinite(v):
        return "null"
    sign = "-" if math.copysign(1.0, v) < 0 else ""
    if v == 0:
        return sign + "0.0"
    t = decimal.Decimal(repr(abs(v))).as_tuple()
    digits = "".join(map(str, t.digits)).lstrip("0")
    k = t.exponent + (len(digits) - len(digits.rstrip("0")))
    digits = digits.rstrip("0")
    n = len(digits)
    kk = n + k
    if 0 <= k and kk <= 16:
        return sign + digits + "0" * k + ".0"
    if 0 < kk <= 16:
        return sign + digits[:kk] + "." + digits[kk:]
    if -5 < kk <= 0:
        return sign + "0." + "0" * (-kk) + digits
    return sign + digits[0] + ("." + digits[1:] if n > 1 else "") + "e" + str(kk - 1)


# outputs documented for serde_json / ryu (and the two in the reference's
# validation/real-header-inspection.json)
KNOWN = [(1.0, "1.0"), (0.3, "0.3"), (-0.0, "-0.0"), (0.0, "0.0"), (1e-7, "1e-7"), (1e23, "1e23"),
         (1e16, "1e16"), (1e15, "1000000000000000.0"), (1e-5, "0.00001"), (1.5e-5, "0.000015"),
         (1e-6, "1e-6"), (123456.789, "123456.789"), (1.7976931348623157e308, "1.7976931348623157e308"),
         (2.2250738585072014e-308, "2.2250738585072014e-308"), (5e-324, "5e-324"),
         (1234567890123456789.0, "1.2345678901234568e18"), (float(np.float32(1e-6)), "9.999999974752427e-7"),
         (float(np.float32(1e7)), "10000000.0"), (float("nan"), "null"), (float("inf"), "null")]

DRIVER = r'''
#include <cstdio>
#include <cstring>
#include <cstdint>
#include "json_fmt.hpp"
int main() {
    unsigned long long b;
    while (std::scanf("%llx", &b) == 1) {
        double v;
        std::memcpy(&v, &b, 8);
        std::printf("%s\n", qh::json_f64(v).c_str());
    }
    return 0;
}
'''


def test_json_number_layout(tmp_path):
    src = tmp_path / "fmt.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "fmt"
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", os.path.join(PKG, "csrc"), str(src), "-o", str(exe)],
                   check=True)
    rng = np.random.default_rng(11)
    f32 = np.concatenate([(rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 9, 3000)).astype(np.float32),
                          np.frombuffer(rng.integers(0, 2**32, 2000, dtype=np.uint64).astype(np.uint32).tobytes(),
                                        np.float32)])
    vals = [v for v, _ in KNOWN] + [float(x) for x in f32] + \
        [struct.unpack("<d", struct.pack("<Q", int(b)))[0] for b in rng.integers(0, 2**63, 2000, dtype=np.uint64)]
    inp = "\n".join("%x" % struct.unpack("<Q", struct.pack("<d", v))[0] for v in vals) + "\n"
    out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True).stdout.split("\n")
    for (v, want), got in zip(KNOWN, out):
        assert got == want, (v, got, want)
    for v, got in zip(vals, out):
        assert got == serde_layout(v), (v, got)
        if got != "null":
            assert float(got) == v or (v != v)


# ------------------------------------------------------------------ GPU ----

@pytest.mark.gpu
@needs_cli
@pytest.mark.parametrize("device", ["hip", "vulkan"])
def test_logits_prefixes_match_reference_fixture(device):
    """tools/reference_fixture.py:123-131 against this binary: every prefix of
    [1, 5, 2, 9] at --ctx 16, rtol 2e-4 / atol 2e-5 against the NumPy
    reference's expected-logits.json."""
    with open(os.path.join(GOLDEN, "expected-logits.json")) as f:
        expected = json.load(f)
    tokens = [1, 5, 2, 9]
    for n in range(1, len(tokens) + 1):
        r = run("logits", "--model", FIXTURE, "--tokens", ",".join(map(str, tokens[:n])), "--ctx", 16,
                "--device", device)
        assert r.returncode == 0, r.stderr
        out = json.loads(r.stdout)
        assert sorted(out) == ["logits", "seconds", "stats"]
        np.testing.assert_allclose(np.array(out["logits"]), expected[n - 1], rtol=2e-4, atol=2e-5)
        st = out["stats"]
        assert sorted(st) == ["cache_hits", "matvec_ms", "matvecs", "uploaded_bytes"]
        # per token: q, k, v, o, router and 3 per routed expert in each of 2
        # layers, then the vocab projection (src/model.rs:230-295)
        assert st["matvecs"] == n * (2 * (5 + 3 * 2) + 1)
        assert out["seconds"] > 0
        # the logits are written as f32 values widened to f64
        assert all(float(np.float32(v)) == v for v in out["logits"])


@pytest.mark.gpu
@needs_cli
def test_devices_and_adapter_selection():
    r = run("devices")
    assert r.returncode == 0 and "gfx950" in r.stdout
    r = run("logits", "--model", FIXTURE, "--tokens", "1", "--ctx", 16, "--adapter", "no-such-adapter")
    assert r.returncode == 1 and "no HIP device matches adapter" in r.stderr
    r = run("logits", "--model", FIXTURE, "--tokens", "1", "--ctx", 16, "--adapter", "gfx950")
    assert r.returncode == 0, r.stderr


def test_python_inspect_matches_reference_output(header_30b):
    engine = importlib.import_module("qwen-30brust_amd")
    with open(os.path.join(GOLDEN, "real-header-inspection.json")) as f:
        want = json.load(f)
    got = engine.inspect(header_30b)
    got["config"] = {k: (float(np.float32(v)) if k in ("eps", "theta") else v) for k, v in got["config"].items()}
    assert got == want
    with pytest.raises(engine.EngineError, match="invalid context"):
        engine.inspect(header_30b, 0)
