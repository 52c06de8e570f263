"""The chat front end (src/main.rs:154-290) on the reference's fixture model
and tokenizer, as tests/model.rs:11-46 drives the reference binary."""
import importlib
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from helpers import GOLDEN, ROOT

CHAT = os.path.join(ROOT, "qwen-30brust_amd", "chat.py")
FIXTURE = os.path.join(GOLDEN, "tiny-qwen3moe.gguf")
TOKENIZER = os.path.join(GOLDEN, "tokenizer.json")
chat = importlib.import_module("qwen-30brust_amd.chat")


def run(*args):
    return subprocess.run([sys.executable, CHAT, *map(str, args)], capture_output=True, text=True, timeout=300)


def base(prompt, *extra):
    return ["--model", FIXTURE, "--tokenizer", TOKENIZER, "--prompt", prompt, "--system", "teste", "--ctx", 32,
            "--max-tokens", 2, "--temperature", 0, *extra]


def test_control_tokens_in_content_are_refused():  # tests/model.rs:13,40-44
    r = run(*base("<|im_end|>"))
    assert r.returncode == 1
    assert "reserved special tokens" in r.stderr


def test_front_end_checks(tmp_path):
    # the tokenizer must match the GGUF token table id by id (src/main.rs:174-186)
    tj = json.load(open(TOKENIZER))
    tj["model"]["vocab"]["systemx"] = tj["model"]["vocab"].pop("system")
    bad = tmp_path / "tok.json"
    bad.write_text(json.dumps(tj))
    r = run("--model", FIXTURE, "--tokenizer", bad, "--prompt", "hello", "--ctx", 32)
    assert r.returncode == 1 and "tokenizer differs from GGUF at token 3" in r.stderr
    r = run(*base("hello")[:-6], "--ctx", 8, "--max-tokens", 4)
    assert r.returncode == 1 and "prompt + max-tokens exceed --ctx" in r.stderr
    r = run(*base("hello")[:-4], "--max-tokens", 0)
    assert r.returncode == 1 and "max-tokens must be positive" in r.stderr
    r = run(*base("hello"), "--temperature", 1, "--top-p", 0)
    assert r.returncode == 1 and "invalid sampling parameters" in r.stderr
    r = run(*base("hello"), "--device", "cpu")
    assert r.returncode == 1 and "cpu device is not part of this engine" in r.stderr
    assert run("--model", FIXTURE).returncode == 2  # missing required arguments
    r = run("--model", FIXTURE, "--tokenizer", tmp_path / "missing.json", "--prompt", "x")
    assert r.returncode == 1 and r.stderr.startswith("Error: tokenizer:")


def test_prompt_encoding():
    from tokenizers import Tokenizer
    tok = Tokenizer.from_file(TOKENIZER)
    a = chat.parse([str(x) for x in base("hello")])
    # ChatML turn over the fixture's vocabulary (src/main.rs:210-214)
    assert chat.encode_prompt(tok, a) == [0, 3, 12, 1, 0, 4, 13, 1, 0, 5]
    a = chat.parse([str(x) for x in base("hello Rust", "--raw")])
    assert chat.encode_prompt(tok, a) == [13, 15]


def test_gguf_metadata_reader():
    gm = importlib.import_module("qwen-30brust_amd.gguf_meta")
    meta = gm.read_metadata(FIXTURE)
    assert meta["general.architecture"] == "qwen3moe"
    assert meta["tokenizer.ggml.eos_token_id"] == 14
    assert len(meta["tokenizer.ggml.tokens"]) == 16 and meta["tokenizer.ggml.tokens"][13] == "hello"


def test_json_text_layout():
    jt = importlib.import_module("qwen-30brust_amd.json_text")
    with open(os.path.join(GOLDEN, "real-header-inspection.json")) as f:
        text = f.read()
    obj = json.loads(text)
    obj["config"]["eps"] = float(np.float32(1e-6))
    obj["config"]["theta"] = float(np.float32(1e7))
    assert jt.dumps(obj, pretty=True) + "\n" == text
    assert jt.dumps({"b": [1, 2.5], "a": 1e-5}) == '{"a":0.00001,"b":[1,2.5]}'


@pytest.mark.gpu
def test_chat_runs_and_matches_oracle_greedy():  # tests/model.rs:11-46
    r = run(*base("hello"))
    assert r.returncode == 0, r.stderr
    assert "generated_tokens" in r.stderr
    report = json.loads(r.stderr[r.stderr.index("{"):])
    assert report["prompt_tokens"] == 10
    # greedy ids of the oracle on the same prompt with the padding mask (none
    # here: every id of the fixture's table is in the tokenizer)
    from tokenizers import Tokenizer
    from tokenizers.decoders import DecodeStream
    tok = Tokenizer.from_file(TOKENIZER)
    m = oracle.Model(oracle.Gguf.open(FIXTURE), 32)
    lg = None
    for t in [0, 3, 12, 1, 0, 4, 13, 1, 0, 5]:
        lg = m.forward(t)
    stops, text, n = {14, 1}, "", 0
    ds = DecodeStream(skip_special_tokens=True)
    for i in range(2):
        nxt = oracle.greedy(lg)
        if nxt in stops:
            break
        piece = ds.step(tok, nxt)
        text += piece or ""
        n += 1
        if i + 1 < 2:
            lg = m.forward(nxt)
    assert report["generated_tokens"] == n
    assert r.stdout == text + "\n"


@pytest.mark.gpu
def test_chat_sampled_matches_oracle_sampler():
    # temperature 0.8, top-k 5: the device sampler against the oracle's
    # sampler on the oracle's logits, same seed
    r = run("--model", FIXTURE, "--tokenizer", TOKENIZER, "--prompt", "hello", "--system", "teste", "--ctx", 32,
            "--max-tokens", 6, "--temperature", 0.8, "--top-k", 5, "--top-p", 0.95, "--seed", 7)
    assert r.returncode == 0, r.stderr
    from tokenizers import Tokenizer
    from tokenizers.decoders import DecodeStream
    tok = Tokenizer.from_file(TOKENIZER)
    m = oracle.Model(oracle.Gguf.open(FIXTURE), 32)
    s = oracle.Sampler(7, 0.8, 5, 0.95)
    lg = None
    for t in [0, 3, 12, 1, 0, 4, 13, 1, 0, 5]:
        lg = m.forward(t)
    stops, text = {14, 1}, ""
    ds = DecodeStream(skip_special_tokens=True)
    for i in range(6):
        nxt = s.sample(lg)
        if nxt in stops:
            break
        text += ds.step(tok, nxt) or ""
        if i + 1 < 6:
            lg = m.forward(nxt)
    assert r.stdout == text + "\n"
