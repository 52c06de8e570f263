"""One-turn chat with the model's tokenizer.json: the `chat` command of the
reference binary (src/main.rs:80-105 arguments, :154-290 behaviour) on the
HIP engine.

    python qwen-30brust_amd/chat.py --model M.gguf --tokenizer tokenizer.json \\
        --prompt "hello" [--system S] [--ctx 4096] [--max-tokens 128] \\
        [--temperature 0.2] [--top-k 20] [--top-p 0.8] [--seed 42] [--raw] \\
        [--device hip] [--adapter SUBSTRING]

Tokenisation uses the `tokenizers` library the reference links (0.22.2, the
Rust crate of src/main.rs:169, through its Python binding), so prompts encode
and generated ids decode exactly as in the reference.  The prompt runs as the
reference runs it, one token step per prompt token (`qh_forward`), so the
logits and therefore the sampled ids follow the FP32 step; sampling, the
padding-vocab mask and the token steps run on the GPU (`qh_sample`,
`qh_set_valid_tokens`).  Generated text goes to stdout, the statistics JSON
(src/main.rs:283-288) to stderr.  Failures print "Error: <message>" and exit
1; argument errors exit 2.
"""
import argparse
import importlib
import os
import sys
import time

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(PKG_DIR))


class ChatError(RuntimeError):
    pass


def ensure(cond, msg):
    if not cond:
        raise ChatError(msg)


def parse(argv):
    ap = argparse.ArgumentParser(prog="chat", description="One-turn chat with the original tokenizer.json.")
    ap.add_argument("--model", required=True)
    ap.add_argument("--tokenizer", required=True)
    ap.add_argument("--prompt", required=True)
    ap.add_argument("--system", default="You are a helpful coding assistant.")
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--max-tokens", type=int, default=128)
    ap.add_argument("--temperature", type=float, default=0.2)
    ap.add_argument("--top-k", type=int, default=20)
    ap.add_argument("--top-p", type=float, default=0.8)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--raw", action="store_true", help="Encode the prompt directly, without ChatML wrappers.")
    ap.add_argument("--device", choices=["hip", "vulkan", "cpu"], default="hip")
    ap.add_argument("--gpu-cache-mib", type=int, default=4096)
    ap.add_argument("--adapter")
    ap.add_argument("--allow-software", action="store_true")
    a = ap.parse_args(argv)
    if a.ctx < 0 or a.max_tokens < 0 or a.top_k < 0 or a.seed < 0 or a.gpu_cache_mib < 0:
        ap.error("sizes and the seed are unsigned integers")
    return a


def encode_prompt(tok, a):
    """Token ids of the prompt: raw, or the ChatML turn (src/main.rs:191-220)."""
    if a.raw:
        return tok.encode(a.prompt, add_special_tokens=False).ids
    ensure(tok.token_to_id("<|im_start|>") is not None, "missing ChatML im_start token")
    ensure(tok.token_to_id("<|im_end|>") is not None, "missing ChatML im_end token")
    # untrusted content is encoded on its own; model control tokens are refused
    special = {i for i, t in tok.get_added_tokens_decoder().items() if t.special}
    for content in (a.system, a.prompt):
        body = tok.encode(content, add_special_tokens=False)
        ensure(not any(i in special for i in body.ids),
               "prompt/system contains reserved special tokens; use --raw for exact tokenized inputs")
    chat = (f"<|im_start|>system\n{a.system}<|im_end|>\n<|im_start|>user\n{a.prompt}<|im_end|>\n"
            "<|im_start|>assistant\n")
    return tok.encode(chat, add_special_tokens=False).ids


def run(argv, out=sys.stdout, err=sys.stderr):
    a = parse(argv)
    from tokenizers import Tokenizer
    from tokenizers.decoders import DecodeStream

    gguf_meta = importlib.import_module("qwen-30brust_amd.gguf_meta")
    json_text = importlib.import_module("qwen-30brust_amd.json_text")
    ensure(a.max_tokens > 0, "max-tokens must be positive")
    try:
        tok = Tokenizer.from_file(a.tokenizer)
    except Exception as e:  # the library's message, as src/main.rs:169-170 passes it on
        raise ChatError(f"tokenizer: {e}")
    meta = gguf_meta.read_metadata(a.model)
    # token-id identity against the GGUF token table, not the vocabulary size alone
    table = meta.get("tokenizer.ggml.tokens")
    ensure(isinstance(table, list), "GGUF has no token table")
    ensure(tok.get_vocab_size(True) <= len(table), "tokenizer vocabulary exceeds GGUF")
    for text, i in tok.get_vocab(True).items():
        ensure(i < len(table) and table[i] == text, f"tokenizer differs from GGUF at token {i}")
    # the embedding may be padded beyond the tokenizer's vocabulary
    valid = np.array([tok.id_to_token(i) is not None for i in range(len(table))], np.uint8)
    ids = encode_prompt(tok, a)
    ensure(len(ids) > 0 and len(ids) + a.max_tokens <= a.ctx,
           "prompt + max-tokens exceed --ctx; reduce the prompt or generation length")
    stops = []
    eos = meta.get("tokenizer.ggml.eos_token_id")
    if isinstance(eos, int):
        stops.append(eos)
    for t in ("<|im_end|>", "<|endoftext|>"):
        i = tok.token_to_id(t)
        if i is not None:
            stops.append(i)
    ensure(stops, "no EOS token found")

    engine = importlib.import_module("qwen-30brust_amd")
    try:
        sampler = engine.Sampler(a.seed, a.temperature, a.top_k, a.top_p)
    except engine.EngineError as e:
        raise ChatError(str(e))
    ensure(a.device != "cpu", "the cpu device is not part of this engine; use --device hip")
    names = engine.devices()
    ensure(names, "no HIP device found")
    dev_i = 0
    if a.adapter is not None:
        match = [i for i, n in enumerate(names) if a.adapter in n]
        ensure(match, f"no HIP device matches adapter '{a.adapter}'")
        dev_i = match[0]
    dev = engine.Device(dev_i)
    model = engine.Model(a.model, a.ctx, device=dev)
    ensure(len(valid) == model.config["vocab"], "GGUF token table length differs from the vocabulary")
    kv = a.ctx * model.config["layers"] * model.config["kvheads"] * model.config["head_dim"] * 8
    print(f"KV cache maximum: {kv / 1048576:.1f} MiB (FP32, GPU HBM)", file=err)
    print(f"HIP device: {names[dev_i]}", file=err)
    model.set_valid_tokens(valid)

    start = time.perf_counter()
    for n, t in enumerate(ids):
        model.forward(t, want_logits=False)
        print(f"\rPrefill {n + 1}/{len(ids)}", end="", file=err, flush=True)
    prefill_seconds = time.perf_counter() - start
    print(file=err)
    decode = time.perf_counter()
    count = 0
    stream = DecodeStream(skip_special_tokens=True)
    for i in range(a.max_tokens):
        nxt = model.sample(sampler)
        if nxt in stops:
            break
        text = stream.step(tok, nxt)
        if text is not None:
            out.write(text)
            out.flush()
        count += 1
        if i + 1 < a.max_tokens:
            model.forward(nxt, want_logits=False)
    print(file=out)
    s = engine._Stats()
    engine.lib().qh_stats(dev.h, engine.C.byref(s))
    stats = {n: getattr(s, n) for n, _ in engine._Stats._fields_}
    report = {"prompt_tokens": len(ids), "generated_tokens": count, "prefill_seconds": prefill_seconds,
              "generation_seconds": time.perf_counter() - decode, "stats": stats,
              "note": "timings include orchestration and host round trips per token; not a pure GPU benchmark"}
    print(json_text.dumps(report, pretty=True), file=err)
    return 0


def main(argv=None):
    try:
        return run(sys.argv[1:] if argv is None else argv)
    except SystemExit:
        raise
    except Exception as e:  # anyhow's "Error: ..." on the way out of main
        msg = str(e)
        if type(e).__name__ == "EngineError" or isinstance(e, (ChatError, ValueError, OSError)):
            print(f"Error: {msg}", file=sys.stderr)
        else:
            print(f"Error: {type(e).__name__}: {msg}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
