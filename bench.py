"""Batch-1 decode benchmark of the random-init Qwen3-30B-A3B Q4_K_M token loop
on one MI355X, plus the four single-matvec HBM cases and the CPU baseline.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--prompt 512]

Prints ONE JSON line (rank 0).  A step is one greedy decode token of the full
48-layer model (embedding, 48 decoder layers, vocab projection, argmax), with
all weights, activations and the FP32 KV cache resident in HBM.  Timed: K
steps after a 512-token sequential prefill and W warmup steps, bracketed by
stream synchronisation, measured with HIP events on the engine's stream.
"""
import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def tensor_bytes(model, name, rows_slice=None):
    t = model.tensor(name)
    blk, size = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
                 14: (256, 210)}[t["kind"]]
    rb = t["dims"][0] // blk * size
    rows = t["dims"][1] if len(t["dims"]) > 1 else 1
    return rb * (rows if rows_slice is None else rows_slice)


def algorithmic_bytes(model, pos_avg):
    """Bytes each kernel class must move per decode token: weights read once,
    activation vectors in/out, and the KV history at the average position."""
    c = model.config
    H, L, top, ff, E = c["hidden"], c["layers"], c["top"], c["intermediate"], c["experts"]
    qd, kvd = c["heads"] * c["head_dim"], c["kvheads"] * c["head_dim"]
    b = dict.fromkeys(model.KERNEL_CLASSES, 0.0)
    b["qkv"] = tensor_bytes(model, "token_embd.weight", 1)
    for i in range(L):
        p = f"blk.{i}."
        b["qkv"] += sum(tensor_bytes(model, p + n) for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight")) + 4 * H + 4 * (qd + 2 * kvd)
        b["attention"] += 2 * 4 * kvd * (pos_avg + 1) + 4 * (qd + 2 * kvd) + 4 * qd
        b["oproj"] += tensor_bytes(model, p + "attn_output.weight") + tensor_bytes(model, p + "ffn_gate_inp.weight") + 4 * qd + 8 * H
        b["gateup"] += top * (tensor_bytes(model, p + "ffn_gate_exps.weight", ff) +
                              tensor_bytes(model, p + "ffn_up_exps.weight", ff)) + 4 * H + 4 * top * ff
        b["down"] += top * tensor_bytes(model, p + "ffn_down_exps.weight", H) + 4 * top * ff + 8 * H
    out = "output.weight"
    try:
        model.tensor(out)
    except Exception:
        out = "token_embd.weight"
    b["vocab"] = tensor_bytes(model, out) + 4 * H + 4 * c["vocab"]
    return b


def active_weight_bytes(model):
    """Weight bytes one decode token must read (no activations, no KV): the
    embedding row, every layer's attention matrices, router and norms, the
    routed experts' gate/up/down rows, the final norm and the vocab matrix."""
    c = model.config
    H, top, ff = c["hidden"], c["top"], c["intermediate"]
    w = tensor_bytes(model, "token_embd.weight", 1) + tensor_bytes(model, "output_norm.weight")
    for i in range(c["layers"]):
        p = f"blk.{i}."
        w += sum(tensor_bytes(model, p + n) for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight",
                                                        "attn_output.weight", "ffn_gate_inp.weight",
                                                        "attn_norm.weight", "attn_q_norm.weight",
                                                        "attn_k_norm.weight", "ffn_norm.weight"))
        w += top * (tensor_bytes(model, p + "ffn_gate_exps.weight", ff) + tensor_bytes(model, p + "ffn_up_exps.weight", ff)
                    + tensor_bytes(model, p + "ffn_down_exps.weight", H))
    out = "output.weight"
    try:
        model.tensor(out)
    except Exception:
        out = "token_embd.weight"
    return w + tensor_bytes(model, out)


def prefill_flops(model, n):
    """Algorithmic flops of a batched prefill of n tokens from position 0:
    every projection (q, k, v, o, F32 router, the top experts' gate/up/down)
    as 2 flops per weight per token, causal attention as 4 flops per
    (query, key, head dim) pair over keys 0..t, and the last token's vocab
    projection."""
    c = model.config
    H, L, top, ff, E = c["hidden"], c["layers"], c["top"], c["intermediate"], c["experts"]
    qd, kvd, heads, d = c["heads"] * c["head_dim"], c["kvheads"] * c["head_dim"], c["heads"], c["head_dim"]
    per_tok_layer = 2 * (qd * H + 2 * kvd * H + H * qd + E * H + top * 3 * ff * H)
    attn = heads * (n * (n + 1) / 2) * d * 4
    return L * (n * per_tok_layer + attn) + 2 * c["vocab"] * H


def prefill_executed_flops(model, n, routes):
    """Flops the prefill's fp16 matrix-core instructions execute for n tokens
    from position 0, tile padding included, from the routes [n][layers][top]
    it logged: the dense GEMMs run 128 x 128 tiles over the token rows; an
    expert's gate/up and down GEMMs run its tokens in 128-row tiles, a
    remainder of at most 64 rows as 64; the attention runs 16-query blocks
    against 64-key blocks up to the block's last query.  The F32 router
    (fp32 matrix cores) is counted apart."""
    c = model.config
    H, L, ff, E = c["hidden"], c["layers"], c["intermediate"], c["experts"]
    qd, kvd, heads, d = c["heads"] * c["head_dim"], c["kvheads"] * c["head_dim"], c["heads"], c["head_dim"]
    up = lambda v, m: -(-v // m) * m
    dense = 2 * up(n, 128) * (up(qd + 2 * kvd, 128) * H + up(H, 128) * qd)
    attn = sum(up(min(q0 + 16, n), 64) for q0 in range(0, n, 16)) * 16 * d * 4 * heads
    expert = 0
    for layer in range(L):
        cnt = np.bincount(routes[:, layer, :].ravel(), minlength=E)
        rows = sum(128 * (k // 128) + (0 if k % 128 == 0 else 64 if k % 128 <= 64 else 128) for k in cnt.tolist())
        expert += rows * 2 * 3 * ff * H  # gate, up and down
    return {"fp16": int(L * (dense + attn) + expert), "router_fp32": int(L * 2 * up(n, 64) * E * H)}


def matvec_cases(engine, synth, dev):
    """Single quantized matvecs at 30B-A3B shapes (W ~ N(0,0.02), k-quantized,
    x ~ N(0,1)), rotating over >= 512 MB of distinct weight copies so every
    launch streams from HBM rather than the 256 MB MALL.  Each case reports the
    median of per-launch event timings, the mean of back-to-back launches and
    the back-to-back floor of an empty kernel.  The last case is the hot
    path's batched form: the 8 routed experts' down projections of one layer
    in one launch."""
    cases = [("q_proj 2048->4096 Q4_K", 12, 4096, 2048, 1), ("o_proj 4096->2048 Q4_K", 12, 2048, 4096, 1),
             ("vocab 2048->151936 Q6_K", 14, 151936, 2048, 1), ("expert_down 768->2048 Q6_K", 14, 2048, 768, 1),
             ("expert_down x8 768->2048 Q6_K (one launch)", 14, 2048, 768, 8)]
    out = []
    # the device's practical read ceiling: a plain stream over as many bytes as the vocab matrix
    rd = dev.bench_read(255868416, 2, 200)
    ceil_gbs = 255868416 / (rd["median_ms"] * 1e-3) / 1e9
    out.append({"case": "read-only stream 255,868,416 B (ceiling)", "bytes": 255868416,
                "us_median": round(rd["median_ms"] * 1e3, 3), "GB_s": round(ceil_gbs, 1),
                "frac_of_peak": round(ceil_gbs / HBM_PEAK_GBS, 4)})
    log(f"read-only stream: median {rd['median_ms']*1e3:.2f} us ({ceil_gbs:.0f} GB/s)")
    for i, (name, kind, rows, cols, nvec) in enumerate(cases):
        w = synth.normal(100 + i, nvec * rows * cols, 0.0, 0.02).reshape(nvec * rows, cols)
        data = synth.quantize(kind, w)
        x = synth.normal(200 + i, nvec * cols)
        copies = max(2, int(np.ceil(512e6 / data.size)))
        t = dev.bench_matvec(data, kind, rows, cols, x, copies, 400 if rows < 100000 else 200, nvec=nvec)
        nbytes = data.size + 4 * nvec * (cols + rows)
        gbs = nbytes / (t["median_ms"] * 1e-3) / 1e9
        out.append({"case": name, "bytes": int(nbytes), "us_median": round(t["median_ms"] * 1e3, 3),
                    "us_mean_back_to_back": round(t["mean_ms"] * 1e3, 3),
                    "us_empty_kernel_floor": round(t["empty_ms"] * 1e3, 3),
                    "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                    "frac_of_read_ceiling": round(gbs / ceil_gbs, 4),
                    "GB_s_back_to_back": round(nbytes / (t["mean_ms"] * 1e-3) / 1e9, 1)})
        log(f"matvec {name}: median {t['median_ms']*1e3:.2f} us ({gbs:.0f} GB/s), back-to-back "
            f"{t['mean_ms']*1e3:.2f} us, empty kernel {t['empty_ms']*1e3:.2f} us")
    return out


def measured_traffic(kernel_class, position):
    """HBM bytes per launch of a step kernel class (reads + writes), from the
    committed rocprofv3 PMC summary (FETCH_SIZE / WRITE_SIZE passes scaled by
    a copy of known size).  For the persistent step the summary holds a
    least-squares line over every launch of the profiled run (the KV history
    grows with the position), evaluated here at the position timed; None when
    the summary is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_decode_30b.json")
    try:
        with open(path) as f:
            d = json.load(f)["per_launch"][kernel_class]
        tot = 0.0
        for k in ("read_bytes", "write_bytes"):
            v = d[k]
            tot += v["intercept"] + v["slope"] * position if isinstance(v, dict) else v
        return int(tot)
    except (OSError, KeyError, ValueError, TypeError):
        return None


def cpu_baseline(img, spec, threads_nt, pos):
    """The oracle (C restatement of the reference CPU backend) on this host:
    faithful single-thread per-element decode, as backend.rs:41-48.  Sample:
    layers 0-15 and the vocab projection of one decode token at position
    `pos` (the position the GPU step is timed at) over a seeded N(0,1) KV
    history of `pos` positions, scaled to the 48-layer token.  Also the
    row-threaded oracle (same bits) on one full token at position 0."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    g = oracle.Gguf(img)
    m = oracle.Model(g, 8, threads=0)
    x = g.row("token_embd.weight", 3)
    kvd = spec.kvheads * spec.head_dim
    hist = np.random.default_rng(7).standard_normal((2, pos * kvd)).astype(np.float32)
    n_sample = 16
    t0 = time.time()
    for layer in range(n_sample):
        x, _, _ = m.layer_forward(layer, x, pos, hist[0], hist[1], threads=0)
    t_layers = time.time() - t0
    t0 = time.time()
    m.matvec("output.weight", None, x, threads=0)
    t_vocab = time.time() - t0
    per_token = t_layers * spec.layers / n_sample + t_vocab
    log(f"cpu faithful: {n_sample} layers {t_layers:.1f}s + vocab {t_vocab:.1f}s -> {per_token:.1f} s/token")
    mt = oracle.Model(g, 8, threads=threads_nt)
    t0 = time.time()
    mt.forward(3)
    t_nt = time.time() - t0
    log(f"cpu oracle {threads_nt} threads: {t_nt:.2f} s/token")
    return {"value": round(1.0 / per_token, 5), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"faithful single-thread oracle, one decode token at position {pos} over a seeded KV history: "
                      f"layers 0-{n_sample-1} ({t_layers:.1f} s) + vocab projection ({t_vocab:.1f} s), layers "
                      f"scaled to {spec.layers}",
            "threaded": {"value": round(1.0 / t_nt, 4), "unit": "tok/s", "cores": threads_nt,
                         "sample": "row-threaded oracle (bit-identical), one full decode token at position 0"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--layers", type=int, default=48, help="decoder layers (48 = the real model)")
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--no-per-phase", action="store_true",
                    help="skip the per-phase kernels' comparison line (profiler runs of k_decode alone)")
    ap.add_argument("--prefill", type=int, default=2048,
                    help="tokens of the batched-prefill measurement (0: skip)")
    ap.add_argument("--long-pos", type=int, default=3584,
                    help="also time decode steps from this position, the KV cache filled by a batched "
                         "prefill (0: skip)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a known-size "
                         "kernel that calibrates HBM byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): "
              "batch-1 decode of a model resident in one GPU's HBM has no multi-GPU path here.",
              file=sys.stderr)
        sys.exit(2)
    engine = importlib.import_module("qwen-30brust_amd")
    synth = importlib.import_module("qwen-30brust_amd.synth")
    if args.copy_mb > 0:
        import torch
        n = args.copy_mb << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {n} bytes device to device")
        del src, dst

    alt_warmup, alt_steps = 4, 32
    ctx = args.prompt + args.warmup + args.steps + 2 * args.profile_steps + alt_warmup + alt_steps + 8
    spec = synth.qwen30b(layers=args.layers, context=max(4096, ctx, args.prefill))
    threads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    img = synth.build_image(spec, threads=threads)
    log(f"built {img.size/1e9:.2f} GB GGUF image ({args.layers} layers) in {time.time()-t0:.1f}s")
    dev = engine.Device(0)
    t0 = time.time()
    model = engine.Model(img, spec.context, device=dev)
    log(f"loaded to HBM in {time.time()-t0:.1f}s; packed weight bytes {model.packed_weight_bytes()}")

    rng = np.random.default_rng(512)
    prompt = rng.integers(0, spec.vocab, args.prompt).astype(np.uint32)
    t0 = time.time()
    model.generate(prompt, 1)
    log(f"prefill {args.prompt} tokens (sequential) in {time.time()-t0:.2f}s")
    pos_start = model.position
    ms = model.bench_decode(args.warmup, args.steps)
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    log(f"decode: {ms_per_step:.3f} ms/token, {tok_s:.1f} tok/s")

    persistent = model.persistent
    decode_launch = None
    if persistent:
        # the k_decode launch alone, timed with HIP events on its stream
        ms_embed, ms_decode = model.profile_decode(args.profile_steps)
        decode_launch = {"ms_embed": round(ms_embed, 4), "ms_decode": round(ms_decode, 4)}
        log(f"persistent step: k_decode {ms_decode*1e3:.1f} us per token (embedding row included; "
            f"empty interval before it {ms_embed*1e3:.1f} us)")
    pos_mid = pos_start + args.warmup + args.steps + (args.profile_steps if persistent else 0)
    # the per-phase kernels: timed as a second line, and profiled one kernel
    # class at a time (HIP events between direct launches)
    if args.no_per_phase and persistent:
        ms_alt, breakdown = None, None
    else:
        model.persistent = False
        ms_alt = model.bench_decode(alt_warmup, alt_steps) / alt_steps
        log(f"per-phase kernels: {ms_alt:.3f} ms/token, {1000.0/ms_alt:.1f} tok/s")
        breakdown = model.profile_step(args.profile_steps)
        model.persistent = persistent
    bytes_cls = algorithmic_bytes(model, pos_mid + args.profile_steps / 2)
    classes = {}
    for k, v in (breakdown or {}).items():
        gbs = bytes_cls[k] / (v * 1e-3) / 1e9 if v > 0 else 0.0
        classes[k] = {"ms_per_token": round(v, 4), "bytes_per_token": int(bytes_cls[k]), "GB_s": round(gbs, 1)}
    if persistent:
        # one k_decode launch (plus the 1-WG embedding kernel) per token: its
        # algorithmic bytes are the whole token's (weights + KV + activations)
        dom = "decode_step"
        pos_dec = pos_start + args.warmup + args.steps + args.profile_steps / 2
        per_launch_bytes = sum(algorithmic_bytes(model, pos_dec).values())
        per_launch_ms = decode_launch["ms_decode"]
    else:
        dom = max(breakdown, key=breakdown.get)
        launches = 1 if dom in ("vocab", "finish") else args.layers
        per_launch_bytes = bytes_cls[dom] / launches
        per_launch_ms = breakdown[dom] / launches
    achieved = per_launch_bytes / (per_launch_ms * 1e-3) / 1e9
    log(f"dominant kernel {dom}: {per_launch_ms*1e3:.1f} us/launch, {achieved:.0f} GB/s")

    prefill = None
    if args.prefill > 0:
        # batched prefill of a fresh sequence (fp16 matrix cores); the
        # reference's prompt loop is one sequential forward per token
        pp = rng.integers(0, spec.vocab, args.prefill).astype(np.uint32)
        times = []
        for _ in range(3):
            model.reset()
            t0 = time.perf_counter()
            model.prefill(pp, want_logits=False)
            times.append(time.perf_counter() - t0)
        pms = sorted(times)[1] * 1e3
        fl = prefill_flops(model, args.prefill)
        tfs = fl / (pms * 1e-3) / 1e12
        ex = prefill_executed_flops(model, args.prefill, model.route_log(0, args.prefill))
        xtfs = ex["fp16"] / (pms * 1e-3) / 1e12
        prefill = {"tokens": args.prefill, "ms": round(pms, 2), "tok_s": round(args.prefill / pms * 1e3, 1),
                   "flops": int(fl), "sequential_decode_ms_estimate": round(args.prefill * ms_per_step, 1),
                   "roofline": {"bound": "mfma", "achieved": round(tfs, 1), "peak": 2500.0, "unit": "TFLOP/s",
                                "frac": round(tfs / 2500.0, 4), "dtype": "f16 operands, f32 accumulate"},
                   "executed": {"fp16_mfma_flops": ex["fp16"], "router_fp32_mfma_flops": ex["router_fp32"],
                                "fp16_TFLOP_s": round(xtfs, 1), "fp16_frac": round(xtfs / 2500.0, 4),
                                "note": "tile padding included: 128-row expert tiles (remainders of <= 64 rows "
                                        "as 64), 16-query x 64-key attention blocks"}}
        log(f"batched prefill {args.prefill} tokens: {pms:.1f} ms, {args.prefill / pms * 1e3:.0f} tok/s, "
            f"{tfs:.0f} TFLOP/s algorithmic, {xtfs:.0f} TFLOP/s executed fp16 MFMA")

    long_ctx = None
    if args.long_pos > 0 and args.long_pos + 24 <= spec.context:
        # decode late in the context (--ctx 4096): the KV cache of the first
        # long_pos positions filled by the batched prefill, then event-timed
        # greedy steps; the KV history read grows by 196,608 B per position
        model.reset()
        model.prefill(rng.integers(0, spec.vocab, args.long_pos).astype(np.uint32), want_logits=False)
        lw, ls = 4, 16
        lms = model.bench_decode(lw, ls) / ls
        lp = args.long_pos + lw + ls / 2
        lbytes = sum(algorithmic_bytes(model, lp).values())
        long_ctx = {"positions": [args.long_pos + lw, args.long_pos + lw + ls], "ms_per_token": round(lms, 4),
                    "tok_s": round(1000.0 / lms, 2), "algorithmic_bytes_per_token": int(lbytes),
                    "GB_s": round(lbytes / (lms * 1e-3) / 1e9, 1),
                    "frac": round(lbytes / (lms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"decode at positions {args.long_pos + lw}-{args.long_pos + lw + ls}: {lms:.3f} ms/token, "
            f"{1000.0 / lms:.1f} tok/s ({long_ctx['GB_s']:.0f} GB/s)")

    w_active = active_weight_bytes(model)
    matvec = [] if args.no_matvec else matvec_cases(engine, synth, dev)
    cpu = None if args.no_cpu else cpu_baseline(img, spec, threads, int(pos_dec) if persistent else int(pos_mid))

    result = {
        "metric": "decode tok/s, 30B-A3B Q4_K_M batch 1; matvec HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init weights, uniform random prompt ids)",
        "config": {"workload": f"Qwen3-30B-A3B Q4_K_M random-init, {args.layers} layers, batch-1 greedy "
                               f"decode after a {args.prompt}-token sequential prefill",
                   "prompt_tokens": args.prompt, "decode_tokens": args.steps,
                   "weights": "Q4_K/Q6_K/F32 (Q4_K_M mix), activations and KV FP32",
                   "positions": [pos_start, pos_start + args.warmup + args.steps]},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(dom, pos_dec if persistent else pos_mid),
                     "algorithmic_bytes_per_launch": int(per_launch_bytes),
                     "launch_us": round(per_launch_ms * 1e3, 2)},
        "weights_roofline": {"active_weight_bytes_per_token": int(w_active),
                             "GB_s": round(w_active * tok_s / 1e9, 1),
                             "frac": round(w_active * tok_s / 1e9 / HBM_PEAK_GBS, 4)},
        "step": "persistent k_decode (one launch per token)" if persistent else "per-phase kernels",
        "decode_launch": decode_launch,
        "per_phase_kernels": None if ms_alt is None else {"ms_per_token": round(ms_alt, 4),
                                                          "tok_s": round(1000.0 / ms_alt, 2), "breakdown": classes},
        "prefill": prefill,
        "long_context": long_ctx,
        "matvec": matvec,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    # release the device before the interpreter (and a profiler's exit
    # handlers) tear the runtime down
    del model
    dev.close()


if __name__ == "__main__":
    main()
