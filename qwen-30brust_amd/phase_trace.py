"""Phase trace of the persistent token step on the random-init 48-layer
Qwen3-30B-A3B Q4_K_M model: per-workgroup wall clock at each phase mark of
the last layer of a token and of the vocab phase, from
libqwen_hip_trace.so (`python qwen-30brust_amd/build.py trace`).

    python qwen-30brust_amd/phase_trace.py [--layers 48] [--prompt 512] [--tokens 8]

Prints, for each mark, the min / median / max over workgroups of the time
since the first workgroup reached the layer (microseconds), the median over
the traced tokens; with --split, separately for the attention workgroups
(key chunk j < chunks, workgroup b = 8 j + XCD) and the others.
"""
import argparse
import ctypes as C
import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

# (part, mark): name, in the order the marks are reached within a layer
MARKS = [
    ((0, 0), "A  loads issued, wait for x''"),
    ((0, 1), "A  x'' gathered"),
    ((0, 2), "A  q|k|v dots done"),
    ((1, 0), "B  attention start"),
    ((1, 1), "B  q|k|v received"),
    ((1, 4), "B  q/k norm, RoPE done"),
    ((1, 5), "B  scores done (last tile)"),
    ((1, 6), "B  softmax done (last tile)"),
    ((1, 2), "B  key tiles done"),
    ((1, 3), "B  partials stored"),
    ((2, 0), "C  loads issued, wait for partials"),
    ((2, 1), "C  chunk partials gathered"),
    ((2, 2), "C  chunks merged"),
    ((7, 0), "D  o-proj partials received (cross-XCD)"),
    ((4, 0), "E  wait for x'"),
    ((4, 1), "E  x' gathered, normed"),
    ((4, 4), "E  top-k keys written"),
    ((4, 5), "E  ranks done"),
    ((4, 2), "E  routed"),
    ((4, 3), "E  SwiGLU done"),
    ((5, 0), "F  wait for h (down rows requested at the end of E)"),
    ((5, 1), "F  h gathered"),
    ((7, 1), "R  down partials received (cross-XCD)"),
    ((6, 0), "V  vocab loads issued, wait for x''"),
    ((6, 1), "V  x'' gathered"),
    ((6, 2), "V  rows done"),
    ((6, 4), "V  argmax partial stored"),
    ((6, 5), "V  (wg 0) partials received"),
    ((6, 3), "V  (wg 0) token written"),
]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--tokens", type=int, default=8)
    ap.add_argument("--split", action="store_true", help="attention workgroups and the others apart")
    ap.add_argument("--lib", default=None, help="trace library to load (default: the in-tree trace build)")
    args = ap.parse_args()
    engine = importlib.import_module("qwen-30brust_amd")
    synth = importlib.import_module("qwen-30brust_amd.synth")
    from importlib import import_module
    build = import_module("qwen-30brust_amd.build")
    trace_so = os.path.abspath(args.lib) if args.lib else build.TRACE_SO
    engine.LIB_PATH = trace_so
    spec = synth.qwen30b(layers=args.layers, context=max(4096, args.prompt + args.tokens + 8))
    img = synth.build_image(spec, threads=min(16, os.cpu_count() or 1))
    m = engine.Model(img, spec.context)
    if not m.persistent:
        raise SystemExit("the persistent step is not selected for this model")
    prompt = np.random.default_rng(1).integers(0, spec.vocab, args.prompt).astype(np.uint32)
    m.generate(prompt, 2)
    lib = C.CDLL(trace_so)
    buf = np.zeros((8, 512, 8), np.uint64)
    classes = ("all", "attention", "other") if args.split else ("all",)
    rows = {(mk, cl): [] for mk, _ in MARKS for cl in classes}
    for _ in range(args.tokens):
        T = m.position + 1
        tc = max((T + 15) // 16, 64)
        nch = (T + tc - 1) // tc  # key chunks per XCD (decode.hip: attn_chunk)
        wg = np.arange(512)
        member = {"all": wg >= 0, "attention": wg // 8 < nch, "other": wg // 8 >= nch}
        assert lib.qh_dtrace_clear() == 0
        m.forward(7, want_logits=False)
        assert lib.qh_dtrace_dump(buf.ctypes.data_as(C.c_void_p)) == 0
        t = buf.astype(np.int64)
        base = t[0, :, 0][t[0, :, 0] > 0].min()
        for (k, p), _ in MARKS:
            for cl in classes:
                col = t[k, :, p][member[cl]]
                col = col[col > 0]
                if col.size:
                    r = (col - base) * 0.01  # 100 MHz ticks -> us
                    rows[((k, p), cl)].append((np.min(r), np.median(r), np.max(r), col.size))
    print(f"persistent step, {args.layers} layers, positions {args.prompt + 1}..{m.position - 1}: "
          f"last layer of the token, us since the first workgroup reached it "
          f"(min / median / max over workgroups; median over {args.tokens} tokens)")
    for (k, p), name in MARKS:
        for cl in classes:
            r = rows[((k, p), cl)]
            if not r:
                continue
            a = np.median(np.array([x[:3] for x in r]), axis=0)
            tag = "" if cl == "all" else f" [{cl}]"
            print(f"  {name + tag:54s} {a[0]:7.2f} {a[1]:7.2f} {a[2]:7.2f}   (workgroups {r[0][3]})")


if __name__ == "__main__":
    main()
