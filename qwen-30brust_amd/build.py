"""Build recipe for the engine (libqwen_hip.so, hipcc for gfx950), its
command-line driver (qwen-hip) and the synthetic-model generator
(libqwen_synth.so, host-only g++).

Usage: python qwen-30brust_amd/build.py         (compiles every time it is called)
       python qwen-30brust_amd/build.py trace   (the phase-trace variant; reuses the objects of a build)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
ENGINE_SO = os.path.join(PKG, "libqwen_hip.so")
SYNTH_SO = os.path.join(PKG, "libqwen_synth.so")
CLI = os.path.join(PKG, "qwen-hip")
TRACE_SO = os.path.join(PKG, "libqwen_hip_trace.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # no packed-FP32 instructions (v_pk_*_f32) anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unknown-pragmas",
    "-I", os.path.join(ROOT, "include"),
]
ENGINE_SOURCES = ["kernels.hip", "matvec.hip", "step.hip", "decode.hip", "prefill.hip", "sample.hip", "engine.hip", "gguf.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


def _compile_one(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if src.endswith(".hip"):
        _run([HIPCC, *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj])
    else:  # host-only C++
        _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_engine():
    os.makedirs(BUILD, exist_ok=True)
    compile_one = _compile_one
    with ThreadPoolExecutor(max_workers=len(ENGINE_SOURCES)) as ex:
        objs = list(ex.map(compile_one, ENGINE_SOURCES))
    tmp = ENGINE_SO + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, ENGINE_SO)
    build_cli()
    return ENGINE_SO


def build_trace():
    """libqwen_hip_trace.so: the engine with the phase-trace build of the
    persistent step (decode_trace.hip) in place of decode.hip, for
    phase_trace.py.  Built on request only (`python build.py trace`)."""
    os.makedirs(BUILD, exist_ok=True)

    def one(src):
        if src == "decode.hip":
            obj = os.path.join(BUILD, "decode_trace.o")
            _run([HIPCC, *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, "decode_trace.hip"), "-o", obj])
            return obj
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        return obj if os.path.exists(obj) else _compile_one(src)  # objects of an earlier build are reused

    with ThreadPoolExecutor(max_workers=len(ENGINE_SOURCES)) as ex:
        objs = list(ex.map(one, ENGINE_SOURCES))
    tmp = TRACE_SO + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, TRACE_SO)
    return TRACE_SO


def build_cli():
    """qwen-hip, the command-line driver over the C ABI (links libqwen_hip.so
    from its own directory)."""
    tmp = CLI + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-Wall", os.path.join(CSRC, "cli.cpp"), "-o", tmp,
          "-L", PKG, "-lqwen_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, CLI)
    return CLI


def build_synth():
    tmp = SYNTH_SO + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall",
          os.path.join(CSRC, "synth.cpp"), "-o", tmp])
    os.replace(tmp, SYNTH_SO)
    return SYNTH_SO


def build():
    with ThreadPoolExecutor(max_workers=2) as ex:
        f1 = ex.submit(build_engine)
        f2 = ex.submit(build_synth)
        return f1.result(), f2.result()


if __name__ == "__main__":
    if sys.argv[1:] == ["trace"]:
        print(build_trace())
    else:
        for p in build():
            print(p)
    sys.exit(0)
