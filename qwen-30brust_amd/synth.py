"""Seeded random-init qwen3moe GGUF images (libqwen_synth.so).

Named shapes:
  tiny_k()      2 layers, hidden 256, 4 Q / 2 KV heads of 64, 8 experts top-2,
                expert FFN 256, vocab 256, ctx 64; Q4_K attn/gate/up, Q6_K
                down/output (K-quants need 256-column rows, src/quant.rs:14-17,
                so the literal 64-wide shape below cannot carry them).
  tiny_lit()    the literal 2 layers, hidden 64, 4/2 heads of 16, 8 experts
                top-2, FFN 32, vocab 256, ctx 64 with Q4_0 (attn/gate/up) and
                Q8_0 (down/output).
  layer30b()    one decoder layer at Qwen3-30B-A3B shapes (hidden 2048, 32/4
                heads of 128, 128 experts top-8, FFN 768), small vocab.
  qwen30b()     the full 48-layer Qwen3-30B-A3B Q4_K_M layout (vocab 151936):
                Q4_K everywhere, Q6_K output, F32 router and norms, Q6_K
                attn_v / ffn_down_exps on llama.cpp's "more bits" layers --
                18,550,716,416 packed weight bytes, as the real file.
"""
import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libqwen_synth.so")
NONE = 0xFFFFFFFF
# GGML type ids (ggml.h)
F32, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 2, 8, 12, 13, 14

ROLES = ["token_embd", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate_inp",
         "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "output"]


class _Spec(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "layers", "heads", "kvheads", "head_dim",
                                          "experts", "top", "ff", "vocab", "context")] + \
               [("eps", C.c_float), ("theta", C.c_float), ("types", C.c_uint32 * 10),
                ("more_bits_type", C.c_uint32), ("tied_output", C.c_uint32),
                ("seed", C.c_uint64), ("wstd", C.c_float), ("norm_mean", C.c_float),
                ("norm_std", C.c_float)]


@dataclass
class Spec:
    hidden: int
    layers: int
    heads: int
    kvheads: int
    head_dim: int
    experts: int
    top: int
    ff: int
    vocab: int
    context: int
    types: dict = field(default_factory=dict)  # role -> GGML kind
    more_bits_type: int = NONE
    tied_output: bool = False
    seed: int = 1
    eps: float = 1e-6
    theta: float = 1e6
    wstd: float = 0.02
    norm_mean: float = 1.0
    norm_std: float = 0.05

    def _c(self):
        s = _Spec()
        for n in ("hidden", "layers", "heads", "kvheads", "head_dim", "experts", "top", "ff",
                  "vocab", "context"):
            setattr(s, n, getattr(self, n))
        s.eps, s.theta = self.eps, self.theta
        for i, r in enumerate(ROLES):
            s.types[i] = self.types.get(r, 0)
        s.more_bits_type = self.more_bits_type
        s.tied_output = int(self.tied_output)
        s.seed, s.wstd, s.norm_mean, s.norm_std = self.seed, self.wstd, self.norm_mean, self.norm_std
        return s


def _k_types(attn=12, down=14, out=14, embd=12, router=0):
    return {"token_embd": embd, "attn_q": attn, "attn_k": attn, "attn_v": attn,
            "attn_output": attn, "ffn_gate_inp": router, "ffn_gate_exps": attn,
            "ffn_up_exps": attn, "ffn_down_exps": down, "output": out}


def tiny_k(seed=7):
    return Spec(256, 2, 4, 2, 64, 8, 2, 256, 256, 64, types=_k_types(), seed=seed)


def tiny_lit(seed=7):
    return Spec(64, 2, 4, 2, 16, 8, 2, 32, 256, 64, types=_k_types(attn=2, down=8, out=8, embd=2),
                seed=seed)


def layer30b(more_bits=True, seed=3, vocab=256, context=2048):
    """One 30B-shaped layer; more_bits=True gives layer 0's types (Q6_K
    attn_v / ffn_down_exps), False a plain Q4_K layer such as layer 6."""
    t = _k_types(attn=12, down=12, out=14, embd=12)
    return Spec(2048, 1, 32, 4, 128, 128, 8, 768, vocab, context, types=t,
                more_bits_type=14 if more_bits else NONE, seed=seed)


def qwen30b(seed=2026, context=4096, layers=48):
    t = _k_types(attn=12, down=12, out=14, embd=12)
    return Spec(2048, layers, 32, 4, 128, 128, 8, 768, 151936, context, types=t,
                more_bits_type=14, seed=seed)


def build_lib():
    tmp = LIB_PATH + ".tmp"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread",
                    os.path.join(PKG_DIR, "csrc", "synth.cpp"), "-o", tmp], check=True)
    os.replace(tmp, LIB_PATH)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build_lib()
        l = C.CDLL(LIB_PATH)
        l.qs_image_size.restype = C.c_size_t
        l.qs_image_size.argtypes = [C.POINTER(_Spec)]
        l.qs_packed_bytes.restype = C.c_uint64
        l.qs_packed_bytes.argtypes = [C.POINTER(_Spec)]
        l.qs_build.restype = C.c_int
        l.qs_build.argtypes = [C.POINTER(_Spec), C.c_void_p, C.c_size_t, C.c_int]
        l.qs_header.restype = C.c_size_t
        l.qs_header.argtypes = [C.POINTER(_Spec), C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]
        l.qs_quantize.restype = C.c_int
        l.qs_quantize.argtypes = [C.c_uint32, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        l.qs_normal.restype = None
        l.qs_normal.argtypes = [C.c_uint64, C.c_void_p, C.c_size_t, C.c_float, C.c_float]
        _lib = l
    return _lib


def image_size(spec):
    s = spec._c()
    return lib().qs_image_size(C.byref(s))


def packed_bytes(spec):
    s = spec._c()
    return lib().qs_packed_bytes(C.byref(s))


def build_image(spec, threads=None):
    """The GGUF image as a uint8 array."""
    s = spec._c()
    n = lib().qs_image_size(C.byref(s))
    if n == 0:
        raise ValueError("invalid synthetic model spec")
    out = np.empty(n, np.uint8)
    threads = threads or min(16, os.cpu_count() or 1)
    if lib().qs_build(C.byref(s), out.ctypes.data, n, threads) != 0:
        raise RuntimeError("qs_build failed")
    return out


def write_header_only(spec, path):
    """Writes the image's header to `path` and extends the file to the full
    image size without writing the tensor data (a sparse file: the data reads
    as zeros).  Enough for header parsing and validation at full size."""
    s = spec._c()
    buf = np.zeros(1 << 20, np.uint8)
    total = C.c_size_t(0)
    n = lib().qs_header(C.byref(s), buf.ctypes.data, buf.size, C.byref(total))
    if n == 0:
        raise ValueError("invalid synthetic model spec")
    with open(path, "wb") as f:
        f.write(buf[:n].tobytes())
        f.truncate(total.value)
    return total.value


def quantize(kind, x):
    """Quantize rows of x (rows, cols) into packed GGML blocks."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, cols = x.shape
    blk, size = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
                 14: (256, 210)}[kind]
    out = np.empty(rows * (cols // blk) * size, np.uint8)
    if lib().qs_quantize(kind, x.ctypes.data, rows, cols, out.ctypes.data) != 0:
        raise ValueError("bad quantize shape")
    return out


def normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    lib().qs_normal(seed, out.ctypes.data, n, mean, std)
    return out
