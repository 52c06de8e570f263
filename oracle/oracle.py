"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the oracle is what the HIP engine is compared
against.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
import this module; the engine never does.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


class OracleError(RuntimeError):
    pass


def build():
    """Compile liboracle.so with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    sz, u32, i32, f32 = C.c_size_t, C.c_uint32, C.c_int, C.c_float
    sig = {
        "or_last_error": (C.c_char_p, []),
        "or_layout": (i32, [u32, C.POINTER(sz), C.POINTER(sz)]),
        "or_row_bytes": (i32, [u32, sz, C.POINTER(sz)]),
        "or_f16": (f32, [C.c_uint16]),
        "or_value": (f32, [_u8p, u32, sz]),
        "or_decode": (i32, [_u8p, sz, u32, sz, _f32p]),
        "or_rms": (i32, [_f32p, _f32p, sz, f32]),
        "or_rope": (None, [_f32p, sz, sz, sz, f32]),
        "or_softmax": (i32, [_f32p, sz]),
        "or_route": (i32, [_f32p, sz, sz, _u32p, _f32p]),
        "or_attention": (i32, [_f32p, _f32p, _f32p, sz, sz, sz, sz, _f32p]),
        "or_greedy": (i32, [_f32p, sz, C.POINTER(u32)]),
        "or_chacha_block": (None, [C.POINTER(u32 * 8), C.c_uint64, C.c_uint64, i32, C.POINTER(u32 * 16)]),
        "or_stdrng_seed": (None, [C.c_uint64, C.POINTER(u32 * 8)]),
        "or_sampler_new": (C.c_void_p, [C.c_uint64, f32, sz, f32]),
        "or_sampler_free": (None, [C.c_void_p]),
        "or_sampler_draw": (f32, [C.c_void_p]),
        "or_sampler_sample": (i32, [C.c_void_p, _f32p, sz, C.POINTER(u32)]),
        "or_packed_matvec": (i32, [_u8p, sz, u32, sz, sz, _f32p, _f32p, i32]),
        "or_gguf_open": (C.c_void_p, [C.c_void_p, sz]),
        "or_gguf_free": (None, [C.c_void_p]),
        "or_gguf_tensor_count": (sz, [C.c_void_p]),
        "or_gguf_tensor": (i32, [C.c_void_p, C.c_char_p, C.POINTER(u32), C.POINTER(sz),
                                 C.POINTER(C.c_uint64 * 3), C.POINTER(sz), C.POINTER(sz)]),
        "or_gguf_row": (i32, [C.c_void_p, C.c_char_p, sz, _f32p, sz]),
        "or_gguf_uint": (i32, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]),
        "or_gguf_float": (f32, [C.c_void_p, C.c_char_p, f32]),
        "or_gguf_packed_bytes": (C.c_uint64, [C.c_void_p]),
        "or_model_new": (C.c_void_p, [C.c_void_p, sz]),
        "or_model_free": (None, [C.c_void_p]),
        "or_model_config": (i32, [C.c_void_p, C.c_void_p]),
        "or_model_reset": (None, [C.c_void_p]),
        "or_model_position": (sz, [C.c_void_p]),
        "or_model_forward": (i32, [C.c_void_p, u32, C.c_void_p, i32]),
        "or_model_step": (i32, [C.c_void_p, u32, i32]),
        "or_model_matvec": (i32, [C.c_void_p, C.c_char_p, C.c_int64, _f32p, sz, _f32p, sz, i32]),
        "or_layer_forward": (i32, [C.c_void_p, sz, _f32p, sz, C.c_void_p, C.c_void_p,
                                   C.c_void_p, C.c_void_p, i32]),
        "or_model_kv": (i32, [C.c_void_p, sz, _f32p, _f32p, sz]),
        "or_model_last_router": (i32, [C.c_void_p, sz, _f32p, sz]),
        "or_model_force_routes": (i32, [C.c_void_p, _u32p, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _err():
    return lib().or_last_error().decode()


def _check(rc):
    if rc != 0:
        raise OracleError(_err())


# ---- quant.rs -------------------------------------------------------------
LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
          14: (256, 210)}


def layout(kind):
    b, n = C.c_size_t(), C.c_size_t()
    _check(lib().or_layout(kind, C.byref(b), C.byref(n)))
    return b.value, n.value


def row_bytes(kind, cols):
    out = C.c_size_t()
    _check(lib().or_row_bytes(kind, cols, C.byref(out)))
    return out.value


def f16(bits):
    return lib().or_f16(bits)


def f16_all():
    return np.array([lib().or_f16(i) for i in range(65536)], dtype=np.float32)


def decode(row, kind, cols):
    row = np.frombuffer(bytes(row), dtype=np.uint8)
    buf = row.copy() if row.size else np.zeros(1, np.uint8)
    out = np.empty(max(cols, 1), np.float32)
    _check(lib().or_decode(buf, row.size, kind, cols, out))
    return out[:cols]


# ---- ops.rs ----------------------------------------------------------------
def rms(x, w, eps):
    x = np.array(x, np.float32)
    _check(lib().or_rms(x, np.ascontiguousarray(w, np.float32), x.size, eps))
    return x


def rope(x, head, pos, theta):
    x = np.array(x, np.float32)
    lib().or_rope(x, x.size, head, pos, theta)
    return x


def softmax(x):
    x = np.array(x, np.float32)
    _check(lib().or_softmax(x, x.size))
    return x


def route(logits, top):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(max(top, 1), np.uint32)
    w = np.zeros(max(top, 1), np.float32)
    _check(lib().or_route(logits, logits.size, top, ids, w))
    return ids[:top], w[:top]


def attention(q, k, v, heads, kvheads, d):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    if k.size != v.size:
        raise OracleError("attention shape mismatch")
    if q.size != heads * d:
        raise OracleError("attention shape mismatch")
    out = np.zeros(heads * d, np.float32)
    kk = k if k.size else np.zeros(1, np.float32)
    vv = v if v.size else np.zeros(1, np.float32)
    _check(lib().or_attention(q, kk, vv, k.size, heads, kvheads, d, out))
    return out


def greedy(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    if logits.size == 0:
        raise OracleError("invalid logits")
    out = C.c_uint32()
    _check(lib().or_greedy(logits, logits.size, C.byref(out)))
    return out.value


def chacha_block(key, counter, stream=0, rounds=12):
    k = (C.c_uint32 * 8)(*key)
    out = (C.c_uint32 * 16)()
    lib().or_chacha_block(C.byref(k), counter, stream, rounds, C.byref(out))
    return list(out)


def stdrng_key(seed):
    k = (C.c_uint32 * 8)()
    lib().or_stdrng_seed(seed, C.byref(k))
    return list(k)


class Sampler:
    """sampling.rs `Sampler` (seeded StdRng stream, top-k, temperature, top-p)."""

    def __init__(self, seed, temperature, top_k, top_p):
        self._p = lib().or_sampler_new(seed, temperature, top_k, top_p)
        if not self._p:
            raise OracleError(_err())

    def __del__(self):
        if getattr(self, "_p", None):
            lib().or_sampler_free(self._p)
            self._p = None

    def draw(self):
        return lib().or_sampler_draw(self._p)

    def sample(self, logits):
        logits = np.ascontiguousarray(logits, np.float32)
        out = C.c_uint32()
        _check(lib().or_sampler_sample(self._p, logits, logits.size, C.byref(out)))
        return out.value


def packed_matvec(data, kind, rows, cols, x, threads=0):
    data = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check(lib().or_packed_matvec(data, data.size, kind, rows, cols, x, y, threads))
    return y


# ---- gguf.rs / model.rs ------------------------------------------------------
class Gguf:
    """A parsed GGUF image (gguf.rs:102-195).  Keeps the bytes alive."""

    def __init__(self, image):
        self._buf = np.frombuffer(image, np.uint8) if not isinstance(image, np.ndarray) else image
        self._buf = np.ascontiguousarray(self._buf)
        h = lib().or_gguf_open(self._buf.ctypes.data, self._buf.size)
        if not h:
            raise OracleError(_err())
        self.h = h

    @classmethod
    def open(cls, path):
        with open(path, "rb") as f:
            return cls(f.read())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_gguf_free(self.h)
            self.h = None

    def tensor_count(self):
        return lib().or_gguf_tensor_count(self.h)

    def tensor(self, name):
        kind, rank, off, ln = C.c_uint32(), C.c_size_t(), C.c_size_t(), C.c_size_t()
        dims = (C.c_uint64 * 3)()
        _check(lib().or_gguf_tensor(self.h, name.encode(), C.byref(kind), C.byref(rank),
                                    C.byref(dims), C.byref(off), C.byref(ln)))
        return dict(kind=kind.value, dims=list(dims)[: rank.value], offset=off.value, len=ln.value)

    def data(self, name):
        t = self.tensor(name)
        return self._buf[t["offset"]: t["offset"] + t["len"]]

    def row(self, name, r):
        t = self.tensor(name)
        out = np.empty(t["dims"][0], np.float32)
        _check(lib().or_gguf_row(self.h, name.encode(), r, out, out.size))
        return out

    def uint(self, key):
        v = C.c_uint64()
        _check(lib().or_gguf_uint(self.h, key.encode(), C.byref(v)))
        return v.value

    def float(self, key, default):
        return lib().or_gguf_float(self.h, key.encode(), default)

    def packed_bytes(self):
        return lib().or_gguf_packed_bytes(self.h)


class _Config(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("hidden", "layers", "heads", "kvheads", "head_dim",
                                          "experts", "top", "intermediate", "vocab", "max_context")] + \
               [("eps", C.c_float), ("theta", C.c_float)]


class Model:
    """Oracle of model.rs `Model` over a parsed Gguf.  threads=0 runs the
    faithful single-thread matvec; threads>=1 the row-threaded one (same bits)."""

    def __init__(self, gguf, context, threads=8):
        self.gguf = gguf
        h = lib().or_model_new(gguf.h, context)
        if not h:
            raise OracleError(_err())
        self.h = h
        self.threads = threads
        c = _Config()
        lib().or_model_config(h, C.byref(c))
        self.config = {n: getattr(c, n) for n, _ in _Config._fields_}

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None

    @property
    def position(self):
        return lib().or_model_position(self.h)

    def reset(self):
        lib().or_model_reset(self.h)

    def force_routes(self, ids):
        """Route the next forward/step to `ids` ([layers][top], in rank
        order) instead of the oracle's own top-k; the weights are the softmax
        of the oracle's own router logits at those ids.  One step only."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        _check(lib().or_model_force_routes(self.h, ids, ids.size))

    def forward(self, token, threads=None, routes=None):
        if routes is not None:
            self.force_routes(routes)
        out = np.empty(self.config["vocab"], np.float32)
        _check(lib().or_model_forward(self.h, token, out.ctypes.data,
                                      self.threads if threads is None else threads))
        return out

    def step(self, token, threads=None, routes=None):
        """forward() without the final norm and vocab projection: the layers,
        the KV append and the position advance only (for long prompts whose
        intermediate logits are not compared)."""
        if routes is not None:
            self.force_routes(routes)
        _check(lib().or_model_step(self.h, token, self.threads if threads is None else threads))

    def routes(self):
        """Top-k expert ids of every layer for the last step, [layers][top]."""
        c = self.config
        return np.stack([route(self.last_router(l), c["top"])[0] for l in range(c["layers"])])

    def matvec(self, name, expert, x, threads=None):
        x = np.ascontiguousarray(x, np.float32)
        t = self.gguf.tensor(name)
        rows = t["dims"][1] if len(t["dims"]) > 1 else 1
        y = np.empty(max(rows, 1), np.float32)
        _check(lib().or_model_matvec(self.h, name.encode(), -1 if expert is None else expert, x,
                                     x.size, y, y.size, self.threads if threads is None else threads))
        return y[:rows]

    def layer_forward(self, layer, x, pos, kprev, vprev, threads=None):
        """Layer loop body at position `pos` over a time-major KV history of
        exactly `pos` positions; returns (x_out, expert_ids, expert_weights)."""
        x = np.array(x, np.float32)
        top = self.config["top"]
        ids = np.zeros(top, np.uint32)
        w = np.zeros(top, np.float32)
        kp = np.ascontiguousarray(kprev, np.float32) if pos else None
        vp = np.ascontiguousarray(vprev, np.float32) if pos else None
        _check(lib().or_layer_forward(self.h, layer, x, pos,
                                      kp.ctypes.data if pos else None,
                                      vp.ctypes.data if pos else None,
                                      ids.ctypes.data, w.ctypes.data,
                                      self.threads if threads is None else threads))
        return x, ids, w

    def kv(self, layer):
        c = self.config
        n = self.position * c["kvheads"] * c["head_dim"]
        k = np.empty(max(n, 1), np.float32)
        v = np.empty(max(n, 1), np.float32)
        _check(lib().or_model_kv(self.h, layer, k, v, k.size))
        return k[:n], v[:n]

    def last_router(self, layer):
        out = np.empty(self.config["experts"], np.float32)
        _check(lib().or_model_last_router(self.h, layer, out, out.size))
        return out
