"""MI355X (gfx950) Qwen3-MoE decode engine: Python host mirror of the
reference's backend interface over the engine's C ABI (include/qwen_hip.h).

The reference exposes (src/backend.rs:14-23, src/model.rs:163-302):

    trait Backend { fn matvec(&mut self, model, name, expert, x) -> Vec<f32>;
                    fn stats(&self) -> &Stats; }
    Model::new(gguf, context) / forward(token, backend) / reset() / position

Here the same surface is `HipBackend.matvec(name, expert, x)` /
`HipBackend.stats()` and `Model(image_or_path, context)` with
`.forward(token)`, `.reset()`, `.position`, all running on the GPU through
libqwen_hip.so.  There is no CPU fallback: without the built library or a
gfx950 device every entry raises.

Import with importlib (the package directory name contains a hyphen):
    qh = importlib.import_module("qwen-30brust_amd")
"""
import atexit
import ctypes as C
import os
import sys
import weakref

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# QH_LIB selects another build of the engine library (same ABI)
LIB_PATH = os.environ.get("QH_LIB") or os.path.join(PKG_DIR, "libqwen_hip.so")

KINDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


class EngineError(RuntimeError):
    """A failure reported by the engine (the reference's anyhow error)."""


class _Stats(C.Structure):
    _fields_ = [("matvecs", C.c_uint64), ("uploaded_bytes", C.c_uint64),
                ("cache_hits", C.c_uint64), ("matvec_ms", C.c_double)]


class _Config(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("hidden", "layers", "heads", "kvheads", "head_dim",
                                          "experts", "top", "intermediate", "vocab",
                                          "max_context")] + \
               [("eps", C.c_float), ("theta", C.c_float)]


class _Inspect(C.Structure):
    _fields_ = [("config", _Config), ("tensor_count", C.c_uint64), ("packed_weight_bytes", C.c_uint64),
                ("kv_f32_bytes_at_context", C.c_uint64)]


_SIGS = {
    "qh_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "qh_inspect": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(_Inspect)]),
    "qh_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "qh_sampler_create": (C.c_int, [C.c_uint64, C.c_float, C.c_size_t, C.c_float, C.POINTER(C.c_void_p)]),
    "qh_sampler_destroy": (None, [C.c_void_p]),
    "qh_sampler_draw": (C.c_int, [C.c_void_p, C.POINTER(C.c_float)]),
    "qh_set_valid_tokens": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "qh_sample": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32)]),
    "qh_sample_logits": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                   C.POINTER(C.c_uint32)]),
    "qh_device_name": (C.c_int, [C.c_int, C.c_char_p, C.c_size_t]),
    "qh_destroy": (None, [C.c_void_p]),
    "qh_last_error": (C.c_char_p, [C.c_void_p]),
    "qh_load_model": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]),
    "qh_load_model_file": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "qh_model_config": (C.c_int, [C.c_void_p, C.POINTER(_Config)]),
    "qh_packed_weight_bytes": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64)]),
    "qh_tensor_info": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_size_t),
                                 C.POINTER(C.c_uint64 * 3)]),
    "qh_matvec": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int64, C.c_void_p, C.c_size_t,
                            C.c_void_p, C.c_size_t]),
    "qh_stats": (C.c_int, [C.c_void_p, C.POINTER(_Stats)]),
    "qh_packed_matvec_batch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint32, C.c_size_t,
                                         C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]),
    "qh_packed_matvec": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint32, C.c_size_t,
                                   C.c_size_t, C.c_void_p, C.c_void_p]),
    "qh_dequant": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint32, C.c_size_t,
                             C.c_size_t, C.c_void_p]),
    "qh_route": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                           C.c_void_p]),
    "qh_argmax": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32)]),
    "qh_attention": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                               C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p]),
    "qh_attention_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                       C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]),
    "qh_forward": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32)]),
    "qh_generate": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                              C.c_void_p, C.c_size_t]),
    "qh_reset": (C.c_int, [C.c_void_p]),
    "qh_position": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "qh_layer_forward": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                                   C.c_void_p, C.c_void_p, C.c_void_p]),
    "qh_bench_decode": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_double)]),
    "qh_persistent": (C.c_int, [C.c_void_p, C.POINTER(C.c_int)]),
    "qh_prefill_batched": (C.c_int, [C.c_void_p, C.POINTER(C.c_int)]),
    "qh_set_persistent": (C.c_int, [C.c_void_p, C.c_int]),
    "qh_profile_decode": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "qh_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t,
                             C.POINTER(C.c_uint32)]),
    "qh_model_generation": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64)]),
    "qh_fault_inject": (C.c_int, [C.c_void_p, C.c_uint32]),
    "qh_route_log": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    "qh_route_gap_log": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    "qh_prefill_reruns": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64)]),
    "qh_prefill_release": (C.c_int, [C.c_void_p]),
    "qh_prefill_bytes": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64)]),
    "qh_read_kv": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]),
    "qh_profile_step": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]),
    "qh_bench_read": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p]),
    "qh_bench_matvec": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint32, C.c_size_t,
                                  C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t, C.c_size_t,
                                  C.c_void_p]),
}

_lib = None


def lib():
    """Loads libqwen_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EngineError(f"{LIB_PATH} is missing: build it with `python -c "
                              f"'import __graft_entry__ as g; g.build()'` (no CPU fallback)")
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _ptr(a):
    return a.ctypes.data if a is not None and a.size else None


def _cap(a):
    return 0 if a is None else a.size


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def inspect(path, ctx=4096):
    """The reference's `inspect` command (src/main.rs:119-131) as a dict:
    config, tensor_count, packed_weight_bytes, kv_f32_bytes_at_context.
    Parses and validates the file without any device work."""
    r = _Inspect()
    if lib().qh_inspect(os.fsencode(str(path)), ctx, C.byref(r)) != 0:
        raise EngineError(lib().qh_last_error(None).decode())
    return {"config": {n: getattr(r.config, n) for n, _ in _Config._fields_},
            "tensor_count": r.tensor_count, "packed_weight_bytes": r.packed_weight_bytes,
            "kv_f32_bytes_at_context": r.kv_f32_bytes_at_context}


def devices():
    """One description per HIP device (the reference's `devices` command)."""
    n = C.c_int(0)
    if lib().qh_device_count(C.byref(n)) != 0:
        raise EngineError(lib().qh_last_error(None).decode())
    out = []
    buf = C.create_string_buffer(512)
    for d in range(n.value):
        if lib().qh_device_name(d, buf, len(buf)) != 0:
            raise EngineError(lib().qh_last_error(None).decode())
        out.append(buf.value.decode())
    return out


class Sampler:
    """== sampling::Sampler (src/sampling.rs:3-65): seeded StdRng stream
    (host), top-k / temperature / top-p selection on the device."""

    def __init__(self, seed, temperature, top_k, top_p):
        h = C.c_void_p()
        if lib().qh_sampler_create(seed, temperature, top_k, top_p, C.byref(h)) != 0:
            raise EngineError(lib().qh_last_error(None).decode())
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().qh_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        if not sys.is_finalizing():
            self.close()

    def draw(self):
        """The stream's next rng.gen::<f32>()."""
        u = C.c_float()
        lib().qh_sampler_draw(self.h, C.byref(u))
        return u.value

    def sample(self, dev, logits, valid=None):
        """Sampler::sample on caller logits (uploaded), optional valid mask."""
        lg = _f32(logits)
        v = None if valid is None else np.ascontiguousarray(valid, np.uint8)
        out = C.c_uint32()
        dev._check(lib().qh_sample_logits(dev.h, self.h, _ptr(lg), _ptr(v), lg.size, C.byref(out)))
        return out.value


_open_devices = weakref.WeakSet()


def _close_all():
    """Destroys every open context while the runtime is still whole: runs
    from atexit, before the interpreter tears modules down and before the
    HIP runtime's (or a profiler's) own exit handlers."""
    for d in list(_open_devices):
        d.close()


atexit.register(_close_all)


class Device:
    """One engine context (one HIP stream) on a gfx950 device.  close()
    releases it (idempotent); open devices are also closed at interpreter
    exit, before the runtime's own teardown."""

    def __init__(self, device=0):
        h = C.c_void_p()
        if lib().qh_create(device, C.byref(h)) != 0:
            raise EngineError(lib().qh_last_error(None).decode())
        self.h = h
        _open_devices.add(self)

    def close(self):
        if getattr(self, "h", None):
            lib().qh_destroy(self.h)
            self.h = None

    def __del__(self):
        if not sys.is_finalizing():
            self.close()

    def _check(self, rc):
        if rc != 0:
            raise EngineError(lib().qh_last_error(self.h).decode())

    # ---- raw test surfaces -------------------------------------------------
    def packed_matvec(self, data, kind, rows, cols, x):
        """== Vulkan::packed_matvec (src/backend.rs:173-182)."""
        d = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data, np.uint8)
        x = _f32(x)
        y = np.empty(max(rows, 1), np.float32)
        self._check(lib().qh_packed_matvec(self.h, _ptr(d), d.size, kind, rows, cols, _ptr(x), _ptr(y)))
        return y[:rows]

    def packed_matvec_batch(self, data, kind, rows, cols, x, nvec):
        """The routed experts' down projections of one layer in one launch:
        y[b] = W_b x[b] (rows of nvec matrices back to back in data)."""
        d = np.ascontiguousarray(data, np.uint8)
        x = _f32(x)
        y = np.empty(max(nvec * rows, 1), np.float32)
        self._check(lib().qh_packed_matvec_batch(self.h, _ptr(d), d.size, kind, rows, cols, nvec, _ptr(x),
                                                 _ptr(y)))
        return y[:nvec * rows].reshape(nvec, rows)

    def dequant(self, data, kind, rows, cols):
        """== quant::decode (src/quant.rs:81-84) for `rows` packed rows."""
        d = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data, np.uint8)
        out = np.empty(max(rows * cols, 1), np.float32)
        self._check(lib().qh_dequant(self.h, _ptr(d), d.size, kind, rows, cols, _ptr(out)))
        return out[: rows * cols].reshape(rows, cols)

    def route(self, logits, top):
        """== ops::route (src/ops.rs:45-56)."""
        lg = _f32(logits)
        ids = np.zeros(max(top, 1), np.uint32)
        w = np.zeros(max(top, 1), np.float32)
        self._check(lib().qh_route(self.h, _ptr(lg), lg.size, top, _ptr(ids), _ptr(w)))
        return ids[:top], w[:top]

    def argmax(self, logits):
        """== Sampler::sample, temperature 0 (src/sampling.rs:26-35)."""
        lg = _f32(logits)
        out = C.c_uint32()
        self._check(lib().qh_argmax(self.h, _ptr(lg), lg.size, C.byref(out)))
        return out.value

    def attention(self, q, k, v, heads, kvheads, d):
        """== ops::attention (src/ops.rs:57-98), time-major k/v."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        if k.size != v.size or q.size != heads * d:
            raise EngineError("attention shape mismatch")
        out = np.empty(heads * d, np.float32)
        self._check(lib().qh_attention(self.h, _ptr(q), _ptr(k), _ptr(v), k.size, heads, kvheads, d, _ptr(out)))
        return out

    def bench_read(self, nbytes, copies, iters):
        """Times a read-only stream over nbytes: {"mean_ms", "median_ms"}."""
        t = (C.c_double * 3)()
        self._check(lib().qh_bench_read(self.h, nbytes, copies, iters, C.cast(t, C.c_void_p)))
        return {"mean_ms": t[0], "median_ms": t[1]}

    def bench_matvec(self, data, kind, rows, cols, x, copies, iters, nvec=1):
        """Times nvec matvecs of rows x cols (one launch) on device-resident
        copies: {"mean_ms", "median_ms", "empty_ms"} per launch."""
        d = np.ascontiguousarray(data, np.uint8)
        xv = np.ascontiguousarray(x, np.float32)
        if xv.size != nvec * cols:
            raise EngineError("x must hold nvec * cols floats")
        t = (C.c_double * 3)()
        self._check(lib().qh_bench_matvec(self.h, _ptr(d), d.size, kind, rows, cols, nvec, _ptr(xv),
                                          copies, iters, C.cast(t, C.c_void_p)))
        return {"mean_ms": t[0], "median_ms": t[1], "empty_ms": t[2]}


class Model:
    """== model::Model on the GPU: `Model(image_or_path, context)`."""

    def __init__(self, source, context, device=None):
        self.dev = device if device is not None else Device(0)
        if isinstance(source, (str, os.PathLike)):
            self.dev._check(lib().qh_load_model_file(self.dev.h, os.fspath(source).encode(), context))
        else:
            buf = np.frombuffer(source, np.uint8) if not isinstance(source, np.ndarray) else source
            buf = np.ascontiguousarray(buf, np.uint8)
            self.dev._check(lib().qh_load_model(self.dev.h, _ptr(buf), buf.size, context))
        c = _Config()
        self.dev._check(lib().qh_model_config(self.dev.h, C.byref(c)))
        self.config = {n: getattr(c, n) for n, _ in _Config._fields_}
        self.context = context
        self.generation = self._generation()

    def _generation(self):
        g = C.c_uint64()
        self.dev._check(lib().qh_model_generation(self.dev.h, C.byref(g)))
        return g.value

    def _live(self):
        """Raises when a later load on the same Device replaced this model
        (the context holds one model at a time)."""
        if self.dev.h is None:
            raise EngineError("the device of this model was closed")
        if self._generation() != self.generation:
            raise EngineError("this model was replaced by a later load on the same device")

    def route_log(self, pos0, n):
        """Routed experts [n][layers][top] recorded for positions pos0..pos0+n
        by the last step that processed them (diagnostics)."""
        self._live()
        c = self.config
        out = np.zeros((max(n, 1), c["layers"], c["top"]), np.uint32)
        self.dev._check(lib().qh_route_log(self.dev.h, pos0, n, _ptr(out)))
        return out[:n]

    def route_gaps(self, pos0, n):
        """[n][layers] relative gap between the top-th and (top+1)-th router
        logit of each routing decision recorded for positions pos0..pos0+n
        (diagnostics: how near a tie each choice was)."""
        self._live()
        c = self.config
        out = np.zeros((max(n, 1), c["layers"]), np.float32)
        self.dev._check(lib().qh_route_gap_log(self.dev.h, pos0, n, _ptr(out)))
        return out[:n]

    def read_kv(self, layer, pos0, n):
        """Layer `layer`'s K and V at positions pos0..pos0+n, time-major
        [n][kvheads][head_dim] (the reference's layout)."""
        self._live()
        c = self.config
        k = np.zeros((max(n, 1), c["kvheads"], c["head_dim"]), np.float32)
        v = np.zeros_like(k)
        self.dev._check(lib().qh_read_kv(self.dev.h, layer, pos0, n, _ptr(k), _ptr(v)))
        return k[:n], v[:n]

    def inject_fault(self, kind=1):
        """Fault injection for failure-path tests (qh_fault_inject): kind 1
        raises the persistent step's abort flag before the next step."""
        self._live()
        self.dev._check(lib().qh_fault_inject(self.dev.h, kind))

    @property
    def position(self):
        p = C.c_size_t()
        lib().qh_position(self.dev.h, C.byref(p))
        return p.value

    def packed_weight_bytes(self):
        v = C.c_uint64()
        self.dev._check(lib().qh_packed_weight_bytes(self.dev.h, C.byref(v)))
        return v.value

    def tensor(self, name):
        """== Gguf::tensor: {"kind", "dims"} of a loaded tensor."""
        kind, rank, dims = C.c_uint32(), C.c_size_t(), (C.c_uint64 * 3)()
        self.dev._check(lib().qh_tensor_info(self.dev.h, name.encode(), C.byref(kind), C.byref(rank), C.byref(dims)))
        return {"kind": kind.value, "dims": list(dims)[: rank.value]}

    def reset(self):
        self._live()
        self.dev._check(lib().qh_reset(self.dev.h))

    def forward(self, token, want_logits=True):
        """== Model::forward: returns the logits (and keeps the argmax)."""
        lg = np.empty(self.config["vocab"], np.float32) if want_logits else None
        am = C.c_uint32()
        self._live()
        self.dev._check(lib().qh_forward(self.dev.h, token, _ptr(lg), _cap(lg), C.byref(am)))
        self.last_argmax = am.value
        return lg

    def sample(self, sampler):
        """Sampler::sample on the logits of the last step, on the device."""
        out = C.c_uint32()
        self.dev._check(lib().qh_sample(self.dev.h, sampler.h, C.byref(out)))
        return out.value

    def set_valid_tokens(self, valid):
        """Padding-vocab mask (src/main.rs:262-266); None clears it."""
        v = None if valid is None else np.ascontiguousarray(valid, np.uint8)
        self.dev._check(lib().qh_set_valid_tokens(self.dev.h, _ptr(v), 0 if v is None else v.size))

    def generate(self, prompt, n_new, want_logits=False):
        """Sequential prefill of `prompt` then `n_new` greedy tokens on device."""
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(n_new, 1), np.uint32)
        lg = np.empty(self.config["vocab"], np.float32) if want_logits else None
        self._live()
        self.dev._check(lib().qh_generate(self.dev.h, _ptr(p), p.size, n_new, _ptr(out), _ptr(lg), _cap(lg)))
        return (out[:n_new], lg) if want_logits else out[:n_new]

    def prefill(self, prompt, want_logits=True):
        """Batched prefill of `prompt` from the current position (fp16 matrix
        cores; models outside its coverage run the exact token step per
        prompt token); returns (greedy id, logits of the last prompt token)."""
        p = np.ascontiguousarray(prompt, np.uint32)
        lg = np.empty(self.config["vocab"], np.float32) if want_logits else None
        am = C.c_uint32()
        self._live()
        self.dev._check(lib().qh_prefill(self.dev.h, _ptr(p), p.size, _ptr(lg), _cap(lg), C.byref(am)))
        return am.value, lg

    def layer_forward(self, layer, x, pos, kprev, vprev):
        self._live()
        x = np.array(x, np.float32)
        top = self.config["top"]
        ids = np.zeros(top, np.uint32)
        w = np.zeros(top, np.float32)
        kp = _f32(kprev) if pos else None
        vp = _f32(vprev) if pos else None
        self.dev._check(lib().qh_layer_forward(self.dev.h, layer, _ptr(x), pos, _ptr(kp), _ptr(vp), _ptr(ids), _ptr(w)))
        return x, ids, w

    KERNEL_CLASSES = ["qkv", "attention", "oproj", "gateup", "down", "vocab", "finish"]

    def profile_step(self, steps):
        """Mean GPU ms per token of each kernel class (events between kernels)."""
        out = np.zeros(len(self.KERNEL_CLASSES), np.float64)
        self.dev._check(lib().qh_profile_step(self.dev.h, steps, _ptr(out), out.size))
        return dict(zip(self.KERNEL_CLASSES, out.tolist()))

    @property
    def persistent(self):
        """True when the token step runs as one persistent launch (k_decode)
        rather than the per-phase kernels."""
        v = C.c_int()
        self.dev._check(lib().qh_persistent(self.dev.h, C.byref(v)))
        return bool(v.value)

    @property
    def prefill_batched(self):
        """True when prefill() runs this model's prompts through the batched
        GEMM path, False when through the exact token step."""
        v = C.c_int()
        self.dev._check(lib().qh_prefill_batched(self.dev.h, C.byref(v)))
        return bool(v.value)

    @property
    def prefill_reruns(self):
        """Prompts the batched prefill ran again through the exact token step
        (an fp16 operand out of range, or non-finite router/output logits)."""
        v = C.c_uint64()
        self.dev._check(lib().qh_prefill_reruns(self.dev.h, C.byref(v)))
        return v.value

    @property
    def prefill_bytes(self):
        """Device bytes the batched prefill holds now: the tile-layout copy of
        the projection matrices plus its chunk buffers (0 before the first
        batched prefill and after prefill_release())."""
        v = C.c_uint64()
        self.dev._check(lib().qh_prefill_bytes(self.dev.h, C.byref(v)))
        return v.value

    def prefill_release(self):
        """Frees the batched prefill's device memory (the tile-layout weight
        copy and the chunk buffers); the KV cache and the position stay, and
        the next batched prefill builds both again."""
        self.dev._check(lib().qh_prefill_release(self.dev.h))

    @persistent.setter
    def persistent(self, enable):
        self.dev._check(lib().qh_set_persistent(self.dev.h, 1 if enable else 0))

    def profile_decode(self, steps):
        """Mean GPU ms of (the embedding kernel, the k_decode launch) per token
        of the persistent step, from HIP events around each kernel."""
        self._live()
        e, d = C.c_double(), C.c_double()
        self.dev._check(lib().qh_profile_decode(self.dev.h, steps, C.byref(e), C.byref(d)))
        return e.value, d.value

    def bench_decode(self, warmup, steps):
        self._live()
        ms = C.c_double()
        self.dev._check(lib().qh_bench_decode(self.dev.h, warmup, steps, C.byref(ms)))
        return ms.value


class HipBackend:
    """== backend::Backend for a loaded Model: matvec(name, expert, x) and
    stats() (src/backend.rs:14-23)."""

    def __init__(self, model):
        self.model = model

    def matvec(self, name, expert, x):
        x = _f32(x)
        dims = self.model.tensor(name)["dims"]
        rows = dims[1] if len(dims) > 1 else 1
        y = np.empty(rows, np.float32)
        dev = self.model.dev
        dev._check(lib().qh_matvec(dev.h, name.encode(), -1 if expert is None else expert,
                                   _ptr(x), x.size, _ptr(y), rows))
        return y

    def stats(self):
        s = _Stats()
        lib().qh_stats(self.model.dev.h, C.byref(s))
        return {n: getattr(s, n) for n, _ in _Stats._fields_}
