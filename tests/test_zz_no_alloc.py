"""The no-allocation entry point qh_attention_noalloc (device buffers, the
kernel's scratch in the library's fixed device array) against qh_attention
(src/ops.rs:57-98 over host buffers) on the same inputs, through the C ABI:
two calls in a row, the second with a smaller shape, bit-identical outputs
(the same kernel and chunking) at history lengths up to 20,000 keys; a
shape whose scratch exceeds the array (one chunk's partials larger than it)
is refused; and a caller-supplied stream."""
import ctypes as C
import importlib

import numpy as np
import pytest

engine = importlib.import_module("qwen-30brust_amd")
synth = importlib.import_module("qwen-30brust_amd.synth")

pytestmark = pytest.mark.gpu
_hip = None


def hip():
    """The HIP runtime libqwen_hip.so is linked against (same instance)."""
    global _hip
    if _hip is None:
        engine.lib()
        h = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipStreamDestroy.argtypes = [C.c_void_p]
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        _hip = h
    return _hip


def hip_check(rc):
    assert rc == 0, f"HIP error {rc}"


class DeviceBuffer:
    """A device copy of a float32 host array."""

    def __init__(self, a):
        self.a = np.ascontiguousarray(a, np.float32)
        self.ptr = C.c_void_p()
        hip_check(hip().hipMalloc(C.byref(self.ptr), max(self.a.nbytes, 4)))
        hip_check(hip().hipMemcpy(self.ptr, self.a.ctypes.data, self.a.nbytes, 1))  # host to device

    def read(self):
        out = np.empty_like(self.a)
        hip_check(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2))  # device to host
        return out

    def free(self):
        if self.ptr:
            hip_check(hip().hipFree(self.ptr))
            self.ptr = C.c_void_p()


@pytest.fixture(scope="module")
def dev():
    d = engine.Device(0)
    yield d
    d.close()


def inputs(seed, T, heads, kvheads, d):
    q = synth.normal(seed, heads * d)
    k = synth.normal(seed + 1, T * kvheads * d)
    v = synth.normal(seed + 2, T * kvheads * d)
    return q, k, v


def noalloc(dev, q, k, v, heads, kvheads, d, stream=None):
    """qh_attention_noalloc on device copies of q, k, v (buffers from the HIP
    runtime the engine itself uses, through ctypes)."""
    bufs = [DeviceBuffer(a) for a in (q, k, v)]
    out = DeviceBuffer(np.full(heads * d, np.nan, np.float32))
    try:
        rc = engine.lib().qh_attention_noalloc(dev.h, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, k.size, heads,
                                               kvheads, d, out.ptr, stream)
        if rc != 0:
            raise engine.EngineError(engine.lib().qh_last_error(dev.h).decode())
        if stream is not None:
            hip_check(hip().hipStreamSynchronize(stream))
        return out.read()
    finally:
        for b in bufs + [out]:
            b.free()


@pytest.mark.parametrize("T,heads,kvheads,d", [(700, 32, 4, 128), (45, 8, 2, 64), (8192, 32, 4, 128),
                                               (20000, 32, 4, 128)])
def test_noalloc_attention_equals_allocating_entry(dev, T, heads, kvheads, d):
    """Bit-identical to qh_attention at any history length (long ones take
    several key tiles per chunk, so the scratch stays within its array), and
    within 1e-5 of a float64 restatement of ops.rs:57-98."""
    q, k, v = inputs(T, T, heads, kvheads, d)
    ref = dev.attention(q, k, v, heads, kvheads, d)
    got = noalloc(dev, q, k, v, heads, kvheads, d)
    assert np.array_equal(got, ref)
    G = heads // kvheads
    kk = k.reshape(T, kvheads, d).astype(np.float64)
    vv = v.reshape(T, kvheads, d).astype(np.float64)
    exp = np.empty((heads, d))
    for h in range(heads):
        s = kk[:, h // G, :] @ q[h * d:(h + 1) * d].astype(np.float64) / np.sqrt(d)
        e = np.exp(s - s.max())
        exp[h] = (e / e.sum()) @ vv[:, h // G, :]
    assert np.max(np.abs(got.reshape(heads, d) - exp)) <= 1e-5 * np.max(np.abs(exp))


def test_noalloc_two_calls_in_a_row_second_smaller(dev):
    a = inputs(11, 1025, 32, 4, 128)
    b = inputs(12, 33, 4, 4, 32)
    ga = noalloc(dev, *a, 32, 4, 128)
    gb = noalloc(dev, *b, 4, 4, 32)
    assert np.array_equal(ga, dev.attention(*a, 32, 4, 128))
    assert np.array_equal(gb, dev.attention(*b, 4, 4, 32))


def test_noalloc_caller_stream(dev):
    s = C.c_void_p()
    hip_check(hip().hipStreamCreate(C.byref(s)))
    try:
        q, k, v = inputs(21, 300, 16, 4, 128)
        got = noalloc(dev, q, k, v, 16, 4, 128, stream=s)
        assert np.array_equal(got, dev.attention(q, k, v, 16, 4, 128))
    finally:
        hip_check(hip().hipStreamDestroy(s))


def test_noalloc_refuses_shapes_beyond_its_scratch(dev):
    # 2048 heads of 128: one chunk's partials alone exceed the 1 MiB array
    q, k, v = inputs(31, 2, 2048, 2048, 128)
    with pytest.raises(engine.EngineError, match="bytes of scratch"):
        noalloc(dev, q, k, v, 2048, 2048, 128)
    # the array is left in a usable state
    q, k, v = inputs(32, 64, 8, 2, 64)
    assert np.array_equal(noalloc(dev, q, k, v, 8, 2, 64), dev.attention(q, k, v, 8, 2, 64))
