"""Shared test helpers: the reference's block-layout fixture and independent
block-wise dequant equations (numpy), used to pin the oracle and the engine."""
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
KINDS = [0, 1, 2, 8, 12, 13, 14]
LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
          14: (256, 210)}
F32 = np.float32


def f16_bits(v):
    return int(np.array(v, np.float16).view(np.uint16))


def _put16(b, p, v):
    bits = f16_bits(v)
    b[p] = bits & 0xFF
    b[p + 1] = bits >> 8


def layout_fixture(kind):
    """The two-block fixture of tests/core.rs:50-143: bytes follow
    (j*73 + block*29 + 19) % 256 with explicit d / dmin, and the expected
    values come from block-wise equations written per format (not from the
    element decoder)."""
    n, size = LAYOUT[kind]
    b = np.zeros(size * 2, np.uint8)
    expected = []
    for block in range(2):
        p = block * size
        for j in range(size):
            b[p + j] = (j * 73 + block * 29 + 19) % 256
        if kind == 0:
            f = F32(0.75 if block == 0 else -1.25)
            b[p:p + 4] = np.frombuffer(np.array([f], "<f4").tobytes(), np.uint8)
            expected.append(f)
        elif kind == 1:
            f = F32(0.75 if block == 0 else -1.25)
            _put16(b, p, f)
            expected.append(f)
        elif kind in (2, 8):
            _put16(b, p, 0.125)
            if kind == 8:
                expected.extend(F32(np.int8(np.uint8(v).view(np.int8))) * F32(0.125) for v in b[p + 2:p + 34])
            else:
                for shift in (0, 4):
                    expected.extend(F32(int((v >> shift) & 15) - 8) * F32(0.125) for v in b[p + 2:p + 18])
        elif kind in (12, 13):
            _put16(b, p, 0.125)
            _put16(b, p + 2, 0.0625)
            packed = b[p + 4:p + 16].astype(np.int64)
            ds = [0] * 8
            ms = [0] * 8
            for j in range(4):
                ds[j] = packed[j] & 63
                ms[j] = packed[j + 4] & 63
                ds[j + 4] = (packed[j + 8] & 15) | ((packed[j] >> 6) * 16)
                ms[j + 4] = (packed[j + 8] >> 4) | ((packed[j + 4] >> 6) * 16)
            qs = p + (16 if kind == 12 else 48)
            for chunk in range(4):
                for upper in range(2):
                    for lane in range(32):
                        q = (int(b[qs + chunk * 32 + lane]) >> (upper * 4)) & 15
                        g = chunk * 2 + upper
                        if kind == 13 and ((int(b[p + 16 + lane]) >> g) & 1):
                            q += 16
                        expected.append(F32(0.125) * F32(ds[g]) * F32(q) - F32(0.0625) * F32(ms[g]))
        elif kind == 14:
            _put16(b, p + 208, 0.125)
            out = [F32(0)] * 256
            for chunk in range(2):
                for lane in range(32):
                    low0 = int(b[p + chunk * 64 + lane])
                    low1 = int(b[p + chunk * 64 + 32 + lane])
                    hi = int(b[p + 128 + chunk * 32 + lane])
                    qs = [(low0 & 15) | ((hi & 3) << 4), (low1 & 15) | (((hi >> 2) & 3) << 4),
                          (low0 >> 4) | (((hi >> 4) & 3) << 4), (low1 >> 4) | (((hi >> 6) & 3) << 4)]
                    for quarter in range(4):
                        sc = int(np.uint8(b[p + 192 + chunk * 8 + quarter * 2 + lane // 16]).view(np.int8))
                        out[chunk * 128 + quarter * 32 + lane] = F32(0.125) * F32(sc) * F32(qs[quarter] - 32)
            expected.extend(out)
    exp = np.array(expected, np.float32)
    assert exp.size == n * 2
    return b, exp


# --- independent vectorised GGML dequant (numpy, from the block layouts) -----
def _h(u8, off):
    return (u8[..., off].astype(np.uint16) | (u8[..., off + 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)


def _kscales(sc12):
    """6-bit scales/mins for the 8 sub-blocks from the 12 packed bytes."""
    s = sc12.astype(np.uint8)
    d = np.zeros(s.shape[:-1] + (8,), np.uint8)
    m = np.zeros_like(d)
    d[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    d[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return d, m


def np_dequant(data, kind, cols):
    """Dequantise rows of packed bytes with array equations per format.
    Same rounding steps as the reference ((d*sc)*q - dmin*m, each rounded)."""
    data = np.asarray(data, np.uint8)
    blk, size = LAYOUT[kind]
    rb = cols // blk * size
    rows = data.size // rb
    u = data[: rows * rb].reshape(rows, cols // blk, size)
    if kind == 0:
        return u.reshape(rows, -1).view(np.float32).reshape(rows, cols)
    if kind == 1:
        return u.reshape(rows, -1).view(np.float16).astype(np.float32).reshape(rows, cols)
    if kind == 2:
        d = _h(u, 0)[..., None]
        q = np.concatenate([u[..., 2:18] & 15, u[..., 2:18] >> 4], axis=-1).astype(np.int32) - 8
        return (d * q.astype(np.float32)).reshape(rows, cols)
    if kind == 8:
        d = _h(u, 0)[..., None]
        q = u[..., 2:34].view(np.int8).astype(np.float32)
        return (d * q).reshape(rows, cols)
    if kind in (12, 13):
        d = _h(u, 0)[..., None, None]
        dmin = _h(u, 2)[..., None, None]
        sc, mn = _kscales(u[..., 4:16])
        qs = u[..., 16:144] if kind == 12 else u[..., 48:176]
        qs = qs.reshape(rows, cols // 256, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=3).reshape(rows, cols // 256, 8, 32).astype(np.int32)
        if kind == 13:
            qh = u[..., 16:48]
            bits = ((qh[..., None, :] >> np.arange(8, dtype=np.uint8)[:, None]) & 1).astype(np.int32)
            q = q + 16 * bits
        ds = d * sc.astype(np.float32)[..., None]
        mm = dmin * mn.astype(np.float32)[..., None]
        return (ds * q.astype(np.float32) - mm).reshape(rows, cols)
    if kind == 14:
        ql = u[..., 0:128].reshape(rows, cols // 256, 2, 64)
        qh = u[..., 128:192].reshape(rows, cols // 256, 2, 32)
        sc = u[..., 192:208].view(np.int8).reshape(rows, cols // 256, 2, 8).astype(np.float32)
        d = _h(u, 208)[..., None, None, None]
        lo = np.stack([ql[..., 0:32] & 15, ql[..., 32:64] & 15, ql[..., 0:32] >> 4, ql[..., 32:64] >> 4], axis=3)
        hi = np.stack([(qh >> (2 * k)) & 3 for k in range(4)], axis=3)
        q = (lo.astype(np.int32) | (hi.astype(np.int32) << 4)) - 32  # [rows, nb, 2, 4, 32]
        scale = sc.reshape(rows, cols // 256, 2, 4, 2)
        scale = np.repeat(scale, 16, axis=-1)  # lane/16 selects
        return ((d * scale) * q.astype(np.float32)).reshape(rows, cols)
    raise ValueError(kind)


def random_blocks(kind, rows, cols, rng):
    """Random packed rows with finite f16 d/dmin (so values are finite)."""
    blk, size = LAYOUT[kind]
    nb = cols // blk
    b = rng.integers(0, 256, size=(rows, nb, size), dtype=np.uint8)
    def put(off, scale):
        v = (rng.standard_normal((rows, nb)) * scale).astype(np.float16).view(np.uint16)
        b[..., off] = v & 0xFF
        b[..., off + 1] = v >> 8
    if kind == 0:
        v = rng.standard_normal((rows, cols)).astype(np.float32)
        return np.frombuffer(v.tobytes(), np.uint8).copy()
    if kind == 1:
        v = rng.standard_normal((rows, cols)).astype(np.float16)
        return np.frombuffer(v.tobytes(), np.uint8).copy()
    if kind in (2, 8):
        put(0, 0.01)
    elif kind in (12, 13):
        put(0, 0.01)
        put(2, 0.01)
    elif kind == 14:
        put(208, 0.01)
    return b.reshape(-1).copy()
