"""Metadata of a GGUF file (the key/value section before the tensor table),
read without touching the tensor data: what the chat front end needs from
`Gguf::open` (src/gguf.rs:102-120) -- the token table and the EOS id.

Value types follow the GGUF specification (the reader of src/gguf.rs:30-99):
0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array,
10 u64, 11 i64, 12 f64."""
import struct

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GgufError(ValueError):
    pass


def _read(f, n):
    b = f.read(n)
    if len(b) != n:
        raise GgufError("truncated GGUF header")
    return b


def _string(f):
    (n,) = struct.unpack("<Q", _read(f, 8))
    if n > 1 << 24:
        raise GgufError("GGUF string too long")
    return _read(f, n).decode("utf-8", errors="replace")


def _value(f, t, depth=0):
    if t in _SCALAR:
        fmt = _SCALAR[t]
        return struct.unpack(fmt, _read(f, struct.calcsize(fmt)))[0]
    if t == 8:
        return _string(f)
    if t == 9:
        if depth > 0:
            raise GgufError("nested GGUF arrays are not supported")
        (et,) = struct.unpack("<I", _read(f, 4))
        (n,) = struct.unpack("<Q", _read(f, 8))
        if n > 1 << 26:
            raise GgufError("GGUF array too long")
        if et in _SCALAR:
            fmt = _SCALAR[et]
            size = struct.calcsize(fmt)
            raw = _read(f, size * n)
            return [v[0] for v in struct.iter_unpack(fmt, raw)]
        return [_value(f, et, depth + 1) for _ in range(n)]
    raise GgufError(f"unknown GGUF value type {t}")


def read_metadata(path):
    """dict of every metadata key of the GGUF file at `path`."""
    with open(path, "rb") as f:
        if _read(f, 4) != b"GGUF":
            raise GgufError("not a GGUF file")
        (ver,) = struct.unpack("<I", _read(f, 4))
        if ver not in (2, 3):
            raise GgufError(f"GGUF version {ver} unsupported")
        _nt, nk = struct.unpack("<QQ", _read(f, 16))
        if nk > 100_000:
            raise GgufError("too many GGUF metadata keys")
        meta = {}
        for _ in range(nk):
            k = _string(f)
            (t,) = struct.unpack("<I", _read(f, 4))
            if k in meta:
                raise GgufError("duplicate metadata key")
            meta[k] = _value(f, t)
        return meta
