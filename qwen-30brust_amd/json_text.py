"""JSON text in serde_json's layout (the reference's command-line outputs,
src/main.rs:124-131,146-151,283-288): object keys in sorted order (its
default map), f64 in the shortest round-trip digits with serde_json's
placement of the decimal point (the ryu crate's format64), non-finite floats
as null; `pretty` uses two-space indentation."""
import decimal
import json
import math


def f64(v):
    v = float(v)
    if not math.isfinite(v):
        return "null"
    sign = "-" if math.copysign(1.0, v) < 0 else ""
    if v == 0:
        return sign + "0.0"
    t = decimal.Decimal(repr(abs(v))).as_tuple()
    digits = "".join(map(str, t.digits)).lstrip("0")
    k = t.exponent + (len(digits) - len(digits.rstrip("0")))
    digits = digits.rstrip("0")
    n = len(digits)
    kk = n + k
    if 0 <= k and kk <= 16:
        return sign + digits + "0" * k + ".0"
    if 0 < kk <= 16:
        return sign + digits[:kk] + "." + digits[kk:]
    if -5 < kk <= 0:
        return sign + "0." + "0" * (-kk) + digits
    return sign + digits[0] + ("." + digits[1:] if n > 1 else "") + "e" + str(kk - 1)


def dumps(obj, pretty=False, _level=0):
    """serde_json::to_string (pretty=False) / to_string_pretty (pretty=True)."""
    if isinstance(obj, dict):
        if not obj:
            return "{}"
        brackets = "{}"
        parts = [json.dumps(str(k)) + (": " if pretty else ":") + dumps(obj[k], pretty, _level + 1)
                 for k in sorted(obj)]
    elif isinstance(obj, (list, tuple)):
        if not obj:
            return "[]"
        brackets = "[]"
        parts = [dumps(v, pretty, _level + 1) for v in obj]
    elif isinstance(obj, bool):
        return "true" if obj else "false"
    elif isinstance(obj, int):
        return str(obj)
    elif isinstance(obj, float):
        return f64(obj)
    elif obj is None:
        return "null"
    else:
        return json.dumps(obj, ensure_ascii=False)
    if pretty:
        ind = "  " * (_level + 1)
        return brackets[0] + "\n" + ",\n".join(ind + p for p in parts) + "\n" + "  " * _level + brackets[1]
    return brackets[0] + ",".join(parts) + brackets[1]
