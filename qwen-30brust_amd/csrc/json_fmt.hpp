// JSON number layout of serde_json (the Rust serializer the reference's
// command-line outputs go through, src/main.rs:124-131,146-151).
#pragma once
#include <charconv>
#include <cmath>
#include <cstdlib>
#include <string>

namespace qh {

// f64 in serde_json's layout (the ryu crate's format64): shortest round-trip
// digits d (length n) and exponent k with value = d * 10^k, kk = n + k;
//   0 <= k, kk <= 16   -> digits, zeros, ".0"        (10000000.0)
//   0 < kk <= 16       -> digits with the point inside (12.34)
//   -5 < kk <= 0       -> "0." zeros digits           (0.001234)
//   else               -> d[.ddd]e<kk-1>              (9.999999974752427e-7)
// Non-finite values are written as null (serde_json's behaviour).
inline std::string json_f64(double v) {
    if (!std::isfinite(v)) return "null";
    std::string out;
    if (std::signbit(v)) {
        out += '-';
        v = -v;
    }
    if (v == 0.0) return out + "0.0";
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
    const std::string sci(buf, r.ptr);
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = 0; i < e; i++)
        if (sci[i] != '.') digits += sci[i];
    const long n = (long)digits.size(), kk = std::strtol(sci.c_str() + e + 1, nullptr, 10) + 1, k = kk - n;
    if (0 <= k && kk <= 16) {
        out += digits;
        out.append((size_t)k, '0');
        out += ".0";
    } else if (0 < kk && kk <= 16) {
        out += digits.substr(0, (size_t)kk);
        out += '.';
        out += digits.substr((size_t)kk);
    } else if (-5 < kk && kk <= 0) {
        out += "0.";
        out.append((size_t)-kk, '0');
        out += digits;
    } else {
        out += digits[0];
        if (n > 1) {
            out += '.';
            out += digits.substr(1);
        }
        out += 'e';
        out += std::to_string(kk - 1);
    }
    return out;
}

}  // namespace qh
