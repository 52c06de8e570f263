// GGUF reader and config validation for the engine (see gguf.hpp).
#include "gguf.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "qh_format.hpp"

namespace qh {

namespace {

std::string fmt(const char* f, const std::string& a) {
    std::string s(f);
    auto p = s.find("{}");
    if (p != std::string::npos) s.replace(p, 2, a);
    return s;
}

struct Reader {
    const uint8_t* p;
    size_t len, pos = 0;
    size_t budget = 128u * 1024 * 1024;  // metadata byte budget (gguf.rs:107)

    void bytes(void* out, size_t n) {
        if (len - pos < n) throw Error("failed to fill whole buffer");
        std::memcpy(out, p + pos, n);
        pos += n;
    }
    uint32_t u32() { uint32_t v; bytes(&v, 4); return v; }
    uint64_t u64() { uint64_t v; bytes(&v, 8); return v; }
    uint64_t count(uint64_t max) {
        uint64_t n = u64();
        if (n > max)
            throw Error("GGUF count " + std::to_string(n) + " exceeds limit " + std::to_string(max));
        return n;
    }
    static bool utf8_ok(const uint8_t* s, size_t n) {
        size_t i = 0;
        while (i < n) {
            uint8_t c = s[i];
            size_t k;
            uint32_t cp;
            if (c < 0x80) { i++; continue; }
            if ((c & 0xe0) == 0xc0) { k = 1; cp = c & 0x1f; }
            else if ((c & 0xf0) == 0xe0) { k = 2; cp = c & 0x0f; }
            else if ((c & 0xf8) == 0xf0) { k = 3; cp = c & 0x07; }
            else return false;
            if (n - i <= k) return false;
            for (size_t j = 1; j <= k; j++) {
                if ((s[i + j] & 0xc0) != 0x80) return false;
                cp = (cp << 6) | (s[i + j] & 0x3f);
            }
            if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) ||
                cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
                return false;
            i += k + 1;
        }
        return true;
    }
    std::string string() {
        uint64_t n = count(16u * 1024 * 1024);
        if (n > budget) throw Error("GGUF metadata budget exceeded");
        budget -= n;
        if (len - pos < n) throw Error("failed to fill whole buffer");
        if (!utf8_ok(p + pos, n)) throw Error("invalid utf-8 sequence");
        std::string s(reinterpret_cast<const char*>(p + pos), n);
        pos += n;
        return s;
    }
    Meta val(uint32_t t, size_t depth) {
        if (!(depth <= 4 && budget >= 8)) throw Error("excessive metadata depth/size");
        budget -= 8;
        Meta m;
        auto sint = [&](int64_t v) {
            m.i = v;
            m.u = (uint64_t)v;
            m.tag = v < 0 ? Meta::INT : Meta::UINT;
        };
        switch (t) {
        case 0: { uint8_t b; bytes(&b, 1); m.tag = Meta::UINT; m.u = b; break; }
        case 1: { uint8_t b; bytes(&b, 1); sint((int8_t)b); break; }
        case 2: { uint16_t b; bytes(&b, 2); m.tag = Meta::UINT; m.u = b; break; }
        case 3: { uint16_t b; bytes(&b, 2); sint((int16_t)b); break; }
        case 4: m.tag = Meta::UINT; m.u = u32(); break;
        case 5: sint((int32_t)u32()); break;
        case 6: {
            float f;
            bytes(&f, 4);
            if (!std::isfinite(f)) throw Error("nonfinite metadata");
            m.tag = Meta::FLOAT;
            m.f = f;
            break;
        }
        case 7: {
            uint8_t b;
            bytes(&b, 1);
            if (b > 1) throw Error("invalid boolean");
            m.tag = Meta::BOOL;
            m.u = b;
            break;
        }
        case 8: m.tag = Meta::STR; m.s = string(); break;
        case 9: {
            uint32_t ty = u32();
            uint64_t n = count(1000000);
            for (uint64_t i = 0; i < n; i++) val(ty, depth + 1);
            m.tag = Meta::ARRAY;
            m.u = n;
            break;
        }
        case 10: m.tag = Meta::UINT; m.u = u64(); break;
        case 11: sint((int64_t)u64()); break;
        case 12: {
            double f;
            bytes(&f, 8);
            if (!std::isfinite(f)) throw Error("nonfinite metadata");
            m.tag = Meta::FLOAT;
            m.f = f;
            break;
        }
        default: throw Error("unknown GGUF metadata type " + std::to_string(t));
        }
        return m;
    }
};

}  // namespace

void check_layout(uint32_t kind) {
    uint32_t b, n;
    if (!layout(kind, b, n))
        throw Error("GGML tensor type " + std::to_string(kind) +
                    " is not supported (supported: F32/F16/Q4_0/Q8_0/Q4_K/Q5_K/Q6_K)");
}

size_t row_bytes_checked(uint32_t kind, uint64_t cols) {
    check_layout(kind);
    uint32_t b, n;
    layout(kind, b, n);
    if (cols == 0 || cols % b)
        throw Error("row width " + std::to_string(cols) + " is not divisible by block size " +
                    std::to_string(b));
    return (size_t)(cols / b) * n;
}

Gguf parse_gguf(const uint8_t* data, size_t len) {
    Gguf g;
    g.data = data;
    g.len = len;
    Reader r{data, len};
    char magic[4];
    r.bytes(magic, 4);
    if (std::memcmp(magic, "GGUF", 4)) throw Error("not a GGUF file");
    uint32_t ver = r.u32();
    if (ver != 2 && ver != 3) throw Error("GGUF version " + std::to_string(ver) + " unsupported");
    uint64_t nt = r.count(100000), nk = r.count(100000);
    for (uint64_t i = 0; i < nk; i++) {
        std::string k = r.string();
        uint32_t t = r.u32();
        Meta v = r.val(t, 0);
        if (!g.meta.emplace(k, v).second) throw Error("duplicate metadata key");
    }
    auto sc = g.meta.find("split.count");
    if (sc != g.meta.end() && sc->second.tag == Meta::UINT && sc->second.u != 1)
        throw Error("split GGUF not supported; merge shards first");
    for (uint64_t i = 0; i < nt; i++) {
        Tensor t;
        t.name = r.string();
        uint32_t nd = r.u32();
        if (nd < 1 || nd > 3) throw Error("unsupported tensor rank " + std::to_string(nd) + ": " + t.name);
        for (uint32_t k = 0; k < nd; k++) {
            uint64_t d = r.u64();
            if (d == 0) throw Error("zero tensor dimension");
            t.dims.push_back(d);
        }
        t.kind = r.u32();
        t.offset = r.u64();
        size_t l = row_bytes_checked(t.kind, t.dims[0]);
        for (uint32_t k = 1; k < nd; k++) {
            if (l > SIZE_MAX / t.dims[k]) throw Error("tensor length overflow");
            l *= t.dims[k];
        }
        t.len = l;
        std::string name = t.name;
        if (!g.tensors.emplace(name, std::move(t)).second) throw Error("duplicate tensor name");
    }
    uint64_t alignment = 32;
    auto al = g.meta.find("general.alignment");
    if (al != g.meta.end() && al->second.tag == Meta::UINT) alignment = al->second.u;
    if (!(alignment && !(alignment & (alignment - 1)) && alignment <= 4096))
        throw Error("invalid GGUF alignment");
    size_t start = (r.pos + alignment - 1) & ~(size_t)(alignment - 1);
    std::vector<std::pair<size_t, size_t>> ranges;
    for (auto& kv : g.tensors) {
        Tensor& t = kv.second;
        if (t.offset % alignment) throw Error("unaligned tensor " + t.name);
        if (t.offset > SIZE_MAX - start) throw Error("tensor offset overflow");
        t.offset += start;
        if (t.len > SIZE_MAX - t.offset) throw Error("tensor end overflow");
        size_t end = t.offset + t.len;
        if (end > len) throw Error("truncated tensor " + t.name);
        ranges.emplace_back(t.offset, end);
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); i++)
        if (ranges[i - 1].second > ranges[i].first) throw Error("overlapping tensors");
    return g;
}

const Tensor& Gguf::tensor(const std::string& name) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) throw Error("missing tensor " + name);
    return it->second;
}
bool Gguf::try_uint(const std::string& key, uint64_t& v) const {
    auto it = meta.find(key);
    if (it == meta.end() || it->second.tag != Meta::UINT) return false;
    v = it->second.u;
    return true;
}
uint64_t Gguf::uint(const std::string& key) const {
    uint64_t v;
    if (!try_uint(key, v)) throw Error("missing integer " + key);
    return v;
}
float Gguf::flt(const std::string& key, float dflt) const {
    auto it = meta.find(key);
    if (it == meta.end()) return dflt;
    const Meta& m = it->second;
    if (m.tag == Meta::UINT) return (float)(double)m.u;
    if (m.tag == Meta::INT) return (float)(double)m.i;
    if (m.tag == Meta::FLOAT) return (float)m.f;
    return dflt;
}
const std::string* Gguf::str(const std::string& key) const {
    auto it = meta.find(key);
    return it != meta.end() && it->second.tag == Meta::STR ? &it->second.s : nullptr;
}
uint64_t Gguf::packed_bytes() const {
    uint64_t s = 0;
    for (auto& kv : tensors) s += kv.second.len;
    return s;
}

Config config_from_gguf(const Gguf& g) {
    const std::string* arch = g.str("general.architecture");
    if (!arch || *arch != "qwen3moe") throw Error("only qwen3moe architecture is implemented");
    auto get = [&](const char* k) { return g.uint(std::string("qwen3moe.") + k); };
    auto tryget = [&](const char* k, uint64_t& v) { return g.try_uint(std::string("qwen3moe.") + k, v); };
    Config c{};
    c.hidden = get("embedding_length");
    c.heads = get("attention.head_count");
    c.top = get("expert_used_count");
    uint64_t v;
    c.head_dim = tryget("attention.key_length", v) ? v : c.hidden / std::max<uint64_t>(c.heads, 1);
    uint64_t vl = tryget("attention.value_length", v) ? v : c.head_dim;
    if (vl != c.head_dim) throw Error("different key/value head sizes unsupported");
    c.layers = get("block_count");
    c.kvheads = get("attention.head_count_kv");
    c.experts = get("expert_count");
    if (tryget("expert_feed_forward_length", v)) c.intermediate = v;
    else c.intermediate = get("feed_forward_length") / std::max<uint64_t>(c.top, 1);
    const Tensor& emb = g.tensor("token_embd.weight");
    if (emb.dims.size() < 2) throw Error("invalid embedding rank");
    c.vocab = emb.dims[1];
    c.max_context = get("context_length");
    c.eps = g.flt("qwen3moe.attention.layer_norm_rms_epsilon", 1e-6f);
    c.theta = g.flt("qwen3moe.rope.freq_base", 1000000.f);
    if (!(c.hidden > 0 && c.layers > 0 && c.layers <= 256 && c.kvheads > 0 && c.heads > 0 &&
          c.heads % c.kvheads == 0 && c.head_dim > 0 && c.head_dim % 2 == 0 && c.top > 0 &&
          c.top <= c.experts && c.experts <= 1024 && c.intermediate > 0 && std::isfinite(c.eps) &&
          c.eps > 0.f && std::isfinite(c.theta) && c.theta > 0.f))
        throw Error("invalid Qwen3 MoE config");
    uint64_t rd = tryget("rope.dimension_count", v) ? v : c.head_dim;
    if (rd != c.head_dim) throw Error("partial rotary dimensions unsupported");
    const std::string* scaling = g.str("qwen3moe.rope.scaling.type");
    if (scaling && *scaling != "none")
        throw Error("RoPE scaling is not implemented; use the original native-context model");
    return c;
}

void validate_tensors(const Config& c, const Gguf& g) {
    auto check = [&](const std::string& name, std::vector<uint64_t> shape) {
        const Tensor& t = g.tensor(name);
        if (t.dims != shape) throw Error(name + ": unexpected shape");
    };
    check("token_embd.weight", {c.hidden, c.vocab});
    check("output_norm.weight", {c.hidden});
    if (g.has("output.weight")) check("output.weight", {c.hidden, c.vocab});
    for (uint64_t i = 0; i < c.layers; i++) {
        std::string p = "blk." + std::to_string(i) + ".";
        check(p + "attn_norm.weight", {c.hidden});
        check(p + "ffn_norm.weight", {c.hidden});
        check(p + "attn_q_norm.weight", {c.head_dim});
        check(p + "attn_k_norm.weight", {c.head_dim});
        check(p + "attn_q.weight", {c.hidden, c.heads * c.head_dim});
        check(p + "attn_k.weight", {c.hidden, c.kvheads * c.head_dim});
        check(p + "attn_v.weight", {c.hidden, c.kvheads * c.head_dim});
        check(p + "attn_output.weight", {c.heads * c.head_dim, c.hidden});
        check(p + "ffn_gate_inp.weight", {c.hidden, c.experts});
        check(p + "ffn_gate_exps.weight", {c.hidden, c.intermediate, c.experts});
        check(p + "ffn_up_exps.weight", {c.hidden, c.intermediate, c.experts});
        check(p + "ffn_down_exps.weight", {c.intermediate, c.hidden, c.experts});
        for (auto& kv : g.tensors) {
            const std::string& n = kv.first;
            if (n.compare(0, p.size(), p) == 0 && n.size() >= 5 && n.compare(n.size() - 5, 5, ".bias") == 0)
                throw Error("unexpected bias tensors");
        }
    }
}

}  // namespace qh
