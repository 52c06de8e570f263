// Synthetic qwen3moe GGUF generator: seeded random-init weights, quantized with
// this project's own block quantizers (the reference ships a decoder only,
// src/quant.rs:1), serialised as a single-file GGUF v3 image that the
// reference reader accepts (src/gguf.rs:102-195).
//
// Used to build the parity and benchmark models (random-init weights; there
// are no checkpoints offline).  Host-only C++; exported with a C ABI.
//
// Determinism: every row of every tensor draws from its own splitmix64 stream
// keyed by (seed, tensor name, row), so the image is identical for any thread
// count.  Weights are approximately N(0, wstd^2) (Irwin-Hall sum of four
// 16-bit uniforms, rescaled to unit variance); norm vectors N(norm_mean,
// norm_std^2).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

enum Kind : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

bool layout(uint32_t k, size_t& blk, size_t& bytes) {
    switch (k) {
    case F32: blk = 1; bytes = 4; return true;
    case F16: blk = 1; bytes = 2; return true;
    case Q4_0: blk = 32; bytes = 18; return true;
    case Q8_0: blk = 32; bytes = 34; return true;
    case Q4_K: blk = 256; bytes = 144; return true;
    case Q5_K: blk = 256; bytes = 176; return true;
    case Q6_K: blk = 256; bytes = 210; return true;
    default: return false;
    }
}

// ---- f32 -> f16, round to nearest even ------------------------------------
uint16_t to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to inf
    if (ax < 0x38800000u) {                                    // f16 subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;
        // value = m * 2^(e-150); in units of 2^-24 that is m >> (126 - e)
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        uint32_t q = m >> shift;
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u;  // rebias 127 -> 15
    uint32_t q = r >> 13, rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

float from_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023, bits;
    if (e == 0) {
        if (!m) bits = sign;
        else {
            int s = -1;
            do { m <<= 1; s++; } while (!(m & 1024));
            bits = sign | ((uint32_t)(112 - s) << 23) | ((m & 1023) << 13);
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e + 112) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

void put16(uint8_t* p, uint16_t v) { p[0] = v & 0xff; p[1] = v >> 8; }

int nearest(float v) { return (int)std::lrintf(v); }

// ---- block quantizers (write exactly `bytes` per block) --------------------
void q4_0_block(const float* x, uint8_t* o) {
    float amax = 0, mx = 0;
    for (int i = 0; i < 32; i++) if (std::fabs(x[i]) > amax) { amax = std::fabs(x[i]); mx = x[i]; }
    float d = mx / -8.f, id = d ? 1.f / d : 0.f;
    put16(o, to_f16(d));
    for (int i = 0; i < 16; i++) {
        int a = std::min(15, std::max(0, nearest(x[i] * id + 8.f)));
        int b = std::min(15, std::max(0, nearest(x[i + 16] * id + 8.f)));
        o[2 + i] = (uint8_t)(a | (b << 4));
    }
}

void q8_0_block(const float* x, uint8_t* o) {
    float amax = 0;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    float d = amax / 127.f, id = d ? 1.f / d : 0.f;
    put16(o, to_f16(d));
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)std::min(127, std::max(-127, nearest(x[i] * id)));
}

// Packs 8 six-bit (scale, min) pairs into the 12-byte K-quant layout read by
// quant.rs:25-34.
void pack_kscales(const uint8_t* sc, const uint8_t* mn, uint8_t* b) {
    for (int j = 0; j < 4; j++) {
        b[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        b[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        b[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

// Q4_K (nbits=4) and Q5_K (nbits=5): 8 sub-blocks of 32 with an asymmetric
// range [min, max] each; 6-bit sub-scales/mins relative to f16 d / dmin.
void qk_block(const float* x, uint8_t* o, int nbits) {
    const int qmax = (1 << nbits) - 1;
    float scale[8], minv[8];
    for (int g = 0; g < 8; g++) {
        float lo = x[g * 32], hi = x[g * 32];
        for (int i = 1; i < 32; i++) { lo = std::min(lo, x[g * 32 + i]); hi = std::max(hi, x[g * 32 + i]); }
        lo = std::min(lo, 0.f);
        scale[g] = (hi - lo) / qmax;
        minv[g] = -lo;
    }
    float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(minv, minv + 8);
    float d = from_f16(to_f16(ms / 63.f)), dmin = from_f16(to_f16(mm / 63.f));
    uint8_t sc[8], mn[8];
    for (int g = 0; g < 8; g++) {
        sc[g] = (uint8_t)std::min(63, std::max(0, d > 0 ? nearest(scale[g] / d) : 0));
        mn[g] = (uint8_t)std::min(63, std::max(0, dmin > 0 ? nearest(minv[g] / dmin) : 0));
    }
    put16(o, to_f16(d));
    put16(o + 2, to_f16(dmin));
    pack_kscales(sc, mn, o + 4);
    uint8_t* qs = o + (nbits == 4 ? 16 : 48);
    uint8_t* qh = o + 16;
    std::memset(qs, 0, 128);
    if (nbits == 5) std::memset(qh, 0, 32);
    for (int g = 0; g < 8; g++) {
        float ds = d * sc[g], mv = dmin * mn[g];
        for (int l = 0; l < 32; l++) {
            int q = ds > 0 ? nearest((x[g * 32 + l] + mv) / ds) : 0;
            q = std::min(qmax, std::max(0, q));
            qs[(g / 2) * 32 + l] |= (uint8_t)((q & 15) << ((g % 2) * 4));
            if (nbits == 5 && (q & 16)) qh[l] |= (uint8_t)(1u << g);
        }
    }
}

// Q6_K: 16 sub-blocks of 16 with signed int8 scales and 6-bit q - 32.
void q6_k_block(const float* x, uint8_t* o) {
    float sub[16];
    for (int s = 0; s < 16; s++) {
        float amax = 0, mx = 0;
        for (int i = 0; i < 16; i++) if (std::fabs(x[s * 16 + i]) > amax) { amax = std::fabs(x[s * 16 + i]); mx = x[s * 16 + i]; }
        sub[s] = mx / -32.f;
    }
    float amax = 0;
    for (int s = 0; s < 16; s++) amax = std::max(amax, std::fabs(sub[s]));
    float d = from_f16(to_f16(amax / 127.f));
    std::memset(o, 0, 210);
    int8_t sc[16];
    for (int s = 0; s < 16; s++) sc[s] = (int8_t)std::min(127, std::max(-128, d > 0 ? nearest(sub[s] / d) : 0));
    for (int i = 0; i < 256; i++) {
        float ds = d * sc[i / 16];
        int q = ds != 0 ? nearest(x[i] / ds) : 0;
        q = std::min(31, std::max(-32, q)) + 32;
        int chunk = i / 128, j = i % 128, quarter = j / 32, lane = j % 32;
        o[chunk * 64 + (quarter % 2) * 32 + lane] |= (uint8_t)((q & 15) << ((quarter / 2) * 4));
        o[128 + chunk * 32 + lane] |= (uint8_t)((q >> 4) << (quarter * 2));
    }
    for (int s = 0; s < 16; s++) o[192 + s] = (uint8_t)sc[s];
    put16(o + 208, to_f16(d));
}

void quantize_row(uint32_t kind, const float* x, size_t cols, uint8_t* o) {
    switch (kind) {
    case F32: std::memcpy(o, x, cols * 4); return;
    case F16: for (size_t i = 0; i < cols; i++) put16(o + 2 * i, to_f16(x[i])); return;
    case Q4_0: for (size_t b = 0; b < cols / 32; b++) q4_0_block(x + 32 * b, o + 18 * b); return;
    case Q8_0: for (size_t b = 0; b < cols / 32; b++) q8_0_block(x + 32 * b, o + 34 * b); return;
    case Q4_K: for (size_t b = 0; b < cols / 256; b++) qk_block(x + 256 * b, o + 144 * b, 4); return;
    case Q5_K: for (size_t b = 0; b < cols / 256; b++) qk_block(x + 256 * b, o + 176 * b, 5); return;
    case Q6_K: for (size_t b = 0; b < cols / 256; b++) q6_k_block(x + 256 * b, o + 210 * b); return;
    }
}

// ---- seeded streams ---------------------------------------------------------
uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t hash_name(uint64_t seed, const std::string& s) {
    uint64_t h = 1469598103934665603ull ^ mix64(seed);
    for (unsigned char c : s) { h ^= c; h *= 1099511628211ull; }
    return mix64(h);
}
struct Stream {
    uint64_t s;
    uint64_t next() { return mix64(s += 0x9E3779B97F4A7C15ull); }
    // Irwin-Hall(4) of 16-bit uniforms, standardised to mean 0, variance 1.
    float normal() {
        uint64_t r = next();
        double sum = (double)(r & 0xffff) + (double)((r >> 16) & 0xffff) + (double)((r >> 32) & 0xffff) +
                     (double)(r >> 48);
        static const double mean = 4 * 32767.5, sd = std::sqrt(4.0 * (65536.0 * 65536.0 - 1.0) / 12.0);
        return (float)((sum - mean) / sd);
    }
};

// ---- GGUF serialisation ----------------------------------------------------
struct TensorSpec {
    std::string name;
    std::vector<uint64_t> dims;  // dims[0] = cols
    uint32_t kind;
    bool norm;
    size_t offset = 0, bytes = 0;  // relative to data start
};

struct Buf {
    std::vector<uint8_t> v;
    void u32(uint32_t x) { for (int i = 0; i < 4; i++) v.push_back((x >> (8 * i)) & 0xff); }
    void u64(uint64_t x) { for (int i = 0; i < 8; i++) v.push_back((x >> (8 * i)) & 0xff); }
    void f32(float f) { uint32_t x; std::memcpy(&x, &f, 4); u32(x); }
    void str(const std::string& s) { u64(s.size()); v.insert(v.end(), s.begin(), s.end()); }
};

}  // namespace

extern "C" {

// Model description.  types[] per role: 0 token_embd, 1 attn_q, 2 attn_k,
// 3 attn_v, 4 attn_output, 5 ffn_gate_inp, 6 ffn_gate_exps, 7 ffn_up_exps,
// 8 ffn_down_exps, 9 output.  more_bits_type (if != 0xffffffff) replaces
// attn_v and ffn_down_exps on the layers llama.cpp's Q4_K_M rule upgrades:
// i < L/8, i >= 7L/8, or (i - L/8) % 3 == 2.
typedef struct {
    uint32_t hidden, layers, heads, kvheads, head_dim, experts, top, ff, vocab, context;
    float eps, theta;
    uint32_t types[10];
    uint32_t more_bits_type;
    uint32_t tied_output;  // 1: omit output.weight (vocab projection uses token_embd)
    uint64_t seed;
    float wstd, norm_mean, norm_std;
} qs_spec;

static std::vector<TensorSpec> plan(const qs_spec* s) {
    std::vector<TensorSpec> t;
    const uint64_t H = s->hidden, Q = (uint64_t)s->heads * s->head_dim, KV = (uint64_t)s->kvheads * s->head_dim;
    t.push_back({"token_embd.weight", {H, s->vocab}, s->types[0], false});
    if (!s->tied_output) t.push_back({"output.weight", {H, s->vocab}, s->types[9], false});
    t.push_back({"output_norm.weight", {H}, F32, true});
    for (uint32_t i = 0; i < s->layers; i++) {
        std::string p = "blk." + std::to_string(i) + ".";
        uint32_t L = s->layers;
        bool more = s->more_bits_type != 0xffffffffu &&
                    (i < L / 8 || i >= 7 * L / 8 || ((int64_t)i - (int64_t)(L / 8)) % 3 == 2);
        uint32_t vt = more ? s->more_bits_type : s->types[3];
        uint32_t dt = more ? s->more_bits_type : s->types[8];
        t.push_back({p + "attn_norm.weight", {H}, F32, true});
        t.push_back({p + "attn_q_norm.weight", {s->head_dim}, F32, true});
        t.push_back({p + "attn_k_norm.weight", {s->head_dim}, F32, true});
        t.push_back({p + "ffn_norm.weight", {H}, F32, true});
        t.push_back({p + "attn_q.weight", {H, Q}, s->types[1], false});
        t.push_back({p + "attn_k.weight", {H, KV}, s->types[2], false});
        t.push_back({p + "attn_v.weight", {H, KV}, vt, false});
        t.push_back({p + "attn_output.weight", {Q, H}, s->types[4], false});
        t.push_back({p + "ffn_gate_inp.weight", {H, s->experts}, s->types[5], false});
        t.push_back({p + "ffn_gate_exps.weight", {H, s->ff, s->experts}, s->types[6], false});
        t.push_back({p + "ffn_up_exps.weight", {H, s->ff, s->experts}, s->types[7], false});
        t.push_back({p + "ffn_down_exps.weight", {s->ff, H, s->experts}, dt, false});
    }
    return t;
}

static bool header(const qs_spec* s, std::vector<TensorSpec>& t, Buf& b, size_t& data_start,
                   size_t& total) {
    const size_t align = 32;
    size_t off = 0;
    for (auto& x : t) {
        size_t blk, bytes;
        if (!layout(x.kind, blk, bytes) || x.dims[0] % blk) return false;
        size_t n = x.dims[0] / blk * bytes;
        for (size_t k = 1; k < x.dims.size(); k++) n *= x.dims[k];
        off = (off + align - 1) / align * align;
        x.offset = off;
        x.bytes = n;
        off += n;
    }
    b.v.insert(b.v.end(), {'G', 'G', 'U', 'F'});
    b.u32(3);
    b.u64(t.size());
    struct KV { std::string k; int type; uint64_t u; float f; std::string s; };
    std::vector<KV> kv = {
        {"general.architecture", 8, 0, 0, "qwen3moe"},
        {"general.alignment", 4, align, 0, ""},
        {"qwen3moe.embedding_length", 4, s->hidden, 0, ""},
        {"qwen3moe.block_count", 4, s->layers, 0, ""},
        {"qwen3moe.attention.head_count", 4, s->heads, 0, ""},
        {"qwen3moe.attention.head_count_kv", 4, s->kvheads, 0, ""},
        {"qwen3moe.attention.key_length", 4, s->head_dim, 0, ""},
        {"qwen3moe.attention.value_length", 4, s->head_dim, 0, ""},
        {"qwen3moe.expert_count", 4, s->experts, 0, ""},
        {"qwen3moe.expert_used_count", 4, s->top, 0, ""},
        {"qwen3moe.expert_feed_forward_length", 4, s->ff, 0, ""},
        {"qwen3moe.context_length", 4, s->context, 0, ""},
        {"qwen3moe.rope.freq_base", 6, 0, s->theta, ""},
        {"qwen3moe.attention.layer_norm_rms_epsilon", 6, 0, s->eps, ""},
    };
    b.u64(kv.size());
    for (auto& e : kv) {
        b.str(e.k);
        b.u32((uint32_t)e.type);
        if (e.type == 8) b.str(e.s);
        else if (e.type == 4) b.u32((uint32_t)e.u);
        else b.f32(e.f);
    }
    for (auto& x : t) {
        b.str(x.name);
        b.u32((uint32_t)x.dims.size());
        for (auto d : x.dims) b.u64(d);
        b.u32(x.kind);
        b.u64(x.offset);
    }
    data_start = (b.v.size() + align - 1) / align * align;
    b.v.resize(data_start, 0);
    total = data_start + off;
    return true;
}

// Exact byte size of the image qs_build writes (0 on an invalid spec).
size_t qs_image_size(const qs_spec* s) {
    auto t = plan(s);
    Buf b;
    size_t ds, total;
    if (!header(s, t, b, ds, total)) return 0;
    return total;
}

// Sum of tensor payload bytes (the reference's `packed_weight_bytes`).
uint64_t qs_packed_bytes(const qs_spec* s) {
    auto t = plan(s);
    Buf b;
    size_t ds, total;
    if (!header(s, t, b, ds, total)) return 0;
    uint64_t n = 0;
    for (auto& x : t) n += x.bytes;
    return n;
}

// Writes only the header of the image (through the alignment padding before
// the tensor data) into out[0..cap); *total receives the full image size.
// Returns the header length, 0 on an invalid spec or a short buffer.
size_t qs_header(const qs_spec* s, uint8_t* out, size_t cap, size_t* total) {
    auto t = plan(s);
    Buf b;
    size_t ds, tot;
    if (!header(s, t, b, ds, tot) || cap < ds) return 0;
    std::memcpy(out, b.v.data(), b.v.size());
    std::memset(out + b.v.size(), 0, ds - b.v.size());
    *total = tot;
    return ds;
}

// Writes the GGUF image into out[0..len).  Returns 0 on success.
int qs_build(const qs_spec* s, uint8_t* out, size_t len, int threads) {
    auto t = plan(s);
    Buf b;
    size_t ds, total;
    if (!header(s, t, b, ds, total) || len < total) return -1;
    std::memcpy(out, b.v.data(), b.v.size());
    std::memset(out + b.v.size(), 0, ds - b.v.size());
    // zero the alignment gaps between tensors
    size_t prev = 0;
    for (auto& x : t) {
        if (x.offset > prev) std::memset(out + ds + prev, 0, x.offset - prev);
        prev = x.offset + x.bytes;
    }
    // work items: (tensor, first row, row count) over all "rows" of every slab
    struct Item { size_t t, r0, n; };
    std::vector<Item> items;
    for (size_t i = 0; i < t.size(); i++) {
        size_t rows = 1;
        for (size_t k = 1; k < t[i].dims.size(); k++) rows *= t[i].dims[k];
        size_t step = std::max<size_t>(1, (1u << 20) / (t[i].dims[0] + 1));
        for (size_t r = 0; r < rows; r += step) items.push_back({i, r, std::min(step, rows - r)});
    }
    std::atomic<size_t> next{0};
    auto work = [&]() {
        std::vector<float> row;
        for (;;) {
            size_t k = next.fetch_add(1);
            if (k >= items.size()) return;
            const Item& it = items[k];
            const TensorSpec& x = t[it.t];
            size_t cols = x.dims[0], blk, bytes;
            layout(x.kind, blk, bytes);
            size_t rb = cols / blk * bytes;
            row.resize(cols);
            uint64_t key = hash_name(s->seed, x.name);
            for (size_t r = it.r0; r < it.r0 + it.n; r++) {
                Stream st{mix64(key + r * 0xD1B54A32D192ED03ull)};
                if (x.norm)
                    for (size_t c = 0; c < cols; c++) row[c] = s->norm_mean + s->norm_std * st.normal();
                else
                    for (size_t c = 0; c < cols; c++) row[c] = s->wstd * st.normal();
                quantize_row(x.kind, row.data(), cols, out + ds + x.offset + r * rb);
            }
        }
    };
    int n = std::max(1, threads);
    std::vector<std::thread> pool;
    for (int i = 1; i < n; i++) pool.emplace_back(work);
    work();
    for (auto& th : pool) th.join();
    return 0;
}

// Quantizes `rows` rows of `cols` floats into packed GGML blocks.
int qs_quantize(uint32_t kind, const float* x, size_t rows, size_t cols, uint8_t* out) {
    size_t blk, bytes;
    if (!layout(kind, blk, bytes) || cols % blk) return -1;
    size_t rb = cols / blk * bytes;
    for (size_t r = 0; r < rows; r++) quantize_row(kind, x + r * cols, cols, out + r * rb);
    return 0;
}

// Seeded approximately-normal floats (same generator as the weights).
void qs_normal(uint64_t seed, float* out, size_t n, float mean, float std) {
    Stream st{mix64(seed)};
    for (size_t i = 0; i < n; i++) out[i] = mean + std * st.normal();
}

}  // extern "C"
