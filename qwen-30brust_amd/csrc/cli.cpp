// qwen-hip: command-line driver over the C ABI (include/qwen_hip.h) with the
// commands and JSON outputs of the reference binary (src/main.rs:15-153):
//
//   qwen-hip devices
//   qwen-hip inspect --model PATH [--ctx N]
//   qwen-hip logits  --model PATH --tokens 1,5,2 [--ctx N] [--device hip]
//                    [--adapter SUBSTRING] [--gpu-cache-mib N] [--allow-software]
//
// `inspect` prints the pretty JSON of src/main.rs:119-131 and `logits` the
// compact JSON of src/main.rs:133-153, byte for byte in layout: object keys in
// sorted order (serde_json's default map), floats widened to f64 and written
// in the shortest round-trip form with serde_json's layout, so harnesses that
// parse the reference's stdout (tools/reference_fixture.py:125-128) read this
// one unchanged.  Failures print "Error: <message>" to stderr and exit 1;
// argument errors exit 2.
#include <charconv>
#include <chrono>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/qwen_hip.h"
#include "json_fmt.hpp"

namespace {

struct Fail : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct Usage : std::runtime_error {
    using std::runtime_error::runtime_error;
};

std::string json_u64(uint64_t v) { return std::to_string(v); }

uint64_t parse_u64(const std::string& flag, const std::string& s) {
    if (s.empty() || s.find_first_not_of("0123456789") != std::string::npos)
        throw Usage("invalid value '" + s + "' for '--" + flag + "': invalid digit found in string");
    uint64_t v = 0;
    const auto r = std::from_chars(s.data(), s.data() + s.size(), v);
    if (r.ec != std::errc()) throw Usage("invalid value '" + s + "' for '--" + flag + "': number too large");
    return v;
}

struct Args {
    std::string command, model, device = "hip", adapter;
    size_t ctx = 4096;
    std::vector<uint32_t> tokens;
    bool have_model = false, have_tokens = false, have_adapter = false;
};

const char* kUsage =
    "MI355X (HIP, gfx950) Qwen3 MoE inference engine: token steps and KV cache on the GPU\n"
    "\n"
    "Usage: qwen-hip <COMMAND>\n"
    "\n"
    "Commands:\n"
    "  devices  Show available HIP devices\n"
    "  inspect  Parse and validate a single-file Qwen3 MoE GGUF, without allocating GPU buffers\n"
    "  logits   Compute logits for explicit token IDs; useful for parity checks\n";

Args parse(int argc, char** argv) {
    Args a;
    if (argc < 2) throw Usage("a subcommand is required");
    a.command = argv[1];
    if (a.command == "--help" || a.command == "-h" || a.command == "help") {
        std::fputs(kUsage, stdout);
        std::exit(0);
    }
    if (a.command == "--version" || a.command == "-V") {
        std::puts("qwen-hip 0.1.0");
        std::exit(0);
    }
    if (a.command == "chat")
        throw Fail("chat is the tokenizer front end qwen-30brust_amd/chat.py (same arguments): "
                   "python qwen-30brust_amd/chat.py --model M --tokenizer T --prompt P");
    if (a.command != "devices" && a.command != "inspect" && a.command != "logits")
        throw Usage("unrecognized subcommand '" + a.command + "'");
    const bool compute = a.command == "logits";
    for (int i = 2; i < argc; i++) {
        std::string f = argv[i], v;
        if (f.rfind("--", 0) != 0) throw Usage("unexpected argument '" + f + "' found");
        f = f.substr(2);
        const size_t eq = f.find('=');
        const bool inline_v = eq != std::string::npos;
        if (inline_v) {
            v = f.substr(eq + 1);
            f = f.substr(0, eq);
        }
        auto value = [&]() -> std::string {
            if (inline_v) return v;
            if (i + 1 >= argc) throw Usage("a value is required for '--" + f + "' but none was supplied");
            return argv[++i];
        };
        const bool takes_model = a.command != "devices";
        if (f == "model" && takes_model) {
            a.model = value();
            a.have_model = true;
        } else if (f == "ctx" && takes_model) {
            a.ctx = (size_t)parse_u64(f, value());
        } else if (f == "tokens" && a.command == "logits") {
            // value_delimiter ',' and repeated occurrences both append (clap)
            const std::string s = value();
            size_t p = 0;
            while (true) {
                const size_t q = s.find(',', p);
                const uint64_t t = parse_u64(f, s.substr(p, q == std::string::npos ? std::string::npos : q - p));
                if (t > UINT32_MAX) throw Usage("invalid value '" + s + "' for '--tokens': number too large");
                a.tokens.push_back((uint32_t)t);
                if (q == std::string::npos) break;
                p = q + 1;
            }
            a.have_tokens = true;
        } else if (f == "device" && compute) {
            a.device = value();
            if (a.device != "hip" && a.device != "vulkan" && a.device != "cpu")
                throw Usage("invalid value '" + a.device + "' for '--device'\n  [possible values: hip, vulkan, cpu]");
        } else if (f == "adapter" && compute) {
            a.adapter = value();
            a.have_adapter = true;
        } else if (f == "gpu-cache-mib" && compute) {
            parse_u64(f, value());  // accepted; every weight stays resident in HBM
        } else if (f == "allow-software" && compute && !inline_v) {
            // accepted; there is no software HIP device
        } else if (f == "help") {
            std::fputs(kUsage, stdout);
            std::exit(0);
        } else {
            throw Usage("unexpected argument '--" + f + "' found");
        }
    }
    if (a.command != "devices" && !a.have_model) throw Usage("the following required arguments were not provided:\n  --model <MODEL>");
    if (a.command == "logits" && !a.have_tokens)
        throw Usage("the following required arguments were not provided:\n  --tokens <TOKENS>");
    return a;
}

std::string last_error(const qh_ctx* c) {
    const char* e = qh_last_error(c);
    return e ? e : "unknown error";
}

// index of the first device whose description contains `sub` (the
// reference's --adapter), else 0; no silent fallback to another device
int pick_device(const Args& a, std::string& name) {
    int n = 0;
    if (qh_device_count(&n) != 0) throw Fail(last_error(nullptr));
    if (n == 0) throw Fail("no HIP device found");
    char buf[512];
    for (int d = 0; d < n; d++) {
        if (qh_device_name(d, buf, sizeof buf) != 0) throw Fail(last_error(nullptr));
        if (!a.have_adapter || std::string(buf).find(a.adapter) != std::string::npos) {
            name = buf;
            return d;
        }
    }
    throw Fail("no HIP device matches adapter '" + a.adapter + "'");
}

int cmd_devices() {
    int n = 0;
    if (qh_device_count(&n) != 0) throw Fail(last_error(nullptr));
    if (n == 0) throw Fail("no HIP device found");
    char buf[512];
    for (int d = 0; d < n; d++) {
        if (qh_device_name(d, buf, sizeof buf) != 0) throw Fail(last_error(nullptr));
        std::printf("%s\n", buf);
    }
    return 0;
}

int cmd_inspect(const Args& a) {
    qh_inspect_t r;
    if (qh_inspect(a.model.c_str(), a.ctx, &r) != 0) throw Fail(last_error(nullptr));
    const qh_config_t& c = r.config;
    std::string s = "{\n  \"config\": {\n";
    const std::pair<const char*, std::string> cfg[] = {
        {"eps", qh::json_f64((double)c.eps)},         {"experts", json_u64(c.experts)},
        {"head_dim", json_u64(c.head_dim)},       {"heads", json_u64(c.heads)},
        {"hidden", json_u64(c.hidden)},           {"intermediate", json_u64(c.intermediate)},
        {"kvheads", json_u64(c.kvheads)},         {"layers", json_u64(c.layers)},
        {"max_context", json_u64(c.max_context)}, {"theta", qh::json_f64((double)c.theta)},
        {"top", json_u64(c.top)},                 {"vocab", json_u64(c.vocab)},
    };
    const size_t nc = sizeof cfg / sizeof cfg[0];
    for (size_t i = 0; i < nc; i++)
        s += std::string("    \"") + cfg[i].first + "\": " + cfg[i].second + (i + 1 < nc ? ",\n" : "\n");
    s += "  },\n";
    s += "  \"kv_f32_bytes_at_context\": " + json_u64(r.kv_f32_bytes_at_context) + ",\n";
    s += "  \"packed_weight_bytes\": " + json_u64(r.packed_weight_bytes) + ",\n";
    s += "  \"tensor_count\": " + json_u64(r.tensor_count) + "\n}\n";
    std::fwrite(s.data(), 1, s.size(), stdout);
    return 0;
}

int cmd_logits(const Args& a) {
    if (a.tokens.size() > a.ctx) throw Fail("tokens exceed context");
    if (a.device == "cpu")
        throw Fail("the cpu device is not part of this engine; use --device hip (the reference's CPU path "
                   "is the oracle of the test suite)");
    std::string name;
    const int dev = pick_device(a, name);
    qh_ctx* ctx = nullptr;
    if (qh_create(dev, &ctx) != 0) throw Fail(last_error(nullptr));
    struct Guard {
        qh_ctx* c;
        ~Guard() { qh_destroy(c); }
    } guard{ctx};
    if (qh_load_model_file(ctx, a.model.c_str(), a.ctx) != 0) throw Fail(last_error(ctx));
    std::fprintf(stderr, "HIP device: %s\n", name.c_str());
    qh_config_t cfg;
    if (qh_model_config(ctx, &cfg) != 0) throw Fail(last_error(ctx));
    std::vector<float> logits(cfg.vocab);
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t id : a.tokens) {
        uint32_t am = 0;
        if (qh_forward(ctx, id, logits.data(), logits.size(), &am) != 0) throw Fail(last_error(ctx));
    }
    const double seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    qh_stats_t st;
    if (qh_stats(ctx, &st) != 0) throw Fail(last_error(ctx));
    std::string s = "{\"logits\":[";
    s.reserve(logits.size() * 24 + 256);
    if (a.tokens.empty()) logits.clear();
    for (size_t i = 0; i < logits.size(); i++) {
        if (i) s += ',';
        s += qh::json_f64((double)logits[i]);
    }
    s += "],\"seconds\":" + qh::json_f64(seconds) + ",\"stats\":{\"cache_hits\":" + json_u64(st.cache_hits) +
         ",\"matvec_ms\":" + qh::json_f64(st.matvec_ms) + ",\"matvecs\":" + json_u64(st.matvecs) +
         ",\"uploaded_bytes\":" + json_u64(st.uploaded_bytes) + "}}\n";
    std::fwrite(s.data(), 1, s.size(), stdout);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const Args a = parse(argc, argv);
        if (a.command == "devices") return cmd_devices();
        if (a.command == "inspect") return cmd_inspect(a);
        return cmd_logits(a);
    } catch (const Usage& e) {
        std::fprintf(stderr, "error: %s\n\nFor more information, try '--help'.\n", e.what());
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
