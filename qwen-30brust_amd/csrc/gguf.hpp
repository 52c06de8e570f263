// GGUF v2/v3 image reader and qwen3moe config validation for the engine.
// Same checks and messages as src/gguf.rs:102-229 and src/model.rs:21-156;
// the image is a host buffer (or a read-only file mapping) instead of memmap2.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace qh {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct Meta {
    enum Tag { UINT, INT, FLOAT, BOOL, STR, ARRAY } tag = UINT;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t kind = 0;
    size_t offset = 0, len = 0;  // absolute offset in the image
};

struct Gguf {
    const uint8_t* data = nullptr;
    size_t len = 0;
    std::map<std::string, Meta> meta;
    std::map<std::string, Tensor> tensors;

    const Tensor& tensor(const std::string& name) const;  // "missing tensor {name}"
    bool has(const std::string& name) const { return tensors.count(name) != 0; }
    uint64_t uint(const std::string& key) const;          // "missing integer {key}"
    bool try_uint(const std::string& key, uint64_t& v) const;
    float flt(const std::string& key, float dflt) const;
    const std::string* str(const std::string& key) const;
    uint64_t packed_bytes() const;
};

// Parses and validates the image (buffer must outlive the result).
Gguf parse_gguf(const uint8_t* data, size_t len);

struct Config {
    uint64_t hidden, layers, heads, kvheads, head_dim, experts, top, intermediate, vocab,
        max_context;
    float eps, theta;
};

Config config_from_gguf(const Gguf& g);           // src/model.rs:21-90
void validate_tensors(const Config& c, const Gguf& g);  // src/model.rs:91-149

// GGML (elements, bytes) per block and row bytes, with the reference errors
// (src/quant.rs:5-21).
void check_layout(uint32_t kind);
size_t row_bytes_checked(uint32_t kind, uint64_t cols);

}  // namespace qh
