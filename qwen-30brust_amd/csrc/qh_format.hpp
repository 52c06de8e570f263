// Block formats and the engine's device row layout.
//
// GGUF stores quantized rows as arrays of self-contained blocks
// (src/quant.rs:5-11).  On the device every row is repacked at load time into
// a struct-of-arrays layout: each block field is gathered into its own
// contiguous run, and the row is padded to a 16-byte multiple.  The bytes are
// the same bytes (dequantized values are bit-identical), but every field run
// starts 16-byte aligned, so a wavefront reads each run with coalesced
// 128-bit loads.  (Q6_K blocks are 210 bytes and otherwise only 2-byte
// aligned.)
//
//   kind   GGUF block                          device row (nb = cols / block)
//   F32    f32                                 f32[cols]
//   F16    f16                                 f16[cols]               (+pad)
//   Q4_0   d f16 | qs[16]                      qs[nb][16] | d[nb]      (+pad)
//   Q8_0   d f16 | qs[32]                      qs[nb][32] | d[nb]      (+pad)
//   Q4_K   d | dmin | sc[12] | qs[128]         hdr[nb][16] | qs[nb][128]
//   Q5_K   d | dmin | sc[12] | qh[32] | qs[128] hdr[nb][16] | qh[nb][32] | qs[nb][128]
//   Q6_K   ql[128] | qh[64] | sc[16] | d f16   ql[nb][128] | qh[nb][64] | sc[nb][16] | d[nb] (+pad)
// where hdr = the first 16 GGUF bytes of the block (d, dmin, 12 scale bytes).
#pragma once
#include <cstddef>
#include <cstdint>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define QH_HD __host__ __device__ __forceinline__
#else
#define QH_HD inline
#endif

namespace qh {

enum Kind : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

// (elements per block, bytes per block); false for unsupported kinds.
QH_HD bool layout(uint32_t kind, uint32_t& block, uint32_t& bytes) {
    switch (kind) {
    case F32: block = 1; bytes = 4; return true;
    case F16: block = 1; bytes = 2; return true;
    case Q4_0: block = 32; bytes = 18; return true;
    case Q8_0: block = 32; bytes = 34; return true;
    case Q4_K: block = 256; bytes = 144; return true;
    case Q5_K: block = 256; bytes = 176; return true;
    case Q6_K: block = 256; bytes = 210; return true;
    default: return false;
    }
}

QH_HD size_t gguf_row_bytes(uint32_t kind, size_t cols) {
    uint32_t b, n;
    layout(kind, b, n);
    return cols / b * n;
}

// Device row stride in bytes (GGUF row bytes rounded up to 16).
QH_HD size_t dev_row_bytes(uint32_t kind, size_t cols) {
    return (gguf_row_bytes(kind, cols) + 15) / 16 * 16;
}

// Byte offsets of the field runs inside one device row.
struct RowGeo {
    uint32_t nb;        // blocks per row
    uint32_t off_a;     // Q4_0/Q8_0: qs   Q4_K/Q5_K: hdr  Q6_K: ql
    uint32_t off_b;     // Q4_0/Q8_0: d    Q4_K: qs  Q5_K: qh  Q6_K: qh
    uint32_t off_c;     // Q5_K: qs  Q6_K: sc
    uint32_t off_d;     // Q6_K: d
};

QH_HD RowGeo row_geo(uint32_t kind, size_t cols) {
    RowGeo g{};
    uint32_t b, n;
    layout(kind, b, n);
    g.nb = (uint32_t)(cols / b);
    switch (kind) {
    case Q4_0: g.off_a = 0; g.off_b = 16 * g.nb; break;
    case Q8_0: g.off_a = 0; g.off_b = 32 * g.nb; break;
    case Q4_K: g.off_a = 0; g.off_b = 16 * g.nb; break;
    case Q5_K: g.off_a = 0; g.off_b = 16 * g.nb; g.off_c = 48 * g.nb; break;
    case Q6_K: g.off_a = 0; g.off_b = 128 * g.nb; g.off_c = 192 * g.nb; g.off_d = 208 * g.nb; break;
    default: break;
    }
    return g;
}

// Where byte `j` of GGUF block `blk` lands in the device row (j < bytes).
QH_HD uint32_t dev_offset(uint32_t kind, const RowGeo& g, uint32_t blk, uint32_t j) {
    switch (kind) {
    case Q4_0: return j < 2 ? g.off_b + 2 * blk + j : g.off_a + 16 * blk + (j - 2);
    case Q8_0: return j < 2 ? g.off_b + 2 * blk + j : g.off_a + 32 * blk + (j - 2);
    case Q4_K: return j < 16 ? g.off_a + 16 * blk + j : g.off_b + 128 * blk + (j - 16);
    case Q5_K:
        return j < 16 ? g.off_a + 16 * blk + j
                      : (j < 48 ? g.off_b + 32 * blk + (j - 16) : g.off_c + 128 * blk + (j - 48));
    case Q6_K:
        return j < 128   ? g.off_a + 128 * blk + j
               : j < 192 ? g.off_b + 64 * blk + (j - 128)
               : j < 208 ? g.off_c + 16 * blk + (j - 192)
                         : g.off_d + 2 * blk + (j - 208);
    default: {
        uint32_t b, n;
        layout(kind, b, n);
        return blk * n + j;  // F32 / F16: unchanged
    }
    }
}

}  // namespace qh
