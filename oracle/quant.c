/*
 * Oracle: GGML block decoding, restated from src/quant.rs.  TEST
 * INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Format table (quant.rs:5-11): kind -> (elements per block, bytes per block)
 *   F32 0 (1,4)  F16 1 (1,2)  Q4_0 2 (32,18)  Q8_0 8 (32,34)
 *   Q4_K 12 (256,144)  Q5_K 13 (256,176)  Q6_K 14 (256,210)
 */
#include "oracle.h"
#include "oracle_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

static _Thread_local char g_err[512];

const char *or_last_error(void) { return g_err; }

int or_fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

/* quant.rs:5-11 */
int or_layout(uint32_t kind, size_t *block, size_t *bytes) {
    size_t b, n;
    switch (kind) {
    case 0: b = 1; n = 4; break;
    case 1: b = 1; n = 2; break;
    case 2: b = 32; n = 18; break;
    case 8: b = 32; n = 34; break;
    case 12: b = 256; n = 144; break;
    case 13: b = 256; n = 176; break;
    case 14: b = 256; n = 210; break;
    default:
        return or_fail("GGML tensor type %u is not supported "
                       "(supported: F32/F16/Q4_0/Q8_0/Q4_K/Q5_K/Q6_K)", kind);
    }
    if (block) *block = b;
    if (bytes) *bytes = n;
    return 0;
}

/* quant.rs:12-21 */
int or_row_bytes(uint32_t kind, size_t cols, size_t *out) {
    size_t block, bytes;
    if (or_layout(kind, &block, &bytes)) return -1;
    if (cols == 0 || cols % block != 0)
        return or_fail("row width %zu is not divisible by block size %zu", cols, block);
    size_t n = cols / block;
    if (n > SIZE_MAX / bytes) return or_fail("row size overflow");
    *out = n * bytes;
    return 0;
}

/* quant.rs:22-24.  IEEE binary16 -> binary32 widening (exact).  NaNs come
 * out quiet with the payload shifted into the top of the f32 mantissa, as
 * both the `half` crate's software path and the x86 F16C instruction do. */
float or_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24; normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man ? (0x00400000u | (man << 13)) : 0);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float h_at(const uint8_t *b, size_t p) {
    return or_f16((uint16_t)(b[p] | (b[p + 1] << 8)));
}

/* quant.rs:25-34: 6-bit (scale, min) of sub-block j from the 12 packed bytes */
void or_kscale(const uint8_t *b, size_t j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = b[j] & 63;
        *m = b[j + 4] & 63;
    } else {
        *sc = (uint8_t)((b[j + 4] & 15) | ((b[j - 4] >> 6) << 4));
        *m = (uint8_t)((b[j + 4] >> 4) | ((b[j] >> 6) << 4));
    }
}

/* quant.rs:36-80.  Caller supplies a validated row and an in-range column. */
float or_value(const uint8_t *b, uint32_t kind, size_t col) {
    switch (kind) {
    case 0: {
        float f;
        memcpy(&f, b + col * 4, 4);
        return f;
    }
    case 1:
        return h_at(b, col * 2);
    case 2: { /* quant.rs:40-45 */
        size_t p = col / 32 * 18, i = col % 32;
        int q = (b[p + 2 + i % 16] >> (i < 16 ? 0 : 4)) & 15;
        return h_at(b, p) * (float)(q - 8);
    }
    case 8: { /* quant.rs:46-49 */
        size_t p = col / 32 * 34;
        return h_at(b, p) * (float)(int8_t)b[p + 2 + col % 32];
    }
    case 12:
    case 13: { /* quant.rs:50-62 */
        size_t size = kind == 12 ? 144 : 176;
        size_t p = col / 256 * size, i = col % 256, group = i / 32;
        uint8_t s, m;
        or_kscale(b + p + 4, group, &s, &m);
        size_t qs = p + (kind == 12 ? 16 : 48);
        unsigned q = (b[qs + (i / 64) * 32 + i % 32] >> ((group % 2) * 4)) & 15;
        if (kind == 13 && (b[p + 16 + i % 32] & (1u << group))) q += 16;
        /* ((d * sc) * q) - (dmin * m), each step rounded */
        return h_at(b, p) * (float)s * (float)q - h_at(b, p + 2) * (float)m;
    }
    case 14: { /* quant.rs:63-77 */
        size_t p = col / 256 * 210, i = col % 256;
        size_t chunk = i / 128, j = i % 128, quarter = j / 32, lane = j % 32;
        uint8_t low = b[p + chunk * 64 + (quarter % 2) * 32 + lane];
        unsigned lo = (low >> ((quarter / 2) * 4)) & 15;
        unsigned hi = (b[p + 128 + chunk * 32 + lane] >> (quarter * 2)) & 3;
        int q = (int)(lo | (hi << 4)) - 32;
        return h_at(b, p + 208) * (float)(int8_t)b[p + 192 + chunk * 8 + quarter * 2 + lane / 16] *
               (float)q;
    }
    default:
        return 0.f; /* unreachable: kinds validated by the reader */
    }
}

/* quant.rs:81-84 */
int or_decode(const uint8_t *b, size_t len, uint32_t kind, size_t cols, float *out) {
    size_t rb;
    if (or_row_bytes(kind, cols, &rb)) return -1;
    if (len < rb) return or_fail("truncated quantized row");
    for (size_t i = 0; i < cols; i++) out[i] = or_value(b, kind, i);
    return 0;
}

/* Block-at-a-time decode of a whole row: the same formulas as or_value with
 * the per-block header decoded once.  Produces the identical floats. */
void or_decode_row_fast(const uint8_t *b, uint32_t kind, size_t cols, float *out) {
    switch (kind) {
    case 12:
    case 13: {
        size_t size = kind == 12 ? 144 : 176;
        for (size_t blk = 0; blk < cols / 256; blk++) {
            const uint8_t *p = b + blk * size;
            float d = h_at(p, 0), dmin = h_at(p, 2);
            const uint8_t *qs = p + (kind == 12 ? 16 : 48);
            for (size_t g = 0; g < 8; g++) {
                uint8_t s, m;
                or_kscale(p + 4, g, &s, &m);
                float ds = d * (float)s, mm = dmin * (float)m;
                for (size_t l = 0; l < 32; l++) {
                    unsigned q = (qs[(g / 2) * 32 + l] >> ((g % 2) * 4)) & 15;
                    if (kind == 13 && (p[16 + l] & (1u << g))) q += 16;
                    out[blk * 256 + g * 32 + l] = ds * (float)q - mm;
                }
            }
        }
        return;
    }
    case 14: {
        for (size_t blk = 0; blk < cols / 256; blk++) {
            const uint8_t *p = b + blk * 210;
            float d = h_at(p, 208);
            for (size_t chunk = 0; chunk < 2; chunk++)
                for (size_t quarter = 0; quarter < 4; quarter++)
                    for (size_t lane = 0; lane < 32; lane++) {
                        uint8_t low = p[chunk * 64 + (quarter % 2) * 32 + lane];
                        unsigned lo = (low >> ((quarter / 2) * 4)) & 15;
                        unsigned hi = (p[128 + chunk * 32 + lane] >> (quarter * 2)) & 3;
                        int q = (int)(lo | (hi << 4)) - 32;
                        float ds = d * (float)(int8_t)p[192 + chunk * 8 + quarter * 2 + lane / 16];
                        out[blk * 256 + chunk * 128 + quarter * 32 + lane] = ds * (float)q;
                    }
        }
        return;
    }
    default:
        for (size_t i = 0; i < cols; i++) out[i] = or_value(b, kind, i);
    }
}
