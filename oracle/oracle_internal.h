/* Oracle internals shared between the oracle's C files.  TEST INFRASTRUCTURE. */
#ifndef QWEN_ORACLE_INTERNAL_H
#define QWEN_ORACLE_INTERNAL_H
#include <stddef.h>
#include <stdint.h>

int or_fail(const char *fmt, ...);
void or_decode_row_fast(const uint8_t *row, uint32_t kind, size_t cols, float *out);

/* Total order of f32 (Rust f32::total_cmp): returns <0, 0, >0. */
static inline int or_total_cmp(float a, float b) {
    union { float f; int32_t i; } ua = {a}, ub = {b};
    int32_t x = ua.i, y = ub.i;
    x ^= (int32_t)(((uint32_t)(x >> 31)) >> 1);
    y ^= (int32_t)(((uint32_t)(y >> 31)) >> 1);
    return (x > y) - (x < y);
}

static inline int or_isfinite(float v) {
    union { float f; uint32_t u; } x = {v};
    return (x.u & 0x7f800000u) != 0x7f800000u;
}

#endif
