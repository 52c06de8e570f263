// Row engine shared by every matvec-shaped kernel.
//
// A wavefront computes dot products for a group of rows of one packed matrix.
// The row's chunks (32 weights, see qh_device.hpp) are spread over L lanes
// (L = next power of two >= chunks per row, capped at 64), so one wave covers
// S = 64 / L rows per "row step" and R row steps per pass: R*S rows share each
// x chunk, which is read once from LDS.  All R weight loads of a chunk are
// issued before any of them is consumed.
#pragma once
#include "qh_device.hpp"

namespace qh {

// Lanes per row for a matrix with `cols` columns.
QH_HD int lanes_per_row(uint32_t cols) {
    uint32_t cpr = (cols + 31) / 32;
    int L = 1;
    while (L < 64 && (uint32_t)L < cpr) L <<= 1;
    return L;
}

// Loads the two 16-float x runs of chunk c from LDS (zero-padded to a
// multiple of 32) and their sums.
template <uint32_t KIND>
__device__ __forceinline__ void x_runs(const float* xs, uint32_t c, float* xa, float* xb, float& sa,
                                       float& sb) {
    const float4* pa = reinterpret_cast<const float4*>(xs + Fmt<KIND>::xoff_a(c));
    const float4* pb = reinterpret_cast<const float4*>(xs + Fmt<KIND>::xoff_b(c));
    sa = 0.f;
    sb = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float4 a = pa[k], b = pb[k];
        xa[4 * k] = a.x; xa[4 * k + 1] = a.y; xa[4 * k + 2] = a.z; xa[4 * k + 3] = a.w;
        xb[4 * k] = b.x; xb[4 * k + 1] = b.y; xb[4 * k + 2] = b.z; xb[4 * k + 3] = b.w;
        sa += (a.x + a.y) + (a.z + a.w);
        sb += (b.x + b.y) + (b.z + b.w);
    }
}

// LDS layout of the gathered activation vectors: element i at px(i) =
// i + 4 (i / 64).  The lanes of one read take the 16-float runs of
// neighbouring chunks of a Q4_K/Q6_K row, 16-64 floats apart; unpadded, four
// of every eight lanes of a 16-byte read met in the same banks.  A run never
// crosses a 64-float block, so it stays contiguous.
__device__ __forceinline__ uint32_t px(uint32_t i) { return i + ((i >> 6) << 2); }

// x_runs (the two 16-float runs of chunk c and their sums) of the vector
// that starts at element `base` of a padded LDS vector.
template <uint32_t KIND>
__device__ __forceinline__ void x_runs_p(const float* xs, uint32_t base, uint32_t c, float* xa, float* xb, float& sa,
                                         float& sb) {
    const uint32_t fa = base + Fmt<KIND>::xoff_a(c), fb = base + Fmt<KIND>::xoff_b(c);
    const float4* pa = reinterpret_cast<const float4*>(xs + px(fa));
    const float4* pb = reinterpret_cast<const float4*>(xs + px(fb));
    sa = 0.f;
    sb = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 a = pa[k], b = pb[k];
        xa[4 * k] = a.x; xa[4 * k + 1] = a.y; xa[4 * k + 2] = a.z; xa[4 * k + 3] = a.w;
        xb[4 * k] = b.x; xb[4 * k + 1] = b.y; xb[4 * k + 2] = b.z; xb[4 * k + 3] = b.w;
        sa += (a.x + a.y) + (a.z + a.w);
        sb += (b.x + b.y) + (b.z + b.w);
    }
}

// Chunk load with a column bound: F32/F16 rows may end inside a chunk; the
// missing weights read as zero.  Quantized formats always hold whole blocks.
template <uint32_t KIND>
__device__ __forceinline__ typename Fmt<KIND>::Raw load_chunk(const uint8_t* row, const RowGeo& g,
                                                              uint32_t c, uint32_t cols) {
    if constexpr (KIND == F32 || KIND == F16) {
        if ((c + 1) * 32 > cols) {
            typename Fmt<KIND>::Raw r;
            uint32_t* w = reinterpret_cast<uint32_t*>(&r);
            if constexpr (KIND == F32) {
                for (int i = 0; i < 32; i++)
                    w[i] = c * 32 + i < cols ? reinterpret_cast<const uint32_t*>(row)[c * 32 + i] : 0u;
            } else {
                for (int i = 0; i < 16; i++) {
                    uint32_t e0 = c * 32 + 2 * i, e1 = e0 + 1;
                    uint32_t lo = e0 < cols ? ld_u16(row + 2 * e0) : 0u;
                    uint32_t hi = e1 < cols ? ld_u16(row + 2 * e1) : 0u;
                    w[i] = lo | (hi << 16);
                }
            }
            return r;
        }
    }
    return Fmt<KIND>::load(row, g, c);
}

// Computes, for k < R, acc[k] = dot(row rowsel(k), x) restricted to the chunks
// owned by this lane (chunk cl, cl+L, ...).  rowsel(k) returns a row pointer
// or nullptr for "no row".  The caller reduces acc over the L-lane segment.
template <uint32_t KIND, int R, typename RowSel>
__device__ __forceinline__ void rows_dot(RowSel rowsel, const RowGeo& g, const float* xs,
                                         uint32_t cols, int L, int cl, float (&acc)[R]) {
    const uint32_t cpr = (cols + 31) / 32;
    const uint8_t* rp[R];
#pragma unroll
    for (int k = 0; k < R; k++) {
        rp[k] = rowsel(k);
        acc[k] = 0.f;
    }
    for (uint32_t c = cl; c < cpr; c += L) {
        typename Fmt<KIND>::Raw raw[R];
#pragma unroll
        for (int k = 0; k < R; k++)
            if (rp[k]) raw[k] = load_chunk<KIND>(rp[k], g, c, cols);
        float xa[16], xb[16], sa, sb;
        x_runs<KIND>(xs, c, xa, xb, sa, sb);
#pragma unroll
        for (int k = 0; k < R; k++)
            if (rp[k]) acc[k] += Fmt<KIND>::dot(raw[k], c, xa, xb, sa, sb);
    }
}

// Dispatches a runtime kind to the templated row engine.
#define QH_DISPATCH_KIND(kind, ...)                                                   \
    switch (kind) {                                                                   \
    case ::qh::F32: { constexpr uint32_t K_ = ::qh::F32; __VA_ARGS__; } break;        \
    case ::qh::F16: { constexpr uint32_t K_ = ::qh::F16; __VA_ARGS__; } break;        \
    case ::qh::Q4_0: { constexpr uint32_t K_ = ::qh::Q4_0; __VA_ARGS__; } break;      \
    case ::qh::Q8_0: { constexpr uint32_t K_ = ::qh::Q8_0; __VA_ARGS__; } break;      \
    case ::qh::Q4_K: { constexpr uint32_t K_ = ::qh::Q4_K; __VA_ARGS__; } break;      \
    case ::qh::Q5_K: { constexpr uint32_t K_ = ::qh::Q5_K; __VA_ARGS__; } break;      \
    case ::qh::Q6_K: { constexpr uint32_t K_ = ::qh::Q6_K; __VA_ARGS__; } break;      \
    default: break;                                                                   \
    }

// The same over the block-quantised kinds only (compact register tiles).
#define QH_DISPATCH_QUANT(kind, ...)                                                  \
    switch (kind) {                                                                   \
    case ::qh::Q4_0: { constexpr uint32_t K_ = ::qh::Q4_0; __VA_ARGS__; } break;      \
    case ::qh::Q8_0: { constexpr uint32_t K_ = ::qh::Q8_0; __VA_ARGS__; } break;      \
    case ::qh::Q4_K: { constexpr uint32_t K_ = ::qh::Q4_K; __VA_ARGS__; } break;      \
    case ::qh::Q5_K: { constexpr uint32_t K_ = ::qh::Q5_K; __VA_ARGS__; } break;      \
    case ::qh::Q6_K: { constexpr uint32_t K_ = ::qh::Q6_K; __VA_ARGS__; } break;      \
    default: break;                                                                   \
    }

QH_HD bool is_quant(uint32_t kind) { return kind == Q4_0 || kind == Q8_0 || kind == Q4_K || kind == Q5_K || kind == Q6_K; }

}  // namespace qh
