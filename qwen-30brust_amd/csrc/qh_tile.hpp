// Register tiles: a wavefront's whole share of a matrix, loaded up front.
//
// Decode matvecs are latency-bound: a load that waits for an earlier
// dependent step costs a full memory round trip.  A RowTile therefore issues
// every chunk load of its R rows (C chunk slots per lane) before any of them
// is consumed, so the kernel can start its activation loads and reductions
// while the weights are in flight, and then compute from registers.
//
// Lane cl of a row owns chunks cl, cl + L, ..., cl + (C-1)L (L = lanes per
// row); rows beyond the matrix or chunks beyond the row are skipped.
#pragma once
#include "qh_rows.hpp"

namespace qh {

// Lane cl of a row owns chunks cl, cl + L, ..., cl + (C-1)L.  C = 0 is the
// general form for any row length and format: only the row pointers are
// kept, and dot() walks the lane's chunks loading each as it goes.
template <uint32_t KIND, int R, int C>
struct RowTile {
    using Raw = typename Fmt<KIND>::Raw;
    static constexpr bool kHeld = C > 0;
    Raw raw[kHeld ? R : 1][kHeld ? C : 1];
    const uint8_t* rp[R];

    template <class RowSel>
    __device__ __forceinline__ void load(RowSel rowsel, const RowGeo& g, uint32_t cols, int L, int cl) {
        const uint32_t cpr = (cols + 31) / 32;
#pragma unroll
        for (int k = 0; k < R; k++) {
            rp[k] = rowsel(k);
            if constexpr (kHeld) {
#pragma unroll
                for (int c = 0; c < C; c++) {
                    const uint32_t ch = cl + c * L;
                    if (rp[k] && ch < cpr) raw[k][c] = load_chunk<KIND>(rp[k], g, ch, cols);
                }
            }
        }
    }

    // acc[k] = this lane's share of row k's dot with xs (zero-padded LDS).
    __device__ __forceinline__ void dot(const float* xs, const RowGeo& g, uint32_t cols, int L, int cl,
                                        float (&acc)[R]) const {
        const uint32_t cpr = (cols + 31) / 32;
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = 0.f;
        if constexpr (kHeld) {
#pragma unroll
            for (int c = 0; c < C; c++) {
                const uint32_t ch = cl + c * L;
                if (ch < cpr) {
                    float xa[16], xb[16], sa, sb;
                    x_runs<KIND>(xs, ch, xa, xb, sa, sb);
#pragma unroll
                    for (int k = 0; k < R; k++)
                        if (rp[k]) acc[k] += Fmt<KIND>::dot(raw[k][c], ch, xa, xb, sa, sb);
                }
            }
        } else {
            for (uint32_t ch = cl; ch < cpr; ch += L) {
                float xa[16], xb[16], sa, sb;
                x_runs<KIND>(xs, ch, xa, xb, sa, sb);
#pragma unroll
                for (int k = 0; k < R; k++)
                    if (rp[k]) acc[k] += Fmt<KIND>::dot(load_chunk<KIND>(rp[k], g, ch, cols), ch, xa, xb, sa, sb);
            }
        }
    }
};

// Runs the body with K_ bound to the format `kind`: over the block-quantised
// formats for a held tile (C > 0), over every format for C = 0.
#define QH_DISPATCH_TILE(C, kind, ...)                            \
    do {                                                          \
        if constexpr ((C) > 0) {                                  \
            QH_DISPATCH_QUANT(kind, __VA_ARGS__);                 \
        } else {                                                  \
            QH_DISPATCH_KIND(kind, __VA_ARGS__);                  \
        }                                                         \
    } while (0)

// Held chunk slots per lane for rows of `cols` columns of format `kind`
// spread over lanes_per_row(cols) lanes: 1 or 2 for block-quantised formats
// (rows of up to 4096 columns), 0 (the general chunk loop) otherwise.
QH_HD int tile_slots(uint32_t kind, uint32_t cols) {
    if (!is_quant(kind)) return 0;
    const uint32_t cpr = (cols + 31) / 32, L = (uint32_t)lanes_per_row(cols);
    const uint32_t c = (cpr + L - 1) / L;
    return c <= 1 ? 1 : c <= 2 ? 2 : 0;
}

}  // namespace qh
