// Device codec for the engine's row layout (qh_format.hpp).
//
// The unit of work is a "chunk": 32 weights of one row whose bytes a lane
// fetches with 16-byte loads.  Chunk c of a row touches two runs of 16
// consecutive columns, xa = x[xoff_a(c) .. +16) and xb = x[xoff_b(c) .. +16),
// because the K-quant formats interleave two sub-blocks per qs byte (low and
// high nibble).  Each format provides
//   load(row, geo, c)             -> Raw (the chunk's packed bytes + scales)
//   dot(raw, c, xa, xb, sa, sb)   -> sum over the chunk of w[i] * x[i]
// where sa / sb are the sums of xa / xb (used to fold the per-sub-block
// offsets: sum x*(ds*q - dm*m) = ds*sum(x*q) - dm*m*sum(x)).
//
// dequant_value() is the bit-exact element decoder (same operation order as
// src/quant.rs:36-80, contraction disabled).
#pragma once
#include <hip/hip_runtime.h>

#include "qh_format.hpp"

namespace qh {

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t k) { return (w >> (8 * k)) & 0xffu; }
__device__ __forceinline__ uint32_t byte_of(const uint4& v, uint32_t k) {
    uint32_t w = k < 4 ? v.x : k < 8 ? v.y : k < 12 ? v.z : v.w;
    return byte_of(w, k & 3);
}

// K-quant 6-bit (scale, min) of sub-block j from the 12 scale bytes held in
// s0 (bytes 0-3), s1 (4-7), s2 (8-11) -- src/quant.rs:25-34.
__device__ __forceinline__ void kscale(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j,
                                       uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = byte_of(s0, j) & 63;
        m = byte_of(s1, j) & 63;
    } else {
        uint32_t k = j - 4;
        sc = (byte_of(s2, k) & 15) | ((byte_of(s0, k) >> 6) << 4);
        m = (byte_of(s2, k) >> 4) | ((byte_of(s1, k) >> 6) << 4);
    }
}

// Loads from device memory through global-address-space pointers: they
// compile to global_load (counted by vmcnt only).  A load through a generic
// pointer of unknown origin compiles to flat_load, which also counts in
// lgkmcnt, so every later LDS wait would wait for it as well.
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ T gld(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(gptr<T>)p;
#else
    return *static_cast<const T*>(p);  // host pass: never executed
#endif
}
__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return gld<uint4>(p); }
// The same load marked non-temporal (the weight chunks of load() below: the
// token step reads each weight row once per token, and keeping those
// streams from allocating as reusable lines in the vector L1 measured 1.5 %
// faster per token).
__device__ __forceinline__ uint4 ld16s(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v t = __builtin_nontemporal_load((gptr<u4v>)p);
    return make_uint4(t.x, t.y, t.z, t.w);
#else
    return *reinterpret_cast<const uint4*>(p);  // host pass: never executed
#endif
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return gld<uint16_t>(p); }

// Hides a value from the optimiser's known-bits analysis, so that byte k of a
// pre-masked word still converts with one v_cvt_f32_ubyte<k> instead of a
// bitfield extract plus convert.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Four bytes of `w` as floats, multiplied into x[0..4) and accumulated.
__device__ __forceinline__ float dot4u8(uint32_t w, const float* x, float acc) {
    w = opaque(w);
    acc = fmaf(x[0], (float)(w & 0xffu), acc);
    acc = fmaf(x[1], (float)((w >> 8) & 0xffu), acc);
    acc = fmaf(x[2], (float)((w >> 16) & 0xffu), acc);
    acc = fmaf(x[3], (float)(w >> 24), acc);
    return acc;
}

// 6-bit (scale, min) of the sub-block pair (2p, 2p+1), p in 0..3, from the
// 12 scale bytes in s0 (bytes 0-3), s1 (4-7), s2 (8-11), branch-free
// (src/quant.rs:25-34).  Returns byte 0 = value of sub-block 2p, byte 1 =
// value of 2p+1.
__device__ __forceinline__ void kscale_pair(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t p,
                                            uint32_t& sc, uint32_t& m) {
    const uint32_t sh = (p & 1) * 16;
    const uint32_t Y = (s0 >> sh) & 0xffffu, Z = (s1 >> sh) & 0xffffu, W = (s2 >> sh) & 0xffffu;
    const uint32_t scA = Y & 0x3f3fu, mA = Z & 0x3f3fu;
    const uint32_t scB = (W & 0x0f0fu) | ((Y >> 2) & 0x3030u);
    const uint32_t mB = ((W >> 4) & 0x0f0fu) | ((Z >> 2) & 0x3030u);
    sc = p < 2 ? scA : scB;
    m = p < 2 ? mA : mB;
}

template <uint32_t KIND> struct Fmt;

// -------------------------------------------------------------------- Q4_K --
template <> struct Fmt<Q4_K> {
    struct Raw { uint4 q, h; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) {
        uint32_t j = c & 7;
        return (c >> 3) * 256 + (j >> 1) * 64 + (j & 1) * 16;
    }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return xoff_a(c) + 32; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo& g, uint32_t c) {
        uint32_t b = c >> 3, j = c & 7;
        return {ld16s(row + g.off_b + b * 128 + j * 16), ld16s(row + g.off_a + b * 16)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t c, const float* xa,
                                                const float* xb, float sa, float sb) {
        uint32_t scp, mp;
        kscale_pair(r.h.y, r.h.z, r.h.w, (c & 7) >> 1, scp, mp);
        const float sca = (float)(scp & 0xffu), scb = (float)(scp >> 8), ma = (float)(mp & 0xffu),
                    mb = (float)(mp >> 8);
        float d = h2f(r.h.x & 0xffff), dm = h2f(r.h.x >> 16);
        uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float pa = 0.f, pb = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            pa = dot4u8(w[k] & 0x0f0f0f0fu, xa + 4 * k, pa);
            pb = dot4u8((w[k] >> 4) & 0x0f0f0f0fu, xb + 4 * k, pb);
        }
        return d * (sca * pa + scb * pb) - dm * (ma * sa + mb * sb);
    }
};

// -------------------------------------------------------------------- Q5_K --
template <> struct Fmt<Q5_K> {
    struct Raw { uint4 q, h, qh; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) { return Fmt<Q4_K>::xoff_a(c); }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return xoff_a(c) + 32; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo& g, uint32_t c) {
        uint32_t b = c >> 3, j = c & 7;
        return {ld16s(row + g.off_c + b * 128 + j * 16), ld16s(row + g.off_a + b * 16),
                ld16s(row + g.off_b + b * 32 + (j & 1) * 16)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t c, const float* xa,
                                                const float* xb, float sa, float sb) {
        const uint32_t ga = ((c & 7) >> 1) * 2;
        uint32_t scp, mp;
        kscale_pair(r.h.y, r.h.z, r.h.w, (c & 7) >> 1, scp, mp);
        const float sca = (float)(scp & 0xffu), scb = (float)(scp >> 8), ma = (float)(mp & 0xffu),
                    mb = (float)(mp >> 8);
        float d = h2f(r.h.x & 0xffff), dm = h2f(r.h.x >> 16);
        uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t hb[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        float pa = 0.f, pb = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t qa = (w[k] & 0x0f0f0f0fu) | (((hb[k] >> ga) & 0x01010101u) << 4);
            uint32_t qb = ((w[k] >> 4) & 0x0f0f0f0fu) | (((hb[k] >> (ga + 1)) & 0x01010101u) << 4);
            pa = dot4u8(qa, xa + 4 * k, pa);
            pb = dot4u8(qb, xb + 4 * k, pb);
        }
        return d * (sca * pa + scb * pb) - dm * (ma * sa + mb * sb);
    }
};

// -------------------------------------------------------------------- Q6_K --
template <> struct Fmt<Q6_K> {
    // ql, qh of the chunk; the 8 scale bytes of its half-block (selected in
    // dot(), so that load() only issues loads); the aligned 32-bit word
    // holding d (a 16-bit load would give the value a 16-bit type, whose
    // widening the compiler then places right after the load, where it waits
    // for it)
    struct Raw { uint4 ql, qh; uint2 s8; uint32_t d; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) {
        uint32_t j = c & 7;
        return (c >> 3) * 256 + (j >> 2) * 128 + ((j & 3) >> 1) * 32 + (j & 1) * 16;
    }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return xoff_a(c) + 64; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo& g, uint32_t c) {
        uint32_t b = c >> 3, j = c & 7;
        return {ld16s(row + g.off_a + b * 128 + j * 16),
                ld16s(row + g.off_b + b * 64 + (j >> 2) * 32 + (j & 1) * 16),
                gld<uint2>(row + g.off_c + b * 16 + (j >> 2) * 8),
                gld<uint32_t>(row + g.off_d + (b >> 1) * 4)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t c, const float* xa,
                                                const float* xb, float sa, float sb) {
        // scales of this chunk: sc[(j>>2)*8 + qa*2 + (j&1)] (quarter qa) and +4
        // (quarter qa+2), bytes sh/8 of the two words of s8
        const uint32_t jj = c & 7, sh = (((jj & 3) >> 1) * 2 + (jj & 1)) * 8;
        const uint32_t rsc = ((r.s8.x >> sh) & 0xffu) | (((r.s8.y >> sh) & 0xffu) << 8);
        uint32_t j = c & 7, qa = (j & 3) >> 1;
        float sca = (float)(int8_t)(rsc & 0xffu), scb = (float)(int8_t)(rsc >> 8);
        // opaque: the conversion stays here, after the caller's waits; hoisted
        // next to the load it made the loading code wait for the load
        const uint32_t dw = opaque(r.d);
        float d = h2f(((c >> 3) & 1) ? dw >> 16 : dw);
        uint32_t l[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
        uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        float pa = 0.f, pb = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t ua = (l[k] & 0x0f0f0f0fu) | ((h[k] << (4 - 2 * qa)) & 0x30303030u);
            uint32_t ub = ((l[k] >> 4) & 0x0f0f0f0fu) | ((h[k] >> (2 * qa)) & 0x30303030u);
            pa = dot4u8(ua, xa + 4 * k, pa);
            pb = dot4u8(ub, xb + 4 * k, pb);
        }
        return d * (sca * (pa - 32.f * sa) + scb * (pb - 32.f * sb));
    }
};

// -------------------------------------------------------------------- Q4_0 --
template <> struct Fmt<Q4_0> {
    struct Raw { uint4 q; uint32_t d; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) { return c * 32; }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return c * 32 + 16; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo& g, uint32_t c) {
        // d in the aligned 32-bit word holding it (the row is padded past it)
        return {ld16s(row + g.off_a + c * 16), gld<uint32_t>(row + g.off_b + (c >> 1) * 4)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t c, const float* xa,
                                                const float* xb, float sa, float sb) {
        uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float p = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            p = dot4u8(w[k] & 0x0f0f0f0fu, xa + 4 * k, p);
            p = dot4u8((w[k] >> 4) & 0x0f0f0f0fu, xb + 4 * k, p);
        }
        return h2f((c & 1) ? r.d >> 16 : r.d) * (p - 8.f * (sa + sb));
    }
};

// -------------------------------------------------------------------- Q8_0 --
template <> struct Fmt<Q8_0> {
    struct Raw { uint4 a, b; uint32_t d; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) { return c * 32; }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return c * 32 + 16; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo& g, uint32_t c) {
        return {ld16s(row + g.off_a + c * 32), ld16s(row + g.off_a + c * 32 + 16),
                gld<uint32_t>(row + g.off_b + (c >> 1) * 4)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t c, const float* xa,
                                                const float* xb, float sa, float sb) {
        // bytes ^ 0x80 = q + 128 (unsigned); subtract 128 * sum(x) afterwards
        uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        float p = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) p = dot4u8(w[k] ^ 0x80808080u, xa + 4 * k, p);
#pragma unroll
        for (int k = 0; k < 4; k++) p = dot4u8(w[4 + k] ^ 0x80808080u, xb + 4 * k, p);
        return h2f((c & 1) ? r.d >> 16 : r.d) * (p - 128.f * (sa + sb));
    }
};

// --------------------------------------------------------------------- F16 --
template <> struct Fmt<F16> {
    struct Raw { uint4 a, b, c, d; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) { return c * 32; }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return c * 32 + 16; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo&, uint32_t c) {
        const uint8_t* p = row + c * 64;
        return {ld16s(p), ld16s(p + 16), ld16s(p + 32), ld16s(p + 48)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t, const float* xa,
                                                const float* xb, float, float) {
        uint32_t w[16] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w,
                          r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
        float p = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            p = fmaf(xa[2 * k], h2f(w[k] & 0xffff), p);
            p = fmaf(xa[2 * k + 1], h2f(w[k] >> 16), p);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            p = fmaf(xb[2 * k], h2f(w[8 + k] & 0xffff), p);
            p = fmaf(xb[2 * k + 1], h2f(w[8 + k] >> 16), p);
        }
        return p;
    }
};

// --------------------------------------------------------------------- F32 --
template <> struct Fmt<F32> {
    struct Raw { float4 v[8]; };
    static __device__ __forceinline__ uint32_t xoff_a(uint32_t c) { return c * 32; }
    static __device__ __forceinline__ uint32_t xoff_b(uint32_t c) { return c * 32 + 16; }
    static __device__ __forceinline__ Raw load(const uint8_t* row, const RowGeo&, uint32_t c) {
        Raw r;
#pragma unroll
        for (int k = 0; k < 8; k++) r.v[k] = gld<float4>(row + c * 128 + 16 * k);
        return r;
    }
    static __device__ __forceinline__ float dot(const Raw& r, uint32_t, const float* xa,
                                                const float* xb, float, float) {
        float p = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            p = fmaf(xa[4 * k], r.v[k].x, p);
            p = fmaf(xa[4 * k + 1], r.v[k].y, p);
            p = fmaf(xa[4 * k + 2], r.v[k].z, p);
            p = fmaf(xa[4 * k + 3], r.v[k].w, p);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            p = fmaf(xb[4 * k], r.v[4 + k].x, p);
            p = fmaf(xb[4 * k + 1], r.v[4 + k].y, p);
            p = fmaf(xb[4 * k + 2], r.v[4 + k].z, p);
            p = fmaf(xb[4 * k + 3], r.v[4 + k].w, p);
        }
        return p;
    }
};

// ------------------------------------------------- bit-exact element decode --
// Same operation order as src/quant.rs:36-80: Q4_K/Q5_K ((d*sc)*q) - (dmin*m),
// Q6_K (d*sc)*q, Q4_0 d*(q-8), Q8_0 d*q; every product and difference
// rounded on its own (no contraction).
__device__ __forceinline__ float dequant_value(const uint8_t* row, uint32_t kind, const RowGeo& g,
                                               uint32_t col) {
#pragma clang fp contract(off)
    switch (kind) {
    case F32: return reinterpret_cast<const float*>(row)[col];
    case F16: return h2f(ld_u16(row + 2 * col));
    case Q4_0: {
        uint32_t b = col / 32, i = col % 32;
        uint32_t q = (row[g.off_a + 16 * b + (i % 16)] >> (i < 16 ? 0 : 4)) & 15;
        return h2f(ld_u16(row + g.off_b + 2 * b)) * (float)((int)q - 8);
    }
    case Q8_0: {
        uint32_t b = col / 32;
        return h2f(ld_u16(row + g.off_b + 2 * b)) * (float)(int8_t)row[g.off_a + 32 * b + col % 32];
    }
    case Q4_K:
    case Q5_K: {
        uint32_t b = col / 256, i = col % 256, grp = i / 32;
        const uint8_t* h = row + g.off_a + 16 * b;
        const uint8_t* s = h + 4;
        uint32_t sc, m;
        if (grp < 4) {
            sc = s[grp] & 63;
            m = s[grp + 4] & 63;
        } else {
            sc = (s[grp + 4] & 15) | ((s[grp - 4] >> 6) << 4);
            m = (s[grp + 4] >> 4) | ((s[grp] >> 6) << 4);
        }
        const uint8_t* qs = row + (kind == Q4_K ? g.off_b : g.off_c) + 128 * b;
        uint32_t q = (qs[(i / 64) * 32 + i % 32] >> ((grp % 2) * 4)) & 15;
        if (kind == Q5_K && (row[g.off_b + 32 * b + i % 32] & (1u << grp))) q += 16;
        float d = h2f(ld_u16(h)), dmin = h2f(ld_u16(h + 2));
        float t = d * (float)sc;
        t = t * (float)q;
        float u = dmin * (float)m;
        return t - u;
    }
    case Q6_K: {
        uint32_t b = col / 256, i = col % 256;
        uint32_t chunk = i / 128, j = i % 128, quarter = j / 32, lane = j % 32;
        uint32_t low = row[g.off_a + 128 * b + chunk * 64 + (quarter % 2) * 32 + lane];
        uint32_t lo = (low >> ((quarter / 2) * 4)) & 15;
        uint32_t hi = (row[g.off_b + 64 * b + chunk * 32 + lane] >> (quarter * 2)) & 3;
        int q = (int)(lo | (hi << 4)) - 32;
        float d = h2f(ld_u16(row + g.off_d + 2 * b));
        float sc = (float)(int8_t)row[g.off_c + 16 * b + chunk * 8 + quarter * 2 + lane / 16];
        float t = d * sc;
        return t * (float)q;
    }
    default: return 0.f;
    }
}

// ------------------------------------------------------------ reductions --
// Cross-lane reductions on the DPP crossbar (VALU latency) rather than
// ds_bpermute (an LDS round trip per step).  Within a row of 16 lanes an xor
// butterfly (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror) leaves every lane with its group's result; the four rows are
// then combined through v_readlane.  Every lane of the wave must be active.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over aligned segments of `width` lanes (a power of two <= 64); every
// lane of a segment receives the segment's sum.
__device__ __forceinline__ float seg_sum(float v, int width) {
    if (width >= 2) v += dpp_f<kDppXor1>(v);
    if (width >= 4) v += dpp_f<kDppXor2>(v);
    if (width >= 8) v += dpp_f<kDppHalfMirror>(v);
    if (width >= 16) v += dpp_f<kDppMirror>(v);
    if (width >= 32) {
        const float a = lane_f(v, 0) + lane_f(v, 16), b = lane_f(v, 32) + lane_f(v, 48);
        v = width == 64 ? a + b : ((threadIdx.x & 32) ? b : a);
    }
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return seg_sum(v, 64); }
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Total-order key of an f32 (Rust f32::total_cmp): larger key = larger value.
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t b = __float_as_int(f);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

__device__ __forceinline__ bool finite_f(float f) {
    return (__float_as_uint(f) & 0x7f800000u) != 0x7f800000u;
}

}  // namespace qh
