// Batched prefill: the reference runs a prompt as one Model::forward per
// token (src/main.rs:250-256, src/model.rs:209-302); here a chunk of S prompt
// tokens goes through each layer at once, so every projection is a GEMM
// (S x K activations times the N x K quantised weight rows) on the fp16
// matrix cores, and attention is a causal flash-attention pass over the
// chunk and the cached history.
//
// Per layer (one launch each): RMSNorm -> fp16; q/k/v GEMMs; Q/K RMSNorm +
// RoPE + KV append (fp32 cache, the decode path's layout); attention;
// o-projection GEMM + residual; RMSNorm (fp16 and fp32); F32 router logits;
// top-k + softmax; grouping of the (token, slot) assignments by expert;
// grouped gate/up GEMM with SwiGLU; grouped down GEMM; routing-weighted
// combine + residual in slot order.
//
// GEMM: 128 x 128 output tiles, 4 waves, K in 64-column slices, fp16
// operands on v_mfma_f32_32x32x16_f16 with fp32 accumulation; the weights
// (Q4_K / Q6_K) are read from a tile-layout copy and dequantised straight into
// the MFMA's B registers, the activations staged through LDS (gemm_tile_r).
#include "qh_block.hpp"

namespace qh {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

// fp16 of an activation, noting a value outside the fp16 range (|v| > 65504,
// or not finite) in bad; a thread that saw one raises kErrRange once, and
// the engine runs that prompt again through the exact FP32 token step.
__device__ __forceinline__ _Float16 to_h(float v, bool& bad) {
    bad |= !(fabsf(v) <= 65504.f);
    return (_Float16)v;
}
__device__ __forceinline__ void note_range(bool bad, uint32_t* err) {
    if (bad) atomicOr(err, kErrRange);
}
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kGM = 128, kGN = 128, kGK = 64, kGT = 256;
constexpr int kGL = kGK + 8;  // LDS row pitch in halfs (144 bytes)

// ------------------------------------------- GEMM, weights in registers --
// The expert and dense GEMMs: 128 x 128 output tiles (rows: activations,
// columns: weight rows), 4 waves; wave w owns weight rows [32w, 32w+32) over
// all 128 tile rows as 4 row blocks of 32, one v_mfma_f32_32x32x16_f16 per
// (row block, matrix, k-step).  K runs in 64-column slices (one sub-block
// pair of a 256-column super-block), four k-steps of 16.
// Lane l supplies weight row 32w + l%32 and column group g = l/32: in k-step
// s its 8 B values are the slice columns 32(s/2) + 16g + 8(s%2) + (0..7).
// The MFMA sums over k, so any assignment of the slice's columns to
// (k-group, k-step) is exact as long as A uses the same one.  The B values
// are dequantised from the lane's weight bytes straight into registers (no
// LDS round trip, no barrier), each value the f32 d*sc*q - dmin*m (Q4_K) or
// d*sc*(q-32) (Q6_K) of one FMA, rounded to fp16 (bytes_affine: a byte
// permute and one mixed-precision FMA per value); the weight bytes come from
// the tile layout (DevMat::wt), where a wave's load of one field for its 32
// rows is one contiguous 1-KB run.  The activations go through LDS,
// double-buffered with two slices in flight in registers, one barrier per
// slice; each A load of a wave covers 8 whole 128-byte slice rows.
typedef float f16v __attribute__((ext_vector_type(16)));

template <uint32_t KIND> struct WReg;

// Four fp16 values a * (byte i of m) + b, i = 0..3, into v[o .. o+3], from
// c = b - 1024 a: v_perm_b32 puts byte i under the fp16 exponent of 1024
// (the half 0x64XX is exactly 1024 + XX), and one v_fma_mix per value
// computes (1024 + XX) * a + c in f32 from that half and rounds it to fp16;
// the product is exact, so the value differs from fma(XX, a, b) only by the
// f32 rounding of c (2^-24 of 1024 |a|).
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bytes_affine(h8v& v, int o, uint32_t m, float a, float c) {
    const h2v lo = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, m, 0x04010400u));  // bytes 0, 1
    const h2v hi = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, m, 0x04030402u));  // bytes 2, 3
    v[o] = (_Float16)fmaf((float)lo[0], a, c);
    v[o + 1] = (_Float16)fmaf((float)lo[1], a, c);
    v[o + 2] = (_Float16)fmaf((float)hi[0], a, c);
    v[o + 3] = (_Float16)fmaf((float)hi[1], a, c);
}
// The bias c of bytes_affine for the value a * q + b.
__device__ __forceinline__ float bias1024(float a, float b) { return fmaf(-1024.f, a, b); }
// w & mk, opaque to the optimiser: knowing the mask, it would narrow each
// byte extraction to a bit-field one and lose the byte-convert form
__device__ __forceinline__ uint32_t and_opaque(uint32_t w, uint32_t mk) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(w), "s"(mk));
    return r;
}

template <> struct WReg<Q4_K> {
    uint4 q, hdr;
    // d*sc and the bytes_affine bias of -dmin*m of sub-blocks 2sl (low
    // nibbles) and 2sl+1 (high nibbles, kept in place: their scale is
    // divided by 16, exactly)
    struct Sc { float a0, b0, a1, b1; };
    // from tile block blk (32 rows, one super-block): the lane's row header
    // and quant bytes 32 sl + 16 g .. of its row
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t sl, uint32_t lane) {
        hdr = ld16(blk + (lane & 31) * 16);
        q = ld16(blk + 512 + sl * 1024 + lane * 16);
    }
    __device__ __forceinline__ Sc prep(uint32_t sl, uint32_t) const {
        uint32_t scp, mp;
        kscale_pair(hdr.y, hdr.z, hdr.w, sl, scp, mp);
        const float d = h2f(hdr.x & 0xffffu), dm = h2f(hdr.x >> 16);
        const float a0 = d * (float)(scp & 0xffu), a1 = d * (float)(scp >> 8) * 0.0625f;
        return {a0, bias1024(a0, -(dm * (float)(mp & 0xffu))), a1, bias1024(a1, -(dm * (float)(mp >> 8)))};
    }
    // k-step S: bytes 8(S%2) .. +7, low nibbles for S < 2, high for S >= 2;
    // d*sc*q - dmin*m (src/quant.rs:50-62) rounded once to fp16
    template <int S>
    __device__ __forceinline__ h8v dequant(const Sc& c, uint32_t) const {
        const uint32_t w0 = (S & 1) ? q.z : q.x, w1 = (S & 1) ? q.w : q.y;
        const uint32_t mk = S < 2 ? 0x0f0f0f0fu : 0xf0f0f0f0u;
        const float a = S < 2 ? c.a0 : c.a1, b = S < 2 ? c.b0 : c.b1;
        h8v v;
        bytes_affine(v, 0, and_opaque(w0, mk), a, b);
        bytes_affine(v, 4, and_opaque(w1, mk), a, b);
        return v;
    }
};

template <> struct WReg<Q6_K> {
    uint4 l0, l1, qh;
    uint32_t sc4, d;
    // d*sc and the bytes_affine bias of -32 d*sc, the lane's two scales
    // (sets l0 and l1)
    struct Sc { float a0, b0, a1, b1; };
    // slice sl = 2c + p of the super-block (half c, nibble p), from tile
    // block blk: low-bit bytes 64c + 16g .. and 64c + 32 + 16g .. of the
    // lane's row (columns 16g.. and 32+16g..), their high-bit bytes
    // 32c + 16g .., the slice's 4 scales and d
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t sl, uint32_t lane) {
        const uint32_t c = sl >> 1;
        l0 = ld16(blk + c * 2048 + lane * 16);
        l1 = ld16(blk + c * 2048 + 1024 + lane * 16);
        qh = ld16(blk + 4096 + c * 1024 + lane * 16);
        sc4 = gld<uint32_t>(blk + 6144 + sl * 128 + (lane & 31) * 4);
        d = ld_u16(blk + 6656 + (lane & 31) * 2);
    }
    __device__ __forceinline__ Sc prep(uint32_t, uint32_t grp) const {
        const float df = h2f(d);
        const float a0 = df * (float)(int8_t)((sc4 >> (8 * grp)) & 0xffu);
        const float a1 = df * (float)(int8_t)((sc4 >> (8 * (grp + 2))) & 0xffu);
        return {a0, -1056.f * a0, a1, -1056.f * a1};  // bias1024(a, -32 a)
    }
    // k-step S: set S/2 (l0 with scale byte g, or l1 with byte g+2), bytes
    // 8(S%2) .. +7; d*sc*(q-32) (src/quant.rs:63-77) with q = nibble p | two
    // high bits << 4, rounded once to fp16
    template <int S>
    __device__ __forceinline__ h8v dequant(const Sc& c, uint32_t p) const {
        const uint4& L = S < 2 ? l0 : l1;
        const uint32_t x0 = (S & 1) ? L.z : L.x, x1 = (S & 1) ? L.w : L.y;
        const uint32_t h0 = (S & 1) ? qh.z : qh.x, h1 = (S & 1) ? qh.w : qh.y;
        const uint32_t hs = 2 * (2 * p + (S < 2 ? 0 : 1)), ls = 4 * p;
        const uint32_t va = and_opaque(x0 >> ls, 0x0f0f0f0fu) | (and_opaque(h0 >> hs, 0x03030303u) << 4);
        const uint32_t vb = and_opaque(x1 >> ls, 0x0f0f0f0fu) | (and_opaque(h1 >> hs, 0x03030303u) << 4);
        const float a = S < 2 ? c.a0 : c.a1, b = S < 2 ? c.b0 : c.b1;
        h8v v;
        bytes_affine(v, 0, va, a, b);
        bytes_affine(v, 4, vb, a, b);
        return v;
    }
};

template <> struct WReg<Q5_K> {
    uint4 q, hdr, qh;
    // d*sc and the bytes_affine bias of -dmin*m of sub-blocks 2sl and 2sl+1;
    // the bit of the qh bytes that holds sub-block 2sl's fifth bits
    struct Sc { float a0, b0, a1, b1; uint32_t hs; };
    // from tile block blk: the lane's row header, quant bytes 32 sl + 16 g ..
    // and high-bit bytes 16 g .. of its row
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t sl, uint32_t lane) {
        hdr = ld16(blk + (lane & 31) * 16);
        q = ld16(blk + 512 + sl * 1024 + lane * 16);
        qh = ld16(blk + 4608 + lane * 16);
    }
    __device__ __forceinline__ Sc prep(uint32_t sl, uint32_t) const {
        uint32_t scp, mp;
        kscale_pair(hdr.y, hdr.z, hdr.w, sl, scp, mp);
        const float d = h2f(hdr.x & 0xffffu), dm = h2f(hdr.x >> 16);
        const float a0 = d * (float)(scp & 0xffu), a1 = d * (float)(scp >> 8);
        return {a0, bias1024(a0, -(dm * (float)(mp & 0xffu))), a1, bias1024(a1, -(dm * (float)(mp >> 8))), 2 * sl};
    }
    // k-step S: bytes 8(S%2) .. +7, low nibbles for S < 2, high for S >= 2,
    // each with its fifth bit (qh bit 2sl + S/2) as bit 4;
    // d*sc*q - dmin*m (src/quant.rs:50-62) rounded once to fp16
    template <int S>
    __device__ __forceinline__ h8v dequant(const Sc& c, uint32_t) const {
        const uint32_t w0 = (S & 1) ? q.z : q.x, w1 = (S & 1) ? q.w : q.y;
        const uint32_t h0 = (S & 1) ? qh.z : qh.x, h1 = (S & 1) ? qh.w : qh.y;
        const uint32_t ls = S < 2 ? 0 : 4, hs = c.hs + (S < 2 ? 0 : 1);
        const uint32_t va = and_opaque(w0 >> ls, 0x0f0f0f0fu) | (and_opaque(h0 >> hs, 0x01010101u) << 4);
        const uint32_t vb = and_opaque(w1 >> ls, 0x0f0f0f0fu) | (and_opaque(h1 >> hs, 0x01010101u) << 4);
        const float a = S < 2 ? c.a0 : c.a1, b = S < 2 ? c.b0 : c.b1;
        h8v v;
        bytes_affine(v, 0, va, a, b);
        bytes_affine(v, 4, vb, a, b);
        return v;
    }
};

// d of blocks 2sl and 2sl+1 (32-column blocks) from the row's eight d
// values of the super-block
__device__ __forceinline__ uint32_t d_pair(const uint4& dd, uint32_t sl) {
    return sl == 0 ? dd.x : sl == 1 ? dd.y : sl == 2 ? dd.z : dd.w;
}

template <> struct WReg<Q4_0> {
    uint4 q0, q1, dd;
    // d and the bytes_affine bias of -8d, blocks 2sl and 2sl+1; the nibble
    // of the lane's group
    // (low for columns 0-15 of a block, high for 16-31)
    struct Sc { float a0, b0, a1, b1; uint32_t sh; };
    // from tile block blk: the lane's row's d values and the 16 quant bytes
    // of blocks 2sl and 2sl+1 (both lane groups read the same bytes)
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t sl, uint32_t lane) {
        dd = ld16(blk + (lane & 31) * 16);
        q0 = ld16(blk + 512 + sl * 1024 + (lane & 31) * 16);
        q1 = ld16(blk + 512 + sl * 1024 + 512 + (lane & 31) * 16);
    }
    __device__ __forceinline__ Sc prep(uint32_t sl, uint32_t grp) const {
        const uint32_t w = d_pair(dd, sl);
        const float d0 = h2f(w & 0xffffu), d1 = h2f(w >> 16);
        return {d0, -1032.f * d0, d1, -1032.f * d1, 4 * grp};  // bias1024(d, -8 d)
    }
    // k-step S: block 2sl + S/2, bytes 8(S%2) .. +7, the group's nibble;
    // d*(q-8) (src/quant.rs:40-45) rounded once to fp16
    template <int S>
    __device__ __forceinline__ h8v dequant(const Sc& c, uint32_t) const {
        const uint4& Q = S < 2 ? q0 : q1;
        const uint32_t w0 = (S & 1) ? Q.z : Q.x, w1 = (S & 1) ? Q.w : Q.y;
        const float a = S < 2 ? c.a0 : c.a1, b = S < 2 ? c.b0 : c.b1;
        h8v v;
        bytes_affine(v, 0, and_opaque(w0 >> c.sh, 0x0f0f0f0fu), a, b);
        bytes_affine(v, 4, and_opaque(w1 >> c.sh, 0x0f0f0f0fu), a, b);
        return v;
    }
};

template <> struct WReg<Q8_0> {
    uint4 q0, q1, dd;
    // d and the bytes_affine bias of -128d, blocks 2sl and 2sl+1
    struct Sc { float a0, b0, a1, b1; };
    // from tile block blk: the lane's row's d values and quant bytes 16g ..
    // of blocks 2sl and 2sl+1
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t sl, uint32_t lane) {
        dd = ld16(blk + (lane & 31) * 16);
        q0 = ld16(blk + 512 + sl * 2048 + lane * 16);
        q1 = ld16(blk + 512 + sl * 2048 + 1024 + lane * 16);
    }
    __device__ __forceinline__ Sc prep(uint32_t sl, uint32_t) const {
        const uint32_t w = d_pair(dd, sl);
        const float d0 = h2f(w & 0xffffu), d1 = h2f(w >> 16);
        return {d0, -1152.f * d0, d1, -1152.f * d1};  // bias1024(d, -128 d)
    }
    // k-step S: block 2sl + S/2, bytes 8(S%2) .. +7; the signed byte q as
    // (q + 128) - 128, so d*q (src/quant.rs:46-49) is one FMA, rounded once to fp16
    template <int S>
    __device__ __forceinline__ h8v dequant(const Sc& c, uint32_t) const {
        const uint4& Q = S < 2 ? q0 : q1;
        const uint32_t w0 = (S & 1) ? Q.z : Q.x, w1 = (S & 1) ? Q.w : Q.y;
        const float a = S < 2 ? c.a0 : c.a1, b = S < 2 ? c.b0 : c.b1;
        h8v v;
        bytes_affine(v, 0, w0 ^ 0x80808080u, a, b);
        bytes_affine(v, 4, w1 ^ 0x80808080u, a, b);
        return v;
    }
};

// Weight row of this thread (tile column): wave w, lane l -> 32w + l%32.
__device__ __forceinline__ uint32_t rtile_row() { return 32 * (threadIdx.x >> 6) + (threadIdx.x & 31); }
// Tile row of this thread's A load i (i < 4): 32w + 8i + l/8.
__device__ __forceinline__ uint32_t arow_row(uint32_t i) {
    return 32 * (threadIdx.x >> 6) + 8 * i + ((threadIdx.x & 63) >> 3);
}

// Output element acc[.][mb][i] of this lane: tile row / tile column.
__device__ __forceinline__ uint32_t racc_row(uint32_t mb, uint32_t i) {
    return 32 * mb + 8 * (i >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (i & 3);
}
__device__ __forceinline__ uint32_t racc_col() { return rtile_row(); }

constexpr int kRA = 2 * kGM * kGL;  // halfs of LDS: the two A buffers

// acc[nb][mb] += A[m0 .. m0+128) x W_nb[n0 .. n0+128)^T over columns
// [kbeg, kbeg + K) (kbeg a multiple of 256, K of 64 * STAGES; STAGES even).
// arows[i]: the A row of tile row arow_row(i) (any valid row past the tile's
// rows: those outputs are not stored); wblk[nb]: tile block (G, 0) of matrix
// nb for this wave's row group G = (n0 + 32w) / 32 (likewise clamped).  STAGES register stages
// of weight loads run ahead; the loads are unconditional (clamped), so each
// wait covers exactly one stage.  With full false (workgroup-uniform: a tile
// whose valid rows fit in the first 64) row blocks 2 and 3 are skipped, and
// acc[.][2..3] stay as they are.
template <uint32_t KIND, int NB, int STAGES>
__device__ __forceinline__ void gemm_tile_r(const _Float16* const (&arows)[4], const uint8_t* const (&wblk)[NB],
                                            uint32_t K, f16v (&acc)[NB][4], _Float16* As, uint32_t kbeg = 0,
                                            bool full = true) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, grp = lane >> 5;
    static_assert(STAGES % 2 == 0, "slice k uses A buffer k % 2 = its stage's parity");
    const uint32_t nsl = K / kGK;
    WReg<KIND> wr[STAGES][NB];
    uint4 av[2][4];  // A slices k+1 and k+2 in flight while slice k is multiplied
    auto wload = [&](int st, uint32_t k) {
        const uint32_t k0 = kbeg + min(k, nsl - 1) * kGK;  // past the end: a harmless reload
#pragma unroll
        for (int nb = 0; nb < NB; nb++) wr[st][nb].load(wblk[nb] + (size_t)(k0 >> 8) * tile_block_bytes(KIND), (k0 >> 6) & 3, lane);
    };
    // A row r, 16-byte chunks 2i + grp of the slice (lanes l and l+32 read
    // adjacent chunks of one row)
    // A: load i of a wave covers 8 whole 128-byte slice rows, rows
    // arow_row(i) (lane l: row 32w + 8i + l/8, 16-byte chunk l%8)
    const uint32_t ach = lane & 7;
    auto aload = [&](int j, uint32_t k) {
        const uint32_t k0 = kbeg + min(k, nsl - 1) * kGK;
#pragma unroll
        for (int i = 0; i < 4; i++) av[j][i] = gld<uint4>(arows[i] + k0 + 8 * ach);
    };
    // A slice held in av[j] to LDS buffer j (slice k sits in buffer k % 2)
    auto astore = [&](int j) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4*>(As + j * kGM * kGL + arow_row(i) * kGL + 8 * ach) = av[j][i];
    };
#pragma unroll
    for (int st = 0; st < STAGES; st++) wload(st, st);
    aload(0, 0);
    astore(0);
    aload(1, 1);
    aload(0, 2);
    __syncthreads();
    for (uint32_t k0 = 0; k0 < nsl; k0 += STAGES) {
#pragma unroll
        for (int st = 0; st < STAGES; st++) {
            const uint32_t k = k0 + st;
            const uint32_t sl = ((kbeg >> 6) + k) & 3, p = sl & 1;
            const _Float16* Ab = As + (k & 1) * kGM * kGL;
            typename WReg<KIND>::Sc sc[NB];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) sc[nb] = wr[st][nb].prep(sl, grp);
            auto kstep = [&](auto S_) {
                constexpr int S = decltype(S_)::value;
                const uint32_t col = 32 * (S >> 1) + 16 * grp + 8 * (S & 1);
                h8v af[4], bf[NB];
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
                    af[mb] = *reinterpret_cast<const h8v*>(Ab + (32 * mb + (lane & 31)) * kGL + col);
#pragma unroll
                for (int nb = 0; nb < NB; nb++) bf[nb] = wr[st][nb].template dequant<S>(sc[nb], p);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
                        acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mb], bf[nb], acc[nb][mb], 0, 0, 0);
                if (full) {
#pragma unroll
                    for (int mb = 2; mb < 4; mb++)
                        af[mb] = *reinterpret_cast<const h8v*>(Ab + (32 * mb + (lane & 31)) * kGL + col);
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
#pragma unroll
                        for (int mb = 2; mb < 4; mb++)
                            acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mb], bf[nb], acc[nb][mb], 0, 0, 0);
                }
            };
            kstep(std::integral_constant<int, 0>{});
            kstep(std::integral_constant<int, 1>{});
            kstep(std::integral_constant<int, 2>{});
            kstep(std::integral_constant<int, 3>{});
            wload(st, k + STAGES);
            astore((st + 1) & 1);  // slice k + 1
            aload((st + 1) & 1, k + 3);
            __syncthreads();
        }
    }
}

// XCD-aware tile order.  Workgroup b runs on XCD b % 8 (each XCD has its own
// L2).  The grid is 1-D: XCD x takes the row tiles t = x, x + 8, ... and, for
// each in turn, all nn column tiles, so that one row tile's activations (read
// by every column tile) stay in that XCD's L2 while its column tiles run.
// Returns (row tile, column tile) of this workgroup; the grid holds
// 8 * ceil(row tiles / 8) * nn workgroups.
__device__ __forceinline__ void xcd_tile(uint32_t nn, uint32_t& t, uint32_t& n) {
    const uint32_t b = blockIdx.x, x = b & 7, i = b >> 3;
    t = x + 8 * (i / nn);
    n = i % nn;
}

// gate/up of the routed experts + SwiGLU (model.rs:266-274):
// Hs[goff[e] + r][n] = silu(g) * u, fp16, for the sorted assignments.
template <uint32_t KIND>
__global__ __launch_bounds__(kGT, 2) void k_gemm_gateup(const _Float16* Xn, uint32_t H, ExpertTiles G, DevMat Wg, DevMat Wu,
                                                     _Float16* Hs, uint32_t* err) {
    __shared__ __align__(16) _Float16 smem[kRA];
    uint32_t ty, tx;
    xcd_tile((Wg.rows + kGN - 1) / kGN, ty, tx);
    if (ty >= *G.ntile) return;
    const uint32_t e = G.te[ty], mt0 = G.tm[ty];
    const uint32_t base = G.goff[e], rows = G.goff[e + 1] - base;
    const uint32_t n0 = tx * kGN, r = rtile_row(), ff = Wg.rows;
    const _Float16* arows[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t ra = mt0 + arow_row(i);
        arows[i] = Xn + (size_t)(ra < rows ? G.tok[base + ra] : 0u) * H;
    }
    const size_t gofs = (size_t)min((n0 >> 5) + (threadIdx.x >> 6), ff / 32 - 1) * tile_group_bytes(KIND, Wg.cols);
    const uint8_t* const wblk[2] = {Wg.wt + e * Wg.expert_stride + gofs, Wu.wt + e * Wu.expert_stride + gofs};
    f16v acc[2][4];
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) acc[nb][mb] = f16v{};
    // a tile of at most 64 valid rows (an expert's remainder past its full
    // tiles) multiplies two row blocks, not four
    gemm_tile_r<KIND, 2, 2>(arows, wblk, Wg.cols, acc, smem, 0, rows - mt0 > 64);
    const uint32_t n = n0 + racc_col();
    bool bad = false;
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t m = mt0 + racc_row(mb, i);
            if (m < rows && n < ff) {
#pragma clang fp contract(off)
                const float gv = acc[0][mb][i], uv = acc[1][mb][i];
                Hs[(size_t)(base + m) * ff + n] = to_h((gv / (1.f + expf(-gv))) * uv, bad);
            }
        }
    note_range(bad, err);
}

// down of the routed experts: Y[asg][n] = Hs[goff[e] + r] . Wd_e[n].
template <uint32_t KIND>
__global__ __launch_bounds__(kGT, 2) void k_gemm_down(const _Float16* Hs, ExpertTiles G, DevMat Wd, float* Y) {
    __shared__ __align__(16) _Float16 smem[kRA];
    __shared__ uint32_t dsts[kGM];  // assignment index of each tile row
    uint32_t ty, tx;
    xcd_tile((Wd.rows + kGN - 1) / kGN, ty, tx);
    if (ty >= *G.ntile) return;
    const uint32_t e = G.te[ty], mt0 = G.tm[ty];
    const uint32_t base = G.goff[e], rows = G.goff[e + 1] - base;
    const uint32_t n0 = tx * kGN, r = rtile_row(), ff = Wd.cols, N = Wd.rows;
    // visible to the epilogue through the GEMM's barriers
    if (threadIdx.x < kGM) dsts[threadIdx.x] = G.asg[base + min(mt0 + threadIdx.x, rows - 1)];
    const _Float16* arows[4];
#pragma unroll
    for (int i = 0; i < 4; i++) arows[i] = Hs + (size_t)(base + min(mt0 + arow_row(i), rows - 1)) * ff;
    const uint8_t* const wblk[1] = {
        Wd.wt + e * Wd.expert_stride +
        (size_t)min((n0 >> 5) + (threadIdx.x >> 6), N / 32 - 1) * tile_group_bytes(KIND, Wd.cols)};
    f16v acc[1][4];
#pragma unroll
    for (int mb = 0; mb < 4; mb++) acc[0][mb] = f16v{};
    gemm_tile_r<KIND, 1, 2>(arows, wblk, ff, acc, smem, 0, rows - mt0 > 64);  // as in k_gemm_gateup
    const uint32_t n = n0 + racc_col();
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t ml = racc_row(mb, i), m = mt0 + ml;
            if (m < rows && n < N) Y[(size_t)dsts[ml] * N + n] = acc[0][mb][i];
        }
}

// Dense projections (the per-token q/k/v and o matvecs of model.rs:230-232,
// 245 over a chunk), up to three matrices of either format in one launch so
// that the small k and v projections share the machine with q:
// C[m][cofs_i + n] = X16[m] . W_i[n] (columns [kbeg, kbeg + K) of W_i, K =
// cols / gridDim.z, split z of the columns writing to C + z * split_stride),
// for m < S, n < W_i.rows.  Column tiles [t_i, t_{i+1}) of gridDim.x belong
// to matrix i.  Tiles as the expert GEMMs.
template <uint32_t KIND>
__device__ __forceinline__ void dense_body(const _Float16* X16, uint32_t S, const DevMat& W, uint32_t m0,
                                           uint32_t n0, uint32_t kbeg, uint32_t K, float* C, uint32_t ldc,
                                           uint32_t cofs, _Float16* smem) {
    const uint32_t r = rtile_row(), N = W.rows, ld = W.cols;
    const _Float16* arows[4];
#pragma unroll
    for (int i = 0; i < 4; i++) arows[i] = X16 + (size_t)min(m0 + arow_row(i), S - 1) * ld;
    const uint8_t* const wblk[1] = {
        W.wt + (size_t)min((n0 >> 5) + (threadIdx.x >> 6), N / 32 - 1) * tile_group_bytes(KIND, W.cols)};
    f16v acc[1][4];
#pragma unroll
    for (int mb = 0; mb < 4; mb++) acc[0][mb] = f16v{};
    gemm_tile_r<KIND, 1, 2>(arows, wblk, K, acc, smem, kbeg);
    const uint32_t n = n0 + racc_col();
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t m = m0 + racc_row(mb, i);
            if (m < S && n < N) C[(size_t)m * ldc + cofs + n] = acc[0][mb][i];
        }
}

// Three workgroups per CU (168 VGPRs, 4 of them spilled): the q|k|v grid of
// 16 x 40 tiles at 2,048 tokens then runs in one round of 768 workgroup slots
// rather than 1.25 rounds of 512.
__global__ __launch_bounds__(kGT, 3) void k_gemm_dense(const _Float16* X16, uint32_t S, DenseSegs G, float* C,
                                                    uint32_t ldc, size_t split_stride) {
    __shared__ __align__(16) _Float16 smem[kRA];
    uint32_t mt, t;
    xcd_tile(G.tile_end[2], mt, t);  // row tile (tokens), column tile
    if (mt * kGM >= S) return;
    const uint32_t i = t < G.tile_end[0] ? 0 : t < G.tile_end[1] ? 1 : 2;  // workgroup-uniform
    const uint32_t t0 = i == 0 ? 0 : G.tile_end[i - 1];
    const DevMat& W = G.W[i];
    const uint32_t K = W.cols / gridDim.z, kbeg = blockIdx.z * K;
    float* Cz = C + blockIdx.z * split_stride;
    switch (W.kind) {
#define QH_DENSE(KD) \
    case KD: dense_body<KD>(X16, S, W, mt * kGM, (t - t0) * kGN, kbeg, K, Cz, ldc, G.cofs[i], smem); break;
        QH_DENSE(Q4_0) QH_DENSE(Q8_0) QH_DENSE(Q4_K) QH_DENSE(Q5_K) QH_DENSE(Q6_K)
#undef QH_DENSE
    default: break;
    }
}

// ------------------------------------------------------- tile layout --
// Row-layout source byte of byte o of tile block (G, b) of a matrix whose
// rows start at w (stride drb): the inverse of the layout described at
// DevMat::wt.
__device__ __forceinline__ const uint8_t* tile_src(const uint8_t* w, uint32_t drb, const RowGeo& g, uint32_t kind,
                                                   uint32_t G, uint32_t b, uint32_t o) {
    uint32_t row, off;
    if (kind == Q6_K) {
        if (o < 4096) {  // low bits
            const uint32_t c = o >> 11, part = (o >> 10) & 1, lane = (o >> 4) & 63;
            row = lane & 31;
            off = g.off_a + b * 128 + c * 64 + part * 32 + (lane >> 5) * 16 + (o & 15);
        } else if (o < 6144) {  // high bits
            const uint32_t u = o - 4096, c = u >> 10, lane = (u >> 4) & 63;
            row = lane & 31;
            off = g.off_b + b * 64 + c * 32 + (lane >> 5) * 16 + (u & 15);
        } else if (o < 6656) {  // scales
            const uint32_t u = o - 6144, sl = u >> 7;
            row = (u >> 2) & 31;
            off = g.off_c + b * 16 + sl * 4 + (u & 3);
        } else {  // d
            const uint32_t u = o - 6656;
            row = u >> 1;
            off = g.off_d + b * 2 + (u & 1);
        }
    } else if (kind == Q4_K || kind == Q5_K) {
        if (o < 512) {  // headers
            row = o >> 4;
            off = g.off_a + b * 16 + (o & 15);
        } else if (o < 4608) {  // quants
            const uint32_t u = o - 512, sl = u >> 10, lane = (u >> 4) & 63;
            row = lane & 31;
            off = (kind == Q4_K ? g.off_b : g.off_c) + b * 128 + sl * 32 + (lane >> 5) * 16 + (u & 15);
        } else {  // Q5_K high bits
            const uint32_t u = o - 4608, lane = (u >> 4) & 63;
            row = lane & 31;
            off = g.off_b + b * 32 + (lane >> 5) * 16 + (u & 15);
        }
    } else {  // Q4_0, Q8_0: eight 32-column blocks per 256 columns
        if (o < 512) {  // d of the eight blocks
            row = o >> 4;
            off = g.off_b + (8 * b + ((o & 15) >> 1)) * 2 + (o & 1);
        } else if (kind == Q4_0) {  // 16 quant bytes of block 2sl + part
            const uint32_t u = o - 512, sl = u >> 10, part = (u >> 9) & 1;
            row = (u >> 4) & 31;
            off = g.off_a + (8 * b + 2 * sl + part) * 16 + (u & 15);
        } else {  // Q8_0: bytes 16g .. of block 2sl + part
            const uint32_t u = o - 512, sl = u >> 11, part = (u >> 10) & 1, lane = (u >> 4) & 63;
            row = lane & 31;
            off = g.off_a + (8 * b + 2 * sl + part) * 32 + (lane >> 5) * 16 + (u & 15);
        }
    }
    return w + (size_t)(32 * G + row) * drb + off;
}

// Whether the 16 tile bytes at o (a multiple of 16) are 16 consecutive source
// bytes: every field but Q6_K's scales (4-byte runs) and d (2-byte runs).
__device__ __forceinline__ bool tile_run16(uint32_t kind, uint32_t o) { return kind != Q6_K || o < 6144; }

// The tile copy of matrix m (every expert): workgroup = one block, 16-byte
// copies where the layout keeps 16 source bytes together (a 16-byte aligned
// matrix), single bytes elsewhere.
__global__ __launch_bounds__(kBlock) void k_tile_gemm(DevMat m, uint32_t experts, uint8_t* __restrict__ dst) {
    const uint32_t nb = m.cols / 256, groups = m.rows / 32, bb = tile_block_bytes(m.kind);
    const size_t nblk = (size_t)experts * groups * nb;
    const bool vec = (reinterpret_cast<uintptr_t>(m.w) % 16 == 0) && m.drb % 16 == 0 && m.expert_stride % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    for (size_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
        const uint32_t e = (uint32_t)(blk / ((size_t)groups * nb)), rem = (uint32_t)(blk % ((size_t)groups * nb));
        const uint32_t G = rem / nb, b = rem % nb;
        const uint8_t* w = m.w + (size_t)e * m.expert_stride;
        uint8_t* out = dst + (size_t)e * m.expert_stride + ((size_t)G * nb + b) * bb;
        for (uint32_t o = 16 * threadIdx.x; o < bb; o += 16 * kBlock) {  // bb is a multiple of 16
            if (vec && tile_run16(m.kind, o)) {
                *reinterpret_cast<uint4*>(out + o) =
                    *reinterpret_cast<const uint4*>(tile_src(w, m.drb, m.geo, m.kind, G, b, o));
            } else {
#pragma unroll 4
                for (uint32_t k = 0; k < 16; k++) out[o + k] = *tile_src(w, m.drb, m.geo, m.kind, G, b, o + k);
            }
        }
    }
}

// ------------------------------------------------------ element kernels --
// X[t] = embedding row of tokens[t] (model.rs:225), bit-exact decode.
__global__ __launch_bounds__(kBlock) void k_pf_embed(DevMat emb, const uint32_t* tokens, uint32_t H, uint32_t vocab,
                                                     float* X, DevState* st) {
    const uint32_t t = blockIdx.x, tok = tokens[t];
    if (tok >= vocab) {
        if (threadIdx.x == 0) atomicOr(&st->err, kErrToken);
        return;
    }
    const uint8_t* row = emb.w + (size_t)tok * emb.drb;
    for (uint32_t i = threadIdx.x; i < H; i += kBlock) X[(size_t)t * H + i] = dequant_value(row, emb.kind, emb.geo, i);
}

// RMSNorm (ops.rs:3-15) of row t: fp16 copy (GEMM input), optional fp32 copy.
// With P: first X[t] += P[0][t] + P[1][t] (the two column halves of the
// o-projection: the residual add of model.rs:246-248, in that order).
__global__ __launch_bounds__(kBlock) void k_pf_norm(float* X, const float* w, uint32_t H, float eps,
                                                    _Float16* Y16, float* Y32, const float* P, size_t pstride,
                                                    uint32_t* err) {
    __shared__ float red[kWaves];
    const size_t t = blockIdx.x;
    float* x = X + t * H;
    if (P) {
        const float* p0 = P + t * H;
        const float* p1 = p0 + pstride;
        for (uint32_t i4 = threadIdx.x; 4 * i4 < H; i4 += kBlock) {
            const float4 v = reinterpret_cast<const float4*>(x)[i4], a = reinterpret_cast<const float4*>(p0)[i4],
                         b = reinterpret_cast<const float4*>(p1)[i4];
            reinterpret_cast<float4*>(x)[i4] =
                make_float4(v.x + (a.x + b.x), v.y + (a.y + b.y), v.z + (a.z + b.z), v.w + (a.w + b.w));
        }
        // each thread reads back only the elements it wrote
    }
    // 4 consecutive elements per thread (H % 64 == 0), the sum of squares in
    // the same element order as k_pf_combine's
    float ss = 0.f;
    for (uint32_t i4 = threadIdx.x; 4 * i4 < H; i4 += kBlock) {
        const float4 v = reinterpret_cast<const float4*>(x)[i4];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
    bool bad = false;
    for (uint32_t i4 = threadIdx.x; 4 * i4 < H; i4 += kBlock) {
        const float4 v = reinterpret_cast<const float4*>(x)[i4], w4 = reinterpret_cast<const float4*>(w)[i4];
        const float4 y = make_float4(v.x * (scale * w4.x), v.y * (scale * w4.y), v.z * (scale * w4.z),
                                     v.w * (scale * w4.w));
        _Float16* o = Y16 + t * H + 4 * i4;
        o[0] = to_h(y.x, bad);
        o[1] = to_h(y.y, bad);
        o[2] = to_h(y.z, bad);
        o[3] = to_h(y.w, bad);
        if (Y32) reinterpret_cast<float4*>(Y32 + t * H)[i4] = y;
    }
    note_range(bad, err);
}

// Q/K RMSNorm per head (model.rs:233-238), NeoX RoPE at position p0 + t
// (ops.rs:16-28), KV append (model.rs:241-243).  Row t of QKV is
// [q (heads*128) | k (kvheads*128) | v (kvheads*128)].  Q goes to
// Q16[head][t][128] (fp16), K and V to the fp32 cache [kvhead][ctx][128].
// Wave w takes head slots w, w + kWaves, ...: 0..heads-1 q, then k, then v;
// lane l holds elements l and l + 64, the rotated pair.
__global__ __launch_bounds__(kBlock) void k_pf_qkrope(const float* QKV, const float* qn, const float* kn,
                                                      const float2* rope, uint32_t p0, uint32_t S, uint32_t heads,
                                                      uint32_t kvheads, uint32_t ctx, float eps, _Float16* Q16,
                                                      float* kcache, float* vcache, _Float16* Kh, _Float16* Vth,
                                                      uint32_t vp, uint32_t* err) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, pos = p0 + t;
    const uint32_t row = (heads + 2 * kvheads) * 128;
    const float* x = QKV + (size_t)t * row;
    const float2 cs = rope[(size_t)pos * 64 + lane];
    const uint32_t nslot = heads + 2 * kvheads;
    const float qw0 = qn[lane], qw1 = qn[lane + 64], kw0 = kn[lane], kw1 = kn[lane + 64];
    constexpr uint32_t kSW = 5;  // slots per wave per round, their loads issued together
    bool bad = false;
    for (uint32_t s0 = w; s0 < nslot; s0 += kSW * kWaves) {  // wave-uniform
        float xa_[kSW], xb_[kSW];
#pragma unroll
        for (uint32_t j = 0; j < kSW; j++) {
            const uint32_t sl = min(s0 + j * kWaves, nslot - 1);
            xa_[j] = x[sl * 128 + lane];
            xb_[j] = x[sl * 128 + lane + 64];
        }
#pragma unroll
        for (uint32_t j = 0; j < kSW; j++) {
            const uint32_t slot = s0 + j * kWaves;
            if (slot >= nslot) break;
            const float xa = xa_[j], xb = xb_[j];
            if (slot >= heads + kvheads) {
                const uint32_t g = slot - heads - kvheads;
                float* dst = vcache + ((size_t)g * ctx + pos) * 128;
                dst[lane] = xa;
                dst[lane + 64] = xb;
                Vth[((size_t)g * 128 + lane) * vp + pos] = to_h(xa, bad);
                Vth[((size_t)g * 128 + lane + 64) * vp + pos] = to_h(xb, bad);
                continue;
            }
            const bool isq = slot < heads;
            const float w0 = isq ? qw0 : kw0, w1 = isq ? qw1 : kw1;
            const float ssq = wave_sum(fmaf(xb, xb, xa * xa));
            const float sc = 1.0f / sqrtf(ssq / 128.0f + eps);
            const float y0 = xa * (sc * w0), y1 = xb * (sc * w1);
            float o0, o1;
            {
#pragma clang fp contract(off)
                o0 = y0 * cs.x - y1 * cs.y;
                o1 = y0 * cs.y + y1 * cs.x;
            }
            if (isq) {
                _Float16* dst = Q16 + ((size_t)slot * S + t) * 128;
                dst[lane] = to_h(o0, bad);
                dst[lane + 64] = to_h(o1, bad);
            } else {
                float* dst = kcache + ((size_t)(slot - heads) * ctx + pos) * 128;
                dst[lane] = o0;
                dst[lane + 64] = o1;
                _Float16* dh = Kh + ((size_t)(slot - heads) * ctx + pos) * 128;
                dh[lane] = to_h(o0, bad);
                dh[lane + 64] = to_h(o1, bad);
            }
        }
    }
    note_range(bad, err);
}

// Router logits (model.rs:249-256) in fp32 on the matrix cores
// (v_mfma_f32_16x16x4_f32: fp32 operands and accumulation): 64 tokens per
// workgroup (the router rows, 1 MB in all, are read once per 64 tokens),
// wave w takes experts [32 w, 32 w + 32) (E <= 128); 64-column slices of x and
// of the F32 router rows are staged in LDS, the next slice's loads issued
// before the current slice's MFMAs.  The columns are split over gridDim.y
// workgroups (split ks writes its partial sums to LR + ks S E; k_pf_topk adds
// them in split order), so that the launch fills the device.
constexpr uint32_t kRT = 64;  // tokens per router workgroup
__global__ __launch_bounds__(kBlock) void k_pf_router(const float* Xn, DevMat R, uint32_t S, uint32_t H, uint32_t E,
                                                      float* LR) {
    constexpr uint32_t kP = 65;  // LDS pitch (floats)
    __shared__ float xs[kRT * kP];
    __shared__ float rs[128 * kP];
    const uint32_t t0 = blockIdx.x * kRT, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t grp = lane >> 4, col = lane & 15;
    float4 xr[4], rr[8];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t idx = tid + kBlock * i, tt = idx >> 4, kk = 4 * (idx & 15);
            xr[i] = t0 + tt < S ? gld<float4>(Xn + (size_t)(t0 + tt) * H + k0 + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t idx = tid + kBlock * i, ee = idx >> 4, k4 = 4 * (idx & 15);
            rr[i] = ee < E ? gld<float4>(R.w + (size_t)ee * R.drb + 4 * (k0 + k4)) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    f4v acc[kRT / 16][2];
#pragma unroll
    for (uint32_t mt = 0; mt < kRT / 16; mt++) acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const uint32_t nsl = H / 64, per = (nsl + gridDim.y - 1) / gridDim.y;
    const uint32_t kb = min(blockIdx.y * per, nsl) * 64, ke = min((blockIdx.y + 1) * per, nsl) * 64;
    LR += (size_t)blockIdx.y * S * E;
    if (kb < ke) gload(kb);
    for (uint32_t k0 = kb; k0 < ke; k0 += 64) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t idx = tid + kBlock * i, tt = idx >> 4, kk = 4 * (idx & 15);
            float* xd = xs + tt * kP + kk;
            xd[0] = xr[i].x;
            xd[1] = xr[i].y;
            xd[2] = xr[i].z;
            xd[3] = xr[i].w;
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t idx = tid + kBlock * i, ee = idx >> 4, k4 = 4 * (idx & 15);
            float* rd = rs + ee * kP + k4;
            rd[0] = rr[i].x;
            rd[1] = rr[i].y;
            rd[2] = rr[i].z;
            rd[3] = rr[i].w;
        }
        __syncthreads();
        if (k0 + 64 < ke) gload(k0 + 64);
#pragma unroll 2
        for (uint32_t kk = 0; kk < 64; kk += 4) {
            float bv[2];
#pragma unroll
            for (uint32_t nt = 0; nt < 2; nt++) bv[nt] = rs[(32 * w + 16 * nt + col) * kP + kk + grp];
#pragma unroll
            for (uint32_t mt = 0; mt < kRT / 16; mt++) {
                const float av = xs[(16 * mt + col) * kP + kk + grp];
#pragma unroll
                for (uint32_t nt = 0; nt < 2; nt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[nt], acc[mt][nt], 0, 0, 0);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (uint32_t mt = 0; mt < kRT / 16; mt++)
#pragma unroll
        for (uint32_t nt = 0; nt < 2; nt++)
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t t = t0 + 16 * mt + 4 * grp + i, e = 32 * w + 16 * nt + col;
                if (t < S && e < E) LR[(size_t)t * E + e] = acc[mt][nt][i];
            }
}

// Top-k routing of one token per wave (ops.rs:45-56): the k largest logits
// under the total order, lower index on ties; softmax over the chosen logits
// in rank order (ops.rs:29-44).  E <= 128.  The logits are the sum of the
// router's kPfRouterSplit partial sums, added in split order; every partial
// is requested before the first is added (one memory round trip, not one
// per split).
__global__ __launch_bounds__(kBlock) void k_pf_topk(const float* LR, uint32_t S, uint32_t E,
                                                    uint32_t top, uint32_t* ids, float* wts, DevState* st,
                                                    uint32_t* route_log, float* gap_log, uint32_t layers,
                                                    uint32_t layer, uint32_t p0) {
    const uint32_t lane = threadIdx.x & 63, t = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (t >= S) return;  // wave-uniform
    // lanes past E read column E - 1 (in the row) and drop it
    const uint32_t c0 = min(lane, E - 1), c1 = min(lane + 64, E - 1);
    float pa[kPfRouterSplit], pb[kPfRouterSplit];
#pragma unroll
    for (uint32_t ks = 0; ks < kPfRouterSplit; ks++) {
        const float* lg = LR + ((size_t)ks * S + t) * E;
        pa[ks] = lg[c0];
        pb[ks] = lg[c1];
    }
    float v0 = lane < E ? pa[0] : 0.f, v1 = lane + 64 < E ? pb[0] : 0.f;
#pragma unroll
    for (uint32_t ks = 1; ks < kPfRouterSplit; ks++) {
        v0 += lane < E ? pa[ks] : 0.f;
        v1 += lane + 64 < E ? pb[ks] : 0.f;
    }
    const bool bad = (lane < E && !finite_f(v0)) || (lane + 64 < E && !finite_f(v1));
    if (__any(bad)) {
        if (lane == 0) atomicOr(&st->err, kErrRouter);
        return;
    }
    bool u0 = lane >= E, u1 = lane + 64 >= E;  // used (or absent)
    float sel = 0.f;
    uint32_t sid = 0;
    for (uint32_t k = 0; k < top; k++) {
        int32_t bk = INT32_MIN;
        uint32_t bi = 0xffffffffu;
        if (!u0) best_merge(bk, bi, total_key(v0), lane);
        if (!u1) best_merge(bk, bi, total_key(v1), lane + 64);
        wave_best(bk, bi);
        if (bi == lane) u0 = true;
        if (bi == lane + 64) u1 = true;
        const float w0 = __shfl(v0, bi & 63, 64), w1 = __shfl(v1, bi & 63, 64);
        if (lane == k) {
            sid = bi;
            sel = bi < 64 ? w0 : w1;
        }
    }
    // the gap log: rank top's logit (the next pick) against rank top - 1's,
    // relative to the largest |logit|
    float gap = INFINITY;
    {
        int32_t bk = INT32_MIN;
        uint32_t bi = 0xffffffffu;
        if (!u0) best_merge(bk, bi, total_key(v0), lane);
        if (!u1) best_merge(bk, bi, total_key(v1), lane + 64);
        wave_best(bk, bi);
        const float amax = wave_max(fmaxf(lane < E ? fabsf(v0) : 0.f, lane + 64 < E ? fabsf(v1) : 0.f));
        const float last = __shfl(sel, top - 1, 64);
        if (bi != 0xffffffffu) gap = (last - __shfl(bi < 64 ? v0 : v1, bi & 63, 64)) / amax;
    }
    // softmax in rank order, sequential like ops.rs
    const float mx = wave_max(lane < top ? sel : -INFINITY);
    const float ex = lane < top ? expf(sel - mx) : 0.f;
    float sum = 0.f;
    {
#pragma clang fp contract(off)
        for (uint32_t k = 0; k < top; k++) sum += __shfl(ex, k, 64);
    }
    if (lane < top) {
        ids[(size_t)t * top + lane] = sid;
        wts[(size_t)t * top + lane] = ex / sum;
        route_log[((size_t)(p0 + t) * layers + layer) * top + lane] = sid;  // routing log (diagnostics)
    }
    if (lane == 0) gap_log[(size_t)(p0 + t) * layers + layer] = gap;
}

// Groups the S*top (token, slot) assignments by expert (one workgroup):
// goff = exclusive prefix of the per-expert counts, tok/asg = the
// assignments sorted by expert (order within an expert is arbitrary), and
// the list of 128-row GEMM tiles (te, tm).  Up to 16,384 assignments are
// placed in LDS first and stored in order (coalesced: stored straight to
// their sorted positions, every store instruction of a wave touched up to 64
// cache lines).
__global__ __launch_bounds__(1024) void k_pf_group(const uint32_t* ids, uint32_t n, uint32_t top, uint32_t E,
                                                   uint32_t* goff, uint32_t* tok, uint32_t* asg, uint32_t* te,
                                                   uint32_t* tm, uint32_t* ntile) {
    __shared__ uint32_t cnt[256], cur[256], tb[256];  // E <= 255
    __shared__ uint32_t srt[16384], ntot;              // sorted assignments, their count
    for (uint32_t e = threadIdx.x; e < 256; e += 1024) cnt[e] = 0;
    // this thread's assignments a = threadIdx.x + 1024 i, all loaded before
    // any is used (one memory round trip instead of one per assignment)
    constexpr uint32_t kPer = 16;  // 1024 x 16 = 16,384 = a 2,048-token chunk's top-8 assignments
    uint32_t myid[kPer], mys[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++) {
        const uint32_t a = threadIdx.x + 1024 * i;
        myid[i] = a < n ? ids[a] : 0xffffffffu;
    }
    __syncthreads();
    // the count's old value is the assignment's slot within its expert
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++)
        if (myid[i] < E) mys[i] = atomicAdd(&cnt[myid[i]], 1u);  // ids < E unless routing failed (reported)
    for (uint32_t a = threadIdx.x + 1024 * kPer; a < n; a += 1024)  // chunks beyond 16,384 assignments
        if (ids[a] < E) atomicAdd(&cnt[ids[a]], 1u);
    __syncthreads();
    if (threadIdx.x < 64) {
        // wave 0: exclusive prefix sums of the counts and of the tile counts,
        // lane l holding experts 4l .. 4l + 3
        const uint32_t lane = threadIdx.x;
        uint32_t c4[4], t4[4], cs = 0, ts = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            c4[k] = cnt[4 * lane + k];  // zero past E
            t4[k] = (c4[k] + kGM - 1) / kGM;
            cs += c4[k];
            ts += t4[k];
        }
        uint32_t ci = cs, ti = ts;
#pragma unroll
        for (uint32_t o = 1; o < 64; o <<= 1) {
            const uint32_t cu = __shfl_up(ci, o, 64), tu = __shfl_up(ti, o, 64);
            if (lane >= o) {
                ci += cu;
                ti += tu;
            }
        }
        uint32_t off = ci - cs, toff = ti - ts;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint32_t e = 4 * lane + k;
            if (e <= E) goff[e] = off;  // goff[E] = total
            cur[e] = off;
            tb[e] = toff;
            off += c4[k];
            toff += t4[k];
        }
        if (lane == 63) {
            *ntile = ti;
            ntot = ci;
        }
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < E; e += 1024)
        for (uint32_t m = 0, t = tb[e]; m < cnt[e]; m += kGM, t++) {
            te[t] = e;
            tm[t] = m;
        }
    const bool staged = n <= 1024 * kPer;  // workgroup-uniform
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++) {
        const uint32_t a = threadIdx.x + 1024 * i;
        if (myid[i] >= E) continue;
        if (staged) {
            srt[cur[myid[i]] + mys[i]] = a;  // cur = the expert's offset
        } else {
            const uint32_t p = atomicAdd(&cur[myid[i]], 1u);
            tok[p] = a / top;
            asg[p] = a;
        }
    }
    if (staged) {
        __syncthreads();
        for (uint32_t p = threadIdx.x; p < ntot; p += 1024) {
            const uint32_t a = srt[p];
            tok[p] = a / top;
            asg[p] = a;
        }
    }
    for (uint32_t a = threadIdx.x + 1024 * kPer; a < n; a += 1024) {
        if (ids[a] >= E) continue;
        const uint32_t p = atomicAdd(&cur[ids[a]], 1u);
        tok[p] = a / top;
        asg[p] = a;
    }
}

// MoE combine + residual (model.rs:281-287): moe = sum_k w_k down_k in rank
// order, then x += moe; 4 consecutive elements per thread.  With nw (the
// next layer's attention RMSNorm weights) the block also writes that norm's
// fp16 output (k_pf_norm's arithmetic, with the sum of squares taken in this
// kernel's element order), so the next layer starts on its GEMM.

// A float4 read once (non-temporal hint): the combine's expert rows, 134 MB
// per layer at 30B, each read by exactly one workgroup.
__device__ __forceinline__ float4 ld4s(const float* p) {
    typedef float f4s __attribute__((ext_vector_type(4)));
    const f4s t = __builtin_nontemporal_load((gptr<f4s>)p);
    return make_float4(t.x, t.y, t.z, t.w);
}

__global__ __launch_bounds__(kBlock) void k_pf_combine(float* X, const float* Y, const float* wts, uint32_t H,
                                                       uint32_t top, const float* nw, float eps, _Float16* Xn16,
                                                       uint32_t* err) {
    __shared__ float red[kWaves];
    const size_t t = blockIdx.x;
    const uint32_t tk = min(top, 8u);  // ranks held in registers; more (top > 8) are read in a loop
    float w[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; k++) w[k] = wts[t * top + min(k, top - 1)];
    float ss = 0.f;
    for (uint32_t i4 = threadIdx.x; 4 * i4 < H; i4 += kBlock) {  // H % 64 == 0
        const size_t i = 4 * (size_t)i4;
        // every rank's row requested before the sum (rows past top clamped,
        // their values unused)
        float4 y[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) y[k] = ld4s(Y + (t * top + min(k, top - 1)) * H + i);
        float4 xv = *reinterpret_cast<const float4*>(X + t * H + i);
        float4 moe = make_float4(0.f, 0.f, 0.f, 0.f);
        {
#pragma clang fp contract(off)
#pragma unroll
            for (uint32_t k = 0; k < 8; k++)
                if (k < tk) {
                    moe.x += w[k] * y[k].x;
                    moe.y += w[k] * y[k].y;
                    moe.z += w[k] * y[k].z;
                    moe.w += w[k] * y[k].w;
                }
            for (uint32_t k = 8; k < top; k++) {
                const float wk = wts[t * top + k];
                const float4 yk = *reinterpret_cast<const float4*>(Y + (t * top + k) * H + i);
                moe.x += wk * yk.x;
                moe.y += wk * yk.y;
                moe.z += wk * yk.z;
                moe.w += wk * yk.w;
            }
            xv.x += moe.x;
            xv.y += moe.y;
            xv.z += moe.z;
            xv.w += moe.w;
        }
        *reinterpret_cast<float4*>(X + t * H + i) = xv;
        ss = fmaf(xv.x, xv.x, ss);
        ss = fmaf(xv.y, xv.y, ss);
        ss = fmaf(xv.z, xv.z, ss);
        ss = fmaf(xv.w, xv.w, ss);
    }
    if (!nw) return;  // uniform
    const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
    bool bad = false;
    for (uint32_t i4 = threadIdx.x; 4 * i4 < H; i4 += kBlock) {  // this thread's own x values
        const size_t i = 4 * (size_t)i4;
        const float4 xv = *reinterpret_cast<const float4*>(X + t * H + i);
        const float4 w4 = *reinterpret_cast<const float4*>(nw + i);
        _Float16* o = Xn16 + t * H + i;
        o[0] = to_h(xv.x * (scale * w4.x), bad);
        o[1] = to_h(xv.y * (scale * w4.y), bad);
        o[2] = to_h(xv.z * (scale * w4.z), bad);
        o[3] = to_h(xv.w * (scale * w4.w), bad);
    }
    note_range(bad, err);
}

// ----------------------------------------------------------- attention --
// Causal GQA attention (ops.rs:57-98) of 16-query blocks of the chunk -- at
// positions p0 + q -- for the G <= 8 query heads of KV head g (wave w: heads
// 2w and 2w + 1, which share every K and V fragment the wave reads from LDS),
// over keys [0, p0 + q], on the fp16 matrix
// cores with an online softmax in fp32.  Keys come from an fp16 copy of the
// layer's K ([kvhead][pos][128]) and V, transposed ([kvhead][128][pos], row
// pitch vp, a multiple of 64), so a
// 64-key block is staged in LDS with straight 16-byte copies, then
//   S^T = K Q^T  (keys x queries: lane = (4 keys, 1 query), so each lane's
//                 probabilities already form the A operand of P V, the key
//                 order inside a 32-key step being the same permutation for
//                 P and V),
//   O  += P V    (queries x 128 dims).
// The causal triangle gives block q about q key blocks.  Blocks nqb-1-i and
// i form pair i, which two workgroups share with about half of its key blocks
// each: workgroup 0 takes the first key blocks of the long block, workgroup
// 1 the rest of them and then the short block, and the two parts of the long
// block are merged by the workgroup that finishes second (through memory, no
// waiting).  So every workgroup of the launch has the same work, and the two
// a CU holds at once (two waves per SIMD) both run to the end; with one long
// and one short block per CU, the long block ran alone for most of the launch
// at one wave per SIMD, about 1.2x as long.  Two heads per wave halve the LDS
// reads per product against one head per wave.
constexpr uint32_t kAQ = 16, kAK = 64;
constexpr uint32_t kQT = 2;  // query heads per wave (index qt), each over the block's 16 queries
// LDS pitches (halfs).  K rows of 272 bytes, their 16-byte column chunks
// swizzled (kchunk) so that the staging writes (four threads per key) spread
// over the banks like the fragment reads (one chunk per 8 lanes); V^T rows of
// 136 bytes, so that the 16 rows one 8-byte fragment read spans fall on
// distinct banks (written 8 bytes at a time).
constexpr uint32_t kKL = 128 + 8, kVL = kAK + 4;
__device__ __forceinline__ uint32_t kchunk(uint32_t c) { return c ^ (2 * (c >> 3)); }

__device__ __forceinline__ uint2 pack4h(float a, float b, float c, float d) {
    h8v t;  // only the first four used
    t[0] = (_Float16)a;
    t[1] = (_Float16)b;
    t[2] = (_Float16)c;
    t[3] = (_Float16)d;
    const uint4 u = __builtin_bit_cast(uint4, t);
    return make_uint2(u.x, u.y);
}

// Hand-over of a split query block: one slot per workgroup, [wave][value][lane]
// floats, values 32 qt + 4 dt + i = o[qt][dt][i], then m and l of head qt at
// 64 + 2 qt and 65 + 2 qt.
constexpr uint32_t kXv = kQT * 32 + 2 * kQT;
static_assert(4 * kXv * 64 == kPfAttnSlot, "hand-over slot size");

__global__ __launch_bounds__(kGT, 2) void k_pf_attn(const _Float16* Q16, const _Float16* Kh, const _Float16* Vth,
                                                 uint32_t p0, uint32_t S, uint32_t G, uint32_t ctx, uint32_t vp,
                                                 uint32_t qd, _Float16* O16, float* xw, uint32_t* xcnt) {
    __shared__ __align__(16) _Float16 Kl[kAK * kKL];
    __shared__ __align__(16) _Float16 Vt[128 * kVL];
    __shared__ uint32_t xlast;  // arrivals before this workgroup's at a split block
    // pair pi of KV head g: long block qL = nqb-1-pi and short block qS = pi
    // (the same block for the middle one of an odd count), two workgroups
    const uint32_t nqb = (S + kAQ - 1) / kAQ, npair = (nqb + 1) / 2, kvh = gridDim.x / (2 * npair);
    const uint32_t role = blockIdx.x & 1, unit = blockIdx.x >> 1, g = unit % kvh, pi = unit / kvh;
    const uint32_t qL = nqb - 1 - pi, qS = pi;
    const uint32_t ntL = (p0 + min(qL * kAQ + kAQ, S) + kAK - 1) / kAK;
    const uint32_t ntS = qS != qL ? (p0 + min(qS * kAQ + kAQ, S) + kAK - 1) / kAK : 0;
    // split of qL: workgroup 0 takes key blocks [0, hs), workgroup 1 [hs, ntL)
    // and then all of qS, hs about half the pair's key blocks and 64 hs <= qL's
    // first query position (each query sees a key of both parts)
    const uint32_t hs = min(min((ntL + ntS + 1) / 2, ntL), (p0 + qL * kAQ) / kAK);
    const bool split = hs > 0 && hs < ntL;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, grp = lane >> 4, col = lane & 15;
    const bool hok = kQT * w < G;  // the wave's first head exists (wave-uniform)
    // scores / sqrt(128) (ops.rs:87), exponentiated base 2
    const float sc2 = 1.4426950408889634f / sqrtf(128.0f);
    const _Float16* kg = Kh + (size_t)g * ctx * 128;
    const _Float16* vg = Vth + (size_t)g * 128 * vp;
    // staging: K thread (key tid/4, 32 dims); V^T thread (dim tid/2, 32 keys)
    const uint32_t skey = tid >> 2, sd0 = (tid & 3) * 32, sdim = tid >> 1, skk0 = (tid & 1) * 32;
    auto run = [&](const uint32_t qb, const uint32_t ta, const uint32_t tb, const bool part) {
        const uint32_t q0 = qb * kAQ;
        h8v qf[kQT][4];
#pragma unroll
        for (uint32_t qt = 0; qt < kQT; qt++) {
            const uint32_t q = q0 + col, hh = kQT * w + qt;
            const bool ok = hh < G && q < S;
            const _Float16* src = Q16 + ((size_t)(g * G + hh) * S + q) * 128 + 8 * grp;
#pragma unroll
            for (uint32_t ks = 0; ks < 4; ks++) {
                if (ok) {  // q scaled once, so the scores come out in base-2 units
                    const h8v t = gld<h8v>(src + 32 * ks);
#pragma unroll
                    for (int i = 0; i < 8; i++) qf[qt][ks][i] = (_Float16)((float)t[i] * sc2);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) qf[qt][ks][i] = (_Float16)0.f;
                }
            }
        }
        // O^T tiles: lane holds dims 16 dt + 4 grp + i of query 16 qt + col, so the
        // softmax statistics of its query are lane-local
        f4v o[kQT][8];
#pragma unroll
        for (int qt = 0; qt < (int)kQT; qt++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[qt][dt] = f4v{0.f, 0.f, 0.f, 0.f};
        float m[kQT], l[kQT];
#pragma unroll
        for (int qt = 0; qt < (int)kQT; qt++) {
            m[qt] = -INFINITY;
            l[qt] = 0.f;
        }
        const uint32_t kend = p0 + min(q0 + kAQ, S);  // keys [0, kend) can be attended
        uint4 kr[4], vr[4];
        auto kvload = [&](uint32_t k0) {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
                kr[i] = k0 + skey < kend ? gld<uint4>(kg + (size_t)(k0 + skey) * 128 + sd0 + 8 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t kk = skk0 + 8 * i;
                if (k0 + kk + 8 <= kend) {
                    vr[i] = gld<uint4>(vg + (size_t)sdim * vp + k0 + kk);
                } else if (k0 + kk < kend) {  // partial group at the end: element by element
                    h8v t;
#pragma unroll
                    for (uint32_t j = 0; j < 8; j++)
                        t[j] = k0 + kk + j < kend ? vg[(size_t)sdim * vp + k0 + kk + j] : (_Float16)0.f;
                    vr[i] = __builtin_bit_cast(uint4, t);
                } else {
                    vr[i] = make_uint4(0, 0, 0, 0);
                }
            }
        };
        const uint32_t kstop = tb * kAK;
        kvload(ta * kAK);
        for (uint32_t k0 = ta * kAK; k0 < kstop; k0 += kAK) {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                *reinterpret_cast<uint4*>(Kl + skey * kKL + 8 * kchunk(sd0 / 8 + i)) = kr[i];
                uint2* vd = reinterpret_cast<uint2*>(Vt + sdim * kVL + skk0 + 8 * i);
                vd[0] = make_uint2(vr[i].x, vr[i].y);
                vd[1] = make_uint2(vr[i].z, vr[i].w);
            }
            __syncthreads();
            if (k0 + kAK < kstop) kvload(k0 + kAK);  // next block, during this one
            if (hok) {  // wave-uniform
                f4v st[4][kQT];
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int qt = 0; qt < (int)kQT; qt++) st[kt][qt] = f4v{0.f, 0.f, 0.f, 0.f};
                // every K fragment of the block first (one LDS wait, not one
                // per product)
                h8v kf[4][4];
#pragma unroll
                for (uint32_t ks = 0; ks < 4; ks++)
#pragma unroll
                    for (uint32_t kt = 0; kt < 4; kt++)
                        kf[ks][kt] = *reinterpret_cast<const h8v*>(Kl + (16 * kt + col) * kKL + 8 * kchunk(4 * ks + grp));
                __builtin_amdgcn_sched_barrier(0);  // keeps the reads together, ahead of the products
#pragma unroll
                for (uint32_t ks = 0; ks < 4; ks++) {
#pragma unroll
                    for (uint32_t kt = 0; kt < 4; kt++) {
#pragma unroll
                        for (uint32_t qt = 0; qt < kQT; qt++)
                            st[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[ks][kt], qf[qt][ks], st[kt][qt], 0, 0, 0);
                    }
                }
                // causal mask (only blocks that reach past the block's first
                // query or past kend have masked keys), online softmax per query
                const bool edge = k0 + kAK > p0 + q0 + 1 || k0 + kAK > kend;  // block-uniform
#pragma unroll
                for (uint32_t qt = 0; qt < kQT; qt++) {
                    const uint32_t qpos = p0 + q0 + col;
                    float mx = -INFINITY;
                    if (edge) {
#pragma unroll
                        for (uint32_t kt = 0; kt < 4; kt++)
#pragma unroll
                            for (uint32_t i = 0; i < 4; i++) {
                                const uint32_t kpos = k0 + 16 * kt + 4 * grp + i;
                                const float v = (kpos <= qpos && kpos < kend) ? st[kt][qt][i] : -INFINITY;
                                st[kt][qt][i] = v;
                                mx = fmaxf(mx, v);
                            }
                    } else {
#pragma unroll
                        for (uint32_t kt = 0; kt < 4; kt++)
#pragma unroll
                            for (uint32_t i = 0; i < 4; i++) mx = fmaxf(mx, st[kt][qt][i]);
                    }
                    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    // Lazy rescale: the reference maximum m moves (and O, l
                    // are rescaled) only when some query of the wave saw a
                    // score above m + 8, so the probabilities stay <= 2^8 (fp16
                    // holds them at full precision) and most blocks skip the
                    // rescale; O / l is the same ratio whichever m it used.
                    // A segment's first block always moves it (m = -inf; every
                    // query sees a key of it).
                    if (__any(mx > m[qt] + 8.f)) {  // wave-uniform
                        const float mn = fmaxf(m[qt], mx);
                        const float alpha = __builtin_amdgcn_exp2f(m[qt] - mn);  // 0 on the first block
                        l[qt] *= alpha;
#pragma unroll
                        for (uint32_t dt = 0; dt < 8; dt++) o[qt][dt] *= alpha;
                        m[qt] = mn;
                    }
                    float ls = 0.f;
#pragma unroll
                    for (uint32_t kt = 0; kt < 4; kt++)
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) {
                            const float pv = __builtin_amdgcn_exp2f(st[kt][qt][i] - m[qt]);
                            st[kt][qt][i] = pv;
                            ls += pv;
                        }
                    l[qt] += ls;
                }
                // O^T += V^T P^T: A = V^T rows (dims) with keys in the same
                // permuted order as this lane's probabilities, B = P^T
#pragma unroll
                for (uint32_t ks2 = 0; ks2 < 2; ks2++) {
                    h8v pb[kQT];
#pragma unroll
                    for (uint32_t qt = 0; qt < kQT; qt++)
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) {
                            pb[qt][i] = (_Float16)st[2 * ks2][qt][i];
                            pb[qt][4 + i] = (_Float16)st[2 * ks2 + 1][qt][i];
                        }
                    // the eight V^T fragments of this key half first
                    h8v va[8];
#pragma unroll
                    for (uint32_t dt = 0; dt < 8; dt++) {
                        const _Float16* vrow = Vt + (16 * dt + col) * kVL + 32 * ks2 + 4 * grp;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vrow), hi = *reinterpret_cast<const uint2*>(vrow + 16);
                        va[dt] = __builtin_bit_cast(h8v, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (uint32_t dt = 0; dt < 8; dt++)
#pragma unroll
                        for (uint32_t qt = 0; qt < kQT; qt++)
                            o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt], pb[qt], o[qt][dt], 0, 0, 0);
                }
            }
            __syncthreads();
        }
        if (part) {
            // Both parts of a split block store (O, m, l) to their slot,
            // written through to memory; the second to arrive merges them
            // with weights 2^(m_part - max m), part 0 first whichever
            // workgroup computes it, so the bits do not depend on the order.
            float* mine = xw + ((size_t)(unit * 2 + role) * 4 + w) * kXv * 64 + lane;
            if (hok)
#pragma unroll
                for (uint32_t qt = 0; qt < kQT; qt++) {
#pragma unroll
                    for (uint32_t dt = 0; dt < 8; dt++)
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) st_sys(mine + (qt * 32 + dt * 4 + i) * 64, o[qt][dt][i]);
                    st_sys(mine + (kQT * 32 + 2 * qt) * 64, m[qt]);
                    st_sys(mine + (kQT * 32 + 2 * qt + 1) * 64, l[qt]);
                }
            __builtin_amdgcn_s_waitcnt(0);  // this wave's write-through stores have completed
            __syncthreads();
            if (tid == 0) {
                const uint32_t old = __hip_atomic_fetch_add(xcnt + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                xlast = old;
                if (old == 1) __hip_atomic_store(xcnt + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            __syncthreads();
            if (xlast != 1) return;  // the other part merges
            const float* other = xw + ((size_t)(unit * 2 + (role ^ 1)) * 4 + w) * kXv * 64 + lane;
            if (hok)
#pragma unroll
                for (uint32_t qt = 0; qt < kQT; qt++) {
                    const float mo = ld_sys(other + (kQT * 32 + 2 * qt) * 64), lo = ld_sys(other + (kQT * 32 + 2 * qt + 1) * 64);
                    const float m0 = role ? mo : m[qt], m1 = role ? m[qt] : mo;
                    const float l0 = role ? lo : l[qt], l1 = role ? l[qt] : lo;
                    const float mm = fmaxf(m0, m1);
                    const float a0 = __builtin_amdgcn_exp2f(m0 - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
                    l[qt] = __builtin_fmaf(a0, l0, a1 * l1);
#pragma unroll
                    for (uint32_t dt = 0; dt < 8; dt++)
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) {
                            const float oo = ld_sys(other + (qt * 32 + dt * 4 + i) * 64);
                            const float o0 = role ? oo : o[qt][dt][i], o1 = role ? o[qt][dt][i] : oo;
                            o[qt][dt][i] = __builtin_fmaf(a0, o0, a1 * o1);
                        }
                }
        }
        if (hok)
#pragma unroll
            for (uint32_t qt = 0; qt < kQT; qt++) {
                float lt = l[qt] + __shfl_xor(l[qt], 16, 64);
                lt += __shfl_xor(lt, 32, 64);
                const float inv = 1.0f / lt;
                const uint32_t q = q0 + col, hh = kQT * w + qt;
                if (q < S && hh < G) {
                    _Float16* dst = O16 + (size_t)q * qd + (g * G + hh) * 128 + 4 * grp;
#pragma unroll
                    for (uint32_t dt = 0; dt < 8; dt++)
                        *reinterpret_cast<uint2*>(dst + 16 * dt) =
                            pack4h(o[qt][dt][0] * inv, o[qt][dt][1] * inv, o[qt][dt][2] * inv, o[qt][dt][3] * inv);
                }
            }
    };
    // the workgroup's segments, as two call sites (a loop over them kept
    // values live across its back edge and spilled): workgroup 0 the long
    // block (its first part when split), workgroup 1 the long block's second
    // part (when split), then the short block
    if (role == 0 || split) run(qL, role ? hs : 0, role || !split ? ntL : hs, split);
    if (role == 1 && qS != qL) run(qS, 0, ntS, false);
}

// fp16 copies of the KV cache positions [r0, r0 + gridDim.x) of one layer for
// the attention: Kh[kvhead][pos][128] and Vth[kvhead][128][pos] (row pitch
// vp, a multiple of 64).  One workgroup per position.
__global__ __launch_bounds__(kBlock) void k_pf_kvh(const float* kcache, const float* vcache, uint32_t r0,
                                                   uint32_t kvheads, uint32_t ctx, uint32_t vp, _Float16* Kh,
                                                   _Float16* Vth) {
    const uint32_t pos = r0 + blockIdx.x;
    for (uint32_t i = threadIdx.x; i < kvheads * 128; i += kBlock) {
        const uint32_t g = i >> 7, d = i & 127;
        Kh[((size_t)g * ctx + pos) * 128 + d] = (_Float16)kcache[((size_t)g * ctx + pos) * 128 + d];
        Vth[((size_t)g * 128 + d) * vp + pos] = (_Float16)vcache[((size_t)g * ctx + pos) * 128 + d];
    }
}

#define QH_INSTANTIATE_PREFILL_GEMM(K)                                                                          \
    template __global__ void k_gemm_gateup<K>(const _Float16*, uint32_t, ExpertTiles, DevMat, DevMat, _Float16*,      \
                                              uint32_t*);                                                           \
    template __global__ void k_gemm_down<K>(const _Float16*, ExpertTiles, DevMat, float*);                          \

QH_INSTANTIATE_PREFILL_GEMM(Q4_0)
QH_INSTANTIATE_PREFILL_GEMM(Q8_0)
QH_INSTANTIATE_PREFILL_GEMM(Q4_K)
QH_INSTANTIATE_PREFILL_GEMM(Q5_K)
QH_INSTANTIATE_PREFILL_GEMM(Q6_K)

}  // namespace qh
