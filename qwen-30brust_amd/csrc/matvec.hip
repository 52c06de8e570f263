// Streaming matvec over block-quantised rows: y_b = W_b x_b for up to
// kMvMaxVec vectors in one launch (Backend::matvec, src/backend.rs:29-52,
// resolved as matrix(), :57-75; the Vulkan packed_matvec surface,
// src/backend.rs:173-182; and, with several vectors, the per-expert down
// projections of one MoE layer, src/model.rs:274-284).
//
// Bandwidth layout.  A row of C*L chunks (32 weights each) is spread over L
// lanes, C chunks per lane (lane cl owns chunks cl, cl + L, ...), so a wave
// covers S = 64 / L rows per row step and R row steps per group.  Each
// workgroup owns a contiguous range of groups, which its waves take in turn.
// Every wave keeps two groups in flight: the next group's loads are issued before
// the current group is reduced, unconditionally (row and chunk clamped into
// the matrix; the surplus results are dropped), so the compiler waits for
// exactly the group it computes.  x is staged once per workgroup in LDS in the
// padded layout px() (conflict-free 16-byte reads of the chunk runs).
#include "qh_block.hpp"

namespace qh {

constexpr int kMvT = 512;                 // threads per workgroup
constexpr int kMvW = kMvT / 64;           // waves per workgroup
constexpr uint32_t kMvMaxVec = 8;         // vectors per launch
constexpr uint32_t kMvMaxXFloats = 12288; // sum over vectors of pad64(cols): 52 KB of LDS with padding

struct MvArgs {
    const uint8_t* mat[kMvMaxVec];  // matrix of vector b (device row layout, m.drb bytes per row)
    DevMat m;                       // rows, cols, format of every matrix
    const float* x;                 // [nb][cols]
    float* y;                       // [nb][rows]
    uint32_t nb;                    // vectors
    uint32_t lshift;                // log2 L (lanes per row)
    uint32_t gpb;                   // row groups per vector
    uint32_t per;                   // row groups per workgroup
    uint32_t xpitch;                // LDS elements between vectors (a multiple of 64, before padding)
    uint32_t single;                // every wave has at most one group
    uint32_t xsum_off;              // LDS float offset of the chunk run sums (even)
};

// x elements staged per thread (float4 loads, issued before the weights):
// the 512-thread form stages up to kMvMaxXFloats, the 64-thread form (small
// matrices, one wave per workgroup) up to 2,048 floats.
template <int NT>
constexpr int mv_xv() { return NT == kMvT ? (int)(kMvMaxXFloats / 4 + kMvT - 1) / kMvT : 8; }

// The two 16-float runs of chunk c of the padded LDS vector that starts at
// element `base` (their sums come precomputed).
template <uint32_t KIND>
__device__ __forceinline__ void x_runs_only(const float* xs, uint32_t base, uint32_t c, float* xa, float* xb) {
    const float4* pa = reinterpret_cast<const float4*>(xs + px(base + Fmt<KIND>::xoff_a(c)));
    const float4* pb = reinterpret_cast<const float4*>(xs + px(base + Fmt<KIND>::xoff_b(c)));
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 u = pa[k], v = pb[k];
        xa[4 * k] = u.x; xa[4 * k + 1] = u.y; xa[4 * k + 2] = u.z; xa[4 * k + 3] = u.w;
        xb[4 * k] = v.x; xb[4 * k + 1] = v.y; xb[4 * k + 2] = v.z; xb[4 * k + 3] = v.w;
    }
}

// FULL: one vector whose rows are exactly 64 C chunks (L = 64 lanes per
// row): every lane takes chunks lane, lane + 64, ..., a wave's rows are
// wave-uniform (their offsets in scalar registers), and no chunk is idle, so
// the group, row and chunk arithmetic of the general form (the lane layout is
// a launch argument there) leaves the vector ALU.  The vocab projection
// (2,048 columns) and the 4,096-column o-projection take it.
template <uint32_t KIND, int C, int R, int NT, bool FULL>
__global__ __launch_bounds__(NT) void k_mv_stream(MvArgs a) {
    constexpr int NW = NT / 64, XV = mv_xv<NT>();
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    float2* xsum = reinterpret_cast<float2*>(xs + a.xsum_off);  // [nb][cpr]
    using Raw = typename Fmt<KIND>::Raw;
    const DevMat& m = a.m;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lsh = FULL ? 6u : a.lshift;
    const uint32_t L = 1u << lsh, S = 64u >> lsh, sub = FULL ? 0u : lane >> lsh, cl = FULL ? lane : lane & (L - 1);
    const uint32_t cpr = m.cols / 32, rpg = R * S;
    const uint32_t ngrp = FULL ? a.gpb : a.nb * a.gpb;
    const uint32_t g0 = min(blockIdx.x * a.per, ngrp), g1 = min(g0 + a.per, ngrp);
    if (g0 >= g1) return;  // the whole workgroup

    const uint32_t mbytes = m.rows * m.drb;  // < 2^32 (checked by the host)
    // vector b and row group rg of group g (FULL: one vector)
    auto split = [&](uint32_t g, uint32_t& b, uint32_t& rg) {
        if constexpr (FULL) {
            b = 0;
            rg = g;
        } else {
            b = g / a.gpb;
            rg = g - b * a.gpb;
        }
    };
    auto load_group = [&](Raw (&t)[R][C], uint32_t g) {
        uint32_t b, rg;
        split(g, b, rg);
        // a select chain, so that the argument array stays in scalar registers
        const uint8_t* base = a.mat[0];
        if constexpr (!FULL) {
#pragma unroll
            for (uint32_t j = 1; j < kMvMaxVec; j++) base = b == j ? a.mat[j] : base;
        }
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(base, mbytes);
#pragma unroll
        for (int k = 0; k < R; k++) {
            const uint32_t ro = min(rg * rpg + sub + k * S, m.rows - 1) * m.drb;
#pragma unroll
            for (int i = 0; i < C; i++) {
                if constexpr (FULL)
                    t[k][i] = bload_u<KIND>(rs, __builtin_amdgcn_readfirstlane(ro), m.geo, cl + i * L);
                else
                    t[k][i] = bload<KIND>(rs, ro, m.geo, min(cl + i * L, cpr - 1));
            }
        }
    };
    auto reduce_store = [&](const Raw (&t)[R][C], uint32_t g) {
        uint32_t b, rg;
        split(g, b, rg);
        float acc[R];
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = 0.f;
#pragma unroll
        for (int i = 0; i < C; i++) {
            const uint32_t ch = cl + i * L;
            if (FULL || ch < cpr) {
                float xa[16], xb[16];
                x_runs_only<KIND>(xs, b * a.xpitch, ch, xa, xb);
                const float2 s2 = xsum[b * cpr + ch];
                const float sa = s2.x, sb = s2.y;
#pragma unroll
                for (int k = 0; k < R; k++) acc[k] += Fmt<KIND>::dot(t[k][i], ch, xa, xb, sa, sb);
            }
        }
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = seg_sum(acc[k], (int)L);
        if (cl == 0) {
#pragma unroll
            for (int k = 0; k < R; k++) {
                const uint32_t r = rg * rpg + sub + k * S;
                if (r < m.rows) a.y[(size_t)b * m.rows + r] = acc[k];
            }
        }
    };

    // x first, then the wave's first group: the LDS writes of x then wait for
    // the x loads only (loads complete in issue order)
    const uint32_t n4 = a.nb * m.cols / 4;
    float4 xv[XV];
#pragma unroll
    for (int k = 0; k < XV; k++) xv[k] = gld<float4>(a.x + 4 * min(tid + (uint32_t)k * NT, n4 - 1));
    asm volatile("" ::: "memory");  // keeps the x loads ahead of the weight loads
    uint32_t gi = g0 + wv;
    Raw ta[R][C], tb[R][C];
    load_group(ta, min(gi, g1 - 1));
#pragma unroll
    for (int k = 0; k < XV; k++) {
        const uint32_t i = tid + (uint32_t)k * NT;
        if (i < n4) {
            const uint32_t e = 4 * i, b = e / m.cols, c = e - b * m.cols;
            *reinterpret_cast<float4*>(xs + px(b * a.xpitch + c)) = xv[k];
        }
    }
    __syncthreads();
    // the sums of every chunk's two runs (the K-quant offsets' factors)
    for (uint32_t i = tid; i < a.nb * cpr; i += NT) {
        const uint32_t b = i / cpr, c = i - b * cpr;
        float xa[16], xb[16], sa, sb;
        x_runs_p<KIND>(xs, b * a.xpitch, c, xa, xb, sa, sb);
        xsum[i] = make_float2(sa, sb);
    }
    __syncthreads();
    if (gi >= g1) return;  // wave-uniform, after the barriers
    if (a.single) {        // one group per wave: nothing to prefetch
        reduce_store(ta, gi);
        return;
    }
    // two groups in flight; the buffers alternate, so no register copy waits
    // for the loads behind it.  Wave wv takes groups g0 + wv, g0 + wv + NW, ...
    // (no workgroup-level step at the end, so a late wave delays only its
    // own rows).  Past the range the current group is loaded again (its lines
    // are cached) and the loop ends.
    while (true) {  // wave-uniform
        const uint32_t gb = gi + NW;
        load_group(tb, gb < g1 ? gb : gi);
        reduce_store(ta, gi);
        if (gb >= g1) break;
        const uint32_t ga = gb + NW;
        load_group(ta, ga < g1 ? ga : gb);
        reduce_store(tb, gb);
        if (ga >= g1) break;
        gi = ga;
    }
}

// ------------------------------------------------------------------ host --
namespace {

struct MvShape {
    int C = 0, R = 0;
    uint32_t lshift = 0;
};

// Chunks per lane C and lanes per row L (a power of two <= 64) with the
// fewest idle (lane, chunk) slots, then the rows per wave step R: 2 when that
// still gives every wave of a full grid two groups.  (Measured on the
// 151,936 x 2,048 Q6_K vocab matrix: R = 2 with up to three resident
// workgroups per CU streams at 4.76 TB/s, R = 4 at 4.38, R = 1 at 4.11.)
MvShape mv_shape(uint32_t cpr, uint64_t rows, uint32_t nb, uint32_t waves) {
    MvShape s;
    uint32_t best = 0xffffffffu;
    for (int C = 1; C <= 4; C++) {
        uint32_t L = 1, sh = 0;
        while (L * (uint32_t)C < cpr) {
            L <<= 1;
            sh++;
        }
        if (L > 64) continue;
        const uint32_t waste = L * (uint32_t)C - cpr;
        if (waste < best) {
            best = waste;
            s.C = C;
            s.lshift = sh;
        }
    }
    if (s.C == 0) return s;
    const uint64_t S = 64u >> s.lshift;
    s.R = 1;
    for (int R : {2}) {  // R C <= 4 register tiles per buffer
        if (R * s.C > 4) continue;
        if ((uint64_t)nb * ((rows + R * S - 1) / (R * S)) >= 2ull * waves) {
            s.R = R;
            break;
        }
    }
    return s;
}

// The 512-thread form: one resident wave of workgroups (as many as fit the
// device at once, from the kernel's register and LDS use), so that no
// workgroup waits for a slot behind another's whole row range.  The 64-thread
// form: one workgroup per group up to 8 per CU, for matrices too small to
// give every CU eight groups (the per-CU request rate, not HBM, bounds those).
// The 512-thread form of k_mv_stream<K, C, R, FULL>: one resident wave of
// workgroups (residency asked once per kernel, at the largest x it stages).
template <uint32_t K, int C, int R, bool FULL>
void launch_512(MvArgs a, uint64_t ngrp, uint32_t ncu, size_t smem, hipStream_t st) {
    static const int per_cu = [] {
        int n = 0;
        const size_t most = (size_t)(kMvMaxXFloats + 4 * (kMvMaxXFloats / 64) + 2 * kMvMaxXFloats / 32) * 4;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_mv_stream<K, C, R, kMvT, FULL>, kMvT, most) !=
            hipSuccess)
            n = 1;
        return std::max(n, 1);
    }();
    const uint64_t max_wg = (uint64_t)std::min(per_cu, 3) * ncu;
    const uint32_t grid = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(max_wg, (ngrp + kMvW - 1) / kMvW));
    a.per = (uint32_t)((ngrp + grid - 1) / grid);
    a.single = a.per <= (uint32_t)kMvW;
    hipLaunchKernelGGL((k_mv_stream<K, C, R, kMvT, FULL>), dim3(grid), dim3(kMvT), smem, st, a);
}

template <uint32_t K, int C, int R>
void launch_one(MvArgs a, uint64_t ngrp, uint32_t num_cu, size_t smem, hipStream_t st) {
    const uint32_t ncu = std::max(num_cu, 1u);
    const uint32_t n4 = a.nb * a.m.cols / 4;
    if (ngrp < 8ull * ncu && n4 <= (uint32_t)mv_xv<64>() * 64 && R == 1) {
        const uint32_t grid = (uint32_t)std::min<uint64_t>(ngrp, 8ull * ncu);
        a.per = (uint32_t)((ngrp + grid - 1) / grid);
        a.single = a.per <= 1;
        hipLaunchKernelGGL((k_mv_stream<K, C, R, 64, false>), dim3(grid), dim3(64), smem, st, a);
        return;
    }
    // one vector of rows exactly 64 C chunks wide: the full-width form
    if (a.nb == 1 && a.lshift == 6 && a.m.cols == 64u * 32u * (uint32_t)C)
        launch_512<K, C, R, true>(a, ngrp, ncu, smem, st);
    else
        launch_512<K, C, R, false>(a, ngrp, ncu, smem, st);
}

template <uint32_t K>
bool launch_kind(const MvShape& s, const MvArgs& a, uint64_t ngrp, uint32_t num_cu, size_t smem, hipStream_t st) {
    switch (s.C * 8 + s.R) {
    case 1 * 8 + 1: launch_one<K, 1, 1>(a, ngrp, num_cu, smem, st); return true;
    case 1 * 8 + 2: launch_one<K, 1, 2>(a, ngrp, num_cu, smem, st); return true;
    case 2 * 8 + 1: launch_one<K, 2, 1>(a, ngrp, num_cu, smem, st); return true;
    case 2 * 8 + 2: launch_one<K, 2, 2>(a, ngrp, num_cu, smem, st); return true;
    case 3 * 8 + 1: launch_one<K, 3, 1>(a, ngrp, num_cu, smem, st); return true;
    case 4 * 8 + 1: launch_one<K, 4, 1>(a, ngrp, num_cu, smem, st); return true;
    default: return false;
    }
}

}  // namespace

// y[b][r] = sum_c W_b[r][c] x[b][c] for b < nb, W_b at mats[b] with the
// shape and format of m.  Returns false (nothing launched) for shapes this
// kernel does not cover: formats that are not block-quantised, rows longer
// than 256 chunks, more than kMvMaxVec vectors, more x than LDS holds, x not
// 16-byte aligned, or a matrix past 32-bit byte offsets.
bool launch_mv_stream(const DevMat& m, const uint8_t* const* mats, uint32_t nb, const float* x, float* y,
                      uint32_t num_cu, hipStream_t st) {
    const bool quant = m.kind == Q4_0 || m.kind == Q8_0 || m.kind == Q4_K || m.kind == Q5_K || m.kind == Q6_K;
    if (!quant || nb == 0 || nb > kMvMaxVec || m.rows == 0 || m.cols % 32 != 0) return false;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return false;  // x is staged with 16-byte loads
    const uint32_t cpr = m.cols / 32, xpitch = (m.cols + 63) / 64 * 64;
    if (cpr > 256 || (uint64_t)nb * xpitch > kMvMaxXFloats) return false;
    if ((uint64_t)m.rows * m.drb + 64 >= (1ull << 32)) return false;  // 32-bit buffer offsets
    const MvShape s = mv_shape(cpr, m.rows, nb, 2 * std::max(num_cu, 1u) * kMvW);
    if (s.C == 0) return false;
    MvArgs a{};
    for (uint32_t b = 0; b < nb; b++) a.mat[b] = mats[b];
    a.m = m;
    a.x = x;
    a.y = y;
    a.nb = nb;
    a.lshift = s.lshift;
    const uint32_t rpg = (uint32_t)s.R * (64u >> s.lshift);
    a.gpb = (m.rows + rpg - 1) / rpg;
    a.xpitch = xpitch;
    const uint64_t ngrp = (uint64_t)nb * a.gpb;
    const uint32_t nx = nb * xpitch;
    a.xsum_off = nx + 4 * (nx / 64);
    const size_t smem = (size_t)(a.xsum_off + 2 * nb * cpr) * 4;
    switch (m.kind) {
    case Q4_0: return launch_kind<Q4_0>(s, a, ngrp, num_cu, smem, st);
    case Q8_0: return launch_kind<Q8_0>(s, a, ngrp, num_cu, smem, st);
    case Q4_K: return launch_kind<Q4_K>(s, a, ngrp, num_cu, smem, st);
    case Q5_K: return launch_kind<Q5_K>(s, a, ngrp, num_cu, smem, st);
    default: return launch_kind<Q6_K>(s, a, ngrp, num_cu, smem, st);
    }
}

// Read-only stream: every 16-byte word of p[0, n16) loaded once (with the
// non-temporal hint, as the matvec's weight loads), folded by xor (a word is
// stored only if the fold hits one fixed value, so the loads cannot be
// dropped).  Each workgroup reads one contiguous range (XCD x, which
// runs workgroups b = x mod 8, covers the x-th eighth), eight 16-byte loads
// in flight per thread.  Its rate is the device's practical read ceiling
// beside the matvec timings.
__global__ __launch_bounds__(kMvT) void k_read_stream(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
    const uint32_t nwg = gridDim.x, b = blockIdx.x;
    const uint32_t slot = nwg % 8 == 0 ? (b % 8) * (nwg / 8) + b / 8 : b;
    const size_t per = (n16 + nwg - 1) / nwg, beg = min((size_t)slot * per, n16), end = min(beg + per, n16);
    uint32_t acc = 0;
    size_t i = beg + threadIdx.x;
    for (; i + 7 * kMvT < end; i += 8 * kMvT) {
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            typedef unsigned int u4v __attribute__((ext_vector_type(4)));
            const u4v t = __builtin_nontemporal_load((gptr<u4v>)(p + i + k * kMvT));
            v[k] = make_uint4(t.x, t.y, t.z, t.w);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < end; i += kMvT) {
        const uint4 v = gld<uint4>(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[0] = acc;  // keeps the loads; almost never stores
}
void launch_read_stream(const void* p, size_t bytes, uint32_t* out, uint32_t grid, hipStream_t st) {
    hipLaunchKernelGGL(k_read_stream, dim3(grid), dim3(kMvT), 0, st, static_cast<const uint4*>(p), bytes / 16, out);
}

// An empty kernel: the launch floor beside the small matvec timings.
__global__ void k_empty() {}
void launch_empty(hipStream_t st) { hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, st); }

}  // namespace qh
