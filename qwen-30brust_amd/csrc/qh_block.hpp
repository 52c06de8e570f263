// Workgroup-level building blocks shared by the API kernels (kernels.hip)
// and the token-step kernels (step.hip): reductions, RMSNorm into LDS, the
// matvec row-group drivers, top-k ranking and argmax merging.
#pragma once
#include "kernels.hpp"
#include "qh_rows.hpp"

namespace qh {

// Phase marks of the token-step kernels: QH_MARK(kernel, phase) records the
// wall clock of thread 0 of each workgroup, QH_MARK_LAST that of its last
// wave to get there, when a translation unit that defines QH_PHASE_TRACE (and
// the two functions) includes the kernels; otherwise they compile to nothing.
#ifdef QH_PHASE_TRACE
__device__ void qh_phase_mark(int kernel, int phase);
__device__ void qh_phase_mark_last(int kernel, int phase);
#define QH_MARK(k, p) ::qh::qh_phase_mark((k), (p))
#define QH_MARK_LAST(k, p) ::qh::qh_phase_mark_last((k), (p))
#else
#define QH_MARK(k, p) ((void)0)
#define QH_MARK_LAST(k, p) ((void)0)
#endif

// ------------------------------------------------------------------ helpers --
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) s += red[i];
    __syncthreads();
    return s;
}

// xs[i] = x[i] * (scale * w[i]) with scale = 1/sqrt(mean(x^2) + eps)
// (src/ops.rs:3-15), zero-padded to npad; ends with a barrier.
__device__ __forceinline__ void rms_to_lds(const float* x, const float* w, uint32_t n, uint32_t npad, float eps,
                           float* xs, float* red) {
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
        float v = x[i];
        ss = fmaf(v, v, ss);
    }
    const float tot = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < npad; i += kBlock) xs[i] = i < n ? x[i] * (scale * w[i]) : 0.f;
    __syncthreads();
}

__device__ __forceinline__ void stage_lds(const float* x, uint32_t n, uint32_t npad, float* xs) {
    for (uint32_t i = threadIdx.x; i < npad; i += kBlock) xs[i] = i < n ? x[i] : 0.f;
    __syncthreads();
}

__device__ __forceinline__ uint32_t pad32(uint32_t n) { return (n + 31) / 32 * 32; }

// True for exactly one workgroup: the last one of `expected` to arrive.
// Performs release before and acquire after the counter update.
__device__ __forceinline__ bool last_arrival(uint32_t* counter, uint32_t expected) {
    __shared__ uint32_t last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t old = atomicAdd(counter, 1u);
        last = (old == expected - 1) ? 1u : 0u;
        if (last) atomicExch(counter, 0u);
    }
    __syncthreads();
    if (last) __threadfence();
    return last != 0;
}

// Row groups of a matrix processed R*S rows at a time by a wave.
struct Groups {
    int L, S;
    uint32_t per, n;
};
__device__ __forceinline__ Groups groups_of(uint32_t rows, uint32_t cols, int R) {
    Groups g;
    g.L = lanes_per_row(cols);
    g.S = 64 / g.L;
    g.per = (uint32_t)(R * g.S);
    g.n = (rows + g.per - 1) / g.per;
    return g;
}

// One group of rows of matrix m against x in LDS; epi(row, value) is called
// by the lane holding each row's result.
template <uint32_t KIND, int R, typename Epi>
__device__ __forceinline__ void mv_group(const DevMat& m, const uint8_t* base, const Groups& gp,
                                         uint32_t grp, const float* xs, Epi epi) {
    const uint32_t lane = threadIdx.x & 63, sub = lane / gp.L, cl = lane % gp.L;
    const uint32_t r0 = grp * gp.per + sub;
    float acc[R];
    rows_dot<KIND, R>(
        [&](int k) -> const uint8_t* {
            uint32_t r = r0 + k * gp.S;
            return r < m.rows ? base + (size_t)r * m.drb : nullptr;
        },
        m.geo, xs, m.cols, gp.L, cl, acc);
#pragma unroll
    for (int k = 0; k < R; k++) acc[k] = seg_sum(acc[k], gp.L);
    if (cl == 0) {
#pragma unroll
        for (int k = 0; k < R; k++) {
            uint32_t r = r0 + k * gp.S;
            if (r < m.rows) epi(r, acc[k]);
        }
    }
}

// All groups of one matrix, spread over every wave of the grid.
template <int R, typename Epi>
__device__ __forceinline__ void mv_all(const DevMat& m, const uint8_t* base, const float* xs, Epi epi) {
    const Groups gp = groups_of(m.rows, m.cols, R);
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    QH_DISPATCH_KIND(m.kind, {
        for (uint32_t grp = gw; grp < gp.n; grp += nw) mv_group<K_, R>(m, base, gp, grp, xs, epi);
    });
}

// Router top-k (src/ops.rs:45-56) inside one workgroup: rank every logit by
// total order with index tie-break, keep ranks < top, then a sequential
// softmax over the chosen logits in rank order.  Non-finite input sets
// kErrRouter and leaves ids/w untouched.
__device__ __forceinline__ void route_block(const float* logits, uint32_t n, uint32_t top, uint32_t* ids, float* w,
                            uint32_t* err, float* sw) {
    __shared__ uint32_t bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
        const float v = logits[i];
        if (!finite_f(v)) bad = 1;
        const int32_t key = total_key(v);
        uint32_t rank = 0;
        for (uint32_t j = 0; j < n; j++) {
            const int32_t kj = total_key(logits[j]);
            rank += (kj > key) || (kj == key && j < i);
        }
        if (rank < top) {
            ids[rank] = i;
            sw[rank] = v;
        }
    }
    __syncthreads();
    if (bad) {
        if (threadIdx.x == 0) atomicOr(err, kErrRouter);
        return;
    }
    if (threadIdx.x == 0) {
#pragma clang fp contract(off)
        float mx = -INFINITY;
        for (uint32_t i = 0; i < top; i++) mx = fmaxf(mx, sw[i]);
        float sum = 0.f;
        for (uint32_t i = 0; i < top; i++) {
            sw[i] = expf(sw[i] - mx);
            sum += sw[i];
        }
        for (uint32_t i = 0; i < top; i++) w[i] = sw[i] / sum;
    }
}

// (key, index) merge for argmax under total order, lowest index on ties.
__device__ __forceinline__ void best_merge(int32_t& k, uint32_t& i, int32_t k2, uint32_t i2) {
    if (k2 > k || (k2 == k && i2 < i)) {
        k = k2;
        i = i2;
    }
}
template <int CTRL>
__device__ __forceinline__ void best_step(int32_t& k, uint32_t& i) {
    best_merge(k, i, dpp_i<CTRL>(k), (uint32_t)dpp_i<CTRL>((int32_t)i));
}
// Wave-wide best; result valid in every lane (all lanes active).
__device__ __forceinline__ void wave_best(int32_t& k, uint32_t& i) {
    best_step<kDppXor1>(k, i);
    best_step<kDppXor2>(k, i);
    best_step<kDppHalfMirror>(k, i);
    best_step<kDppMirror>(k, i);
    int32_t bk = __builtin_amdgcn_readlane(k, 0);
    uint32_t bi = (uint32_t)__builtin_amdgcn_readlane((int32_t)i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        best_merge(bk, bi, __builtin_amdgcn_readlane(k, r), (uint32_t)__builtin_amdgcn_readlane((int32_t)i, r));
    k = bk;
    i = bi;
}
// Block-wide best; result valid in every thread.
__device__ __forceinline__ void block_best(int32_t& k, uint32_t& i) {
    __shared__ int32_t sk[kWaves];
    __shared__ uint32_t si[kWaves];
    wave_best(k, i);
    if ((threadIdx.x & 63) == 0) {
        sk[threadIdx.x >> 6] = k;
        si[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    k = sk[0];
    i = si[0];
    for (int w = 1; w < kWaves; w++) best_merge(k, i, sk[w], si[w]);
    __syncthreads();
}

// Chunk loads of a row through a buffer resource: the row's byte offset is
// one 32-bit add per lane, the field offsets (RowGeo) go in the scalar offset.
// The loads carry the non-temporal hint (cache policy nt): every weight byte
// is read once per launch, and streams that do not allocate as reusable
// lines in the vector L1 measured 5-7 % faster on the 256 MB vocab matrix.
constexpr int kMvAux = 2;  // cache policy nt (non-temporal)
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kMvAux);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ uint2 bld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, kMvAux);
    return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kMvAux);
}

// The same bytes as Fmt<KIND>::load (qh_device.hpp), for the row at byte
// offset ro of the buffer.
template <uint32_t KIND>
__device__ __forceinline__ typename Fmt<KIND>::Raw bload(__amdgpu_buffer_rsrc_t r, uint32_t ro, const RowGeo& g,
                                                         uint32_t c) {
    const uint32_t b = c >> 3, j = c & 7;
    if constexpr (KIND == Q4_K) {
        return {bld16(r, ro + b * 128 + j * 16, g.off_b), bld16(r, ro + b * 16, g.off_a)};
    } else if constexpr (KIND == Q5_K) {
        return {bld16(r, ro + b * 128 + j * 16, g.off_c), bld16(r, ro + b * 16, g.off_a),
                bld16(r, ro + b * 32 + (j & 1) * 16, g.off_b)};
    } else if constexpr (KIND == Q6_K) {
        return {bld16(r, ro + b * 128 + j * 16, g.off_a), bld16(r, ro + b * 64 + (j >> 2) * 32 + (j & 1) * 16, g.off_b),
                bld8(r, ro + b * 16 + (j >> 2) * 8, g.off_c), bld4(r, ro + (b >> 1) * 4, g.off_d)};
    } else if constexpr (KIND == Q4_0) {
        return {bld16(r, ro + c * 16, g.off_a), bld4(r, ro + (c >> 1) * 4, g.off_b)};
    } else {
        static_assert(KIND == Q8_0, "block-quantised formats only");
        return {bld16(r, ro + c * 32, g.off_a), bld16(r, ro + c * 32 + 16, g.off_a), bld4(r, ro + (c >> 1) * 4, g.off_b)};
    }
}

// The same bytes for a wave-uniform row offset ro: ro and the field offset go
// in the scalar offset, the lane's chunk offset in the vector offset (which
// then stays the same from row to row).
template <uint32_t KIND>
__device__ __forceinline__ typename Fmt<KIND>::Raw bload_u(__amdgpu_buffer_rsrc_t r, uint32_t ro, const RowGeo& g,
                                                           uint32_t c) {
    const uint32_t b = c >> 3, j = c & 7;
    if constexpr (KIND == Q4_K) {
        return {bld16(r, b * 128 + j * 16, ro + g.off_b), bld16(r, b * 16, ro + g.off_a)};
    } else if constexpr (KIND == Q5_K) {
        return {bld16(r, b * 128 + j * 16, ro + g.off_c), bld16(r, b * 16, ro + g.off_a),
                bld16(r, b * 32 + (j & 1) * 16, ro + g.off_b)};
    } else if constexpr (KIND == Q6_K) {
        return {bld16(r, b * 128 + j * 16, ro + g.off_a), bld16(r, b * 64 + (j >> 2) * 32 + (j & 1) * 16, ro + g.off_b),
                bld8(r, b * 16 + (j >> 2) * 8, ro + g.off_c), bld4(r, (b >> 1) * 4, ro + g.off_d)};
    } else if constexpr (KIND == Q4_0) {
        return {bld16(r, c * 16, ro + g.off_a), bld4(r, (c >> 1) * 4, ro + g.off_b)};
    } else {
        static_assert(KIND == Q8_0, "block-quantised formats only");
        return {bld16(r, c * 32, ro + g.off_a), bld16(r, c * 32 + 16, ro + g.off_a), bld4(r, (c >> 1) * 4, ro + g.off_b)};
    }
}

// ------------------------------------------- cross-workgroup data exchange --
// Workgroups on different XCDs do not share an L2, so data handed from one
// workgroup to another inside a kernel is written through to memory with
// system-scope stores and read with loads that bypass the caches (sc0 sc1).
// A producer waits for its stores (s_waitcnt 0) before publishing a flag or
// counter; a consumer reads the data only after it has seen the flag.
__device__ __forceinline__ void st_sys(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys_u(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float ld_sys(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t ld_sys_u(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// 16-byte load that bypasses the caches (sc0 sc1).
__device__ __forceinline__ float4 ld_sys4(__amdgpu_buffer_rsrc_t r, uint32_t off_bytes) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off_bytes, 0, 17);
    return *reinterpret_cast<float4*>(&v);
}

}  // namespace qh
