// gfx950 kernels behind the engine's raw test surfaces: repack of GGUF rows
// into the device layout, bit-exact dequantisation, single matvecs
// (Backend::matvec, src/backend.rs:29-52), router top-k (src/ops.rs:45-56),
// greedy argmax (src/sampling.rs:26-35) and GQA attention
// (src/ops.rs:57-98).  The token-step kernels live in step.hip.
#include "qh_block.hpp"

namespace qh {

// ============================================================ API kernels ==

// GGUF block rows -> device row layout (one thread per source byte).
__global__ __launch_bounds__(kBlock) void k_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                   uint32_t kind, uint32_t cols, size_t rows,
                                                   size_t src_rb, size_t dst_rb) {
    uint32_t blk_el, blk_bytes;
    layout(kind, blk_el, blk_bytes);
    const RowGeo g = row_geo(kind, cols);
    const size_t total = rows * src_rb;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (size_t)gridDim.x * kBlock) {
        size_t r = i / src_rb, o = i % src_rb;
        uint32_t b = (uint32_t)(o / blk_bytes), j = (uint32_t)(o % blk_bytes);
        dst[r * dst_rb + dev_offset(kind, g, b, j)] = src[i];
    }
}

// p[i] = v for i < n: clears device memory inside a stream (or a captured
// graph) without a memset node.
__global__ __launch_bounds__(kBlock) void k_fill_u32(uint32_t* __restrict__ p, size_t n, uint32_t v) {
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (size_t)gridDim.x * kBlock) p[i] = v;
}

// Bit-exact dequantisation of rows [0, rows) (src/quant.rs:81-84).
__global__ __launch_bounds__(kBlock) void k_dequant(DevMat m, size_t row0, size_t rows, float* __restrict__ out) {
    const size_t total = rows * m.cols;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (size_t)gridDim.x * kBlock) {
        size_t r = i / m.cols;
        uint32_t c = (uint32_t)(i % m.cols);
        out[i] = dequant_value(m.w + (row0 + r) * m.drb, m.kind, m.geo, c);
    }
}

// Router fold of one layer: F[e][k] = sum_j (router[e][j] ffn_norm[j]) wo[j][k]
// for 8 experts e0..e0+7 per workgroup and one column k per thread, f64
// accumulation of exact f64 products, rounded once to f32.  wo is the
// dequantised attn_output ([rows][cols] f32).
__global__ __launch_bounds__(kBlock) void k_router_fold(DevMat router, const float* __restrict__ norm,
                                                        const float* __restrict__ wo, uint32_t rows, uint32_t cols,
                                                        uint32_t experts, float* __restrict__ out) {
    const uint32_t k = blockIdx.x * kBlock + threadIdx.x, e0 = blockIdx.y * 8;
    if (k >= cols) return;
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t j = 0; j < rows; j++) {
        const double w = (double)wo[(size_t)j * cols + k], g = (double)norm[j];
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            if (e0 + i < experts) {
                const float r = reinterpret_cast<const float*>(router.w + (size_t)(e0 + i) * router.drb)[j];
                acc[i] = fma((double)r * g, w, acc[i]);
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 8; i++)
        if (e0 + i < experts) out[(size_t)(e0 + i) * cols + k] = (float)acc[i];
}

// y = W x for one matrix (Backend::matvec, src/backend.rs:29-52).  x is
// staged in LDS (x_global = false) or read from a zero-padded global copy.
template <int R>
__global__ __launch_bounds__(kBlock) void k_matvec(DevMat m, const float* __restrict__ x,
                                                   float* __restrict__ y, int x_in_lds) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    const float* xp = x;
    if (x_in_lds) {
        stage_lds(x, m.cols, pad32(m.cols), xs);
        xp = xs;
    }
    mv_all<R>(m, m.w, xp, [&](uint32_t r, float v) { y[r] = v; });
}
template __global__ void k_matvec<1>(DevMat, const float*, float*, int);
template __global__ void k_matvec<2>(DevMat, const float*, float*, int);
template __global__ void k_matvec<4>(DevMat, const float*, float*, int);
template __global__ void k_matvec<8>(DevMat, const float*, float*, int);

__global__ __launch_bounds__(kBlock) void k_route(const float* logits, uint32_t n, uint32_t top,
                                                  uint32_t* ids, float* w, uint32_t* err) {
    extern __shared__ float4 smem4[];
    route_block(logits, n, top, ids, w, err, reinterpret_cast<float*>(smem4));
}

// Greedy argmax (src/sampling.rs:26-35) over n logits: per-block partials,
// the last block reduces them.
__global__ __launch_bounds__(kBlock) void k_argmax(const float* logits, uint32_t n, int32_t* pkey,
                                                   uint32_t* pidx, uint32_t* counter, uint32_t* out,
                                                   uint32_t* err) {
    int32_t k = INT32_MIN;
    uint32_t idx = 0xffffffffu;
    bool bad = false;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
        float v = logits[i];
        bad |= !finite_f(v);
        best_merge(k, idx, total_key(v), i);
    }
    if (bad) atomicOr(err, kErrLogits);
    block_best(k, idx);
    if (threadIdx.x == 0) {
        pkey[blockIdx.x] = k;
        pidx[blockIdx.x] = idx;
    }
    if (!last_arrival(counter, gridDim.x)) return;
    k = INT32_MIN;
    idx = 0xffffffffu;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += kBlock) best_merge(k, idx, pkey[b], pidx[b]);
    block_best(k, idx);
    if (threadIdx.x == 0) *out = idx;
}

// ================================================================ attention ==
// GQA causal attention for one query vector over T cached positions
// (src/ops.rs:57-98).  Grid (kvheads, chunks); chunk c covers keys
// [c*span, min(T, (c+1)*span)), taken in tiles of tc keys with an online
// softmax (running max m, running sum l, exp-weighted V sum rescaled by
// exp(m_old - m_new) per tile), so the chunk count, and with it the partial
// buffer, stays bounded for any T.  Element j of head g at time t lives at
// K[g*sh + t*st + j].  Each block computes, for the G = heads/kvheads query
// heads of its KV head, the chunk's (m, l, o); the last block of each KV
// head merges the chunks.  Scores are (q . k) / sqrt(d), as the reference
// divides (ops.rs:87).

__device__ __forceinline__ void attention_block(const AttnArgs& a, uint32_t T) {
    extern __shared__ float4 smem4[];
    float* sm = reinterpret_cast<float*>(smem4);
    const uint32_t g = blockIdx.x, ch = blockIdx.y;
    const uint32_t span = a.span, nch = (T + span - 1) / span;
    if (nch > a.max_chunks || nch > gridDim.y) {  // never index past the partial buffer
        if (a.err && g == 0 && ch == 0 && threadIdx.x == 0) atomicOr(a.err, kErrContext);
        return;
    }
    if (ch >= nch) return;
    const uint32_t G = a.heads / a.kvheads, d = a.d, tc = a.tc;
    const uint32_t k0 = ch * span, k1 = min(T, k0 + span);
    float* qs = sm;                    // [G][d]
    float* ks = qs + G * d;            // [tc][d+1]
    float* vs = ks + tc * (d + 1);     // [tc][d]
    float* ps = vs + tc * d;           // [G][tc]
    float* ml = ps + G * tc;           // [G][2]  running max and sum
    float* al = ml + 2 * G;            // [G]     rescale factor of the current tile
    float* os = al + G;                // [G][d]  running exp-weighted V sum
    for (uint32_t i = threadIdx.x; i < G * d; i += kBlock) {
        qs[i] = a.q[(g * G) * d + i];
        os[i] = 0.f;
    }
    for (uint32_t h = threadIdx.x; h < G; h += kBlock) {
        ml[2 * h] = -INFINITY;
        ml[2 * h + 1] = 0.f;
    }
    const float root = sqrtf((float)d);
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (uint32_t t0 = k0; t0 < k1; t0 += tc) {
        const uint32_t n = min(k1, t0 + tc) - t0;
        __syncthreads();  // the previous tile's readers are done
        for (uint32_t i = threadIdx.x; i < n * d; i += kBlock) {
            uint32_t t = i / d, j = i % d;
            size_t off = (size_t)g * a.sh + (size_t)(t0 + t) * a.st + j;
            ks[t * (d + 1) + j] = a.k[off];
            vs[t * d + j] = a.v[off];
        }
        __syncthreads();
        for (uint32_t p = threadIdx.x; p < G * n; p += kBlock) {
            uint32_t h = p / n, t = p % n;
            const float* qh = qs + h * d;
            const float* kt = ks + t * (d + 1);
            float s = 0.f;
            for (uint32_t j = 0; j < d; j++) s = fmaf(qh[j], kt[j], s);
            ps[h * tc + t] = s / root;
        }
        __syncthreads();
        for (uint32_t h = wv; h < G; h += kWaves) {
            float mt = -INFINITY;
            for (uint32_t t = lane; t < n; t += 64) mt = fmaxf(mt, ps[h * tc + t]);
            const float mo = ml[2 * h], M = fmaxf(mo, wave_max(mt));
            float l = 0.f;
            for (uint32_t t = lane; t < n; t += 64) {
                float e = expf(ps[h * tc + t] - M);
                ps[h * tc + t] = e;
                l += e;
            }
            l = wave_sum(l);
            const float alpha = expf(mo - M);  // 0 on the first tile
            if (lane == 0) {
                ml[2 * h] = M;
                ml[2 * h + 1] = fmaf(ml[2 * h + 1], alpha, l);
                al[h] = alpha;
            }
        }
        __syncthreads();
        for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
            uint32_t h = p / d, j = p % d;
            float o = os[p] * al[h];
            for (uint32_t t = 0; t < n; t++) o = fmaf(ps[h * tc + t], vs[t * d + j], o);
            os[p] = o;
        }
    }
    // each thread writes the os entries it owns; ml was written before the
    // last barrier
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
        uint32_t h = p / d, j = p % d;
        float* dst = a.part + ((size_t)(g * G + h) * a.max_chunks + ch) * (d + 2);
        dst[2 + j] = os[p];
        if (j == 0) {
            dst[0] = ml[2 * h];
            dst[1] = ml[2 * h + 1];
        }
    }
    if (!last_arrival(&a.counter[g], nch)) return;
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
        uint32_t h = p / d, j = p % d;
        const float* base = a.part + (size_t)(g * G + h) * a.max_chunks * (d + 2);
        float M = -INFINITY;
        for (uint32_t c = 0; c < nch; c++) M = fmaxf(M, base[c * (d + 2)]);
        float L = 0.f, O = 0.f;
        for (uint32_t c = 0; c < nch; c++) {
            const float* pc = base + c * (d + 2);
            float e = expf(pc[0] - M);
            L = fmaf(pc[1], e, L);
            O = fmaf(pc[2 + j], e, O);
        }
        a.out[(g * G + h) * d + j] = O / L;
    }
}

__global__ __launch_bounds__(kBlock) void k_attention_api(AttnArgs a, uint32_t T) { attention_block(a, T); }

}  // namespace qh
