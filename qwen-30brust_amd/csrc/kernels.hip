// gfx950 kernels of the decode engine.
//
// Layout of one token step (src/model.rs:217-302), per layer:
//   k_rms_qkv          RMSNorm(x) -> q, k, v matvecs                 (model.rs:229-232)
//   k_qk_norm_rope     per-head Q/K RMSNorm, NeoX RoPE, KV append    (model.rs:233-243)
//   k_attention        split-T GQA attention, last-block combine     (model.rs:244, ops.rs:57-98)
//   k_oproj            attn_output matvec + residual add             (model.rs:245-248)
//   k_router           RMSNorm(x), router matvec, top-k + softmax    (model.rs:249-257, ops.rs:45-56)
//   k_gateup           gate/up matvecs of the routed experts + SwiGLU (model.rs:259-274)
//   k_down             down matvecs, weighted combine, residual      (model.rs:275-287)
// and around the layers k_embed (model.rs:225) and k_final (final RMSNorm,
// vocab projection, finite check, greedy argmax, position += 1;
// model.rs:289-300 and sampling.rs:26-35).
//
// Every kernel reads the position from device memory, so one captured graph
// serves every step.  Cross-workgroup reductions (attention combine, router
// top-k, vocab argmax) use the "last workgroup to arrive" pattern: release
// fence, atomic counter, acquire fence, and the last arrival resets the
// counter, so no host-side clearing is needed between steps.
#include "kernels.hpp"
#include "qh_rows.hpp"

namespace qh {

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
__device__ void rms_to_lds(const float* x, const float* w, uint32_t n, uint32_t npad, float eps,
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

__device__ void stage_lds(const float* x, uint32_t n, uint32_t npad, float* xs) {
    for (uint32_t i = threadIdx.x; i < npad; i += kBlock) xs[i] = i < n ? x[i] : 0.f;
    __syncthreads();
}

__device__ __forceinline__ uint32_t pad32(uint32_t n) { return (n + 31) / 32 * 32; }

// True for exactly one workgroup: the last one of `expected` to arrive.
// Performs release before and acquire after the counter update.
__device__ bool last_arrival(uint32_t* counter, uint32_t expected) {
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
__device__ void mv_all(const DevMat& m, const uint8_t* base, const float* xs, Epi epi) {
    const Groups gp = groups_of(m.rows, m.cols, R);
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    QH_DISPATCH_KIND(m.kind, {
        for (uint32_t grp = gw; grp < gp.n; grp += nw) mv_group<K_, R>(m, base, gp, grp, xs, epi);
    });
}

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

// Bit-exact dequantisation of rows [0, rows) (src/quant.rs:81-84).
__global__ __launch_bounds__(kBlock) void k_dequant(DevMat m, size_t row0, size_t rows, float* __restrict__ out) {
    const size_t total = rows * m.cols;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (size_t)gridDim.x * kBlock) {
        size_t r = i / m.cols;
        uint32_t c = (uint32_t)(i % m.cols);
        out[i] = dequant_value(m.w + (row0 + r) * m.drb, m.kind, m.geo, c);
    }
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

// Router top-k (src/ops.rs:45-56) inside one workgroup: rank every logit by
// total order with index tie-break, keep ranks < top, then a sequential
// softmax over the chosen logits in rank order.  Non-finite input sets
// kErrRouter and leaves ids/w untouched.
__device__ void route_block(const float* logits, uint32_t n, uint32_t top, uint32_t* ids, float* w,
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

__global__ __launch_bounds__(kBlock) void k_route(const float* logits, uint32_t n, uint32_t top,
                                                  uint32_t* ids, float* w, uint32_t* err) {
    extern __shared__ float4 smem4[];
    route_block(logits, n, top, ids, w, err, reinterpret_cast<float*>(smem4));
}

// (key, index) merge for argmax under total order, lowest index on ties.
__device__ __forceinline__ void best_merge(int32_t& k, uint32_t& i, int32_t k2, uint32_t i2) {
    if (k2 > k || (k2 == k && i2 < i)) {
        k = k2;
        i = i2;
    }
}
__device__ __forceinline__ void wave_best(int32_t& k, uint32_t& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        int32_t k2 = __shfl_xor(k, o, 64);
        uint32_t i2 = __shfl_xor(i, o, 64);
        best_merge(k, i, k2, i2);
    }
}
// Block-wide best; result valid in every thread.
__device__ void block_best(int32_t& k, uint32_t& i) {
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
// [c*tc, min(T, (c+1)*tc)).  Element j of head g at time t lives at
// K[g*sh + t*st + j].  Each block computes, for the G = heads/kvheads query
// heads of its KV head, the chunk's max score m, sum of exp(s - m) and the
// exp-weighted V sum; the last block of each KV head merges the chunks.
// Scores are (q . k) / sqrt(d), as the reference divides (ops.rs:87).

__device__ void attention_block(const AttnArgs& a, uint32_t T) {
    extern __shared__ float4 smem4[];
    float* sm = reinterpret_cast<float*>(smem4);
    const uint32_t g = blockIdx.x, ch = blockIdx.y;
    const uint32_t nch = (T + a.tc - 1) / a.tc;
    if (nch > a.max_chunks || nch > gridDim.y) {  // never index past the partial buffer
        if (a.err && g == 0 && ch == 0 && threadIdx.x == 0) atomicOr(a.err, kErrContext);
        return;
    }
    if (ch >= nch) return;
    const uint32_t G = a.heads / a.kvheads, d = a.d, tc = a.tc;
    const uint32_t t0 = ch * tc, n = min(T, t0 + tc) - t0;
    float* qs = sm;                    // [G][d]
    float* ks = qs + G * d;            // [tc][d+1]
    float* vs = ks + tc * (d + 1);     // [tc][d]
    float* ps = vs + tc * d;           // [G][tc]
    float* ml = ps + G * tc;           // [G][2]
    for (uint32_t i = threadIdx.x; i < G * d; i += kBlock) qs[i] = a.q[(g * G) * d + i];
    for (uint32_t i = threadIdx.x; i < n * d; i += kBlock) {
        uint32_t t = i / d, j = i % d;
        size_t off = (size_t)g * a.sh + (size_t)(t0 + t) * a.st + j;
        ks[t * (d + 1) + j] = a.k[off];
        vs[t * d + j] = a.v[off];
    }
    __syncthreads();
    const float root = sqrtf((float)d);
    for (uint32_t p = threadIdx.x; p < G * n; p += kBlock) {
        uint32_t h = p / n, t = p % n;
        const float* qh = qs + h * d;
        const float* kt = ks + t * (d + 1);
        float s = 0.f;
        for (uint32_t j = 0; j < d; j++) s = fmaf(qh[j], kt[j], s);
        ps[h * tc + t] = s / root;
    }
    __syncthreads();
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (uint32_t h = wv; h < G; h += kWaves) {
        float m = -INFINITY;
        for (uint32_t t = lane; t < n; t += 64) m = fmaxf(m, ps[h * tc + t]);
        m = wave_max(m);
        float l = 0.f;
        for (uint32_t t = lane; t < n; t += 64) {
            float e = expf(ps[h * tc + t] - m);
            ps[h * tc + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            ml[2 * h] = m;
            ml[2 * h + 1] = l;
        }
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
        uint32_t h = p / d, j = p % d;
        float o = 0.f;
        for (uint32_t t = 0; t < n; t++) o = fmaf(ps[h * tc + t], vs[t * d + j], o);
        float* dst = a.part + ((size_t)(g * G + h) * a.max_chunks + ch) * (d + 2);
        dst[2 + j] = o;
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

// ============================================================ layer kernels ==

// x = token_embd row of tokens[pos] (src/model.rs:225 via gguf.rs:204-213).
__global__ __launch_bounds__(kBlock) void k_embed(DevMat emb, Acts a, ModelDims dm) {
    const uint32_t pos = a.st->pos;
    const uint32_t tok = a.tokens[pos];
    if (tok >= dm.vocab) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrToken);
        return;
    }
    for (uint32_t c = blockIdx.x * kBlock + threadIdx.x; c < dm.hidden; c += gridDim.x * kBlock)
        a.x[c] = dequant_value(emb.w + (size_t)tok * emb.drb, emb.kind, emb.geo, c);
}

// xn = RMSNorm(x) in LDS, then the q, k and v matvecs (model.rs:229-232).
template <int R>
__global__ __launch_bounds__(kBlock) void k_rms_qkv(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    __shared__ float red[kWaves];
    rms_to_lds(a.x, L.attn_norm, dm.hidden, pad32(dm.hidden), dm.eps, xs, red);
    const Groups gq = groups_of(L.q.rows, L.q.cols, R), gk = groups_of(L.k.rows, L.k.cols, R),
                 gv = groups_of(L.v.rows, L.v.cols, R);
    const uint32_t total = gq.n + gk.n + gv.n;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    for (uint32_t grp = gw; grp < total; grp += nw) {
        if (grp < gq.n) {
            QH_DISPATCH_KIND(L.q.kind, mv_group<K_, R>(L.q, L.q.w, gq, grp, xs, [&](uint32_t r, float v) { a.q[r] = v; }));
        } else if (grp < gq.n + gk.n) {
            QH_DISPATCH_KIND(L.k.kind, mv_group<K_, R>(L.k, L.k.w, gk, grp - gq.n, xs, [&](uint32_t r, float v) { a.k[r] = v; }));
        } else {
            QH_DISPATCH_KIND(L.v.kind, mv_group<K_, R>(L.v, L.v.w, gv, grp - gq.n - gk.n, xs, [&](uint32_t r, float v) { a.v[r] = v; }));
        }
    }
}

// Per-head RMSNorm of q and k, NeoX RoPE at pos, KV append
// (model.rs:233-243, ops.rs:17-28).  One block per head: blocks [0, heads)
// are q heads, [heads, heads+kvheads) k heads, then kvheads v heads.  The
// (cos, sin) table holds the reference's angle pos * theta^(-2i/d).
__global__ __launch_bounds__(kBlock) void k_qk_norm_rope(LayerW L, Acts a, ModelDims dm) {
    __shared__ float red[kWaves];
    __shared__ float y[512];
    const uint32_t pos = a.st->pos;
    const uint32_t d = dm.head_dim, b = blockIdx.x;
    if (pos >= dm.ctx) {
        if (b == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrContext);
        return;
    }
    if (b >= dm.heads + dm.kvheads) {  // v head: append only
        const uint32_t h = b - dm.heads - dm.kvheads;
        for (uint32_t j = threadIdx.x; j < d; j += kBlock)
            L.vcache[((size_t)h * dm.ctx + pos) * d + j] = a.v[h * d + j];
        return;
    }
    const bool isq = b < dm.heads;
    const uint32_t h = isq ? b : b - dm.heads;
    float* vec = isq ? a.q + h * d : a.k + h * d;
    const float* w = isq ? L.q_norm : L.k_norm;
    float ss = 0.f;
    for (uint32_t j = threadIdx.x; j < d; j += kBlock) {
        float v = vec[j];
        ss = fmaf(v, v, ss);
    }
    const float tot = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(tot / (float)d + dm.eps);
    for (uint32_t j = threadIdx.x; j < d; j += kBlock) y[j] = vec[j] * (scale * w[j]);
    __syncthreads();
    const uint32_t half = d / 2;
    const float2* cs = a.rope + (size_t)pos * half;
    for (uint32_t i = threadIdx.x; i < half; i += kBlock) {
#pragma clang fp contract(off)
        const float c = cs[i].x, s = cs[i].y, p = y[i], q = y[i + half];
        const float r0 = p * c - q * s, r1 = p * s + q * c;
        vec[i] = r0;
        vec[i + half] = r1;
        if (!isq) {
            L.kcache[((size_t)h * dm.ctx + pos) * d + i] = r0;
            L.kcache[((size_t)h * dm.ctx + pos) * d + i + half] = r1;
        }
    }
}

// Attention of the current query over positions [0, pos] of this layer.
__global__ __launch_bounds__(kBlock) void k_attention(AttnArgs aa, Acts a, ModelDims dm) {
    const uint32_t pos = a.st->pos;
    if (pos >= dm.ctx) return;
    attention_block(aa, pos + 1);
}

// x += W_o attn (model.rs:245-248).
template <int R>
__global__ __launch_bounds__(kBlock) void k_oproj(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    stage_lds(a.attn, L.o.cols, pad32(L.o.cols), xs);
    mv_all<R>(L.o, L.o.w, xs, [&](uint32_t r, float v) { a.x[r] += v; });
}

// xn = RMSNorm(x) (also written out for the expert kernels), router logits,
// then top-k + softmax by the last block (model.rs:249-257).
template <int R>
__global__ __launch_bounds__(kBlock) void k_router(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    __shared__ float red[kWaves];
    const uint32_t hp = pad32(dm.hidden);
    rms_to_lds(a.x, L.ffn_norm, dm.hidden, hp, dm.eps, xs, red);
    if (blockIdx.x == 0)
        for (uint32_t i = threadIdx.x; i < hp; i += kBlock) a.xn[i] = xs[i];
    mv_all<R>(L.router, L.router.w, xs, [&](uint32_t r, float v) { a.logits_r[r] = v; });
    if (!last_arrival(&a.st->cnt_router, gridDim.x)) return;
    route_block(a.logits_r, dm.experts, dm.top, a.ids, a.wts, &a.st->err, xs + hp);
}

// h[s] = silu(gate_e xn) * (up_e xn) for the routed experts e = ids[s]
// (model.rs:259-274): SwiGLU as (g / (1 + exp(-g))) * u.
template <int P>
__global__ __launch_bounds__(kBlock) void k_gateup(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    stage_lds(a.xn, dm.hidden, pad32(dm.hidden), xs);
    const int Lw = lanes_per_row(dm.hidden), S = 64 / Lw;
    const uint32_t per = (uint32_t)(P * S), gps = (dm.ff + per - 1) / per, total = gps * dm.top;
    const uint32_t lane = threadIdx.x & 63, sub = lane / Lw, cl = lane % Lw;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    for (uint32_t grp = gw; grp < total; grp += nw) {
        const uint32_t s = grp / gps, rb = (grp % gps) * per + sub;
        const uint32_t e = a.ids[s];
        const uint8_t* gb = L.gate.w + (size_t)e * L.gate.expert_stride;
        const uint8_t* ub = L.up.w + (size_t)e * L.up.expert_stride;
        float g[P], u[P];
        QH_DISPATCH_KIND(L.gate.kind, rows_dot<K_, P>([&](int k) -> const uint8_t* {
            uint32_t r = rb + k * S;
            return r < dm.ff ? gb + (size_t)r * L.gate.drb : nullptr;
        }, L.gate.geo, xs, dm.hidden, Lw, cl, g));
        QH_DISPATCH_KIND(L.up.kind, rows_dot<K_, P>([&](int k) -> const uint8_t* {
            uint32_t r = rb + k * S;
            return r < dm.ff ? ub + (size_t)r * L.up.drb : nullptr;
        }, L.up.geo, xs, dm.hidden, Lw, cl, u));
#pragma unroll
        for (int k = 0; k < P; k++) {
            float gv = seg_sum(g[k], Lw), uv = seg_sum(u[k], Lw);
            uint32_t r = rb + k * S;
            if (cl == 0 && r < dm.ff) {
#pragma clang fp contract(off)
                a.h[s * pad32(dm.ff) + r] = (gv / (1.f + expf(-gv))) * uv;
            }
        }
    }
}

// x[r] += sum_s w_s * (down_{ids[s]} h_s)[r] (model.rs:275-287).  A wave owns
// R output rows; its lanes stride over the (slot, chunk) units of all routed
// experts, so the weighted combine happens inside the lane reduction.
template <uint32_t KIND, int R>
__device__ void down_rows(const LayerW& L, const Acts& a, const ModelDims& dm, const float* hs,
                          const float* wts, const uint32_t* ids) {
    const uint32_t fp = pad32(dm.ff), cpr = fp / 32, U = dm.top * cpr;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t ngrp = (dm.hidden + R - 1) / R;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    for (uint32_t grp = gw; grp < ngrp; grp += nw) {
        const uint32_t r0 = grp * R;
        float acc[R];
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = 0.f;
        for (uint32_t u = lane; u < U; u += 64) {
            const uint32_t s = u / cpr, c = u % cpr;
            const uint8_t* eb = L.down.w + (size_t)ids[s] * L.down.expert_stride;
            typename Fmt<KIND>::Raw raw[R];
#pragma unroll
            for (int k = 0; k < R; k++)
                if (r0 + k < dm.hidden) raw[k] = load_chunk<KIND>(eb + (size_t)(r0 + k) * L.down.drb, L.down.geo, c, dm.ff);
            float xa[16], xb[16], sa, sb;
            x_runs<KIND>(hs + s * fp, c, xa, xb, sa, sb);
            const float ws = wts[s];
#pragma unroll
            for (int k = 0; k < R; k++)
                if (r0 + k < dm.hidden) acc[k] = fmaf(ws, Fmt<KIND>::dot(raw[k], c, xa, xb, sa, sb), acc[k]);
        }
#pragma unroll
        for (int k = 0; k < R; k++) {
            float v = wave_sum(acc[k]);
            if (lane == 0 && r0 + k < dm.hidden) a.x[r0 + k] += v;
        }
    }
}

template <int R>
__global__ __launch_bounds__(kBlock) void k_down(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* hs = reinterpret_cast<float*>(smem4);
    const uint32_t fp = pad32(dm.ff);
    float* wts = hs + dm.top * fp;
    uint32_t* ids = reinterpret_cast<uint32_t*>(wts + dm.top);
    for (uint32_t i = threadIdx.x; i < dm.top; i += kBlock) {
        wts[i] = a.wts[i];
        ids[i] = a.ids[i];
    }
    for (uint32_t i = threadIdx.x; i < dm.top * fp; i += kBlock) {
        uint32_t s = i / fp, j = i % fp;
        hs[i] = j < dm.ff ? a.h[s * fp + j] : 0.f;
    }
    __syncthreads();
    QH_DISPATCH_KIND(L.down.kind, (down_rows<K_, R>(L, a, dm, hs, wts, ids)));
}

// Final RMSNorm, vocab projection, finite check, greedy argmax and
// position += 1 (model.rs:289-300, sampling.rs:26-35).  When the next
// position is not a caller-given token, the argmax becomes the next token.
template <int R>
__global__ __launch_bounds__(kBlock) void k_final(DevMat out, const float* onorm, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    __shared__ float red[kWaves];
    __shared__ uint32_t bad;
    if (threadIdx.x == 0) bad = 0;
    rms_to_lds(a.x, onorm, dm.hidden, pad32(dm.hidden), dm.eps, xs, red);
    int32_t bk = INT32_MIN;
    uint32_t bi = 0xffffffffu;
    bool nf = false;
    mv_all<R>(out, out.w, xs, [&](uint32_t r, float v) {
        a.logits[r] = v;
        nf |= !finite_f(v);
        best_merge(bk, bi, total_key(v), r);
    });
    if (nf) bad = 1;
    block_best(bk, bi);
    if (threadIdx.x == 0) {
        a.fin_key[blockIdx.x] = (uint32_t)bk;
        a.fin_idx[blockIdx.x] = bi;
        if (bad) atomicOr(&a.st->err, kErrLogits);
    }
    if (!last_arrival(&a.st->cnt_final, gridDim.x)) return;
    bk = INT32_MIN;
    bi = 0xffffffffu;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += kBlock) best_merge(bk, bi, (int32_t)a.fin_key[b], a.fin_idx[b]);
    block_best(bk, bi);
    if (threadIdx.x == 0) {
        const uint32_t pos = a.st->pos;
        a.st->argmax = bi;
        if (pos + 1 >= a.st->n_given && pos + 1 <= dm.ctx) a.tokens[pos + 1] = bi;
        a.st->pos = pos + 1;
    }
}

// Explicit instantiations used by the engine.
template __global__ void k_rms_qkv<2>(LayerW, Acts, ModelDims);
template __global__ void k_oproj<2>(LayerW, Acts, ModelDims);
template __global__ void k_router<1>(LayerW, Acts, ModelDims);
template __global__ void k_gateup<2>(LayerW, Acts, ModelDims);
template __global__ void k_down<2>(LayerW, Acts, ModelDims);
template __global__ void k_final<4>(DevMat, const float*, Acts, ModelDims);

}  // namespace qh
