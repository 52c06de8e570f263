// gfx950 kernels of one decode token step (src/model.rs:217-302).
//
// Per decoder layer, five kernels:
//   k_qkv     RMSNorm(x) -> q, k, v projections; on layer 0 the embedding row
//             of tokens[pos] is dequantised in every workgroup first
//             (model.rs:225-232)
//   k_attn    per-head Q/K RMSNorm + NeoX RoPE + KV append, then split-T GQA
//             attention with an online softmax; the last of a KV head's
//             chunk workgroups merges the chunks (model.rs:233-244,
//             ops.rs:57-98)
//   k_oproj   attention output projection + residual (model.rs:245-248); each
//             workgroup also emits the router dot products restricted to
//             its output rows and their sum of squares -- the router logits
//             are linear in x' up to the RMSNorm scale, so they need no
//             separate pass (model.rs:249-256)
//   k_gateup  every workgroup folds the router partials in one fixed order,
//             selects the top-k and renormalises (identically everywhere, so
//             no cross-workgroup reduction), then the gate/up projections of
//             one routed expert + SwiGLU (ops.rs:45-56, model.rs:257-274)
//   k_down    down projections, routing-weighted combine, residual
//             (model.rs:275-287)
// and per token k_vocab (final RMSNorm, vocab projection, per-workgroup
// argmax partials, model.rs:289-299) plus k_finish (argmax, next token,
// position += 1; sampling.rs:26-35).
//
// Decode is latency-bound, so every kernel issues all the global loads a
// wave needs (weights, activations, norm vectors, KV tiles) before it
// consumes any of them: a kernel costs about one or two memory round trips
// instead of one per dependent step.  Every kernel reads the position from
// device memory, so one captured graph replays for any position.
#include "qh_block.hpp"
#include "qh_tile.hpp"

namespace qh {

constexpr uint32_t kAttnTile = 32;          // keys per tile
constexpr uint32_t kAttnMinChunk = 32;      // fewest keys per attention workgroup
constexpr uint32_t kAttnMaxChunksDev = 32;  // most chunk workgroups per KV head

template <int NT>
__device__ __forceinline__ float bsum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) s += red[i];
    __syncthreads();
    return s;
}

// xs[i] = x[i] * (scale * w[i]), scale = 1/sqrt(mean(x^2) + eps)
// (ops.rs:3-15), zero-padded to npad; x and w are loaded in one batch when
// n <= 8*NT.  Ends with a barrier.
template <int NT>
__device__ __forceinline__ void rms_stage(const float* x, const float* w, uint32_t n, uint32_t npad, float eps,
                                          float* xs, float* red) {
    if (n <= 8u * NT) {
        float xv[8], wv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = threadIdx.x + k * NT;
            xv[k] = i < n ? x[i] : 0.f;
            wv[k] = i < n ? w[i] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) ss = fmaf(xv[k], xv[k], ss);
        const float scale = 1.0f / sqrtf(bsum<NT>(ss, red) / (float)n + eps);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = threadIdx.x + k * NT;
            if (i < npad) xs[i] = xv[k] * (scale * wv[k]);
        }
    } else {
        float ss = 0.f;
        for (uint32_t i = threadIdx.x; i < n; i += NT) ss = fmaf(x[i], x[i], ss);
        const float scale = 1.0f / sqrtf(bsum<NT>(ss, red) / (float)n + eps);
        for (uint32_t i = threadIdx.x; i < npad; i += NT) xs[i] = i < n ? x[i] * (scale * w[i]) : 0.f;
    }
    __syncthreads();
}

// RMSNorm of a vector held in LDS, in place (ops.rs:3-15).
template <int NT>
__device__ __forceinline__ void rms_inplace(float* xs, const float* w, uint32_t n, float eps, float* red) {
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += NT) ss = fmaf(xs[i], xs[i], ss);
    const float scale = 1.0f / sqrtf(bsum<NT>(ss, red) / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += NT) xs[i] = xs[i] * (scale * w[i]);
    __syncthreads();
}

// Copies n floats to LDS (zero-padded to npad), one load batch per thread.
template <int NT>
__device__ __forceinline__ void stage_vec(const float* x, uint32_t n, uint32_t npad, float* xs) {
    for (uint32_t base = 0; base < npad; base += 16u * NT) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const uint32_t i = base + threadIdx.x + k * NT;
            v[k] = i < n ? x[i] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const uint32_t i = base + threadIdx.x + k * NT;
            if (i < npad) xs[i] = v[k];
        }
    }
    __syncthreads();
}

// =================================================================== k_qkv ==
// Workgroups [0, nq) serve attn_q, [nq, nq+nk) attn_k, the rest attn_v, so a
// workgroup's waves share one weight format; wave w of a workgroup owns row
// group (b - first) * 4 + w of its matrix.
template <uint32_t KIND, int R, int C>
__device__ __forceinline__ void qkv_body(const LayerW& L, const DevMat& emb, const Acts& a, const ModelDims& dm,
                                         int first, const DevMat& m, float* out, uint32_t grp, float* xs,
                                         float* red) {
    constexpr int NT = kBlock;
    const uint32_t H = dm.hidden, hp = pad32(H);
    const Groups gp = groups_of(m.rows, m.cols, R);
    const uint32_t lane = threadIdx.x & 63, sub = lane / gp.L, cl = lane % gp.L;
    const uint32_t r0 = grp * gp.per + sub;
    RowTile<KIND, R, C> tile;
    tile.load([&](int k) -> const uint8_t* {
        const uint32_t r = r0 + k * gp.S;
        return grp < gp.n && r < m.rows ? m.w + (size_t)r * m.drb : nullptr;
    }, m.geo, m.cols, gp.L, cl);
    if (first) {
        const uint32_t tok = a.tokens[a.st->pos];
        const bool ok = tok < dm.vocab;
        const uint8_t* row = emb.w + (size_t)(ok ? tok : 0) * emb.drb;
        for (uint32_t i = threadIdx.x; i < hp; i += NT) xs[i] = i < H ? dequant_value(row, emb.kind, emb.geo, i) : 0.f;
        __syncthreads();
        if (!ok) {
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrToken);
            return;
        }
        for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < H; i += gridDim.x * NT) a.x[i] = xs[i];
        rms_inplace<NT>(xs, L.attn_norm, H, dm.eps, red);
    } else {
        rms_stage<NT>(a.x, L.attn_norm, H, hp, dm.eps, xs, red);
    }
    QH_MARK(0, 1);
    float acc[R];
    tile.dot(xs, m.geo, m.cols, gp.L, cl, acc);
    QH_MARK(0, 3);
#pragma unroll
    for (int k = 0; k < R; k++) acc[k] = seg_sum(acc[k], gp.L);
    QH_MARK(0, 4);
    if (cl == 0 && grp < gp.n) {
#pragma unroll
        for (int k = 0; k < R; k++) {
            const uint32_t r = r0 + k * gp.S;
            if (r < m.rows) out[r] = acc[k];
        }
    }
    QH_MARK(0, 2);
}

constexpr int kQkvRows = 2;

template <int C>
__global__ __launch_bounds__(kBlock) void k_qkv(LayerW L, DevMat emb, Acts a, ModelDims dm, int first) {
    constexpr int R = kQkvRows;
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    __shared__ float red[kWaves];
    const uint32_t nq = (groups_of(L.q.rows, L.q.cols, R).n + kWaves - 1) / kWaves;
    const uint32_t nk = (groups_of(L.k.rows, L.k.cols, R).n + kWaves - 1) / kWaves;
    QH_MARK(0, 0);
    const uint32_t b = blockIdx.x, w = threadIdx.x >> 6;
    DevMat m = L.q;
    float* out = a.q;
    uint32_t wg = b;
    if (b >= nq && b < nq + nk) {
        m = L.k;
        out = a.k;
        wg = b - nq;
    } else if (b >= nq + nk) {
        m = L.v;
        out = a.v;
        wg = b - nq - nk;
    }
    const uint32_t grp = wg * kWaves + w;
    QH_DISPATCH_TILE(C, m.kind, (qkv_body<K_, R, C>(L, emb, a, dm, first, m, out, grp, xs, red)));
}

// ================================================================== k_attn ==
// Grid (kvheads, max_chunks).  With T = pos + 1 keys, nch = min(max_chunks,
// ceil(T / 32)) workgroups per KV head cover consecutive chunks of
// ceil(T / nch) keys; the others exit.  Each workgroup normalises and
// rotates the G = heads/kvheads query heads of its KV head and the new key,
// appends the new key/value at pos (the chunk that holds pos), then runs an
// online softmax over its keys in 32-key tiles (each tile's loads issued
// before the previous tile is consumed), keeping per head the running max m,
// the running sum l of exp(s - m) and the exp-weighted V sum.  Scores are
// (q . k) / sqrt(d) (ops.rs:81-88).
struct KVRegs {
    float4 k[4], v[4];  // up to 16 floats of K and V per thread per tile
};

__device__ __forceinline__ void attn_tile_load(KVRegs& r, const float* kc, const float* vc, uint32_t g, uint32_t ctx,
                                               uint32_t d, uint32_t tt, uint32_t nt, uint32_t pos) {
    const uint32_t d4 = d / 4, n4 = nt * d4;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t i = threadIdx.x + k * kBlock;
        if (i < n4) {
            const uint32_t t = i / d4, j = (i % d4) * 4, key = tt + t;
            if (key != pos) {
                const size_t off = ((size_t)g * ctx + key) * d + j;
                r.k[k] = *reinterpret_cast<const float4*>(kc + off);
                r.v[k] = *reinterpret_cast<const float4*>(vc + off);
            }
        }
    }
}

__device__ __forceinline__ void attn_tile_store(const KVRegs& r, float* ks, float* vs, const float* kn, const float* vn,
                                                uint32_t d, uint32_t tt, uint32_t nt, uint32_t pos) {
    const uint32_t d4 = d / 4, n4 = nt * d4;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t i = threadIdx.x + k * kBlock;
        if (i < n4) {
            const uint32_t t = i / d4, j = (i % d4) * 4, key = tt + t;
            float4 kv = r.k[k], vv = r.v[k];
            if (key == pos) {
                kv = make_float4(kn[j], kn[j + 1], kn[j + 2], kn[j + 3]);
                vv = make_float4(vn[j], vn[j + 1], vn[j + 2], vn[j + 3]);
            }
            float* kd = ks + t * (d + 1) + j;
            kd[0] = kv.x;
            kd[1] = kv.y;
            kd[2] = kv.z;
            kd[3] = kv.w;
            *reinterpret_cast<float4*>(vs + t * d + j) = vv;
        }
    }
}

__global__ __launch_bounds__(kBlock) void k_attn(LayerW L, AttnArgs aa, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* sm = reinterpret_cast<float*>(smem4);
    QH_MARK(1, 0);
    const uint32_t pos = a.st->pos;
    if (pos >= dm.ctx) {
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrContext);
        return;
    }
    const uint32_t T = pos + 1, g = blockIdx.x, c = blockIdx.y;
    uint32_t nch = (T + kAttnMinChunk - 1) / kAttnMinChunk;
    nch = min(nch, min(aa.max_chunks, kAttnMaxChunksDev));
    if (c >= nch) return;
    const uint32_t tc = (T + nch - 1) / nch;
    const uint32_t t0 = min(T, c * tc), t1 = min(T, t0 + tc);
    const uint32_t G = dm.heads / dm.kvheads, d = dm.head_dim, half = d / 2, ctx = dm.ctx;
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool vec4 = (d & 3) == 0 && kAttnTile * d <= 16u * kBlock;
    float* qs = sm;                        // [G][d]  normalised, rotated queries
    float* kn = qs + G * d;                // [d]     new key
    float* vn = kn + d;                    // [d]     new value
    float* ks = vn + d;                    // [tile][d+1]
    float* vs = ks + kAttnTile * (d + 1);  // [tile][d]
    float* ps = vs + kAttnTile * d;        // [G][tile] scores, then exp weights
    float* os = ps + G * kAttnTile;        // [G][d]  running V sums
    float* mh = os + G * d;                // [G] running max
    float* lh = mh + G;                    // [G] running sum
    float* al = lh + G;                    // [G] rescale factor of the current tile

    // 0. issue the first K/V tile (history only; the new key comes later)
    KVRegs tile;
    if (vec4 && t1 > t0) attn_tile_load(tile, L.kcache, L.vcache, g, ctx, d, t0, min(kAttnTile, t1 - t0), pos);
    // 1. Q/K RMSNorm (model.rs:233-238): wave w handles vectors w, w+4, ...
    for (uint32_t vi = wv; vi <= G; vi += kWaves) {
        const bool isk = vi == G;
        const float* src = isk ? a.k + g * d : a.q + (g * G + vi) * d;
        const float* w = isk ? L.k_norm : L.q_norm;
        float* dst = isk ? kn : qs + vi * d;
        float sv[4], wv4[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t j = lane + 64 * k;
            sv[k] = j < d ? src[j] : 0.f;
            wv4[k] = j < d ? w[j] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) ss = fmaf(sv[k], sv[k], ss);
        for (uint32_t j = lane + 256; j < d; j += 64) ss = fmaf(src[j], src[j], ss);
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / (float)d + dm.eps);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t j = lane + 64 * k;
            if (j < d) dst[j] = sv[k] * (scale * wv4[k]);
        }
        for (uint32_t j = lane + 256; j < d; j += 64) dst[j] = src[j] * (scale * w[j]);
    }
    for (uint32_t j = threadIdx.x; j < d; j += kBlock) vn[j] = a.v[g * d + j];
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) os[p] = 0.f;
    for (uint32_t h = threadIdx.x; h < G; h += kBlock) {
        mh[h] = -INFINITY;
        lh[h] = 0.f;
    }
    __syncthreads();
    QH_MARK(1, 1);
    // 2. NeoX RoPE at pos (ops.rs:17-28) with the (cos, sin) table
    const float2* cs = a.rope + (size_t)pos * half;
    for (uint32_t p = threadIdx.x; p < (G + 1) * half; p += kBlock) {
#pragma clang fp contract(off)
        const uint32_t vi = p / half, i = p % half;
        float* vec = vi == G ? kn : qs + vi * d;
        const float co = cs[i].x, si = cs[i].y, x0 = vec[i], x1 = vec[i + half];
        vec[i] = x0 * co - x1 * si;
        vec[i + half] = x0 * si + x1 * co;
    }
    __syncthreads();
    QH_MARK(1, 2);
    // 3. KV append (model.rs:241-243) by the chunk that holds pos
    if (t0 <= pos && pos < t1) {
        for (uint32_t j = threadIdx.x; j < d; j += kBlock) {
            L.kcache[((size_t)g * ctx + pos) * d + j] = kn[j];
            L.vcache[((size_t)g * ctx + pos) * d + j] = vn[j];
        }
    }
    const float root = sqrtf((float)d);
    // 4. online softmax over the chunk's keys
    for (uint32_t tt = t0; tt < t1; tt += kAttnTile) {
        const uint32_t nt = min(kAttnTile, t1 - tt);
        if (vec4) {
            attn_tile_store(tile, ks, vs, kn, vn, d, tt, nt, pos);
            const uint32_t tn = tt + kAttnTile;
            if (tn < t1) attn_tile_load(tile, L.kcache, L.vcache, g, ctx, d, tn, min(kAttnTile, t1 - tn), pos);
        } else {
            for (uint32_t i = threadIdx.x; i < nt * d; i += kBlock) {
                const uint32_t t = i / d, j = i % d, key = tt + t;
                const size_t off = ((size_t)g * ctx + key) * d + j;
                ks[t * (d + 1) + j] = key == pos ? kn[j] : L.kcache[off];
                vs[t * d + j] = key == pos ? vn[j] : L.vcache[off];
            }
        }
        __syncthreads();
        for (uint32_t p = threadIdx.x; p < G * nt; p += kBlock) {
            const uint32_t h = p / nt, t = p % nt;
            const float* qh = qs + h * d;
            const float* kt = ks + t * (d + 1);
            float s = 0.f;
            for (uint32_t j = 0; j < d; j++) s = fmaf(qh[j], kt[j], s);
            ps[h * kAttnTile + t] = s / root;
        }
        __syncthreads();
        for (uint32_t h = wv; h < G; h += kWaves) {
            float mt = -INFINITY;
            for (uint32_t t = lane; t < nt; t += 64) mt = fmaxf(mt, ps[h * kAttnTile + t]);
            mt = wave_max(mt);
            const float M = fmaxf(mh[h], mt);
            float sum = 0.f;
            for (uint32_t t = lane; t < nt; t += 64) {
                const float e = expf(ps[h * kAttnTile + t] - M);
                ps[h * kAttnTile + t] = e;
                sum += e;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                const float alpha = expf(mh[h] - M);  // 0 on the first tile (mh = -inf)
                al[h] = alpha;
                lh[h] = fmaf(lh[h], alpha, sum);
                mh[h] = M;
            }
        }
        __syncthreads();
        for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
            const uint32_t h = p / d, j = p % d;
            float o = os[p] * al[h];
            const float* ph = ps + h * kAttnTile;
            for (uint32_t t = 0; t < nt; t++) o = fmaf(ph[t], vs[t * d + j], o);
            os[p] = o;
        }
        __syncthreads();
    }
    QH_MARK(1, 3);
    // 5. chunk partials; an empty chunk contributes (m = -inf, l = 0, o = 0).
    //    Layout: o[h][chunk][d] for all heads, then ml[h][chunk][2].
    const uint32_t mc = aa.max_chunks;
    float* po = aa.part;
    float* pml = aa.part + (size_t)dm.heads * mc * d;
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
        const uint32_t h = p / d, j = p % d;
        po[((size_t)(g * G + h) * mc + c) * d + j] = os[p];
    }
    for (uint32_t h = threadIdx.x; h < G; h += kBlock) {
        pml[((size_t)(g * G + h) * mc + c) * 2] = mh[h];
        pml[((size_t)(g * G + h) * mc + c) * 2 + 1] = lh[h];
    }
    // 6. the last chunk workgroup of this KV head merges the chunks: all
    //    (m, l) pairs and o rows requested in one round, then per-chunk
    //    factors exp(m_c - M) / L
    QH_MARK(1, 4);
    if (!last_arrival(&aa.counter[g], nch)) return;
    QH_MARK(1, 5);
    float* fac = ps;  // [G][nch], nch <= 32 = tile
    for (uint32_t p = threadIdx.x; p < G * nch; p += kBlock) {
        const uint32_t h = p / nch, cc = p % nch;
        const float* src = pml + ((size_t)(g * G + h) * mc + cc) * 2;
        ks[h * kAttnTile + cc] = src[0];  // m
        vs[h * kAttnTile + cc] = src[1];  // l
    }
    __syncthreads();
    for (uint32_t h = wv; h < G; h += kWaves) {
        float M = -INFINITY;
        for (uint32_t cc = lane; cc < nch; cc += 64) M = fmaxf(M, ks[h * kAttnTile + cc]);
        M = wave_max(M);
        float Ls = 0.f;
        for (uint32_t cc = lane; cc < nch; cc += 64) {
            const float e = expf(ks[h * kAttnTile + cc] - M);
            fac[h * kAttnTile + cc] = e;
            Ls = fmaf(vs[h * kAttnTile + cc], e, Ls);
        }
        Ls = wave_sum(Ls);
        for (uint32_t cc = lane; cc < nch; cc += 64) fac[h * kAttnTile + cc] /= Ls;
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < G * d; p += kBlock) {
        const uint32_t h = p / d, j = p % d;
        const float* base = po + (size_t)(g * G + h) * mc * d + j;
        float v[kAttnMaxChunksDev];
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++) v[cc] = cc < nch ? base[(size_t)cc * d] : 0.f;
        float O = 0.f;
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++) O = fmaf(v[cc], cc < nch ? fac[h * kAttnTile + cc] : 0.f, O);
        a.attn[(g * G + h) * d + j] = O;
    }
    QH_MARK(1, 6);
}

// ------------------------------------------------------------- k_attn128 --
// The same step for head_dim 128 and at most 8 query heads per KV head (the
// Qwen3-MoE shapes), built around register-held key slices:
//   * Q/K RMSNorm + RoPE per wave from registers: lane l holds elements l and
//     l + 64, which are exactly the rotated pairs;
//   * scores: thread (key t = tid/8, part p = tid%8) holds 16 dims of its key
//     and reads the matching 16 dims of every query head from LDS; the eight
//     parts of a key are reduced on the DPP crossbar;
//   * online softmax per head on one wave; P.V with thread (4 dims, head);
//   * chunk partials are published with write-through (system-scope) stores
//     and a system-scope arrival counter, so the merging workgroup reads them
//     from memory without device-wide cache flushes.
constexpr uint32_t kFD = 128;  // head_dim of this path
constexpr uint32_t kFG = 8;    // most query heads per KV head
constexpr uint32_t kFQ = 160;  // LDS stride of one query head: 8 parts of 16 dims, padded to 20
constexpr uint32_t kFP = 36;   // LDS stride of one head's score row

// K and V slices (16 dims at part*16) of key tt + tid/8 of KV head g.
__device__ __forceinline__ void kv_slice_load(float4 (&kr)[4], float4 (&vr)[4], const float* kc, const float* vc,
                                              uint32_t g, uint32_t ctx, uint32_t tt, uint32_t t1, uint32_t pos) {
    const uint32_t key = tt + (threadIdx.x >> 3), j = (threadIdx.x & 7) * 16;
    if (key < t1 && key != pos) {
        const float4* ks = reinterpret_cast<const float4*>(kc + ((size_t)g * ctx + key) * kFD + j);
        const float4* vs = reinterpret_cast<const float4*>(vc + ((size_t)g * ctx + key) * kFD + j);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = ks[i];
            vr[i] = vs[i];
        }
    }
}

__global__ __launch_bounds__(kBlock) void k_attn128(LayerW L, AttnArgs aa, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* sm = reinterpret_cast<float*>(smem4);
    float* qs = sm;                  // [kFG][kFQ]   normalised, rotated queries
    float* kn = qs + kFG * kFQ;      // [kFQ]        new key, same part layout
    float* vn = kn + kFQ;            // [kFD]        new value
    float* vs = vn + kFD;            // [kAttnTile][kFD] value tile
    float* ps = vs + kAttnTile * kFD;  // [kFG][kFP]  scores, then exp weights
    float* al = ps + kFG * kFP;      // [kFG]        rescale factor of the tile
    float* ml = al + kFG;            // [kFG][2]     final (m, l) per head
    __shared__ uint32_t last;
    QH_MARK(1, 0);
    const uint32_t pos = a.st->pos;
    if (pos >= dm.ctx) {
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrContext);
        return;
    }
    const uint32_t T = pos + 1, g = blockIdx.x, c = blockIdx.y;
    uint32_t nch = (T + kAttnMinChunk - 1) / kAttnMinChunk;
    nch = min(nch, min(aa.max_chunks, kAttnMaxChunksDev));
    if (c >= nch) return;
    const uint32_t tc = (T + nch - 1) / nch;
    const uint32_t t0 = min(T, c * tc), t1 = min(T, t0 + tc);
    const uint32_t G = dm.heads / dm.kvheads, ctx = dm.ctx;
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63, part = threadIdx.x & 7, kt = threadIdx.x >> 3;
    const bool holds = t0 <= pos && pos < t1;

    // 0. every load of the first phase: K/V slices of the first tile, the
    //    q/k vectors this wave normalises, norm weights, the RoPE row, new v
    float4 kr[4], vr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    kv_slice_load(kr, vr, L.kcache, L.vcache, g, ctx, t0, t1, pos);
    float xa[3], xb[3];
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const uint32_t vi = wv + 4 * r;
        const float* src = vi == G ? a.k + g * kFD : a.q + (g * G + vi) * kFD;
        xa[r] = vi <= G ? src[lane] : 0.f;
        xb[r] = vi <= G ? src[lane + 64] : 0.f;
    }
    const float qw0 = L.q_norm[lane], qw1 = L.q_norm[lane + 64];
    const float kw0 = L.k_norm[lane], kw1 = L.k_norm[lane + 64];
    const float2 cs = a.rope[(size_t)pos * (kFD / 2) + lane];
    float4 vnew = make_float4(0.f, 0.f, 0.f, 0.f);
    if (threadIdx.x < kFD / 4) vnew = reinterpret_cast<const float4*>(a.v + g * kFD)[threadIdx.x];

    // 1. Q/K RMSNorm (model.rs:233-238) and NeoX RoPE at pos (ops.rs:17-28)
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const uint32_t vi = wv + 4 * r;
        if (vi > G) continue;  // wave-uniform
        const float ss = wave_sum(fmaf(xb[r], xb[r], xa[r] * xa[r]));
        const float scale = 1.0f / sqrtf(ss / (float)kFD + dm.eps);
        const bool isk = vi == G;
        const float y0 = xa[r] * (scale * (isk ? kw0 : qw0));
        const float y1 = xb[r] * (scale * (isk ? kw1 : qw1));
        float r0, r1;
        {
#pragma clang fp contract(off)
            r0 = y0 * cs.x - y1 * cs.y;
            r1 = y0 * cs.y + y1 * cs.x;
        }
        float* dst = isk ? kn : qs + vi * kFQ;
        dst[(lane / 16) * 20 + lane % 16] = r0;
        dst[((lane + 64) / 16) * 20 + lane % 16] = r1;
        if (isk && holds) {  // KV append (model.rs:241-243)
            L.kcache[((size_t)g * ctx + pos) * kFD + lane] = r0;
            L.kcache[((size_t)g * ctx + pos) * kFD + lane + 64] = r1;
        }
    }
    if (threadIdx.x < kFD / 4) {
        reinterpret_cast<float4*>(vn)[threadIdx.x] = vnew;
        if (holds) reinterpret_cast<float4*>(L.vcache + ((size_t)g * ctx + pos) * kFD)[threadIdx.x] = vnew;
    }
    __syncthreads();
    QH_MARK(1, 1);

    const float root = sqrtf((float)kFD);
    float mh[2] = {-INFINITY, -INFINITY}, lh[2] = {0.f, 0.f};  // heads wv, wv + 4 (softmax waves)
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);              // head tid/32, dims 4*(tid%32)
    const uint32_t hq = threadIdx.x >> 5, j4 = threadIdx.x & 31;
    for (uint32_t tt = t0; tt < t1; tt += kAttnTile) {
        const uint32_t nt = min(kAttnTile, t1 - tt);
        // 2. scores of key kt against every query head, and the V tile
        const uint32_t key = tt + kt;
        if (key == pos) {
            const float4* k4 = reinterpret_cast<const float4*>(kn + part * 20);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = k4[i];
                vr[i] = reinterpret_cast<const float4*>(vn + part * 16)[i];
            }
        }
        float sc[kFG];
#pragma unroll
        for (uint32_t h = 0; h < kFG; h++) {
            float acc = 0.f;
            if (h < G) {
                const float4* q4 = reinterpret_cast<const float4*>(qs + h * kFQ + part * 20);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 q = q4[i];
                    acc = fmaf(q.x, kr[i].x, acc);
                    acc = fmaf(q.y, kr[i].y, acc);
                    acc = fmaf(q.z, kr[i].z, acc);
                    acc = fmaf(q.w, kr[i].w, acc);
                }
            }
            acc += dpp_f<kDppXor1>(acc);
            acc += dpp_f<kDppXor2>(acc);
            acc += dpp_f<kDppHalfMirror>(acc);
            sc[h] = acc;
        }
        if (kt < nt) {
#pragma unroll
            for (int i = 0; i < 4; i++) reinterpret_cast<float4*>(vs + kt * kFD + part * 16)[i] = vr[i];
            float mine = sc[0];
#pragma unroll
            for (uint32_t h = 1; h < kFG; h++) mine = part == h ? sc[h] : mine;
            if (part < G) ps[part * kFP + kt] = mine / root;
        }
        // next tile's slices are requested before this one is consumed
        if (tt + kAttnTile < t1) kv_slice_load(kr, vr, L.kcache, L.vcache, g, ctx, tt + kAttnTile, t1, pos);
        __syncthreads();
        // 3. online softmax, one wave per head
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t h = wv + 4 * r;
            if (h >= G) continue;  // wave-uniform
            const float sv = lane < nt ? ps[h * kFP + lane] : -INFINITY;
            const float M = fmaxf(mh[r], wave_max(sv));
            const float e = lane < nt ? expf(sv - M) : 0.f;
            const float sum = wave_sum(e);
            const float alpha = expf(mh[r] - M);  // 0 on the first tile (mh = -inf)
            lh[r] = fmaf(lh[r], alpha, sum);
            mh[r] = M;
            if (lane < nt) ps[h * kFP + lane] = e;
            if (lane == 0) al[h] = alpha;
        }
        __syncthreads();
        // 4. P.V for head hq, dims 4*j4 .. 4*j4+3
        if (hq < G) {
            const float alpha = al[hq];
            o4.x *= alpha;
            o4.y *= alpha;
            o4.z *= alpha;
            o4.w *= alpha;
            const float* ph = ps + hq * kFP;
            for (uint32_t t = 0; t < nt; t++) {
                const float p = ph[t];
                const float4 v = reinterpret_cast<const float4*>(vs + t * kFD)[j4];
                o4.x = fmaf(p, v.x, o4.x);
                o4.y = fmaf(p, v.y, o4.y);
                o4.z = fmaf(p, v.z, o4.z);
                o4.w = fmaf(p, v.w, o4.w);
            }
        }
        __syncthreads();
    }
    QH_MARK(1, 3);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t h = wv + 4 * r;
            if (h < G) {
                ml[h * 2] = mh[r];
                ml[h * 2 + 1] = lh[r];
            }
        }
    }
    __syncthreads();
    if (nch == 1) {
        if (hq < G) {
            const float inv = 1.0f / ml[hq * 2 + 1];
            float* out = a.attn + (g * G + hq) * kFD + 4 * j4;
            *reinterpret_cast<float4*>(out) = make_float4(o4.x * inv, o4.y * inv, o4.z * inv, o4.w * inv);
        }
        QH_MARK(1, 6);
        return;
    }
    // 5. chunk partials: o[h][chunk][d], then (m, l)[h][chunk], written through
    const uint32_t mc = aa.max_chunks;
    float* po = aa.part;
    float* pml = aa.part + (size_t)dm.heads * mc * kFD;
    if (hq < G) {
        float* dst = po + ((size_t)(g * G + hq) * mc + c) * kFD + 4 * j4;
        st_sys(dst, o4.x);
        st_sys(dst + 1, o4.y);
        st_sys(dst + 2, o4.z);
        st_sys(dst + 3, o4.w);
    }
    if (threadIdx.x < 2 * G) st_sys(pml + ((size_t)(g * G + threadIdx.x / 2) * mc + c) * 2 + (threadIdx.x & 1), ml[threadIdx.x]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's write-through stores have completed
    __syncthreads();
    QH_MARK(1, 4);
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&aa.counter[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        last = old == nch - 1;
        if (last) __hip_atomic_store(&aa.counter[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    if (!last) return;
    QH_MARK(1, 5);
    // 6. merge: all (m, l) and o partials of head hq requested at once, then
    //    O = sum_c o_c * exp(m_c - M) / L, L = sum_c l_c exp(m_c - M)
    if (hq < G) {
        float m[kAttnMaxChunksDev], l[kAttnMaxChunksDev];
        float4 o[kAttnMaxChunksDev];
        const float* mlh = pml + (size_t)(g * G + hq) * mc * 2;
        const __amdgpu_buffer_rsrc_t orsrc =
            __builtin_amdgcn_make_buffer_rsrc(po, (short)0, (int)((size_t)dm.heads * mc * kFD * 4), 0x00020000);
        const uint32_t obase = ((g * G + hq) * mc * kFD + 4 * j4) * 4;
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++) {
            if (cc < nch) {
                m[cc] = ld_sys(mlh + cc * 2);
                l[cc] = ld_sys(mlh + cc * 2 + 1);
                o[cc] = ld_sys4(orsrc, obase + cc * kFD * 4);
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++)
            if (cc < nch) M = fmaxf(M, m[cc]);
        float Ls = 0.f;
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++) {
            if (cc < nch) {
                m[cc] = expf(m[cc] - M);
                Ls = fmaf(l[cc], m[cc], Ls);
            }
        }
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (uint32_t cc = 0; cc < kAttnMaxChunksDev; cc++) {
            if (cc < nch) {
                const float f = m[cc] / Ls;
                O.x = fmaf(o[cc].x, f, O.x);
                O.y = fmaf(o[cc].y, f, O.y);
                O.z = fmaf(o[cc].z, f, O.z);
                O.w = fmaf(o[cc].w, f, O.w);
            }
        }
        *reinterpret_cast<float4*>(a.attn + (g * G + hq) * kFD + 4 * j4) = O;
    }
    QH_MARK(1, 6);
}

// ================================================================= k_oproj ==
// 512-thread workgroups.  Workgroup b owns output rows [b*H/nb, (b+1)*H/nb):
// x'[r] = x[r] + (W_o a)[r].  It then emits, for every expert e,
// sum_r Wr[e][r] * ffn_norm[r] * x'[r] over its rows, plus sum_r x'[r]^2, into
// rpart[b][0..E].
constexpr int kOprojThreads = 512;
constexpr int kOprojRows = 4;

template <uint32_t KIND, int C>
__device__ __forceinline__ void oproj_body(const LayerW& L, const Acts& a, const ModelDims& dm, float* xs,
                                           float* xo, float* wn) {
    constexpr int NT = kOprojThreads, R = kOprojRows, NW = NT / 64;
    const uint32_t qd = dm.heads * dm.head_dim, qp = pad32(qd), H = dm.hidden, E = dm.experts;
    const uint32_t nb = gridDim.x, b = blockIdx.x;
    const uint32_t r0 = (uint32_t)((uint64_t)b * H / nb), r1 = (uint32_t)((uint64_t)(b + 1) * H / nb), nr = r1 - r0;
    const DevMat& m = L.o;
    const Groups gp = groups_of(nr, m.cols, R);
    const uint32_t lane = threadIdx.x & 63, sub = lane / gp.L, cl = lane % gp.L, wv = threadIdx.x >> 6;
    const uint8_t* base = m.w + (size_t)r0 * m.drb;
    // weights of this wave's first group, then the activation vector
    RowTile<KIND, R, C> tile;
    uint32_t grp = wv;
    auto sel = [&](uint32_t gi) {
        return [&, gi](int k) -> const uint8_t* {
            const uint32_t r = gi * gp.per + sub + k * gp.S;
            return gi < gp.n && r < nr ? base + (size_t)r * m.drb : nullptr;
        };
    };
    QH_MARK(2, 0);
    tile.load(sel(grp), m.geo, m.cols, gp.L, cl);
    // router weights of this workgroup's rows (F32 router, E <= 128): thread
    // (e = tid/4, q = tid%4) owns rows [q*per_q, q*per_q + per_q)
    const uint32_t q = threadIdx.x & 3, per_q = (nr + 3) / 4, ew = threadIdx.x >> 2;
    const bool fast_router = L.router.kind == F32 && per_q <= 16 && E <= (uint32_t)NT / 4;
    float rw[16];
    if (fast_router) {
        const float* wr = reinterpret_cast<const float*>(L.router.w + (size_t)min(ew, E - 1) * L.router.drb) + r0 + q * per_q;
#pragma unroll
        for (uint32_t i = 0; i < 16; i++) rw[i] = ew < E && i < per_q && q * per_q + i < nr ? wr[i] : 0.f;
    }
    for (uint32_t r = threadIdx.x; r < nr; r += NT) {
        xo[r] = a.x[r0 + r];
        wn[r] = L.ffn_norm[r0 + r];
    }
    stage_vec<NT>(a.attn, qd, qp, xs);
    QH_MARK(2, 1);
    for (;;) {
        float acc[R];
        tile.dot(xs, m.geo, m.cols, gp.L, cl, acc);
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = seg_sum(acc[k], gp.L);
        if (cl == 0 && grp < gp.n) {
#pragma unroll
            for (int k = 0; k < R; k++) {
                const uint32_t r = grp * gp.per + sub + k * gp.S;
                if (r < nr) {
                    const float xn = xo[r] + acc[k];
                    a.x[r0 + r] = xn;
                    xo[r] = xn;
                }
            }
        }
        grp += NW;
        if (grp >= gp.n) break;
        tile.load(sel(grp), m.geo, m.cols, gp.L, cl);
    }
    __syncthreads();
    QH_MARK(2, 2);
    for (uint32_t r = threadIdx.x; r < nr; r += NT) wn[r] *= xo[r];
    __syncthreads();
    // router partials rpart[b][e] = sum_r Wr[e][r] * ffn_norm[r] * x'[r] over
    // this workgroup's rows, and rpart[b][E] = sum_r x'[r]^2
    if (fast_router) {
        float acc = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 16; i++) acc = fmaf(rw[i], i < per_q && q * per_q + i < nr ? wn[q * per_q + i] : 0.f, acc);
        acc += dpp_f<kDppXor1>(acc);
        acc += dpp_f<kDppXor2>(acc);
        if (q == 0 && ew < E) a.rpart[(size_t)b * (E + 1) + ew] = acc;
    } else {
        for (uint32_t e = threadIdx.x; e < E; e += NT) {
            const uint8_t* row = L.router.w + (size_t)e * L.router.drb;
            float acc = 0.f;
            for (uint32_t r = 0; r < nr; r++) acc = fmaf(dequant_value(row, L.router.kind, L.router.geo, r0 + r), wn[r], acc);
            a.rpart[(size_t)b * (E + 1) + e] = acc;
        }
    }
    if (wv == 0) {
        float v = 0.f;
        for (uint32_t r = lane; r < nr; r += 64) v = fmaf(xo[r], xo[r], v);
        v = wave_sum(v);
        if (lane == 0) a.rpart[(size_t)b * (E + 1) + E] = v;
    }
    QH_MARK(2, 3);
}

template <int C>
__global__ __launch_bounds__(kOprojThreads) void k_oproj(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    const uint32_t qd = dm.heads * dm.head_dim, qp = pad32(qd), H = dm.hidden;
    const uint32_t rmax = (H + gridDim.x - 1) / gridDim.x;
    float* xo = xs + qp;
    float* wn = xo + rmax;
    QH_DISPATCH_TILE(C, L.o.kind, (oproj_body<K_, C>(L, a, dm, xs, xo, wn)));
}

// ================================================================ k_gateup ==
// 512-thread workgroups.  Router logits: s * sum_b rpart[b][e] folded in the
// fixed order b = 0..nparts-1, s = 1/sqrt(sum_b rpart[b][E] / H + eps); top-k
// by total order with lower index on ties and a sequential softmax over the
// chosen logits (ops.rs:45-56).  Workgroup b serves routed slot b % top and
// a contiguous range of its rows: h[slot][r] = silu(gate xn) * (up xn), xn =
// x' * (s * ffn_norm), SwiGLU as (g / (1 + exp(-g))) * u (model.rs:272).
constexpr int kGateupThreads = 512;
constexpr int kGateupRows = 2;

template <uint32_t KIND, int C>
__device__ __forceinline__ void gateup_rows(const LayerW& L, const Acts& a, const ModelDims& dm, const float* xs,
                                            uint32_t slot, uint32_t e, uint32_t rlo, uint32_t rhi) {
    constexpr int NT = kGateupThreads, P = kGateupRows, NW = NT / 64;
    const uint32_t H = dm.hidden;
    const int Lw = lanes_per_row(H), S = 64 / Lw;
    const uint32_t lane = threadIdx.x & 63, sub = lane / Lw, cl = lane % Lw, wv = threadIdx.x >> 6;
    const uint8_t* gb = L.gate.w + (size_t)e * L.gate.expert_stride;
    const uint8_t* ub = L.up.w + (size_t)e * L.up.expert_stride;
    const uint32_t per = (uint32_t)(P * S), n = (rhi - rlo + per - 1) / per;
    for (uint32_t gi = wv; gi < n; gi += NW) {
        const uint32_t rb = rlo + gi * per + sub;
        RowTile<KIND, P, C> tg, tu;
        tg.load([&](int k) -> const uint8_t* {
            const uint32_t r = rb + k * S;
            return r < rhi ? gb + (size_t)r * L.gate.drb : nullptr;
        }, L.gate.geo, H, Lw, cl);
        tu.load([&](int k) -> const uint8_t* {
            const uint32_t r = rb + k * S;
            return r < rhi ? ub + (size_t)r * L.up.drb : nullptr;
        }, L.up.geo, H, Lw, cl);
        float gv[P], uv[P];
        tg.dot(xs, L.gate.geo, H, Lw, cl, gv);
        tu.dot(xs, L.up.geo, H, Lw, cl, uv);
#pragma unroll
        for (int k = 0; k < P; k++) {
            const float g = seg_sum(gv[k], Lw), u = seg_sum(uv[k], Lw);
            const uint32_t r = rb + k * S;
            if (cl == 0 && r < rhi) {
#pragma clang fp contract(off)
                a.h[slot * pad32(dm.ff) + r] = (g / (1.f + expf(-g))) * u;
            }
        }
    }
}

template <int C>
__global__ __launch_bounds__(kGateupThreads) void k_gateup(LayerW L, Acts a, ModelDims dm, uint32_t nparts) {
    constexpr int NT = kGateupThreads;
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    const uint32_t H = dm.hidden, hp = pad32(H), E = dm.experts, top = dm.top, E1 = E + 1;
    float* lg = xs + hp;                                    // [E+1]
    float* sv = lg + E1;                                    // [top]
    uint32_t* sid = reinterpret_cast<uint32_t*>(sv + top);  // [top]
    __shared__ uint32_t bad;
    __shared__ float s9, slast;  // logits of rank top and E - 1 (the gap log)
    QH_MARK(3, 0);
    if (threadIdx.x == 0) {
        bad = 0;
        s9 = -INFINITY;  // stays when every expert is routed
    }
    // 1. every load of the routing phase in one round.  Logit e (and the sum
    //    of squares, column E) is folded by the four threads (e, q): thread q
    //    sums partial rows [q*pq, q*pq + pq) in order, then the quarters are
    //    combined as (s0 + s1) + (s2 + s3).  E + 1 <= 256, nparts <= 64.
    const uint32_t q = threadIdx.x & 3, pq = (nparts + 3) / 4;
    float pv[2][16];
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const uint32_t e = it * (NT / 4) + (threadIdx.x >> 2);
#pragma unroll
        for (uint32_t k = 0; k < 16; k++) {
            const uint32_t b = q * pq + k;
            pv[it][k] = e < E1 && k < pq && b < nparts ? a.rpart[(size_t)b * E1 + e] : 0.f;
        }
    }
    float xv[8], fv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t i = threadIdx.x + k * NT;
        xv[k] = i < H ? a.x[i] : 0.f;
        fv[k] = i < H ? L.ffn_norm[i] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const uint32_t e = it * (NT / 4) + (threadIdx.x >> 2);
        float acc = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < 16; k++) acc += pv[it][k];
        acc += dpp_f<kDppXor1>(acc);
        acc += dpp_f<kDppXor2>(acc);
        if (q == 0 && e < E1) lg[e] = acc;
    }
    __syncthreads();
    QH_MARK(3, 1);
    const float s = 1.0f / sqrtf(lg[E] / (float)H + dm.eps);
    float lv = 0.f;
    if (threadIdx.x < E) lv = s * lg[threadIdx.x];
    __syncthreads();
    if (threadIdx.x < E) lg[threadIdx.x] = lv;
    __syncthreads();
    QH_MARK(3, 2);
    // 2. top-k by rank under the total order, lower index first on ties
    //    (bit-exact on these logits).  Composite key (total_key << 32 | ~i):
    //    j outranks i exactly when key_j > key_i.  Four threads share one
    //    logit's comparisons (a quarter of j each).
    __shared__ __align__(16) long long ck[256];
    const uint32_t Ep = (E + 7) & ~7u;
    if (threadIdx.x < E) {
        if (!finite_f(lv)) bad = 1;
        ck[threadIdx.x] = (long long)(((uint64_t)(uint32_t)total_key(lv) << 32) | (uint32_t)~threadIdx.x);
    } else if (threadIdx.x < Ep) {
        ck[threadIdx.x] = LLONG_MIN;
    }
    __syncthreads();
    for (uint32_t i0 = 0; i0 < E; i0 += NT / 4) {
        const uint32_t i = i0 + (threadIdx.x >> 2), J = Ep / 4, j0 = q * J;
        const long long ki = ck[min(i, Ep - 1)];
        int32_t rank = 0;
#pragma unroll 4
        for (uint32_t j = j0; j < j0 + J; j += 2) {
            const longlong2 w2 = *reinterpret_cast<const longlong2*>(ck + j);
            rank += (w2.x > ki) + (w2.y > ki);
        }
        rank += dpp_i<kDppXor1>(rank);
        rank += dpp_i<kDppXor2>(rank);
        if (q == 0 && i < E && (uint32_t)rank < top) {
            sid[rank] = i;
            sv[rank] = lg[i];
        }
        if (q == 0 && i < E && (uint32_t)rank == top) s9 = lg[i];
        if (q == 0 && i < E && (uint32_t)rank == E - 1) slast = lg[i];
    }
    __syncthreads();
    const float gap = (sv[top - 1] - s9) / fmaxf(fabsf(sv[0]), fabsf(slast));  // before the softmax rewrites sv
    if (bad) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(&a.st->err, kErrRouter);
        return;
    }
    if (threadIdx.x == 0) {
#pragma clang fp contract(off)
        float mx = -INFINITY;
        for (uint32_t i = 0; i < top; i++) mx = fmaxf(mx, sv[i]);
        float sum = 0.f;
        for (uint32_t i = 0; i < top; i++) {
            sv[i] = expf(sv[i] - mx);
            sum += sv[i];
        }
        for (uint32_t i = 0; i < top; i++) sv[i] = sv[i] / sum;
    }
    // xn = x' * (s * ffn_norm)
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t i = threadIdx.x + k * NT;
        if (i < hp) xs[i] = xv[k] * (s * fv[k]);
    }
    if (H > 8u * NT)
        for (uint32_t i = threadIdx.x + 8 * NT; i < hp; i += NT) xs[i] = i < H ? a.x[i] * (s * L.ffn_norm[i]) : 0.f;
    __syncthreads();
    QH_MARK(3, 3);
    if (blockIdx.x == 0) {
        const uint32_t pos = a.st->pos;
        for (uint32_t i = threadIdx.x; i < top; i += NT) {
            a.ids[i] = sid[i];
            a.wts[i] = sv[i];
            if (pos < dm.ctx) a.route_log[((size_t)pos * dm.layers + L.index) * top + i] = sid[i];
        }
        if (threadIdx.x == 0 && pos < dm.ctx) a.gap_log[(size_t)pos * dm.layers + L.index] = gap;
        if (threadIdx.x < E) a.logits_r[threadIdx.x] = lv;
    }
    // 3. this workgroup's rows of its routed expert
    const uint32_t slot = blockIdx.x % top, wps = max(1u, gridDim.x / top);
    const uint32_t idx = blockIdx.x / top;
    if (idx >= wps) return;
    const uint32_t rlo = (uint32_t)((uint64_t)idx * dm.ff / wps), rhi = (uint32_t)((uint64_t)(idx + 1) * dm.ff / wps);
    const uint32_t e = sid[slot];
    if constexpr (C > 0) {
        // gate and up share one block-quantised format
        QH_DISPATCH_QUANT(L.gate.kind, (gateup_rows<K_, C>(L, a, dm, xs, slot, e, rlo, rhi)));
    } else {
        // any formats: one row at a time per lane segment
        constexpr int NW = NT / 64;
        const int Lw = lanes_per_row(H), S = 64 / Lw;
        const uint32_t lane = threadIdx.x & 63, sub = lane / Lw, cl = lane % Lw;
        const uint8_t* gb = L.gate.w + (size_t)e * L.gate.expert_stride;
        const uint8_t* ub = L.up.w + (size_t)e * L.up.expert_stride;
        for (uint32_t rb = rlo + (threadIdx.x >> 6) * S; rb < rhi; rb += NW * S) {
            const uint32_t r = rb + sub;
            float gv[1] = {0.f}, uv[1] = {0.f};
            if (r < rhi) {
                QH_DISPATCH_KIND(L.gate.kind, (rows_dot<K_, 1>([&](int) { return gb + (size_t)r * L.gate.drb; }, L.gate.geo, xs, H, Lw, cl, gv)));
                QH_DISPATCH_KIND(L.up.kind, (rows_dot<K_, 1>([&](int) { return ub + (size_t)r * L.up.drb; }, L.up.geo, xs, H, Lw, cl, uv)));
            }
            const float g = seg_sum(gv[0], Lw), u = seg_sum(uv[0], Lw);
            if (cl == 0 && r < rhi) {
#pragma clang fp contract(off)
                a.h[slot * pad32(dm.ff) + r] = (g / (1.f + expf(-g))) * u;
            }
        }
    }
    QH_MARK(3, 4);
}

// ================================================================== k_down ==
// x[r] += sum_s w_s * (down_{ids[s]} h_s)[r] (model.rs:275-287).  A wave owns
// R output rows; its lanes stride over the (slot, chunk) units of all routed
// experts (up to 4 per lane, all loaded before use), so the weighted combine
// happens inside the lane reduction.
constexpr int kDownRows = 2;

template <uint32_t KIND, int R, int NU>
__device__ __forceinline__ void down_rows(const LayerW& L, const Acts& a, const ModelDims& dm, const float* hs,
                                          const float* wts, const uint32_t* ids) {
    const uint32_t fp = pad32(dm.ff), cpr = fp / 32, U = dm.top * cpr;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t ngrp = (dm.hidden + R - 1) / R;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    for (uint32_t grp = gw; grp < ngrp; grp += nw) {
        const uint32_t r0 = grp * R;
        float acc[R], xr[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
            acc[k] = 0.f;
            xr[k] = r0 + k < dm.hidden ? a.x[r0 + k] : 0.f;  // requested with the weights
        }
        for (uint32_t u0 = 0; u0 < U; u0 += NU * 64) {
            typename Fmt<KIND>::Raw raw[NU][R];
#pragma unroll
            for (int i = 0; i < NU; i++) {
                const uint32_t u = u0 + lane + 64 * i;
                if (u < U) {
                    const uint32_t s = u / cpr, c = u % cpr;
                    const uint8_t* eb = L.down.w + (size_t)ids[s] * L.down.expert_stride;
#pragma unroll
                    for (int k = 0; k < R; k++)
                        if (r0 + k < dm.hidden) raw[i][k] = load_chunk<KIND>(eb + (size_t)(r0 + k) * L.down.drb, L.down.geo, c, dm.ff);
                }
            }
#pragma unroll
            for (int i = 0; i < NU; i++) {
                const uint32_t u = u0 + lane + 64 * i;
                if (u < U) {
                    const uint32_t s = u / cpr, c = u % cpr;
                    float xa[16], xb[16], sa, sb;
                    x_runs<KIND>(hs + s * fp, c, xa, xb, sa, sb);
                    const float ws = wts[s];
#pragma unroll
                    for (int k = 0; k < R; k++)
                        if (r0 + k < dm.hidden) acc[k] = fmaf(ws, Fmt<KIND>::dot(raw[i][k], c, xa, xb, sa, sb), acc[k]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < R; k++) {
            const float v = wave_sum(acc[k]);
            if (lane == 0 && r0 + k < dm.hidden) a.x[r0 + k] = xr[k] + v;
        }
    }
}

// C > 0: block-quantised weights, 4 units per lane held at once; C = 0: any
// format, one unit at a time.
template <int C>
__global__ __launch_bounds__(kBlock) void k_down(LayerW L, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* hs = reinterpret_cast<float*>(smem4);
    const uint32_t fp = pad32(dm.ff);
    float* wts = hs + dm.top * fp;
    uint32_t* ids = reinterpret_cast<uint32_t*>(wts + dm.top);
    QH_MARK(4, 0);
    for (uint32_t i = threadIdx.x; i < dm.top; i += kBlock) {
        wts[i] = a.wts[i];
        ids[i] = a.ids[i];
    }
    stage_vec<kBlock>(a.h, dm.top * fp, dm.top * fp, hs);  // padding columns of h are zero
    QH_MARK(4, 1);
    constexpr int NU = C > 0 ? 4 : 1;
    QH_DISPATCH_TILE(C, L.down.kind, (down_rows<K_, kDownRows, NU>(L, a, dm, hs, wts, ids)));
    QH_MARK(4, 2);
}

// ================================================================= k_vocab ==
// Final RMSNorm, vocab projection, finite check, and each workgroup's
// (total-order key, index) maximum into fin_key/fin_idx[blockIdx].  Waves
// stride over row groups with the next group's loads issued before the
// current group is consumed.
template <uint32_t KIND, int R, int C>
__device__ __forceinline__ void vocab_rows(const DevMat& m, const float* xs, Acts& a, int32_t& bk, uint32_t& bi,
                                           bool& nf) {
    const Groups gp = groups_of(m.rows, m.cols, R);
    const uint32_t lane = threadIdx.x & 63, sub = lane / gp.L, cl = lane % gp.L;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6), nw = gridDim.x * kWaves;
    auto sel = [&](uint32_t gi) {
        return [&, gi](int k) -> const uint8_t* {
            const uint32_t r = gi * gp.per + sub + k * gp.S;
            return gi < gp.n && r < m.rows ? m.w + (size_t)r * m.drb : nullptr;
        };
    };
    RowTile<KIND, R, C> cur, nxt;
    cur.load(sel(gw), m.geo, m.cols, gp.L, cl);
    for (uint32_t grp = gw; grp < gp.n; grp += nw) {
        const uint32_t gn = grp + nw;
        if (gn < gp.n) nxt.load(sel(gn), m.geo, m.cols, gp.L, cl);
        float acc[R];
        cur.dot(xs, m.geo, m.cols, gp.L, cl, acc);
#pragma unroll
        for (int k = 0; k < R; k++) acc[k] = seg_sum(acc[k], gp.L);
        if (cl == 0) {
#pragma unroll
            for (int k = 0; k < R; k++) {
                const uint32_t r = grp * gp.per + sub + k * gp.S;
                if (r < m.rows) {
                    a.logits[r] = acc[k];
                    nf |= !finite_f(acc[k]);
                    best_merge(bk, bi, total_key(acc[k]), r);
                }
            }
        }
        cur = nxt;
    }
}

constexpr int kVocabRows = 2;

template <int C>
__global__ __launch_bounds__(kBlock) void k_vocab(DevMat out, const float* onorm, Acts a, ModelDims dm) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    __shared__ float red[kWaves];
    __shared__ uint32_t bad;
    QH_MARK(5, 0);
    if (threadIdx.x == 0) bad = 0;
    rms_stage<kBlock>(a.x, onorm, dm.hidden, pad32(dm.hidden), dm.eps, xs, red);
    int32_t bk = INT32_MIN;
    uint32_t bi = 0xffffffffu;
    bool nf = false;
    QH_MARK(5, 1);
    QH_DISPATCH_TILE(C, out.kind, (vocab_rows<K_, kVocabRows, C>(out, xs, a, bk, bi, nf)));
    if (nf) bad = 1;
    block_best(bk, bi);
    if (threadIdx.x == 0) {
        a.fin_key[blockIdx.x] = (uint32_t)bk;
        a.fin_idx[blockIdx.x] = bi;
        if (bad) atomicOr(&a.st->err, kErrLogits);
    }
    QH_MARK(5, 2);
}

// Greedy id over the k_vocab partials; the next token (unless the caller
// supplied it) and position += 1.
__global__ __launch_bounds__(kBlock) void k_finish(Acts a, ModelDims dm, uint32_t nparts) {
    int32_t bk = INT32_MIN;
    uint32_t bi = 0xffffffffu;
    for (uint32_t base = 0; base < nparts; base += 8 * kBlock) {
        int32_t kv[8];
        uint32_t iv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t b = base + threadIdx.x + k * kBlock;
            kv[k] = b < nparts ? (int32_t)a.fin_key[b] : INT32_MIN;
            iv[k] = b < nparts ? a.fin_idx[b] : 0xffffffffu;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) best_merge(bk, bi, kv[k], iv[k]);
    }
    block_best(bk, bi);
    if (threadIdx.x == 0) {
        const uint32_t pos = a.st->pos;
        a.st->argmax = bi;
        if (pos + 1 >= a.st->n_given && pos + 1 <= dm.ctx) a.tokens[pos + 1] = bi;
        a.st->pos = pos + 1;
    }
}

#define QH_INSTANTIATE_STEP(C)                                                    \
    template __global__ void k_qkv<C>(LayerW, DevMat, Acts, ModelDims, int);      \
    template __global__ void k_oproj<C>(LayerW, Acts, ModelDims);                 \
    template __global__ void k_gateup<C>(LayerW, Acts, ModelDims, uint32_t);      \
    template __global__ void k_vocab<C>(DevMat, const float*, Acts, ModelDims);
QH_INSTANTIATE_STEP(0)
QH_INSTANTIATE_STEP(1)
QH_INSTANTIATE_STEP(2)
template __global__ void k_down<0>(LayerW, Acts, ModelDims);
template __global__ void k_down<1>(LayerW, Acts, ModelDims);

}  // namespace qh
