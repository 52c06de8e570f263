// Persistent token step (src/model.rs:227-302 and the greedy sampler,
// src/sampling.rs:26-35) as ONE launch of one 512-thread workgroup per CU,
// preceded by k_embed (the embedding row of tokens[pos], model.rs:225).
//
// The workgroups run six phases per layer and hand data to each other
// through memory instead of through kernel boundaries:
//   A  RMSNorm + q/k/v projections
//   B  Q/K RMSNorm, RoPE, KV append, split-T GQA attention, chunk merge
//   C  output projection + residual for this workgroup's rows of x, and the
//      router partial dots over those rows
//   D  router fold: workgroup e folds logit e over all partial rows
//   E  top-k routing (every workgroup, identically), gate/up + SwiGLU rows
//   F  down projections + routing-weighted combine + residual, own rows
// then V: final RMSNorm, vocab projection and argmax partials, and the
// argmax / next token / position advance by workgroup 0.
//
// Synchronisation: after a phase a workgroup waits for its own
// write-through stores and publishes flags[b] = base + phase; a workgroup that
// needs phase p polls every flag until it reaches base + p.  Before it polls,
// a workgroup issues every load that does not depend on the awaited phase --
// the weights it will use next, norm vectors, the KV history, and once the
// routing is known the down-projection rows -- so their latency overlaps the
// wait.  Each wait is bounded: on timeout the workgroup raises abort_flag
// and every other wait returns, so the grid always drains.
//
// Each phase body is instantiated for the formats of the Q4_K_M mix (q, k,
// o, gate, up: Q4_K; v, down, vocab: Q4_K or Q6_K) and selected once per
// phase, so a wave's register tiles have the exact chunk size.  The host
// launches this path only for models and shapes it covers (engine.hip:
// persist_supported); everything else runs the per-phase kernels.
#include "qh_block.hpp"
#include "qh_tile.hpp"

namespace qh {

constexpr int kDT = 512;
constexpr int kDW = kDT / 64;
constexpr uint32_t kFlagStride = 32;        // flags 128 bytes apart
constexpr uint32_t kSpinLimit = 1u << 22;   // polls before a wait gives up
constexpr uint32_t kDChunks = 32;           // most attention chunk workgroups per KV head
constexpr uint32_t kDTile = 32;             // keys per attention tile
constexpr uint32_t kDSmem = 8192;           // floats of phase scratch
constexpr uint32_t kQkvPerWave = 3;         // q/k/v rows per wave
constexpr uint32_t kPairsPerWave = 3;       // gate/up row pairs per wave
constexpr uint32_t kDownUnits = 3;          // (expert, chunk) units per lane in F
constexpr uint32_t kVocabRows = 4;          // vocab rows per wave group

// Formats of the Q4_K_M mix; the host routes other models to the per-phase
// kernels.
#define QH_DISPATCH_KM(kind, K, ...)                                            \
    switch (kind) {                                                             \
    case ::qh::Q4_K: { constexpr uint32_t K = ::qh::Q4_K; __VA_ARGS__; } break; \
    default: { constexpr uint32_t K = ::qh::Q6_K; __VA_ARGS__; } break;         \
    }

struct DecodeLds {
    long long ck[256];        // composite top-k keys
    float big[kDSmem];        // phase scratch (x, attention tiles, h)
    float xo[8];              // this workgroup's rows of the residual stream
    float wn[8];              // ffn_norm of those rows
    float red[kDW];
    float lg[256];            // router logits, then [E] = RMS scale
    float sv[8];
    uint32_t sid[8];
    float ex[8];
    float wts[8];             // routing weights of the current layer
    uint32_t ids[8];          // routed experts of the current layer
    int32_t bk[kDW];
    uint32_t bi[kDW];
    uint32_t abort;
    uint32_t last;
    uint32_t bad;
};

// Per-workgroup constants of one launch.
struct Ctx {
    uint32_t b, nwg, tid, wv, lane, gw, NWV;
    uint32_t pos, T, H, E, E1, top, ff, fp, G, qd, ctx;
    uint32_t r0, nr;  // this workgroup's rows of x
};

// A copy of the launch constants whose per-lane fields are opaque to the
// optimiser: values derived from them inside a phase cannot be hoisted out of
// the layer loop, so each phase recomputes its few index expressions instead
// of every phase's indices staying live in registers for the whole kernel.
__device__ __forceinline__ Ctx fresh(const Ctx& c0) {
    Ctx c = c0;
    asm volatile("" : "+v"(c.tid));
    asm volatile("" : "+v"(c.lane));
    return c;
}

__device__ __forceinline__ float dsum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kDW; i++) s += red[i];
    __syncthreads();
    return s;
}

// Publishes "phase value done" for this workgroup.
__device__ __forceinline__ void signal(const DecodeArgs& A, uint32_t value) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's write-through stores have completed
    __syncthreads();
    if (threadIdx.x == 0) st_sys_u(A.flags + blockIdx.x * kFlagStride, value);
}

// Waits until every workgroup has published `value`; false when the step was
// aborted (a wait timed out somewhere).
__device__ __forceinline__ bool wait_all(const DecodeArgs& A, DecodeLds& S, uint32_t value) {
    if (threadIdx.x < gridDim.x) {
        const uint32_t* f = A.flags + threadIdx.x * kFlagStride;
        uint32_t spins = 0;
        while ((int32_t)(ld_sys_u(f) - value) < 0) {
            if ((++spins & 63) == 0) {
                if (ld_sys_u(A.abort_flag) != 0) {
                    S.abort = 1;
                    break;
                }
                if (spins > kSpinLimit) {
                    st_sys_u(A.abort_flag, 1u);
                    atomicOr(&A.a.st->err, kErrSync);
                    S.abort = 1;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    return S.abort == 0;
}

// x (H floats, written through) into LDS as RMSNorm(x) * w; returns this
// thread's raw float4 of x.  H <= 2048: one float4 per thread.
__device__ __forceinline__ float4 load_norm_x(const Ctx& c, const float* x, float4 w, float eps, float* xs,
                                             float* red) {
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < c.H) xv = ld_sys4(buf_rsrc(x, c.H * 4), c.tid * 16);
    const float ss = dsum(fmaf(xv.w, xv.w, fmaf(xv.z, xv.z, fmaf(xv.y, xv.y, xv.x * xv.x))), red);
    const float scale = 1.0f / sqrtf(ss / (float)c.H + eps);
    if (4 * c.tid < c.H) {
        xs[4 * c.tid] = xv.x * (scale * w.x);
        xs[4 * c.tid + 1] = xv.y * (scale * w.y);
        xs[4 * c.tid + 2] = xv.z * (scale * w.z);
        xs[4 * c.tid + 3] = xv.w * (scale * w.w);
    }
    __syncthreads();
    return xv;
}

// ================================================================== A: qkv ==
// Flat rows [q | k | v]; wave gw owns rows gw, gw + NWV, gw + 2 NWV.  q and k
// share format KQ, v has KV.  Rows have H <= 2048 columns: lane = chunk.
template <uint32_t KQ, uint32_t KV>
__device__ __forceinline__ bool phase_qkv(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          bool wait_x, uint32_t& ph) {
    const Ctx c = fresh(c0);
    const uint32_t nq = L.q.rows, nk = L.k.rows, nt = nq + nk + L.v.rows, cpr = c.H / 32;
    typename Fmt<KQ>::Raw wq[kQkvPerWave];
    typename Fmt<KV>::Raw wvv[kQkvPerWave];
#pragma unroll
    for (uint32_t k = 0; k < kQkvPerWave; k++) {
        const uint32_t r = c.gw + k * c.NWV;
        if (r < nq + nk && c.lane < cpr) {
            const DevMat& m = r < nq ? L.q : L.k;
            wq[k] = Fmt<KQ>::load(m.w + (size_t)(r < nq ? r : r - nq) * m.drb, m.geo, c.lane);
        } else if (r < nt && c.lane < cpr) {
            wvv[k] = Fmt<KV>::load(L.v.w + (size_t)(r - nq - nk) * L.v.drb, L.v.geo, c.lane);
        }
    }
    float4 nw = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < c.H) nw = reinterpret_cast<const float4*>(L.attn_norm)[c.tid];
    QH_MARK(0, 0);
    if (wait_x && !wait_all(A, S, ph)) return false;  // x of the previous layer (phase F)
    QH_MARK(0, 1);
    float* xs = S.big;
    const float4 xv = load_norm_x(c, A.a.x, nw, A.dm.eps, xs, S.red);
    // this workgroup's residual rows, kept in LDS through the layer
    if (4 * c.tid < c.H) {
        const float e4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = 4 * c.tid + i;
            if (r >= c.r0 && r < c.r0 + c.nr) S.xo[r - c.r0] = e4[i];
        }
    }
    float xa[16], xb[16], sa, sb;
    if (c.lane < cpr) x_runs<KQ>(xs, c.lane, xa, xb, sa, sb);
#pragma unroll
    for (uint32_t k = 0; k < kQkvPerWave; k++) {
        const uint32_t r = c.gw + k * c.NWV;
        if (r < nt) {  // wave-uniform
            float acc = 0.f;
            if (c.lane < cpr) {
                if (r < nq + nk) {
                    acc = Fmt<KQ>::dot(wq[k], c.lane, xa, xb, sa, sb);
                } else {
                    float ya[16], yb[16], ta, tb;
                    x_runs<KV>(xs, c.lane, ya, yb, ta, tb);
                    acc = Fmt<KV>::dot(wvv[k], c.lane, ya, yb, ta, tb);
                }
            }
            acc = wave_sum(acc);
            float* out = r < nq ? A.a.q + r : r < nq + nk ? A.a.k + (r - nq) : A.a.v + (r - nq - nk);
            if (c.lane == 0) st_sys(out, acc);
        }
    }
    QH_MARK(0, 2);
    signal(A, ++ph);
    return true;
}

// ============================================================ B: attention ==
// KV head g = b / 32, chunk b % 32 (the k_attn128 scheme, reading the q/k/v
// projections written through by phase A).
__device__ __forceinline__ void kv_slice(float4 (&kr)[4], float4 (&vr)[4], const float* kc, const float* vc,
                                         uint32_t g, uint32_t ctx, uint32_t tt, uint32_t t1, uint32_t pos) {
    const uint32_t key = tt + ((threadIdx.x & 255) >> 3), j = (threadIdx.x & 7) * 16;
    if (threadIdx.x < 256 && key < t1 && key != pos) {
        const float4* ks = reinterpret_cast<const float4*>(kc + ((size_t)g * ctx + key) * 128 + j);
        const float4* vs = reinterpret_cast<const float4*>(vc + ((size_t)g * ctx + key) * 128 + j);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = ks[i];
            vr[i] = vs[i];
        }
    }
}

__device__ __forceinline__ bool phase_attn(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                           uint32_t& ph) {
    const Ctx c = fresh(c0);
    const Acts& a = A.a;
    const ModelDims& dm = A.dm;
    const uint32_t nch = min((c.T + 31) / 32, A.max_chunks);
    const uint32_t g = c.b / kDChunks, ch = c.b % kDChunks;
    const bool active = g < dm.kvheads && ch < nch;
    if (!active) {
        signal(A, ++ph);
        return true;
    }
    const uint32_t tid = c.tid, wv = c.wv, lane = c.lane, G = c.G, pos = c.pos, ctx = c.ctx;
    const uint32_t tc = (c.T + nch - 1) / nch;
    const uint32_t t0 = min(c.T, ch * tc), t1 = min(c.T, t0 + tc);
    float4 kr[4], vr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    kv_slice(kr, vr, L.kcache, L.vcache, g, ctx, t0, t1, pos);
    const float qw0 = L.q_norm[lane], qw1 = L.q_norm[lane + 64];
    const float kw0 = L.k_norm[lane], kw1 = L.k_norm[lane + 64];
    const float2 cs = a.rope[(size_t)pos * 64 + lane];
    QH_MARK(1, 0);
    if (!wait_all(A, S, ph)) return false;  // q/k/v (phase A)
    QH_MARK(1, 1);
    float* qs = S.big;              // [8][160]  normalised, rotated queries (parts padded to 20)
    float* kn = qs + 8 * 160;       // [160]     new key, same layout
    float* vn = kn + 160;           // [128]     new value
    float* vs = vn + 128;           // [32][128] value tile
    float* ps = vs + kDTile * 128;  // [8][36]   scores, then exp weights
    float* al = ps + 8 * 36;        // [8]       rescale factor of the tile
    float* ml = al + 8;             // [8][2]    final (m, l) per head
    const bool holds = t0 <= pos && pos < t1;
    // Q/K RMSNorm (model.rs:233-238) + NeoX RoPE (ops.rs:17-28): lane l holds
    // elements l and l + 64, the rotated pair
    for (uint32_t vi = wv; vi <= G; vi += kDW) {
        const bool isk = vi == G;
        const float* src = isk ? a.k + g * 128 : a.q + (g * G + vi) * 128;
        const float xa = ld_sys(src + lane), xb = ld_sys(src + lane + 64);
        const float ssq = wave_sum(fmaf(xb, xb, xa * xa));
        const float sc = 1.0f / sqrtf(ssq / 128.0f + dm.eps);
        const float y0 = xa * (sc * (isk ? kw0 : qw0));
        const float y1 = xb * (sc * (isk ? kw1 : qw1));
        float o0, o1;
        {
#pragma clang fp contract(off)
            o0 = y0 * cs.x - y1 * cs.y;
            o1 = y0 * cs.y + y1 * cs.x;
        }
        float* dst = isk ? kn : qs + vi * 160;
        dst[(lane / 16) * 20 + lane % 16] = o0;
        dst[((lane + 64) / 16) * 20 + lane % 16] = o1;
        if (isk && holds) {  // KV append (model.rs:241-243)
            L.kcache[((size_t)g * ctx + pos) * 128 + lane] = o0;
            L.kcache[((size_t)g * ctx + pos) * 128 + lane + 64] = o1;
        }
    }
    QH_MARK(1, 4);
    if (tid < 32) {
        const float* vsrc = a.v + g * 128 + 4 * tid;
        const float4 v4 = make_float4(ld_sys(vsrc), ld_sys(vsrc + 1), ld_sys(vsrc + 2), ld_sys(vsrc + 3));
        reinterpret_cast<float4*>(vn)[tid] = v4;
        if (holds) reinterpret_cast<float4*>(L.vcache + ((size_t)g * ctx + pos) * 128)[tid] = v4;
    }
    __syncthreads();
    QH_MARK(1, 5);
    const float root = sqrtf(128.0f);
    float mh = -INFINITY, lh = 0.f;               // head wv (softmax wave)
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);  // threads < 256: head tid/32, dims 4*(tid%32)
    const uint32_t hq = tid >> 5, j4 = tid & 31, part = tid & 7, kt = (tid & 255) >> 3;
    for (uint32_t tt = t0; tt < t1; tt += kDTile) {
        const uint32_t nt = min(kDTile, t1 - tt);
        if (wv < 4) {  // threads 0..255 = (key kt, 16-dim part): scores + V tile
            if (tt + kt == pos) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    kr[i] = reinterpret_cast<const float4*>(kn + part * 20)[i];
                    vr[i] = reinterpret_cast<const float4*>(vn + part * 16)[i];
                }
            }
            float mine = 0.f;
#pragma unroll
            for (uint32_t h = 0; h < 8; h++) {
                float acc = 0.f;
                if (h < G) {
                    const float4* q4 = reinterpret_cast<const float4*>(qs + h * 160 + part * 20);
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
                mine = part == h ? acc : mine;
            }
            if (kt < nt) {
#pragma unroll
                for (int i = 0; i < 4; i++) reinterpret_cast<float4*>(vs + kt * 128 + part * 16)[i] = vr[i];
                if (part < G) ps[part * 36 + kt] = mine / root;
            }
            if (tt + kDTile < t1) kv_slice(kr, vr, L.kcache, L.vcache, g, ctx, tt + kDTile, t1, pos);
        }
        __syncthreads();
        if (wv < G) {  // online softmax: wave wv owns head wv
            const float sv = lane < nt ? ps[wv * 36 + lane] : -INFINITY;
            const float M = fmaxf(mh, wave_max(sv));
            const float e = lane < nt ? expf(sv - M) : 0.f;
            const float sum = wave_sum(e);
            const float alpha = expf(mh - M);  // 0 on the first tile
            lh = fmaf(lh, alpha, sum);
            mh = M;
            if (lane < nt) ps[wv * 36 + lane] = e;
            if (lane == 0) al[wv] = alpha;
        }
        __syncthreads();
        if (wv < 4 && hq < G) {  // P.V
            const float alpha = al[hq];
            o4.x *= alpha;
            o4.y *= alpha;
            o4.z *= alpha;
            o4.w *= alpha;
            const float* phh = ps + hq * 36;
            for (uint32_t t = 0; t < nt; t++) {
                const float p = phh[t];
                const float4 v = reinterpret_cast<const float4*>(vs + t * 128)[j4];
                o4.x = fmaf(p, v.x, o4.x);
                o4.y = fmaf(p, v.y, o4.y);
                o4.z = fmaf(p, v.z, o4.z);
                o4.w = fmaf(p, v.w, o4.w);
            }
        }
        __syncthreads();
    }
    if (lane == 0 && wv < G) {
        ml[wv * 2] = mh;
        ml[wv * 2 + 1] = lh;
    }
    __syncthreads();
    QH_MARK(1, 2);
    if (nch == 1) {
        if (wv < 4 && hq < G) {
            const float inv = 1.0f / ml[hq * 2 + 1];
            float* out = a.attn + (g * G + hq) * 128 + 4 * j4;
            st_sys(out, o4.x * inv);
            st_sys(out + 1, o4.y * inv);
            st_sys(out + 2, o4.z * inv);
            st_sys(out + 3, o4.w * inv);
        }
        signal(A, ++ph);
        return true;
    }
    // chunk partials written through; the last chunk of the head merges them
    const uint32_t mc = A.max_chunks;
    float* po = a.part;
    float* pml = a.part + (size_t)dm.heads * mc * 128;
    if (wv < 4 && hq < G) {
        float* dst = po + ((size_t)(g * G + hq) * mc + ch) * 128 + 4 * j4;
        st_sys(dst, o4.x);
        st_sys(dst + 1, o4.y);
        st_sys(dst + 2, o4.z);
        st_sys(dst + 3, o4.w);
    }
    if (tid < 2 * G) st_sys(pml + ((size_t)(g * G + tid / 2) * mc + ch) * 2 + (tid & 1), ml[tid]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.attn_cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        S.last = old == nch - 1;
        if (S.last) st_sys_u(&a.attn_cnt[g], 0u);
    }
    __syncthreads();
    if (S.last && wv < 4 && hq < G) {
        // online merge over chunk groups of 16 (all loads of a group at once):
        // O = sum_c o_c exp(m_c - M) / L, L = sum_c l_c exp(m_c - M)
        constexpr uint32_t kGrp = 16;
        const float* mlh = pml + (size_t)(g * G + hq) * mc * 2;
        const __amdgpu_buffer_rsrc_t orsrc = buf_rsrc(po, (uint32_t)((size_t)dm.heads * mc * 128 * 4));
        const uint32_t obase = ((g * G + hq) * mc * 128 + 4 * j4) * 4;
        float M = -INFINITY, Ls = 0.f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t c0 = 0; c0 < nch; c0 += kGrp) {
            float m[kGrp], l[kGrp];
            float4 o[kGrp];
#pragma unroll
            for (uint32_t k = 0; k < kGrp; k++) {
                if (c0 + k < nch) {
                    m[k] = ld_sys(mlh + (c0 + k) * 2);
                    l[k] = ld_sys(mlh + (c0 + k) * 2 + 1);
                    o[k] = ld_sys4(orsrc, obase + (c0 + k) * 128 * 4);
                }
            }
            float Mg = M;
#pragma unroll
            for (uint32_t k = 0; k < kGrp; k++)
                if (c0 + k < nch) Mg = fmaxf(Mg, m[k]);
            const float f0 = expf(M - Mg);  // 0 for the first group
            Ls *= f0;
            O.x *= f0;
            O.y *= f0;
            O.z *= f0;
            O.w *= f0;
#pragma unroll
            for (uint32_t k = 0; k < kGrp; k++) {
                if (c0 + k < nch) {
                    const float e = expf(m[k] - Mg);
                    Ls = fmaf(l[k], e, Ls);
                    O.x = fmaf(o[k].x, e, O.x);
                    O.y = fmaf(o[k].y, e, O.y);
                    O.z = fmaf(o[k].z, e, O.z);
                    O.w = fmaf(o[k].w, e, O.w);
                }
            }
            M = Mg;
        }
        const float inv = 1.0f / Ls;
        float* out = a.attn + (g * G + hq) * 128 + 4 * j4;
        st_sys(out, O.x * inv);
        st_sys(out + 1, O.y * inv);
        st_sys(out + 2, O.z * inv);
        st_sys(out + 3, O.w * inv);
    }
    QH_MARK(1, 3);
    signal(A, ++ph);
    return true;
}

// ======================================================== C: o-projection ==
// Wave wv owns row r0 + wv (qd <= 4096 columns: chunks lane, lane + 64).
template <uint32_t KO>
__device__ __forceinline__ bool phase_oproj(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                            uint32_t& ph) {
    const Ctx c = fresh(c0);
    const uint32_t ocpr = c.qd / 32, E = c.E;
    typename Fmt<KO>::Raw w0, w1;
    const bool rowok = c.wv < c.nr;
    const uint8_t* orow = L.o.w + (size_t)(c.r0 + c.wv) * L.o.drb;
    if (rowok) {
        if (c.lane < ocpr) w0 = Fmt<KO>::load(orow, L.o.geo, c.lane);
        if (c.lane + 64 < ocpr) w1 = Fmt<KO>::load(orow, L.o.geo, c.lane + 64);
    }
    // F32 router weights of this workgroup's rows: thread (e = tid/4, q = tid%4)
    // owns rows 2q, 2q + 1
    const uint32_t e = c.tid >> 2, q = c.tid & 3;
    float rw0 = 0.f, rw1 = 0.f;
    if (e < E) {
        const float* wr = reinterpret_cast<const float*>(L.router.w + (size_t)e * L.router.drb) + c.r0;
        if (2 * q < c.nr) rw0 = wr[2 * q];
        if (2 * q + 1 < c.nr) rw1 = wr[2 * q + 1];
    }
    if (c.tid < c.nr) S.wn[c.tid] = L.ffn_norm[c.r0 + c.tid];
    QH_MARK(2, 0);
    if (!wait_all(A, S, ph)) return false;  // attention output (phase B)
    QH_MARK(2, 1);
    float* xs = S.big;
    {
        const __amdgpu_buffer_rsrc_t ar = buf_rsrc(A.a.attn, c.qd * 4);
        for (uint32_t i = c.tid; i < c.qd / 4; i += kDT) reinterpret_cast<float4*>(xs)[i] = ld_sys4(ar, i * 16);
    }
    __syncthreads();
    if (rowok) {  // wave-uniform
        float acc = 0.f;
        float xa[16], xb[16], sa, sb;
        if (c.lane < ocpr) {
            x_runs<KO>(xs, c.lane, xa, xb, sa, sb);
            acc = Fmt<KO>::dot(w0, c.lane, xa, xb, sa, sb);
        }
        if (c.lane + 64 < ocpr) {
            x_runs<KO>(xs, c.lane + 64, xa, xb, sa, sb);
            acc += Fmt<KO>::dot(w1, c.lane + 64, xa, xb, sa, sb);
        }
        acc = wave_sum(acc);
        if (c.lane == 0) {
            const float xn = S.xo[c.wv] + acc;  // residual (model.rs:246-248)
            S.xo[c.wv] = xn;
            st_sys(A.a.x + c.r0 + c.wv, xn);
        }
    }
    __syncthreads();
    // router partial dots over the rows (the logits are linear in x')
    float p = 0.f;
    if (2 * q < c.nr) p = rw0 * (S.wn[2 * q] * S.xo[2 * q]);
    if (2 * q + 1 < c.nr) p = fmaf(rw1, S.wn[2 * q + 1] * S.xo[2 * q + 1], p);
    p += dpp_f<kDppXor1>(p);
    p += dpp_f<kDppXor2>(p);
    if (q == 0 && e < E) st_sys(A.rpart + (size_t)c.b * c.E1 + e, p);
    if (c.wv == 0) {
        float v = c.lane < c.nr ? S.xo[c.lane] * S.xo[c.lane] : 0.f;
        v = wave_sum(v);
        if (c.lane == 0) st_sys(A.rpart + (size_t)c.b * c.E1 + E, v);
    }
    QH_MARK(2, 2);
    signal(A, ++ph);
    return true;
}

// ========================================================== D: router fold ==
// Workgroup e <= E folds column e (and the sum of squares) over the partial
// rows of every workgroup, in one fixed order.
__device__ __forceinline__ bool phase_fold(const DecodeArgs& A, DecodeLds& S, const Ctx& c0, uint32_t& ph) {
    const Ctx c = fresh(c0);
    if (c.b < c.E1) {
        QH_MARK(3, 0);
        if (!wait_all(A, S, ph)) return false;  // router partials (phase C)
        QH_MARK(3, 1);
        float v = 0.f, vs = 0.f;
        if (c.tid < c.nwg) {
            v = ld_sys(A.rpart + (size_t)c.tid * c.E1 + c.b);
            vs = ld_sys(A.rpart + (size_t)c.tid * c.E1 + c.E);
        }
        const float fold = dsum(v, S.red);
        const float fsq = dsum(vs, S.red);
        if (c.tid == 0) {
            const float s = 1.0f / sqrtf(fsq / (float)c.H + A.dm.eps);
            st_sys(A.rlog + c.b, c.b < c.E ? s * fold : s);
        }
        QH_MARK(3, 2);
    }
    signal(A, ++ph);
    return true;
}

// ============================================== E + F: routed expert FFN ==
template <uint32_t KG, uint32_t KD>
__device__ __forceinline__ bool phase_moe(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          uint32_t& ph) {
    const Ctx c = fresh(c0);
    const Acts& a = A.a;
    const uint32_t E = c.E, top = c.top, ff = c.ff, fp = c.fp, H = c.H, cpr = H / 32;
    float4 fn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < H) fn = reinterpret_cast<const float4*>(L.ffn_norm)[c.tid];
    QH_MARK(4, 0);
    if (!wait_all(A, S, ph)) return false;  // folded logits (phase D)
    QH_MARK(4, 1);
    if (c.tid <= E) S.lg[c.tid] = ld_sys(A.rlog + c.tid);
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < H) xv = ld_sys4(buf_rsrc(a.x, H * 4), c.tid * 16);
    __syncthreads();
    // top-k by rank under the total order, lower index on ties (ops.rs:45-56;
    // bit-exact on these logits): j outranks i iff ck[j] > ck[i]
    const uint32_t Ep = (E + 7) & ~7u;
    if (c.tid < E) {
        const float lv = S.lg[c.tid];
        if (!finite_f(lv)) S.bad = 1;
        S.ck[c.tid] = (long long)(((uint64_t)(uint32_t)total_key(lv) << 32) | (uint32_t)~c.tid);
    } else if (c.tid < Ep) {
        S.ck[c.tid] = LLONG_MIN;
    }
    __syncthreads();
    if (S.bad) {
        if (c.b == 0 && c.tid == 0) atomicOr(&a.st->err, kErrRouter);
        return false;  // every workgroup sees the same logits
    }
    {
        const uint32_t i = c.tid >> 2, q = c.tid & 3, J = Ep / 4, j0 = q * J;
        const long long ki = S.ck[min(i, Ep - 1)];
        int32_t rank = 0;
        for (uint32_t j = j0; j < j0 + J; j += 2) {
            const longlong2 w2 = *reinterpret_cast<const longlong2*>(S.ck + j);
            rank += (w2.x > ki) + (w2.y > ki);
        }
        rank += dpp_i<kDppXor1>(rank);
        rank += dpp_i<kDppXor2>(rank);
        if (q == 0 && i < E && (uint32_t)rank < top) {
            S.sid[rank] = i;
            S.sv[rank] = S.lg[i];
        }
    }
    __syncthreads();
    // softmax over the selected logits, in order (ops.rs:29-44)
    if (c.tid < top) {
        float mx = -INFINITY;
        for (uint32_t i = 0; i < top; i++) mx = fmaxf(mx, S.sv[i]);
        S.ex[c.tid] = expf(S.sv[c.tid] - mx);
        S.ids[c.tid] = S.sid[c.tid];
    }
    __syncthreads();
    if (c.tid < top) {
#pragma clang fp contract(off)
        float sum = 0.f;
        for (uint32_t i = 0; i < top; i++) sum += S.ex[i];
        S.wts[c.tid] = S.ex[c.tid] / sum;
    }
    QH_MARK(4, 2);
    // gate/up rows of pairs p = gw*3 + k: (slot p / ff, row p % ff)
    typename Fmt<KG>::Raw wg[kPairsPerWave], wu[kPairsPerWave];
#pragma unroll
    for (uint32_t k = 0; k < kPairsPerWave; k++) {
        const uint32_t pr = c.gw * kPairsPerWave + k;
        if (pr < top * ff && c.lane < cpr) {
            const uint32_t ex = S.ids[pr / ff], rr = pr % ff;
            wg[k] = Fmt<KG>::load(L.gate.w + (size_t)ex * L.gate.expert_stride + (size_t)rr * L.gate.drb, L.gate.geo,
                                  c.lane);
            wu[k] = Fmt<KG>::load(L.up.w + (size_t)ex * L.up.expert_stride + (size_t)rr * L.up.drb, L.up.geo, c.lane);
        }
    }
    // xn = x' * (s * ffn_norm)
    float* xs = S.big;
    const float s = S.lg[E];
    if (4 * c.tid < H) {
        xs[4 * c.tid] = xv.x * (s * fn.x);
        xs[4 * c.tid + 1] = xv.y * (s * fn.y);
        xs[4 * c.tid + 2] = xv.z * (s * fn.z);
        xs[4 * c.tid + 3] = xv.w * (s * fn.w);
    }
    __syncthreads();
    if (c.b == 0) {
        if (c.tid < top) {
            a.ids[c.tid] = S.ids[c.tid];
            a.wts[c.tid] = S.wts[c.tid];
        }
        if (c.tid < E) a.logits_r[c.tid] = S.lg[c.tid];
    }
    QH_MARK(4, 4);
    {
        float xa[16], xb[16], sa, sb;
        if (c.lane < cpr) x_runs<KG>(xs, c.lane, xa, xb, sa, sb);
#pragma unroll
        for (uint32_t k = 0; k < kPairsPerWave; k++) {
            const uint32_t pr = c.gw * kPairsPerWave + k;
            if (pr < top * ff) {  // wave-uniform
                float gv = 0.f, uv = 0.f;
                if (c.lane < cpr) {
                    gv = Fmt<KG>::dot(wg[k], c.lane, xa, xb, sa, sb);
                    uv = Fmt<KG>::dot(wu[k], c.lane, xa, xb, sa, sb);
                }
                gv = wave_sum(gv);
                uv = wave_sum(uv);
                if (c.lane == 0) {
#pragma clang fp contract(off)
                    const float hv = (gv / (1.f + expf(-gv))) * uv;  // SwiGLU (model.rs:272)
                    st_sys(a.h + (pr / ff) * fp + pr % ff, hv);
                }
            }
        }
    }
    QH_MARK(4, 5);
    // down rows of phase F (row r0 + wv of each routed expert), requested
    // before the wait: lane units u = lane + 64 i = (slot u / dcpr, chunk u % dcpr)
    const uint32_t dcpr = ff / 32, U = top * dcpr;
    typename Fmt<KD>::Raw wd[kDownUnits];
#pragma unroll
    for (uint32_t i = 0; i < kDownUnits; i++) {
        const uint32_t u = c.lane + 64 * i;
        if (c.wv < c.nr && u < U) {
            const uint8_t* drow = L.down.w + (size_t)S.ids[u / dcpr] * L.down.expert_stride +
                                  (size_t)(c.r0 + c.wv) * L.down.drb;
            wd[i] = Fmt<KD>::load(drow, L.down.geo, u % dcpr);
        }
    }
    QH_MARK(4, 3);
    signal(A, ++ph);
    QH_MARK(5, 0);
    if (!wait_all(A, S, ph)) return false;  // SwiGLU outputs (phase E)
    QH_MARK(5, 1);
    {
        const uint32_t nh = top * fp;
        const __amdgpu_buffer_rsrc_t hr = buf_rsrc(a.h, nh * 4);
        for (uint32_t i = c.tid; i < nh / 4; i += kDT) reinterpret_cast<float4*>(xs)[i] = ld_sys4(hr, i * 16);
    }
    __syncthreads();
    QH_MARK(5, 3);
    if (c.wv < c.nr) {  // wave-uniform
        float acc = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < kDownUnits; i++) {
            const uint32_t u = c.lane + 64 * i;
            if (u < U) {
                const uint32_t sl = u / dcpr, chn = u % dcpr;
                float xa[16], xb[16], sa, sb;
                x_runs<KD>(xs + sl * fp, chn, xa, xb, sa, sb);
                acc = fmaf(S.wts[sl], Fmt<KD>::dot(wd[i], chn, xa, xb, sa, sb), acc);
            }
        }
        acc = wave_sum(acc);
        if (c.lane == 0) {
            const float xn = S.xo[c.wv] + acc;  // x += sum_s w_s down_s (model.rs:281-287)
            S.xo[c.wv] = xn;
            st_sys(a.x + c.r0 + c.wv, xn);
        }
    }
    QH_MARK(5, 2);
    signal(A, ++ph);
    return true;
}

// =========================================================== V: vocab ==
template <uint32_t KV>
__device__ __forceinline__ void phase_vocab(const DecodeArgs& A, DecodeLds& S, const Ctx& c0, uint32_t& ph) {
    const Ctx c = fresh(c0);
    const Acts& a = A.a;
    const DevMat& mv = A.out;
    const uint32_t V = A.dm.vocab, ngrp = (V + kVocabRows - 1) / kVocabRows, cpr = c.H / 32;
    using Raw = typename Fmt<KV>::Raw;
    auto load_group = [&](Raw (&t)[kVocabRows], uint32_t gi) {
#pragma unroll
        for (uint32_t k = 0; k < kVocabRows; k++) {
            const uint32_t r = gi * kVocabRows + k;
            if (gi < ngrp && r < V && c.lane < cpr) t[k] = Fmt<KV>::load(mv.w + (size_t)r * mv.drb, mv.geo, c.lane);
        }
    };
    Raw cur[kVocabRows], nxt[kVocabRows];
    load_group(cur, c.gw);
    float4 on = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < c.H) on = reinterpret_cast<const float4*>(A.onorm)[c.tid];
    QH_MARK(6, 0);
    if (!wait_all(A, S, ph)) return;  // x after the last layer
    QH_MARK(6, 1);
    float* xs = S.big;
    load_norm_x(c, a.x, on, A.dm.eps, xs, S.red);
    float xa[16], xb[16], sa, sb;
    if (c.lane < cpr) x_runs<KV>(xs, c.lane, xa, xb, sa, sb);
    int32_t bk = INT32_MIN;
    uint32_t bi = 0xffffffffu;
    bool nf = false;
    for (uint32_t gi = c.gw; gi < ngrp; gi += c.NWV) {
        if (gi + c.NWV < ngrp) load_group(nxt, gi + c.NWV);
        float acc[kVocabRows];
#pragma unroll
        for (uint32_t k = 0; k < kVocabRows; k++) {
            acc[k] = c.lane < cpr ? Fmt<KV>::dot(cur[k], c.lane, xa, xb, sa, sb) : 0.f;
            acc[k] = wave_sum(acc[k]);
        }
        if (c.lane == 0) {
#pragma unroll
            for (uint32_t k = 0; k < kVocabRows; k++) {
                const uint32_t r = gi * kVocabRows + k;
                if (r < V) {
                    a.logits[r] = acc[k];
                    nf |= !finite_f(acc[k]);
                    best_merge(bk, bi, total_key(acc[k]), r);
                }
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kVocabRows; k++) cur[k] = nxt[k];
    }
    QH_MARK(6, 2);
    if (nf) S.bad = 1;
    wave_best(bk, bi);
    if (c.lane == 0) {
        S.bk[c.wv] = bk;
        S.bi[c.wv] = bi;
    }
    __syncthreads();
    if (c.tid == 0) {
        int32_t k0 = S.bk[0];
        uint32_t i0 = S.bi[0];
        for (int w = 1; w < kDW; w++) best_merge(k0, i0, S.bk[w], S.bi[w]);
        st_sys_u(a.fin_key + c.b, (uint32_t)k0);
        st_sys_u(a.fin_idx + c.b, i0);
        if (S.bad) atomicOr(&a.st->err, kErrLogits);
    }
    signal(A, ++ph);
    if (c.b != 0) return;
    if (!wait_all(A, S, ph)) return;  // every workgroup's argmax partial
    int32_t k1 = INT32_MIN;
    uint32_t i1 = 0xffffffffu;
    if (c.tid < c.nwg) {
        k1 = (int32_t)ld_sys_u(a.fin_key + c.tid);
        i1 = ld_sys_u(a.fin_idx + c.tid);
    }
    wave_best(k1, i1);
    if (c.lane == 0) {
        S.bk[c.wv] = k1;
        S.bi[c.wv] = i1;
    }
    __syncthreads();
    if (c.tid == 0) {
        int32_t k0 = S.bk[0];
        uint32_t i0 = S.bi[0];
        for (int w = 1; w < kDW; w++) best_merge(k0, i0, S.bk[w], S.bi[w]);
        a.st->argmax = i0;
        if (c.pos + 1 >= a.st->n_given && c.pos + 1 <= A.dm.ctx) a.tokens[c.pos + 1] = i0;
        a.st->pos = c.pos + 1;
    }
    QH_MARK(6, 3);
}

// ================================================================= kernels ==
// Embedding row of tokens[pos] into x (model.rs:225), bit-exact decode.
__global__ __launch_bounds__(kBlock) void k_embed(DevMat emb, Acts a, ModelDims dm) {
    const uint32_t pos = a.st->pos;
    if (pos >= dm.ctx) return;  // reported by the step kernel
    const uint32_t tok = a.tokens[pos];
    if (tok >= dm.vocab) {
        if (threadIdx.x == 0) atomicOr(&a.st->err, kErrToken);
        return;
    }
    const uint8_t* row = emb.w + (size_t)tok * emb.drb;
    for (uint32_t i = threadIdx.x; i < dm.hidden; i += kBlock) a.x[i] = dequant_value(row, emb.kind, emb.geo, i);
}

__global__ __launch_bounds__(kDT) void k_decode(DecodeArgs A) {
    __shared__ __align__(16) DecodeLds S;
    Ctx c;
    c.b = blockIdx.x;
    c.nwg = gridDim.x;
    c.tid = threadIdx.x;
    c.lane = c.tid & 63;
    // wave-uniform: derived values stay in scalar registers
    c.wv = __builtin_amdgcn_readfirstlane(c.tid >> 6);
    c.gw = c.b * kDW + c.wv;
    c.NWV = c.nwg * kDW;
    const ModelDims& dm = A.dm;
    if (c.tid == 0) {
        S.abort = 0;
        S.bad = 0;
    }
    c.pos = A.a.st->pos;
    const uint32_t err0 = A.a.st->err;
    __syncthreads();
    if (c.pos >= dm.ctx || (err0 & kErrToken)) {
        if (c.b == 0 && c.tid == 0 && c.pos >= dm.ctx) atomicOr(&A.a.st->err, kErrContext);
        return;
    }
    c.T = c.pos + 1;
    c.H = dm.hidden;
    c.E = dm.experts;
    c.E1 = c.E + 1;
    c.top = dm.top;
    c.ff = dm.ff;
    c.fp = pad32(dm.ff);
    c.G = dm.heads / dm.kvheads;
    c.qd = dm.heads * 128;
    c.ctx = dm.ctx;
    const uint32_t rpw = (c.H + c.nwg - 1) / c.nwg;
    c.r0 = c.b * rpw;
    c.nr = c.r0 < c.H ? min(rpw, c.H - c.r0) : 0;
    uint32_t ph = A.base;
    for (uint32_t l = A.l0; l < A.l1; l++) {
        const LayerW& L = A.layers[l];
        const bool wait_x = l != A.l0;
        bool ok = true;
        QH_DISPATCH_KM(L.v.kind, KV, ok = phase_qkv<Q4_K, KV>(A, S, L, c, wait_x, ph));
        if (!ok || !phase_attn(A, S, L, c, ph)) return;
        ok = phase_oproj<Q4_K>(A, S, L, c, ph);
        if (!ok || !phase_fold(A, S, c, ph)) return;
        QH_DISPATCH_KM(L.down.kind, KD, ok = phase_moe<Q4_K, KD>(A, S, L, c, ph));
        if (!ok) return;
    }
    if (A.vocab) QH_DISPATCH_KM(A.out.kind, KV, phase_vocab<KV>(A, S, c, ph));
}

}  // namespace qh
