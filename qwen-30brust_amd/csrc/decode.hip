// Persistent token step (src/model.rs:227-302 and the greedy sampler,
// src/sampling.rs:26-35) as ONE launch of one 512-thread workgroup per CU,
// preceded by k_embed (the embedding row of tokens[pos], model.rs:225).
//
// Per layer the workgroups run five phases:
//   A  RMSNorm + q/k/v projections; router workgroup e also reduces
//      sum_j router[e][j] ffn_norm[j] x[j]
//   B  Q/K RMSNorm, RoPE, KV append, split-T GQA attention; chunk 0 of each
//      KV head merges the other chunks' partials
//   C  output projection + residual for this workgroup's rows of x; router
//      workgroup e adds its row of the precomputed router fold times the
//      attention output, giving the unscaled router logit e of x'
//   E  every workgroup reads x' and the unscaled logits, scales them by the
//      RMS scale of x', top-k routing (identically everywhere), gate/up +
//      SwiGLU rows
//   F  down projections + routing-weighted combine + residual, own rows
// then V: final RMSNorm, vocab projection and argmax partials, and the
// argmax / next token / position advance by workgroup 0.
//
// Hand-over without flags or barriers: every value one workgroup passes to
// another is a 64-bit word (tag << 32) | bits written through to memory with
// a system-scope store, where tag = base + the number of the writing phase
// (6 numbers per layer, 1 for V; base grows by the launch's phase count, so tags
// never repeat between launches).  A reader polls exactly the words it needs
// until each carries the tag it expects: a phase starts as soon as its own
// inputs exist, and no producer waits for its stores to complete.  Before it
// polls, a workgroup issues every load that does not depend on the awaited
// words (its next weights, norm vectors, the KV history, and once the routing
// is known the down-projection rows).  Every wait is bounded: on timeout the
// workgroup raises abort_flag and every other wait returns, so the grid
// always drains.
//
// Reuse of a buffer in the next layer is safe without any barrier: every
// workgroup owns rows of x (the host checks it), so a workgroup that has read
// all of x'' (or x') of layer l knows every workgroup has finished phase F
// (or C) of layer l, and with it every read of the buffers it overwrites next.
//
// Each phase body is instantiated for the formats of the Q4_K_M mix (q, k,
// o, gate, up: Q4_K; v, down, vocab: Q4_K or Q6_K) and selected once per
// phase.  The host launches this path only for models and shapes it covers
// (engine.hip: persist_supported); everything else runs the per-phase kernels.
#include "qh_block.hpp"
#include "qh_tile.hpp"

namespace qh {

typedef float f4v __attribute__((ext_vector_type(4)));  // one MFMA accumulator tile per lane

constexpr int kDT = 512;
constexpr int kDW = kDT / 64;
constexpr uint32_t kSpinLimit = 1u << 22;   // polls before a wait gives up
constexpr uint32_t kDChunks = 32;           // most attention chunk workgroups per KV head
constexpr uint32_t kDTile = 64;             // keys per attention tile (and at least per chunk)
constexpr uint32_t kTP = 132;               // LDS pitch of the key and value tiles (floats)
constexpr uint32_t kPP = 68;                // LDS pitch of the per-head scores (floats)
constexpr uint32_t kDSmem = 11776;          // floats of phase scratch
constexpr uint32_t kQkvPerWave = 3;         // q/k/v rows per wave (at most)
constexpr uint32_t kPairsPerWave = 3;       // gate/up row pairs per wave
constexpr uint32_t kHBlock = kPairsPerWave * kDW;  // SwiGLU outputs per workgroup
constexpr uint32_t kDownUnits = 3;          // (expert, chunk) units per lane in F
constexpr uint32_t kVocabRows = 4;          // vocab rows per wave group
constexpr uint32_t kGatherPairs = 6;        // word pairs in flight per thread in a gather

// Formats of the Q4_K_M mix; the host routes other models to the per-phase
// kernels.
#define QH_DISPATCH_KM(kind, K, ...)                                            \
    switch (kind) {                                                             \
    case ::qh::Q4_K: { constexpr uint32_t K = ::qh::Q4_K; __VA_ARGS__; } break; \
    default: { constexpr uint32_t K = ::qh::Q6_K; __VA_ARGS__; } break;         \
    }

struct DecodeLds {
    float big[kDSmem];        // phase scratch (x, attention tiles, h)
    float xo[8];              // this workgroup's rows of the residual stream
    float hv[kHBlock];        // this workgroup's phase A rows, then its SwiGLU outputs
    float red[2 * kDW];
    float lg[256];            // router logits
    alignas(16) long long ck[128];  // composite top-k keys
    float ra;                 // router workgroup: sum_j router[e][j] ffn_norm[j] x[j] of this layer
    float sv[8];
    uint32_t sid[8];
    float ex[8];
    float wts[8];             // routing weights of the current layer
    uint32_t ids[8];          // routed experts of the current layer
    int32_t bk[kDW];
    uint32_t bi[kDW];
    uint32_t abort;
    uint32_t bad;
    uint32_t vq;              // next vocab row group of this workgroup to hand out
};

// Per-workgroup constants of one launch.
struct Ctx {
    uint32_t b, nwg, tid, wv, lane, gw;
    uint32_t pos, T, H, E, top, ff, G, qd, kvd, ctx;
    uint32_t r0, nr, rpw;  // this workgroup's rows of x: [r0, r0 + nr), rpw per workgroup
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

// ------------------------------------------------------------ tagged words --
__device__ __forceinline__ void put(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Bookkeeping of one poll round: every 64th round checks the abort flag and
// the time limit (on timeout raises the abort flag and kErrSync).  False when
// the wait must stop (ab = true).
__device__ __forceinline__ bool keep_polling(const DecodeArgs& A, uint32_t& spins, bool& ab) {
    if ((++spins & 63) == 0) {
        if (ld_sys_u(A.abort_flag) != 0) {
            ab = true;
            return false;
        }
        if (spins > kSpinLimit) {
            st_sys_u(A.abort_flag, 1u);
            atomicOr(&A.a.st->err, kErrSync);
            ab = true;
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// Two adjacent words (16 bytes, 16-byte aligned) read past the caches.
__device__ __forceinline__ void ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t word, uint64_t& w0, uint64_t& w1) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(word * 8), 0, 17);
    w0 = ((uint64_t)(uint32_t)v[1] << 32) | (uint32_t)v[0];
    w1 = ((uint64_t)(uint32_t)v[3] << 32) | (uint32_t)v[2];
}

// Waits for N word pairs at once: pair k (words word[k], word[k] + 1 of r)
// is awaited when bit k of need is set, its second word only when bit k of
// hi is set too.  Every round re-reads all pairs still missing with one batch
// of loads, so a wait costs one memory round trip per round however many
// words it covers.  v[2k], v[2k + 1] receive the values.
template <uint32_t N>
__device__ __forceinline__ void poll_pairs(const DecodeArgs& A, __amdgpu_buffer_rsrc_t r, const uint32_t (&word)[N],
                                           uint32_t need, uint32_t hi, uint32_t tag, float (&v)[2 * N], bool& ab) {
    uint32_t spins = 0;
    while (need != 0) {
        uint64_t w[2 * N];
#pragma unroll
        for (uint32_t k = 0; k < N; k++)
            if ((need >> k) & 1) ld_pair(r, word[k], w[2 * k], w[2 * k + 1]);
#pragma unroll
        for (uint32_t k = 0; k < N; k++) {
            if (((need >> k) & 1) && has_tag(w[2 * k], tag) && (!((hi >> k) & 1) || has_tag(w[2 * k + 1], tag))) {
                v[2 * k] = __uint_as_float((uint32_t)w[2 * k]);
                v[2 * k + 1] = __uint_as_float((uint32_t)w[2 * k + 1]);
                need &= ~(1u << k);
            }
        }
        if (need == 0 || !keep_polling(A, spins, ab)) break;
    }
}

// The same for N single words base[idx[k]].
template <uint32_t N>
__device__ __forceinline__ void poll_words(const DecodeArgs& A, const uint64_t* base, const uint32_t (&idx)[N],
                                           uint32_t need, uint32_t tag, float (&v)[N], bool& ab) {
    uint32_t spins = 0;
    while (need != 0) {
        uint64_t w[N];
#pragma unroll
        for (uint32_t k = 0; k < N; k++)
            if ((need >> k) & 1) w[k] = __hip_atomic_load(base + idx[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
        for (uint32_t k = 0; k < N; k++) {
            if (((need >> k) & 1) && has_tag(w[k], tag)) {
                v[k] = __uint_as_float((uint32_t)w[k]);
                need &= ~(1u << k);
            }
        }
        if (need == 0 || !keep_polling(A, spins, ab)) break;
    }
}

// LDS layout of the gathered activation vectors: element i at px(i) =
// i + 4 (i / 64).  The lanes of one read take the 16-float runs of
// neighbouring chunks of a Q4_K/Q6_K row, 16-64 floats apart; unpadded, four
// of every eight lanes of a 16-byte read met in the same banks.  A run never
// crosses a 64-float block, so it stays contiguous.
__device__ __forceinline__ uint32_t px(uint32_t i) { return i + ((i >> 6) << 2); }

// dst[i] (dst[px(i)] with PAD) = value of src[i] for i < n, every word
// awaited with `tag` (src is 16-byte aligned with room for an even number of
// words).  Ends with a barrier; false when the step was aborted.
template <bool PAD = false>
__device__ __forceinline__ bool gather(const DecodeArgs& A, DecodeLds& S, const uint64_t* src, uint32_t n,
                                       uint32_t tag, float* dst, uint32_t tid) {
    const uint32_t np = (n + 1) / 2;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(src, np * 16);
    bool ab = false;
    for (uint32_t p0 = tid; p0 < np; p0 += kGatherPairs * kDT) {
        uint32_t word[kGatherPairs], need = 0, hi = 0;
#pragma unroll
        for (uint32_t k = 0; k < kGatherPairs; k++) {
            const uint32_t p = p0 + k * kDT;
            word[k] = 2 * p;
            if (p < np) need |= 1u << k;
            if (2 * p + 1 < n) hi |= 1u << k;
        }
        float v[2 * kGatherPairs];
        poll_pairs<kGatherPairs>(A, r, word, need, hi, tag, v, ab);
        if (ab) break;
#pragma unroll
        for (uint32_t k = 0; k < kGatherPairs; k++) {
            const uint32_t p = p0 + k * kDT, d = PAD ? px(2 * p) : 2 * p;  // a pair stays adjacent
            if (p < np) dst[d] = v[2 * k];
            if (2 * p + 1 < n) dst[d + 1] = v[2 * k + 1];
        }
    }
    if (ab) S.abort = 1;
    __syncthreads();
    return S.abort == 0;
}

// gather<true>() (padded layout) preceded by a cheap readiness check: wave 0 polls ns <= 256
// sample words src[first + j * stride] (one per producer block, each block
// written by one store instruction) until a quarter of the producers have
// written, and only then does the workgroup read all n words (gather() then
// re-reads only what is still missing).  A workgroup that waits long (for
// attention, say) thus polls a few hundred bytes per round instead of the
// whole vector and does not flood the memory channels the producers are
// using, while the later producers overlap the bulk read.  (Measured over the
// 30B step: a quarter and an eighth are best, 1 % ahead of three quarters;
// all producers or none are slower.)
__device__ __forceinline__ bool gather_s(const DecodeArgs& A, DecodeLds& S, const uint64_t* src, uint32_t n,
                                         uint32_t tag, float* dst, uint32_t tid, uint32_t ns, uint32_t first,
                                         uint32_t stride) {
    if (tid < 64) {  // wave 0
        bool ab = false;
        uint32_t idx[4], need = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint32_t j = tid + 64 * k;
            idx[k] = first + j * stride;
            if (j < ns) need |= 1u << k;
        }
        const float want = (float)(ns / 4);
        uint32_t spins = 0;
        while (true) {
            uint64_t w[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; k++)
                if ((need >> k) & 1) w[k] = __hip_atomic_load(src + idx[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (uint32_t k = 0; k < 4; k++)
                if (((need >> k) & 1) && has_tag(w[k], tag)) need &= ~(1u << k);
            const float done = (float)ns - wave_sum((float)__builtin_popcount(need));  // wave-uniform
            if (done >= want || !keep_polling(A, spins, ab)) break;
        }
        if (ab) S.abort = 1;
    }
    __syncthreads();
    if (S.abort) return false;
    return gather<true>(A, S, src, n, tag, dst, tid);
}

// Block sum.  It ends without a barrier: every caller reaches another
// barrier before anything writes red again.
__device__ __forceinline__ float dsum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kDW; i++) s += red[i];
    return s;
}
// Two block sums in one round (the same rule for red).
__device__ __forceinline__ float2 dsum2(float u, float v, float* red) {
    u = wave_sum(u);
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = u;
        red[kDW + (threadIdx.x >> 6)] = v;
    }
    __syncthreads();
    float su = 0.f, sv = 0.f;
#pragma unroll
    for (int i = 0; i < kDW; i++) {
        su += red[i];
        sv += red[kDW + i];
    }
    return make_float2(su, sv);
}

__device__ __forceinline__ float sumsq4(float4 v) { return fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x))); }

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

// RMSNorm (ops.rs:3-15) of the raw x in LDS (padded layout, elements
// [0, H)), in place, with weights w (this thread's float4); returns this
// thread's raw float4.  H <= 2048.
__device__ __forceinline__ float4 norm_in_lds(const Ctx& c, float* xs, float4 w, float eps, float* red) {
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    float* x4 = xs + px(4 * c.tid);
    if (4 * c.tid < c.H) xv = *reinterpret_cast<const float4*>(x4);
    const float scale = 1.0f / sqrtf(dsum(sumsq4(xv), red) / (float)c.H + eps);
    if (4 * c.tid < c.H) {
        x4[0] = xv.x * (scale * w.x);
        x4[1] = xv.y * (scale * w.y);
        x4[2] = xv.z * (scale * w.z);
        x4[3] = xv.w * (scale * w.w);
    }
    __syncthreads();
    return xv;
}

// Router workgroups follow every possible attention workgroup: workgroup
// kvheads * kDChunks + e folds router row e (e < experts) into phases A and C.
__device__ __forceinline__ bool router_wg(const DecodeArgs& A, const Ctx& c, uint32_t& e) {
    e = c.b - A.dm.kvheads * kDChunks;
    return c.b >= A.dm.kvheads * kDChunks && e < c.E;
}

// norm_in_lds that also reduces sum_i rw[i] x[i] (raw x) in the same round.
__device__ __forceinline__ float4 norm_in_lds_dot(const Ctx& c, float* xs, float4 w, float eps, float* red,
                                                  float4 rw, float& rdot) {
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    float* x4 = xs + px(4 * c.tid);
    if (4 * c.tid < c.H) xv = *reinterpret_cast<const float4*>(x4);
    const float dt = fmaf(rw.w, xv.w, fmaf(rw.z, xv.z, fmaf(rw.y, xv.y, rw.x * xv.x)));
    const float2 r = dsum2(sumsq4(xv), dt, red);
    const float scale = 1.0f / sqrtf(r.x / (float)c.H + eps);
    if (4 * c.tid < c.H) {
        x4[0] = xv.x * (scale * w.x);
        x4[1] = xv.y * (scale * w.y);
        x4[2] = xv.z * (scale * w.z);
        x4[3] = xv.w * (scale * w.w);
    }
    __syncthreads();
    rdot = r.y;
    return xv;
}

// Tag of phase k (1..6) of layer l.
__device__ __forceinline__ uint32_t ptag(const DecodeArgs& A, uint32_t l, uint32_t k) {
    return A.base + 6 * (l - A.l0) + k;
}

// Chunk geometry of the attention workgroups: KV head g = b / 32, chunk
// b % 32; a chunk covers >= 64 keys, at most max_chunks chunks per head.
struct AttnChunk {
    uint32_t nch, g, ch, t0, t1;
    bool active;
};
__device__ __forceinline__ AttnChunk attn_chunk(const DecodeArgs& A, const Ctx& c) {
    AttnChunk k;
    k.nch = min((c.T + kDTile - 1) / kDTile, A.max_chunks);
    k.g = c.b / kDChunks;
    k.ch = c.b % kDChunks;
    k.active = k.g < A.dm.kvheads && k.ch < k.nch;
    const uint32_t tc = (c.T + k.nch - 1) / k.nch;
    k.t0 = min(c.T, k.ch * tc);
    k.t1 = min(c.T, k.t0 + tc);
    return k;
}

// What an attention workgroup loads before it has q/k/v: the first K/V
// slice of its chunk, the q/k norm weights and the rotary table row.
struct AttnPre {
    float4 kr[4], vr[4];
    float qw0, qw1, kw0, kw1;
    float2 cs;
};

__device__ __forceinline__ void kv_slice(float4 (&kr)[4], float4 (&vr)[4], const float* kc, const float* vc,
                                         uint32_t g, uint32_t ctx, uint32_t tt, uint32_t t1, uint32_t pos,
                                         uint32_t tid) {
    const uint32_t key = tt + (tid >> 3), j = (tid & 7) * 16;
    if (key < t1 && key != pos) {
        const float* ks = kc + ((size_t)g * ctx + key) * 128 + j;
        const float* vs = vc + ((size_t)g * ctx + key) * 128 + j;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = gld<float4>(ks + 4 * i);
            vr[i] = gld<float4>(vs + 4 * i);
        }
    }
}

// Issued by attention workgroups in phase A, before they wait for x.
__device__ __forceinline__ void attn_prefetch(const DecodeArgs& A, const LayerW& L, const Ctx& c, AttnPre& P) {
    const AttnChunk k = attn_chunk(A, c);
    if (!k.active) return;
#pragma unroll
    for (int i = 0; i < 4; i++) P.kr[i] = P.vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    kv_slice(P.kr, P.vr, L.kcache, L.vcache, k.g, c.ctx, k.t0, k.t1, c.pos, c.tid);
    P.qw0 = gld<float>(L.q_norm + c.lane);
    P.qw1 = gld<float>(L.q_norm + c.lane + 64);
    P.kw0 = gld<float>(L.k_norm + c.lane);
    P.kw1 = gld<float>(L.k_norm + c.lane + 64);
    P.cs = gld<float2>(A.a.rope + (size_t)c.pos * 64 + c.lane);
}

// ================================================================== A: qkv ==
// Flat rows [q | k | v]; q and k share format KQ, v has KV.  Rows have
// H <= 2048 columns: lane = chunk.  Participating workgroup wi owns two
// contiguous blocks, q|k rows [wi Rqk, wi Rqk + Rqk) and v rows
// [wi Rv, wi Rv + Rv) (Rqk = ceil(nqk / workgroups), Rv likewise, so the
// heavier v rows spread over all workgroups), Rqk + Rv <= 24 slots; wave wv
// computes slots wv + 8 k, and the workgroup passes each block on with one
// store instruction.  Phase A rows go to the workgroups that are not
// attention workgroups this step (those start on their K/V history instead)
// when the blocks fit there; otherwise to every workgroup.  Returns false for
// a workgroup without A rows.
struct QkvRows {
    uint32_t qk0, nqk, v0, nv;  // first row and count of each block (counts may be 0)
};

__device__ __forceinline__ uint32_t qkv_slots(uint32_t nqk, uint32_t nv, uint32_t nw) {
    return (nqk + nw - 1) / nw + (nv + nw - 1) / nw;
}

__device__ __forceinline__ bool qkv_rows(const DecodeArgs& A, const Ctx& c, uint32_t nqk, uint32_t nv,
                                         QkvRows& q) {
    const AttnChunk k = attn_chunk(A, c);
    const uint32_t nattn = A.dm.kvheads * k.nch;
    uint32_t wi, nw;
    if (qkv_slots(nqk, nv, c.nwg - nattn) > kQkvPerWave * kDW) {
        wi = c.b;
        nw = c.nwg;
    } else {
        if (k.active) return false;
        const uint32_t g0 = c.b / kDChunks;
        const uint32_t below = g0 < A.dm.kvheads ? g0 * k.nch + min(c.b % kDChunks, k.nch) : nattn;
        wi = c.b - below;
        nw = c.nwg - nattn;
    }
    const uint32_t Rqk = (nqk + nw - 1) / nw, Rv = (nv + nw - 1) / nw;
    q.qk0 = min(wi * Rqk, nqk);
    q.nqk = min(nqk - q.qk0, Rqk);
    q.v0 = min(wi * Rv, nv);
    q.nv = min(nv - q.v0, Rv);
    return true;
}

template <uint32_t KQ, uint32_t KV>
__device__ __forceinline__ bool phase_qkv(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          uint32_t l, AttnPre& P) {
    const Ctx c = fresh(c0);
    const uint32_t nq = L.q.rows, nk = L.k.rows, nt = nq + nk + L.v.rows, cpr = c.H / 32;
    QkvRows B;
    if (!qkv_rows(A, c, nq + nk, L.v.rows, B)) {
        // attention workgroup without A rows: its residual rows are still in
        // S.xo from phase F, or come from x on the launch's first layer
        attn_prefetch(A, L, c, P);
        if (l == A.l0 && c.tid < c.nr) S.xo[c.tid] = ld_sys(A.a.x + c.r0 + c.tid);
        __syncthreads();
        return true;
    }
    typename Fmt<KQ>::Raw wq[kQkvPerWave];
    typename Fmt<KV>::Raw wvv[kQkvPerWave];
    // slot j: q|k row qk0 + j (j < nqk), else v row v0 + j - nqk; flat row r
#pragma unroll
    for (uint32_t k = 0; k < kQkvPerWave; k++) {
        const uint32_t j = c.wv + kDW * k;
        if (j >= B.nqk + B.nv) continue;
        const uint32_t r = j < B.nqk ? B.qk0 + j : nq + nk + B.v0 + (j - B.nqk);
        if (r < nq + nk && c.lane < cpr) {
            const DevMat& m = r < nq ? L.q : L.k;
            wq[k] = Fmt<KQ>::load(m.w + (size_t)(r < nq ? r : r - nq) * m.drb, m.geo, c.lane);
        } else if (r < nt && c.lane < cpr) {
            wvv[k] = Fmt<KV>::load(L.v.w + (size_t)(r - nq - nk) * L.v.drb, L.v.geo, c.lane);
        }
    }
    float4 nw = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < c.H) nw = gld<float4>(L.attn_norm + 4 * c.tid);
    // router workgroup e: router[e] * ffn_norm, for its share of logit e
    uint32_t re;
    const bool rt = router_wg(A, c, re);
    // (multiplied after the wait for x'': a product here made the loads wait)
    float4 wr = make_float4(0.f, 0.f, 0.f, 0.f), fw = wr;
    if (rt && 4 * c.tid < c.H) {
        wr = gld<float4>(L.router.w + (size_t)re * L.router.drb + 16 * c.tid);
        fw = gld<float4>(L.ffn_norm + 4 * c.tid);
    }
    attn_prefetch(A, L, c, P);
    float* xs = S.big;
    QH_MARK(0, 0);
    if (l == A.l0) {
        // x as the embedding kernel (or the host) left it before this launch
        if (4 * c.tid < c.H)
            *reinterpret_cast<float4*>(xs + px(4 * c.tid)) = ld_sys4(buf_rsrc(A.a.x, c.H * 4), c.tid * 16);
        __syncthreads();
    } else if (!gather_s(A, S, A.tx2, c.H, ptag(A, l - 1, 6), xs, c.tid, c.nwg, 0, c.rpw)) {
        return false;  // x'' of the previous layer (phase F)
    }
    QH_MARK(0, 1);
    const float4 rw = make_float4(wr.x * fw.x, wr.y * fw.y, wr.z * fw.z, wr.w * fw.w);
    float rdot;
    const float4 xv = norm_in_lds_dot(c, xs, nw, A.dm.eps, S.red, rw, rdot);
    if (rt && c.tid == 0) S.ra = rdot;
    // this workgroup's residual rows, kept in LDS through the layer
    if (4 * c.tid < c.H) {
        const float e4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = 4 * c.tid + i;
            if (r >= c.r0 && r < c.r0 + c.nr) S.xo[r - c.r0] = e4[i];
        }
    }
    const uint32_t tag = ptag(A, l, 1);
    float xa[16], xb[16], sa, sb;
    if (c.lane < cpr) x_runs_p<KQ>(xs, 0, c.lane, xa, xb, sa, sb);
#pragma unroll
    for (uint32_t k = 0; k < kQkvPerWave; k++) {
        const uint32_t j = c.wv + kDW * k;
        const uint32_t r = j < B.nqk ? B.qk0 + j : nq + nk + B.v0 + (j - B.nqk);
        if (j < B.nqk + B.nv) {  // wave-uniform
            float acc = 0.f;
            if (c.lane < cpr) {
                if (r < nq + nk) {
                    acc = Fmt<KQ>::dot(wq[k], c.lane, xa, xb, sa, sb);
                } else {
                    float ya[16], yb[16], ta, tb;
                    x_runs_p<KV>(xs, 0, c.lane, ya, yb, ta, tb);
                    acc = Fmt<KV>::dot(wvv[k], c.lane, ya, yb, ta, tb);
                }
            }
            acc = wave_sum(acc);
            if (c.lane == 0) S.hv[j] = acc;
        }
    }
    QH_MARK(0, 2);
    QH_MARK_LAST(2, 4);
    __syncthreads();  // S.hv complete; xs is reused by the next phase
    // the two blocks, one store instruction each (waves 0 and 1)
    if (c.tid < B.nqk) put(A.tqkv + B.qk0 + c.tid, S.hv[c.tid], tag);
    if (c.tid >= 64 && c.tid - 64 < B.nv) put(A.tqkv + nq + nk + B.v0 + (c.tid - 64), S.hv[B.nqk + c.tid - 64], tag);
    return true;
}

// ============================================================ B: attention ==
// KV head g = b / 32, chunk b % 32.  A chunk covers >= 64 keys (at most
// max_chunks chunks per head) and runs 64-key tiles on all eight waves:
//   scores   thread (key tid/8, 16-dim part tid%8) holds its K slice in
//            registers and reduces the 8 parts of each head on DPP;
//   softmax  wave h owns head h (lane = key), online over the tiles;
//   P.V      wave h, lane (4 dims j4, key half kh): the weights of keys t and
//            t + 32 are broadcast with v_readlane, V is read from LDS.
// Chunks > 0 pass their partial (o[128], m, l) on as tagged words; chunk 0
// merges them (each half of a wave takes half of the chunks, 8 per round of
// loads), or with a single chunk writes the output directly.
__device__ __forceinline__ float shfl32(float v) { return __shfl_xor(v, 32, 64); }

__device__ __forceinline__ bool phase_attn(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                           uint32_t l, AttnPre& P) {
    const Ctx c = fresh(c0);
    const ModelDims& dm = A.dm;
    const AttnChunk k = attn_chunk(A, c);
    if (!k.active) return true;  // not an attention workgroup this step
    QH_MARK(2, 3);
    const uint32_t nch = k.nch, g = k.g, ch = k.ch, t0 = k.t0, t1 = k.t1;
    const uint32_t tid = c.tid, wv = c.wv, lane = c.lane, G = c.G, pos = c.pos, ctx = c.ctx;
    const bool holds = t0 <= pos && pos < t1;
    const uint32_t tag_in = ptag(A, l, 1), tag = ptag(A, l, 2);
    float4(&kr)[4] = P.kr;
    float4(&vr)[4] = P.vr;
    const float2 cs = P.cs;
    // Wave w: q head w (w < G); the new key by wave G % 8; the new value by
    // wave 7.  Lane l holds elements l and l + 64 (the rotated pair).
    const bool hasq = wv < G, hask = wv == G % kDW, hasv = wv == kDW - 1;
    const uint32_t qo = (g * G + wv) * 128 + lane, ko = c.qd + g * 128 + lane, vo = c.qd + c.kvd + g * 128 + lane;
    QH_MARK(1, 0);
    bool ab = false;
    float qkv[6];
    {
        const uint32_t idx[6] = {qo, qo + 64, ko, ko + 64, vo, vo + 64};
        poll_words<6>(A, A.tqkv, idx, (hasq ? 3u : 0u) | (hask ? 12u : 0u) | (hasv ? 48u : 0u), tag_in, qkv, ab);
    }
    const float qa = qkv[0], qb = qkv[1], ka = qkv[2], kb = qkv[3], va = qkv[4], vb = qkv[5];
    QH_MARK(1, 1);
    float* qs = S.big;               // [8][160]  normalised, rotated queries (16-dim parts padded to 20)
    float* kn = qs + 8 * 160;        // [160]     new key, same layout
    float* vn = kn + 160;            // [128]     new value
    float* vs = vn + 128;            // [64][kTP] value tile
    float* ps = vs + kDTile * kTP;   // [8][kPP]  scores, then probabilities
    float* al = ps + 8 * kPP;        // [8]       rescale factor of each head for this tile
    float* ot = al + 8;              // [8][128]  output of the chunk
    // Q/K RMSNorm (model.rs:233-238) + NeoX RoPE (ops.rs:17-28)
    auto norm_rope = [&](float xa, float xb, float w0, float w1, float* dst, bool append) {
        const float ssq = wave_sum(fmaf(xb, xb, xa * xa));
        const float sc = 1.0f / sqrtf(ssq / 128.0f + dm.eps);
        const float y0 = xa * (sc * w0), y1 = xb * (sc * w1);
        float o0, o1;
        {
#pragma clang fp contract(off)
            o0 = y0 * cs.x - y1 * cs.y;
            o1 = y0 * cs.y + y1 * cs.x;
        }
        dst[(lane / 16) * 20 + lane % 16] = o0;
        dst[((lane + 64) / 16) * 20 + lane % 16] = o1;
        if (append) {  // KV append (model.rs:241-243)
            L.kcache[((size_t)g * ctx + pos) * 128 + lane] = o0;
            L.kcache[((size_t)g * ctx + pos) * 128 + lane + 64] = o1;
        }
    };
    if (hasq) norm_rope(qa, qb, P.qw0, P.qw1, qs + wv * 160, false);
    if (hask) norm_rope(ka, kb, P.kw0, P.kw1, kn, holds);
    if (hasv) {
        vn[lane] = va;
        vn[lane + 64] = vb;
        if (holds) {
            L.vcache[((size_t)g * ctx + pos) * 128 + lane] = va;
            L.vcache[((size_t)g * ctx + pos) * 128 + lane + 64] = vb;
        }
    }
    if (ab) S.abort = 1;
    __syncthreads();
    if (S.abort) return false;
    QH_MARK(1, 4);
    const float root = sqrtf(128.0f);
    const uint32_t part = tid & 7, kt = tid >> 3, j4 = lane & 31, grp = lane >> 4, col = lane & 15;
    float mh = -INFINITY, lh = 0.f;     // softmax state of head wv
    f4v oacc = {0.f, 0.f, 0.f, 0.f};    // O[head 4 grp + i][dim 16 wv + col]
    for (uint32_t tt = t0; tt < t1; tt += kDTile) {
        const uint32_t nt = min(kDTile, t1 - tt);
        if (tt + kt == pos) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = reinterpret_cast<const float4*>(kn + part * 20)[i];
                vr[i] = reinterpret_cast<const float4*>(vn + part * 16)[i];
            }
        }
        // scores: thread (key kt, 16-dim part) holds its K slice in registers;
        // the 8 parts of each head reduce on DPP
        // (heads past G read head G - 1 and are dropped: no branch between the
        // q reads, so they are issued together)
        float mine = 0.f;
#pragma unroll
        for (uint32_t h = 0; h < 8; h++) {
            float acc = 0.f;
            {
                const float4* q4 = reinterpret_cast<const float4*>(qs + min(h, G - 1) * 160 + part * 20);
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
        {
            // the value tile; keys beyond nt as zero rows (probability 0, and a
            // zero row keeps P V finite)
            const bool in = kt < nt;
#pragma unroll
            for (int i = 0; i < 4; i++)
                reinterpret_cast<float4*>(vs + kt * kTP + part * 16)[i] = in ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (in && part < G) ps[part * kPP + kt] = mine / root;
        }
        if (tt + kDTile < t1) kv_slice(kr, vr, L.kcache, L.vcache, g, ctx, tt + kDTile, t1, pos, tid);
        QH_MARK(1, 5);
        __syncthreads();
        QH_MARK(1, 6);
        if (wv < G) {  // wave-uniform: online softmax of head wv
            const float sv = lane < nt ? ps[wv * kPP + lane] : -INFINITY;
            const float M = fmaxf(mh, wave_max(sv));
            const float e = lane < nt ? expf(sv - M) : 0.f;
            const float alpha = expf(mh - M);  // 0 on the first tile
            lh = fmaf(lh, alpha, wave_sum(e));
            mh = M;
            ps[wv * kPP + lane] = e;
            if (lane == 0) al[wv] = alpha;
        }
        QH_MARK(1, 7);
        __syncthreads();
        // O[h][d] = alpha_h O[h][d] + sum_key P[h][key] V[key][d]: M = heads,
        // N = 16 dims per wave, K = 64 keys
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) oacc[i] *= 4 * grp + i < G ? al[4 * grp + i] : 0.f;
#pragma unroll 8
        for (uint32_t k4 = 0; k4 < kDTile / 4; k4++) {
            const uint32_t key = 4 * k4 + grp;
            const float pa = col < G ? ps[col * kPP + key] : 0.f;
            const float vb = vs[key * kTP + 16 * wv + col];
            oacc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vb, oacc, 0, 0, 0);
        }
        __syncthreads();
    }
    QH_MARK(1, 2);
    // O to LDS as [head][128], then lane (head wv, dims 4 j4)
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
        if (4 * grp + i < G) ot[(4 * grp + i) * 128 + 16 * wv + col] = oacc[i];
    __syncthreads();
    const float4 o4 = wv < G ? reinterpret_cast<const float4*>(ot + wv * 128)[j4] : make_float4(0.f, 0.f, 0.f, 0.f);
    const uint32_t kh = lane >> 5;
    const uint32_t mc = A.max_chunks;
    if (ch > 0) {  // pass the partial on to chunk 0: lane writes dims lane, lane + 64
        if (wv < G) {
            uint64_t* dst = A.tpart + ((size_t)(g * G + wv) * mc + ch) * kPartWords;
            put(dst + lane, ot[wv * 128 + lane], tag);
            put(dst + 64 + lane, ot[wv * 128 + 64 + lane], tag);
            if (lane < 2) put(dst + 128 + lane, lane == 0 ? mh : lh, tag);
        }
        QH_MARK(2, 6);
        return true;
    }
    if (wv < G) {  // wave-uniform
        // O = sum_c o_c exp(m_c - M) / L,  L = sum_c l_c exp(m_c - M); half kh
        // takes chunks kh + 2i (chunk 0 from registers), 8 per round of loads
        float M = kh == 0 ? mh : -INFINITY, Ls = kh == 0 ? lh : 0.f;
        float4 O = kh == 0 ? o4 : make_float4(0.f, 0.f, 0.f, 0.f);
        const uint64_t* hb = A.tpart + (size_t)(g * G + wv) * mc * kPartWords;
        const __amdgpu_buffer_rsrc_t pr = buf_rsrc(hb, mc * kPartWords * 8);
        for (uint32_t cb = kh; cb < nch; cb += 16) {
            uint32_t word[24], need = 0;
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) {
                const uint32_t cc = cb + 2 * k;
                word[3 * k] = cc * kPartWords + 128;  // m, l
                word[3 * k + 1] = cc * kPartWords + 4 * j4;
                word[3 * k + 2] = cc * kPartWords + 4 * j4 + 2;
                if (cc > 0 && cc < nch) need |= 7u << (3 * k);
            }
            float v[48];
            poll_pairs<24>(A, pr, word, need, need, tag, v, ab);
            QH_MARK(2, 5);
            if (ab) break;
            float Mn = M;
#pragma unroll
            for (uint32_t k = 0; k < 8; k++)
                if (cb + 2 * k > 0 && cb + 2 * k < nch) Mn = fmaxf(Mn, v[6 * k]);
            const float f = expf(M - Mn);  // 0 while M = -inf
            Ls *= f;
            O.x *= f;
            O.y *= f;
            O.z *= f;
            O.w *= f;
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) {
                if (cb + 2 * k > 0 && cb + 2 * k < nch) {
                    const float e = expf(v[6 * k] - Mn);
                    Ls = fmaf(v[6 * k + 1], e, Ls);
                    O.x = fmaf(v[6 * k + 2], e, O.x);
                    O.y = fmaf(v[6 * k + 3], e, O.y);
                    O.z = fmaf(v[6 * k + 4], e, O.z);
                    O.w = fmaf(v[6 * k + 5], e, O.w);
                }
            }
            M = Mn;
        }
        // the two halves (a half without chunks has M = -inf and adds 0)
        const float Mo = shfl32(M), Lo = shfl32(Ls);
        const float4 Oo = make_float4(shfl32(O.x), shfl32(O.y), shfl32(O.z), shfl32(O.w));
        if (kh == 0) {  // back into this wave's own row of ot (read above by this wave only)
            const float Mn = fmaxf(M, Mo);
            const float f0 = expf(M - Mn), f1 = expf(Mo - Mn);
            const float inv = 1.0f / fmaf(Ls, f0, Lo * f1);
            reinterpret_cast<float4*>(ot + wv * 128)[j4] =
                make_float4(fmaf(O.x, f0, Oo.x * f1) * inv, fmaf(O.y, f0, Oo.y * f1) * inv,
                            fmaf(O.z, f0, Oo.z * f1) * inv, fmaf(O.w, f0, Oo.w * f1) * inv);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // each store instruction writes 64 consecutive words (whole lines)
        uint64_t* out = A.tatt + (g * G + wv) * 128;
        put(out + lane, ot[wv * 128 + lane], tag);
        put(out + 64 + lane, ot[wv * 128 + 64 + lane], tag);
    }
    if (ab) S.abort = 1;
    QH_MARK(1, 3);
    __syncthreads();
    return S.abort == 0;
}

// ======================================================== C: o-projection ==
// Wave wv owns row r0 + wv (qd <= 4096 columns: chunks lane, lane + 64).
template <uint32_t KO>
__device__ __forceinline__ bool phase_oproj(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                            uint32_t l) {
    const Ctx c = fresh(c0);
    const uint32_t ocpr = c.qd / 32;
    // chunks lane and lane + 64 of the row, loaded unconditionally (row and
    // chunks clamped, results of clamped ones dropped)
    const bool rowok = c.wv < c.nr;
    const uint8_t* orow = L.o.w + (size_t)min(c.r0 + c.wv, c.H - 1) * L.o.drb;
    const uint32_t ch0 = min(c.lane, ocpr - 1), ch1 = min(c.lane + 64, ocpr - 1);
    const typename Fmt<KO>::Raw w0 = Fmt<KO>::load(orow, L.o.geo, ch0), w1 = Fmt<KO>::load(orow, L.o.geo, ch1);
    // router workgroup e: row e of the fold, elements 8 tid .. 8 tid + 7
    uint32_t re;
    const bool rt = router_wg(A, c, re);
    float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
    if (rt && 8 * c.tid < c.qd) {
        const float* fr = L.rfold + (size_t)re * c.qd + 8 * c.tid;
        f0 = gld<float4>(fr);
        f1 = gld<float4>(fr + 4);
    }
    QH_MARK(2, 0);
    float* xs = S.big;
    if (!gather_s(A, S, A.tatt, c.qd, ptag(A, l, 2), xs, c.tid, c.qd / 128, 127, 128))
        return false;  // attention output (phase B)
    QH_MARK(2, 1);
    if (rowok) {  // wave-uniform
        // both chunks' x runs read before either dot (no branch between them)
        float xa[16], xb[16], sa, sb, ya[16], yb[16], ta, tb;
        x_runs_p<KO>(xs, 0, ch0, xa, xb, sa, sb);
        x_runs_p<KO>(xs, 0, ch1, ya, yb, ta, tb);
        const float d0 = Fmt<KO>::dot(w0, ch0, xa, xb, sa, sb), d1 = Fmt<KO>::dot(w1, ch1, ya, yb, ta, tb);
        float acc = c.lane < ocpr ? d0 : 0.f;
        if (c.lane + 64 < ocpr) acc += d1;
        acc = wave_sum(acc);
        if (c.lane == 0) S.xo[c.wv] += acc;  // residual (model.rs:246-248)
    }
    if (rt) {  // workgroup-uniform
        float fd = 0.f;
        if (8 * c.tid < c.qd) {
            const float4 a0 = *reinterpret_cast<const float4*>(xs + px(8 * c.tid));
            const float4 a1 = *reinterpret_cast<const float4*>(xs + px(8 * c.tid + 4));
            fd = fmaf(f0.w, a0.w, fmaf(f0.z, a0.z, fmaf(f0.y, a0.y, f0.x * a0.x)));
            fd = fmaf(f1.w, a1.w, fmaf(f1.z, a1.z, fmaf(f1.y, a1.y, fmaf(f1.x, a1.x, fd))));
        }
        fd = wave_sum(fd);
        if (c.lane == 0) S.red[c.wv] = fd;
    }
    QH_MARK(2, 2);
    __syncthreads();
    if (c.tid < c.nr) put(A.tx1 + c.r0 + c.tid, S.xo[c.tid], ptag(A, l, 3));  // one store instruction
    if (rt && c.tid == 64) {
        // unscaled router logit e of x' (model.rs:249-256 with the RMS scale left out)
        float u = S.ra;
#pragma unroll
        for (uint32_t w = 0; w < kDW; w++) u += S.red[w];
        put(A.tx1 + c.H + re, u, ptag(A, l, 3));
    }
    return true;
}

// ============================================ D-F: routing, routed expert FFN ==
// Gathers x' and the unscaled router logits u (phase C); the ffn RMSNorm
// scale s = 1/sqrt(mean(x'^2) + eps) (ops.rs:3-15) gives logit e = s u_e.
template <uint32_t KG, uint32_t KD>
__device__ __forceinline__ bool phase_moe(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          uint32_t l, bool last) {
    const Ctx c = fresh(c0);
    const Acts& a = A.a;
    const uint32_t E = c.E, top = c.top, ff = c.ff, H = c.H, cpr = H / 32;
    float4 fn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < H) fn = gld<float4>(L.ffn_norm + 4 * c.tid);
    QH_MARK(4, 0);
    float* xs = S.big;
    if (!gather_s(A, S, A.tx1, H + E, ptag(A, l, 3), xs, c.tid, c.nwg, 0, c.rpw))
        return false;  // x' and u (phase C)
    float4 x1 = make_float4(0.f, 0.f, 0.f, 0.f);
    float* x4 = xs + px(4 * c.tid);
    if (4 * c.tid < H) x1 = *reinterpret_cast<const float4*>(x4);
    const float s = 1.0f / sqrtf(dsum(sumsq4(x1), S.red) / (float)H + A.dm.eps);
    if (c.tid < E) S.lg[c.tid] = s * xs[px(H + c.tid)];  // router logits (model.rs:249-256)
    // xn = x' * (s * ffn_norm), in place (each thread rewrites its own float4;
    // the routing barriers below order it before the dots)
    if (4 * c.tid < H) {
        x4[0] = x1.x * (s * fn.x);
        x4[1] = x1.y * (s * fn.y);
        x4[2] = x1.z * (s * fn.z);
        x4[3] = x1.w * (s * fn.w);
    }
    QH_MARK(4, 1);
    // top-k by rank under the total order, lower index on ties (ops.rs:45-56;
    // bit-exact on these logits): j outranks i iff ck[j] > ck[i], with the
    // composite key ck = (total-order key of the logit, ~index); experts
    // E..127 get the smallest key and outrank nothing (E <= 128)
    if (c.tid < 128) {
        const float lv = c.tid < E ? S.lg[c.tid] : 0.f;
        if (!finite_f(lv)) S.bad = 1;
        S.ck[c.tid] = c.tid < E ? (long long)(((uint64_t)(uint32_t)total_key(lv) << 32) | (uint32_t)~c.tid)
                                : LLONG_MIN;
    }
    __syncthreads();
    if (S.bad) {
        if (c.b == 0 && c.tid == 0) atomicOr(&a.st->err, kErrRouter);
        return false;  // every workgroup sees the same logits
    }
    {
        // thread (i, q) counts the keys of quarter q (32 of them) above expert i's
        const uint32_t i = c.tid >> 2, q = c.tid & 3;
        const long long ki = S.ck[i];
        int32_t rank = 0;
#pragma unroll
        for (uint32_t j = 32 * q; j < 32 * q + 32; j += 2) {
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
    // softmax over the selected logits (ops.rs:29-44), in every wave, lane k =
    // rank k; wave 0 keeps the result in LDS for phase F
    {
        const float v = c.lane < top ? S.sv[c.lane] : -INFINITY;
        const float mx = wave_max(v);
        const float e = c.lane < top ? expf(v - mx) : 0.f;
        const float w = e / wave_sum(e);
        if (c.wv == 0 && c.lane < top) {
            S.ids[c.lane] = S.sid[c.lane];
            S.wts[c.lane] = w;
        }
    }
    QH_MARK(4, 2);
    // gate/up rows of pairs p = gw*3 + k: (slot p / ff, row p % ff); the
    // loads are unconditional (pair and chunk clamped, results of clamped
    // pairs dropped) so that each pair's dots wait only for that pair
    typename Fmt<KG>::Raw wg[kPairsPerWave], wu[kPairsPerWave];
    const uint32_t gch = min(c.lane, cpr - 1);
#pragma unroll
    for (uint32_t k = 0; k < kPairsPerWave; k++) {
        const uint32_t pr = min(c.gw * kPairsPerWave + k, top * ff - 1);
        const uint32_t ex = S.sid[pr / ff], rr = pr % ff;
        wg[k] = Fmt<KG>::load(L.gate.w + (size_t)ex * L.gate.expert_stride + (size_t)rr * L.gate.drb, L.gate.geo, gch);
        wu[k] = Fmt<KG>::load(L.up.w + (size_t)ex * L.up.expert_stride + (size_t)rr * L.up.drb, L.up.geo, gch);
    }
    QH_MARK(4, 4);
    const uint32_t tag_h = ptag(A, l, 5);
    {
        float xa[16], xb[16], sa, sb;
        if (c.lane < cpr) x_runs_p<KG>(xs, 0, c.lane, xa, xb, sa, sb);
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
                    S.hv[c.wv * kPairsPerWave + k] = (gv / (1.f + expf(-gv))) * uv;  // SwiGLU (model.rs:272)
                }
            }
        }
    }
    QH_MARK_LAST(4, 5);
    __syncthreads();  // S.hv complete; every wave is done with xn, which the gather overwrites
    {
        // this workgroup's outputs [slot][ff] flat at b * kHBlock, one store instruction
        const uint32_t i = c.b * kHBlock + c.tid;
        if (c.tid < kHBlock && i < top * ff) put(A.th + i, S.hv[c.tid], tag_h);
    }
    // down rows of phase F (row r0 + wv of each routed expert), requested
    // before the wait for the SwiGLU outputs, so that they arrive during the
    // hand-over (issued with the gate/up rows they slowed those down): lane
    // units u = lane + 64 i = (slot u / dcpr, chunk u % dcpr).  Unconditional,
    // in straight-line code (row and unit clamped, results of clamped units
    // dropped): loads issued under a branch made the compiler wait for each
    // unit's loads before issuing the next, one memory round trip per unit.
    const uint32_t dcpr = ff / 32, U = top * dcpr;
    const uint8_t* dbase = L.down.w + (size_t)min(c.r0 + c.wv, H - 1) * L.down.drb;
    typename Fmt<KD>::Raw wd[kDownUnits];
#pragma unroll
    for (uint32_t i = 0; i < kDownUnits; i++) {
        const uint32_t u = min(c.lane + 64 * i, U - 1);
        wd[i] = Fmt<KD>::load(dbase + (size_t)S.sid[u / dcpr] * L.down.expert_stride, L.down.geo, u % dcpr);
    }
    QH_MARK(4, 3);
    // ================================================ F: down + combine
    QH_MARK(5, 0);
    if (!gather_s(A, S, A.th, top * ff, tag_h, xs, c.tid, (top * ff + kHBlock - 1) / kHBlock, 0, kHBlock))
        return false;  // SwiGLU outputs (phase E)
    QH_MARK(5, 1);
    if (c.wv < c.nr) {  // wave-uniform
        // every unit computed (clamped ones dropped by the select), so that the
        // x runs of all units are read without a branch between them
        float acc = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < kDownUnits; i++) {
            const uint32_t u = min(c.lane + 64 * i, U - 1), sl = u / dcpr, chn = u % dcpr;
            float xa[16], xb[16], sa, sb;
            x_runs_p<KD>(xs, sl * ff, chn, xa, xb, sa, sb);
            const float d = fmaf(S.wts[sl], Fmt<KD>::dot(wd[i], chn, xa, xb, sa, sb), acc);
            acc = c.lane + 64 * i < U ? d : acc;
        }
        acc = wave_sum(acc);
        if (c.lane == 0) S.xo[c.wv] += acc;  // x += sum_s w_s down_s (model.rs:281-287)
    }
    QH_MARK_LAST(5, 2);
    __syncthreads();
    if (c.tid < c.nr) {
        put(A.tx2 + c.r0 + c.tid, S.xo[c.tid], ptag(A, l, 6));  // one store instruction
        if (last) a.x[c.r0 + c.tid] = S.xo[c.tid];            // x after the launch, for the host
    }
    // the routing of the layer, for the host (stored last: a later use of a
    // store's registers waits for the store, and these wait for nothing else)
    if (c.b == 0) {
        if (c.tid < top) {
            a.ids[c.tid] = S.ids[c.tid];
            a.wts[c.tid] = S.wts[c.tid];
        }
        if (c.tid < E) a.logits_r[c.tid] = S.lg[c.tid];
    }
    return true;
}

// =========================================================== V: vocab ==
template <uint32_t KV>
__device__ __forceinline__ void phase_vocab(const DecodeArgs& A, DecodeLds& S, const Ctx& c0) {
    const Ctx c = fresh(c0);
    const Acts& a = A.a;
    const DevMat& mv = A.out;
    const uint32_t V = A.dm.vocab, ngrp = (V + kVocabRows - 1) / kVocabRows, cpr = c.H / 32;
    const uint32_t tag = A.base + 6 * (A.l1 - A.l0) + 1;
    using Raw = typename Fmt<KV>::Raw;
    // unconditional loads (row and chunk clamped into the matrix; results of
    // clamped rows are dropped): the compiler then waits for exactly the group
    // it computes, not for the prefetched one behind it
    const uint32_t ch = min(c.lane, cpr - 1);
    auto load_group = [&](Raw (&t)[kVocabRows], uint32_t gi) {
#pragma unroll
        for (uint32_t k = 0; k < kVocabRows; k++) {
            const uint32_t r = min(gi * kVocabRows + k, V - 1);
            t[k] = Fmt<KV>::load(mv.w + (size_t)r * mv.drb, mv.geo, ch);
        }
    };
    // the workgroup's groups [g0, g1): the first kDW to its waves in turn, the
    // rest to whichever wave asks first (LDS counter), so that a wave whose
    // rows arrive late does not hold the workgroup's argmax partial back
    const uint32_t per = (ngrp + c.nwg - 1) / c.nwg;
    const uint32_t g0 = min(c.b * per, ngrp), g1 = min(g0 + per, ngrp);
    if (c.tid == 0) S.vq = g0 + kDW;  // ordered before use by the gather's barriers
    uint32_t gi = g0 + c.wv;
    Raw cur[kVocabRows], nxt[kVocabRows];
    load_group(cur, min(gi, ngrp - 1));
    // read now, used by workgroup 0 after the argmax hand-over
    const uint32_t n_given = a.st->n_given;
    float4 on = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * c.tid < c.H) on = gld<float4>(A.onorm + 4 * c.tid);
    QH_MARK(6, 0);
    float* xs = S.big;
    if (!gather_s(A, S, A.tx2, c.H, ptag(A, A.l1 - 1, 6), xs, c.tid, c.nwg, 0, c.rpw))
        return;  // x after the last layer
    QH_MARK(6, 1);
    norm_in_lds(c, xs, on, A.dm.eps, S.red);
    float xa[16], xb[16], sa, sb;
    if (c.lane < cpr) x_runs_p<KV>(xs, 0, c.lane, xa, xb, sa, sb);
    int32_t bk = INT32_MIN;
    uint32_t bi = 0xffffffffu;
    bool nf = false;
    while (gi < g1) {  // wave-uniform
        uint32_t gn = 0;
        if (c.lane == 0) gn = atomicAdd(&S.vq, 1u);
        gn = __builtin_amdgcn_readfirstlane(gn);
        load_group(nxt, min(gn, ngrp - 1));
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
        gi = gn;
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
        put(A.tfin + 2 * c.b, __int_as_float(k0), tag);
        put(A.tfin + 2 * c.b + 1, __uint_as_float(i0), tag);
        if (S.bad) atomicOr(&a.st->err, kErrLogits);
    }
    QH_MARK(6, 4);
    if (c.b != 0) return;
    // workgroup 0: argmax over every workgroup's partial
    float* fin = S.big + 4096;  // clear of the padded x (px(2047) = 2171)
    if (!gather(A, S, A.tfin, 2 * c.nwg, tag, fin, c.tid)) return;
    QH_MARK(6, 5);
    int32_t k1 = INT32_MIN;
    uint32_t i1 = 0xffffffffu;
    if (c.tid < c.nwg) {
        k1 = __float_as_int(fin[2 * c.tid]);
        i1 = __float_as_uint(fin[2 * c.tid + 1]);
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
        if (c.pos + 1 >= n_given && c.pos + 1 <= A.dm.ctx) a.tokens[c.pos + 1] = i0;
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
    c.top = dm.top;
    c.ff = dm.ff;
    c.G = dm.heads / dm.kvheads;
    c.qd = dm.heads * 128;
    c.kvd = dm.kvheads * 128;
    c.ctx = dm.ctx;
    const uint32_t rpw = (c.H + c.nwg - 1) / c.nwg;
    c.rpw = rpw;
    c.r0 = c.b * rpw;
    c.nr = c.r0 < c.H ? min(rpw, c.H - c.r0) : 0;
    for (uint32_t l = A.l0; l < A.l1; l++) {
        // read through the constant address space: scalar loads, which do
        // not wait behind this wave's outstanding vector loads and stores
        const LayerW& L = *(const LayerW*)((const __attribute__((address_space(4))) LayerW*)A.layers + l);
        bool ok = true;
        AttnPre P;
        QH_DISPATCH_KM(L.v.kind, KV, ok = phase_qkv<Q4_K, KV>(A, S, L, c, l, P));
        if (!ok || !phase_attn(A, S, L, c, l, P)) return;
        if (!phase_oproj<Q4_K>(A, S, L, c, l)) return;
        QH_DISPATCH_KM(L.down.kind, KD, ok = phase_moe<Q4_K, KD>(A, S, L, c, l, l + 1 == A.l1));
        if (!ok) return;
    }
    if (A.vocab) QH_DISPATCH_KM(A.out.kind, KV, phase_vocab<KV>(A, S, c));
}

}  // namespace qh
