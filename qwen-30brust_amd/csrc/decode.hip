// Persistent token step (src/model.rs:222-302 and the greedy sampler,
// src/sampling.rs:26-35) as ONE launch of one 512-thread workgroup per CU,
// the embedding row of tokens[pos] (model.rs:225) included.
//
// Placement.  MI355X has 8 XCDs of 32 CUs, each XCD with its own L2, and the
// dispatcher hands workgroups to the XCDs in turn: workgroup b runs on XCD
// (b + s) % 8, where the starting XCD s carries over from earlier dispatches
// (0 for cooperative launches; checked at set-up for one launch).  Workgroup
// b is (X, j) = (its XCD, read from the hardware register, b / 8): every XCD
// then holds j = 0..31 once whatever s is.  (Were the order ever broken, some
// (X, j) would be held twice and another not at all; the waits for the
// missing one time out and the step fails with kErrSync, no value is wrong.)
// Values
// handed between the 32 workgroups of one XCD go through that XCD's L2
// (plain stores, loads that skip L1: about 0.4 us per hand-over); values that
// cross XCDs are written through to memory and read past the caches (about
// 1.6 us).  The layer is laid out so that only two of its seven hand-overs
// cross XCDs:
//
//   XCD X owns query heads 4X..4X+3, which share KV head X/2 (Qwen3-30B-A3B:
//   32 query heads, 4 KV heads), and expert rank X of the layer's top 8.
//   Every XCD holds its own copy of the residual stream x; workgroup j of
//   every XCD computes rows [64j, 64j+64) of each cross-XCD reduction.
//
// Per layer (L = inside one XCD, G = across XCDs):
//   A  RMSNorm of x; this XCD's 768 q|k|v rows (24 per workgroup); the
//      router term sum_c router[e][c] ffn_norm[c] x[c] over this XCD's
//      256 columns for experts 4j..4j+3                        -> L qkv
//   B  Q/K RMSNorm, RoPE, KV append, GQA attention of the XCD's 4 heads over
//      key chunk j (online softmax, P.V on MFMA; at most 32 chunks)
//                                                              -> L partials
//   C  merge of the chunk partials (every workgroup); o-projection partial
//      over this XCD's 512 attention columns for rows [64j, 64j+64), and the
//      router fold F[e] . a over the same columns              -> G partials
//   D  x' = x + sum over XCDs of the partials (rows of j), unscaled router
//      logits u of experts 4j..4j+3                            -> L x', u
//   E  RMS scale s of x', router logits s u, top-k (every workgroup, bit-exact
//      rank), softmax; gate/up rows 24j..24j+23 of expert rank X, SwiGLU
//                                                              -> L h
//   F  down projection of expert rank X for rows [64j, 64j+64) times its
//      routing weight                                          -> G partials
//   R  x'' = x' + sum in rank order of the 8 partials (rows of j) -> L x''
// then V: final RMSNorm, vocab projection and argmax partials (every
// workgroup a range of rows), and the argmax / next token / position advance
// by workgroup 0.
//
// Hand-over without flags or barriers: every value passed on is a 64-bit
// word (tag << 32) | bits, with tag = base + 7 (layer - l0) + phase (1..7;
// the vocab phase uses the next one; base grows by the launch's phase count,
// so tags never repeat between launches).  A reader polls exactly the words
// it needs until each carries the tag it expects.  Every wait is bounded: on
// timeout the workgroup raises the abort flag and kErrSync, and every other
// wait returns (also raising kErrSync), so the grid always drains and the
// step reports the failure.
//
// Reuse of a buffer in the next layer needs no barrier: a workgroup writes
// an L buffer of layer l+1 only after it has read x'' of layer l from every
// workgroup of its XCD, each of which had finished reading the layer-l
// contents by then; a G buffer slice of layer l+1 is written by workgroup
// (X, j) only after it has read the other phase's slice j from every
// workgroup (X', j), which those wrote after reading the layer-l contents.
//
// The kernel is instantiated per main format KM (Q4_0, Q8_0, Q4_K, Q5_K or
// Q6_K: the format of q, k, o, gate and up, as llama.cpp's mixes keep them);
// v and down are KM or Q6_K per layer (the "more bits" layers of the K-quant
// mixes), held in one register block so that one copy of each phase serves
// both; the vocab projection may be any of the five.  The host launches this
// path only for models and shapes it covers (engine.hip: persist_supported);
// everything else runs the per-phase kernels.
#include "qh_block.hpp"
#include "qh_tile.hpp"

namespace qh {

typedef float f4v __attribute__((ext_vector_type(4)));  // one MFMA accumulator tile per lane

constexpr int kDT = 512;
constexpr int kDW = kDT / 64;
constexpr uint32_t kSpinLimit = 1u << 22;   // polls before a wait gives up
constexpr uint32_t kNJ = kDecodeWgPerXcd;   // workgroups per XCD (32)
constexpr uint32_t kNX = kDecodeXcds;       // XCDs (8)
constexpr uint32_t kHX = 4;                 // query heads per XCD
constexpr uint32_t kQkvX = kDecodeQkvX;     // q|k|v rows per XCD (4 q heads + k + v of one KV head)
constexpr uint32_t kQkvWg = kQkvX / kNJ;    // 24 per workgroup, 3 per wave
constexpr uint32_t kRowsWg = 64;            // rows of x per workgroup slice (2048 / 32)
constexpr uint32_t kExpWg = 4;              // router experts per workgroup slice (128 / 32)
constexpr uint32_t kDTile = 64;             // keys per attention tile
constexpr uint32_t kMinKeys = 64;           // fewest keys per attention chunk (one tile)
constexpr uint32_t kMaxChunks = 32;         // most attention chunks per XCD (one per workgroup)
constexpr uint32_t kTP = 132;               // LDS pitch of the value tile (floats)
constexpr uint32_t kPP = 68;                // LDS pitch of the per-head scores (floats)
constexpr uint32_t kDSmem = 18560;          // floats of phase scratch (phase C: 32 chunk partials + the merged output)
constexpr uint32_t kFfWg = 24;              // gate/up rows per workgroup (768 / 32), 3 per wave
constexpr uint32_t kDownUnits = 3;          // chunks per lane in F (8 rows x 24 chunks per wave)
constexpr uint32_t kVocabRows = 4;          // vocab rows per wave group
constexpr uint32_t kGatherPairs = 5;        // word pairs in flight per thread in a gather (one round up to 5120 words)
constexpr int kAuxL = 3;                    // sc0 nt: skip L1, served by the XCD's L2
constexpr int kAuxG = 17;                   // sc0 sc1: past every cache

static_assert(kQkvWg == 24 && kQkvWg % kDW == 0, "three q|k|v rows per wave");

// A layer's v or down format: KM, or Q6_K (the host checks it is one of them).
#define QH_DISPATCH_KM(kind, KM, K, ...)                                      \
    do {                                                                      \
        if ((kind) == ::qh::Q6_K) {                                           \
            constexpr uint32_t K = ::qh::Q6_K;                                \
            __VA_ARGS__;                                                      \
        } else {                                                              \
            constexpr uint32_t K = KM;                                        \
            __VA_ARGS__;                                                      \
        }                                                                     \
    } while (0)
// The vocab projection's format: any block-quantised one.
#define QH_DISPATCH_BLOCK(kind, K, ...)                                         \
    switch (kind) {                                                             \
    case ::qh::Q4_0: { constexpr uint32_t K = ::qh::Q4_0; __VA_ARGS__; } break; \
    case ::qh::Q8_0: { constexpr uint32_t K = ::qh::Q8_0; __VA_ARGS__; } break; \
    case ::qh::Q4_K: { constexpr uint32_t K = ::qh::Q4_K; __VA_ARGS__; } break; \
    case ::qh::Q5_K: { constexpr uint32_t K = ::qh::Q5_K; __VA_ARGS__; } break; \
    default: { constexpr uint32_t K = ::qh::Q6_K; __VA_ARGS__; } break;         \
    }

// One chunk of format KM or of Q6_K in one block of registers (v and down
// rows), so that one copy of a phase serves both layer kinds.  Every put
// writes all three words whole: the two branches then store the same fields
// and the compiler keeps the box in registers (a byte copy, or stores of
// different extents, would place it in scratch memory).
template <uint32_t KM> struct ChunkBox {
    uint4 v[3];
    template <uint32_t K> __device__ __forceinline__ void put(const typename Fmt<K>::Raw& r) {
        static_assert(K == KM || K == Q6_K, "the box holds KM or Q6_K");
        if constexpr (K == Q4_K) {
            v[0] = r.q, v[1] = r.h, v[2] = make_uint4(0u, 0u, 0u, 0u);
        } else if constexpr (K == Q5_K) {
            v[0] = r.q, v[1] = r.h, v[2] = r.qh;
        } else if constexpr (K == Q6_K) {
            v[0] = r.ql, v[1] = r.qh, v[2] = make_uint4(r.s8.x, r.s8.y, r.d, 0u);
        } else if constexpr (K == Q4_0) {
            v[0] = r.q, v[1] = make_uint4(r.d, 0u, 0u, 0u), v[2] = make_uint4(0u, 0u, 0u, 0u);
        } else {
            static_assert(K == Q8_0, "block formats only");
            v[0] = r.a, v[1] = r.b, v[2] = make_uint4(r.d, 0u, 0u, 0u);
        }
    }
    template <uint32_t K> __device__ __forceinline__ typename Fmt<K>::Raw get() const {
        static_assert(K == KM || K == Q6_K, "the box holds KM or Q6_K");
        if constexpr (K == Q4_K) {
            return {v[0], v[1]};
        } else if constexpr (K == Q5_K) {
            return {v[0], v[1], v[2]};
        } else if constexpr (K == Q6_K) {
            return {v[0], v[1], make_uint2(v[2].x, v[2].y), v[2].z};
        } else if constexpr (K == Q4_0) {
            return {v[0], v[1].x};
        } else {
            return {v[0], v[1], v[2].x};
        }
    }
};

struct DecodeLds {
    float xo[kRowsWg];        // rows [64j, 64j+64) of the residual stream x (then x'')
    float x1[kRowsWg];        // the same rows of x'
    float po[kRowsWg];        // o-projection partial / weighted down partial of those rows
    float hv[kQkvWg];         // phase A rows, then the SwiGLU outputs
    float red[2 * kDW];
    float ra[kExpWg];         // router term of this XCD's columns for experts 4j..4j+3
    float lg[128];            // router logits
    alignas(16) long long ck[128];  // composite top-k keys
    float sv[8];
    float s9;                 // router logit of rank top (+inf gap when none), for the gap log
    float slast;              // smallest router logit
    uint32_t sid[8];
    float wts[8];             // routing weights of the current layer
    uint32_t ids[8];          // routed experts of the current layer
    int32_t bk[kDW];
    uint32_t bi[kDW];
    uint32_t abort;
    uint32_t bad;
    uint32_t vq;              // next vocab row group of this workgroup to hand out
    // phase scratch (x, attention tiles, h, reductions) last: the small
    // fields above stay within the 64-KB reach of an LDS instruction's offset
    alignas(16) float big[kDSmem];
};

// Per-workgroup constants of one launch.
struct Ctx {
    uint32_t b, nwg, X, j, tid, wv, lane, gw;
    uint32_t pos, T, H, E, top, ff, qd, ctx;
    uint32_t tok;  // tokens[pos]
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
__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
    return ((uint64_t)tag << 32) | __float_as_uint(v);
}
// Across XCDs: written through to memory.
__device__ __forceinline__ void put_g(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, tagged(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Inside one XCD: a plain store, which lands in the XCD's L2.
__device__ __forceinline__ void put_l(uint64_t* p, float v, uint32_t tag) {
    *(__attribute__((address_space(1))) uint64_t*)p = tagged(v, tag);
}

// Bookkeeping of one poll round: every 64th round checks the abort flag and
// the time limit (on timeout raises the abort flag).  Either way the step is
// marked failed (kErrSync).  False when the wait must stop (ab = true).
__device__ __forceinline__ bool keep_polling(const DecodeArgs& A, uint32_t& spins, bool& ab) {
    if ((++spins & 63) == 0) {
        const bool other = ld_sys_u(A.abort_flag) != 0;
        if (other || spins > kSpinLimit) {
            if (!other) st_sys_u(A.abort_flag, 1u);
            atomicOr(&A.a.st->err, kErrSync);
            ab = true;
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// Two adjacent words (16 bytes, 16-byte aligned): AUX selects the caches the
// load skips (kAuxL or kAuxG).
template <int AUX>
__device__ __forceinline__ void ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t word, uint64_t& w0, uint64_t& w1) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(word * 8), 0, AUX);
    w0 = ((uint64_t)(uint32_t)v[1] << 32) | (uint32_t)v[0];
    w1 = ((uint64_t)(uint32_t)v[3] << 32) | (uint32_t)v[2];
}

// One word (8 bytes), the caches skipped as for ld_pair.
template <int AUX>
__device__ __forceinline__ uint64_t ld_word(__amdgpu_buffer_rsrc_t r, uint32_t word) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)(word * 8), 0, AUX);
    return ((uint64_t)(uint32_t)v[1] << 32) | (uint32_t)v[0];
}

// Waits for N word pairs at once: pair k (words word[k], word[k] + 1 of r)
// is awaited when bit k of need is set, its second word only when bit k of
// hi is set too.  Every round re-reads all pairs still missing with one batch
// of loads, so a wait costs one memory round trip per round however many
// words it covers.  v[2k], v[2k + 1] receive the values.
template <int AUX, uint32_t N>
__device__ __forceinline__ void poll_pairs(const DecodeArgs& A, __amdgpu_buffer_rsrc_t r, const uint32_t (&word)[N],
                                           uint32_t need, uint32_t hi, uint32_t tag, float (&v)[2 * N], bool& ab) {
    uint32_t spins = 0;
    while (need != 0) {
        uint64_t w[2 * N];
#pragma unroll
        for (uint32_t k = 0; k < N; k++)
            if ((need >> k) & 1) ld_pair<AUX>(r, word[k], w[2 * k], w[2 * k + 1]);
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

// dst[px(i)] = value of src[i] for i < n, every word awaited with `tag`
// through the XCD's L2 (src is 16-byte aligned with room for an even number
// of words).  Starts and ends with a barrier; false when the step was
// aborted.
__device__ __forceinline__ bool gather_l(const DecodeArgs& A, DecodeLds& S, const uint64_t* src, uint32_t n,
                                         uint32_t tag, float* dst, uint32_t tid) {
    const uint32_t np = (n + 1) / 2;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(src, np * 16);
    bool ab = false;
    __syncthreads();  // every wave is done with what the previous phase kept in dst's region
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
        poll_pairs<kAuxL, kGatherPairs>(A, r, word, need, hi, tag, v, ab);
        if (ab) break;
#pragma unroll
        for (uint32_t k = 0; k < kGatherPairs; k++) {
            const uint32_t p = p0 + k * kDT, d = px(2 * p);  // a pair stays adjacent
            if (p < np) dst[d] = v[2 * k];
            if (2 * p + 1 < n) dst[d + 1] = v[2 * k + 1];
        }
    }
    if (ab) S.abort = 1;
    __syncthreads();
    return S.abort == 0;
}

// gather_l of an RMSNorm input x (n elements, n even) with its weights w:
// dst[px(i)] = x_i w_i and, with raw, raw[px(i)] = x_i; red[wave] receives the
// wave's sum of x_i^2.  The RMS scale (rms_scale, after the closing barrier)
// then multiplies what a caller computes from dst: s (W . (x w)) instead of
// W . (x (s w)), which takes the normalisation's own reduction and barrier
// out of the way between the gather and the dot products.  (Used where the
// gathered vector arrives last, x'' from across the XCDs; on x', whose
// hand-over inside the XCD is short, the same form measured slower.)
__device__ __forceinline__ bool gather_l_norm(const DecodeArgs& A, DecodeLds& S, const uint64_t* src, uint32_t n,
                                              uint32_t tag, const float* w, float* dst, float* raw, uint32_t tid) {
    const uint32_t np = n / 2;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(src, np * 16);
    bool ab = false;
    float ss = 0.f;
    __syncthreads();  // every wave is done with what the previous phase kept in dst's region
    for (uint32_t p0 = tid; p0 < np; p0 += kGatherPairs * kDT) {
        uint32_t word[kGatherPairs], need = 0;
        float2 wp[kGatherPairs];
#pragma unroll
        for (uint32_t k = 0; k < kGatherPairs; k++) {
            const uint32_t p = p0 + k * kDT;
            word[k] = 2 * p;
            if (p < np) need |= 1u << k;
            wp[k] = p < np ? gld<float2>(w + 2 * p) : make_float2(0.f, 0.f);
        }
        float v[2 * kGatherPairs];
        poll_pairs<kAuxL, kGatherPairs>(A, r, word, need, need, tag, v, ab);
        if (ab) break;
#pragma unroll
        for (uint32_t k = 0; k < kGatherPairs; k++) {
            const uint32_t p = p0 + k * kDT, d = px(2 * p);  // a pair stays adjacent
            if (p < np) {
                dst[d] = v[2 * k] * wp[k].x;
                dst[d + 1] = v[2 * k + 1] * wp[k].y;
                if (raw) {
                    raw[d] = v[2 * k];
                    raw[d + 1] = v[2 * k + 1];
                }
                ss = fmaf(v[2 * k + 1], v[2 * k + 1], fmaf(v[2 * k], v[2 * k], ss));
            }
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) S.red[tid >> 6] = ss;
    if (ab) S.abort = 1;
    __syncthreads();
    return S.abort == 0;
}

// RMSNorm scale 1/sqrt(mean(x^2) + eps) (ops.rs:3-15) from gather_l_norm's
// per-wave sums (the same order in every thread).
__device__ __forceinline__ float rms_scale(const DecodeLds& S, uint32_t n, float eps) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kDW; i++) t += S.red[i];
    return 1.0f / sqrtf(t / (float)n + eps);
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

__device__ __forceinline__ float sumsq4(float4 v) { return fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x))); }

// RMSNorm (ops.rs:3-15) of the raw x in LDS (padded layout, elements
// [0, H)), in place, with weights w (this thread's float4).  H = 2048.
__device__ __forceinline__ void norm_in_lds(const Ctx& c, float* xs, float4 w, float eps, float* red) {
    float* x4 = xs + px(4 * c.tid);
    const float4 xv = *reinterpret_cast<const float4*>(x4);
    const float scale = 1.0f / sqrtf(dsum(sumsq4(xv), red) / (float)c.H + eps);
    x4[0] = xv.x * (scale * w.x);
    x4[1] = xv.y * (scale * w.y);
    x4[2] = xv.z * (scale * w.z);
    x4[3] = xv.w * (scale * w.w);
    __syncthreads();
}

// Tag of phase k (1..kDecodePhases) of layer l.
__device__ __forceinline__ uint32_t ptag(const DecodeArgs& A, uint32_t l, uint32_t k) {
    return A.base + kDecodePhases * (l - A.l0) + k;
}

// Per-XCD and cross-XCD exchange buffers of this workgroup's XCD.
__device__ __forceinline__ uint64_t* lbuf(uint64_t* base, uint32_t stride, uint32_t X) { return base + (size_t)X * stride; }

// Chunk geometry of the attention: chunk j of T keys.  A chunk's time grows
// with its 64-key tiles (each waits for its K/V slice) and hardly with how
// many of a tile's keys are used, and fewer chunks are cheaper to merge: up to
// 16 chunks of at least one tile (T <= 2048: one or two tiles each), then up
// to 32 chunks of two tiles (T <= 4096), then 32 chunks of T/32 keys.
struct AttnChunk {
    uint32_t nch, t0, t1;
    bool active;
};
__device__ __forceinline__ AttnChunk attn_chunk(const Ctx& c) {
    AttnChunk k;
    const uint32_t tc = max((c.T + kMaxChunks - 1) / kMaxChunks, min(max((c.T + 15) / 16, kMinKeys), 2 * kDTile));
    k.nch = (c.T + tc - 1) / tc;
    k.active = c.j < k.nch;
    k.t0 = min(c.T, c.j * tc);
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
    // part p = tid % 8 holds dims 32 i + 4 p .. 32 i + 4 p + 3 (i < 4): load
    // i of the 8 parts of a key is one contiguous 128-byte run
    const uint32_t key = tt + (tid >> 3), j = (tid & 7) * 4;
    if (key < t1 && key != pos) {
        const float* ks = kc + ((size_t)g * ctx + key) * 128 + j;
        const float* vs = vc + ((size_t)g * ctx + key) * 128 + j;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = gld<float4>(ks + 32 * i);
            vr[i] = gld<float4>(vs + 32 * i);
        }
    }
}

// Issued in phase A, before the wait for x.
__device__ __forceinline__ void attn_prefetch(const DecodeArgs& A, const LayerW& L, const Ctx& c, AttnPre& P) {
    const AttnChunk k = attn_chunk(c);
    if (!k.active) return;
#pragma unroll
    for (int i = 0; i < 4; i++) P.kr[i] = P.vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    kv_slice(P.kr, P.vr, L.kcache, L.vcache, c.X / 2, c.ctx, k.t0, k.t1, c.pos, c.tid);
    P.qw0 = gld<float>(L.q_norm + c.lane);
    P.qw1 = gld<float>(L.q_norm + c.lane + 64);
    P.kw0 = gld<float>(L.k_norm + c.lane);
    P.kw1 = gld<float>(L.k_norm + c.lane + 64);
    P.cs = gld<float2>(A.a.rope + (size_t)c.pos * 64 + c.lane);
}

// ================================================================== A: qkv ==
// This XCD's rows: local row r < 512 is q row 512 X + r (heads 4X..4X+3),
// then 128 k rows and 128 v rows of KV head X/2.  Workgroup j computes local
// rows [24j, 24j+24), wave wv rows 24j + wv + 8k (k < 3); lane = chunk
// (2048 columns = 64 chunks).  The router term of experts 4j..4j+3 over
// columns [256X, 256X+256) is reduced in the same pass (waves 0-3, one
// expert each).
template <uint32_t KQ>
__device__ __forceinline__ bool phase_qkv(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          uint32_t l, AttnPre& P) {
    const Ctx c = fresh(c0);
    const uint32_t g = c.X / 2;
    // v rows are Q6_K or KQ (one register block either way): one copy of
    // the phase for both layer kinds keeps the step's code small
    const bool v6 = L.v.kind == Q6_K;
    typename Fmt<KQ>::Raw wq[3];
    ChunkBox<KQ> wvv[3];
#pragma unroll
    for (uint32_t k = 0; k < 3; k++) {
        const uint32_t r = kQkvWg * c.j + c.wv + kDW * k;  // wave-uniform, < 768
        if (r < 512) {
            wq[k] = Fmt<KQ>::load(L.q.w + (size_t)(512 * c.X + r) * L.q.drb, L.q.geo, c.lane);
        } else if (r < 640) {
            wq[k] = Fmt<KQ>::load(L.k.w + (size_t)(128 * g + r - 512) * L.k.drb, L.k.geo, c.lane);
        } else {
            const uint8_t* vrow = L.v.w + (size_t)(128 * g + r - 640) * L.v.drb;
            if (v6)
                wvv[k].template put<Q6_K>(Fmt<Q6_K>::load(vrow, L.v.geo, c.lane));
            else
                wvv[k].template put<KQ>(Fmt<KQ>::load(vrow, L.v.geo, c.lane));
        }
    }
    const float4 nw = gld<float4>(L.attn_norm + 4 * c.tid);
    // router rows of experts 4j + wv (waves 0-3), columns 256X + 4 lane
    const uint32_t rcol = 256 * c.X + 4 * c.lane, re = kExpWg * c.j + c.wv;
    float4 wr = make_float4(0.f, 0.f, 0.f, 0.f), fw = wr;
    if (c.wv < kExpWg && re < c.E) {
        wr = gld<float4>(L.router.w + (size_t)re * L.router.drb + 4 * rcol);
        fw = gld<float4>(L.ffn_norm + rcol);
    }
    attn_prefetch(A, L, c, P);
    float* xs = S.big;
    // the raw x of layers after the first (xs holds x * attn_norm there, and
    // `post` the RMS scale that multiplies the dot products); px(2047) = 2171
    float* const xraw = S.big + 2304;
    const float* xr = xs;
    float post = 1.f;
    QH_MARK(0, 0);
    if (l == A.l0) {
        if (A.embed) {
            // the embedding row of tokens[pos] (model.rs:225), bit-exact
            // decode, four elements per thread
            const uint8_t* row = A.emb.w + (size_t)c.tok * A.emb.drb;
            float4 e;
            e.x = dequant_value(row, A.emb.kind, A.emb.geo, 4 * c.tid);
            e.y = dequant_value(row, A.emb.kind, A.emb.geo, 4 * c.tid + 1);
            e.z = dequant_value(row, A.emb.kind, A.emb.geo, 4 * c.tid + 2);
            e.w = dequant_value(row, A.emb.kind, A.emb.geo, 4 * c.tid + 3);
            *reinterpret_cast<float4*>(xs + px(4 * c.tid)) = e;
        } else {
            // x as the host left it before this launch
            *reinterpret_cast<float4*>(xs + px(4 * c.tid)) = ld_sys4(buf_rsrc(A.a.x, c.H * 4), c.tid * 16);
        }
        __syncthreads();
    } else {
        if (!gather_l_norm(A, S, lbuf(A.lx2, kDecodeStrideX2, c.X), c.H, ptag(A, l - 1, 7), L.attn_norm, xs, xraw,
                           c.tid))
            return false;  // x'' of the previous layer (phase R)
        xr = xraw;
        post = rms_scale(S, c.H, A.dm.eps);
    }
    QH_MARK(0, 1);
    // raw values: this workgroup's rows of x and the router columns
    if (c.tid < kRowsWg / 4)
        *reinterpret_cast<float4*>(S.xo + 4 * c.tid) = *reinterpret_cast<const float4*>(xr + px(kRowsWg * c.j + 4 * c.tid));
    if (c.wv < kExpWg) {
        const float4 xv = *reinterpret_cast<const float4*>(xr + px(rcol));
        float rd = (wr.x * fw.x) * xv.x;
        rd = fmaf(wr.y * fw.y, xv.y, rd);
        rd = fmaf(wr.z * fw.z, xv.z, rd);
        rd = fmaf(wr.w * fw.w, xv.w, rd);
        rd = wave_sum(rd);
        if (c.lane == 0) S.ra[c.wv] = rd;
    }
    if (l == A.l0) norm_in_lds(c, xs, nw, A.dm.eps, S.red);  // in place, scale included
    float xa[16], xb[16], sa, sb;
    x_runs_p<KQ>(xs, 0, c.lane, xa, xb, sa, sb);
#pragma unroll
    for (uint32_t k = 0; k < 3; k++) {
        const uint32_t r = kQkvWg * c.j + c.wv + kDW * k;
        float acc;
        if (r < 640) {
            acc = Fmt<KQ>::dot(wq[k], c.lane, xa, xb, sa, sb);
        } else if (v6) {
            float ya[16], yb[16], ta, tb;
            x_runs_p<Q6_K>(xs, 0, c.lane, ya, yb, ta, tb);
            acc = Fmt<Q6_K>::dot(wvv[k].template get<Q6_K>(), c.lane, ya, yb, ta, tb);
        } else {
            acc = Fmt<KQ>::dot(wvv[k].template get<KQ>(), c.lane, xa, xb, sa, sb);  // the q|k rows' x runs
        }
        acc = wave_sum(acc) * post;
        if (c.lane == 0) S.hv[c.wv + kDW * k] = acc;
    }
    QH_MARK(0, 2);
    __syncthreads();  // S.hv complete; xs is reused by the next phase
    if (c.tid < kQkvWg)  // one store instruction
        put_l(lbuf(A.lqkv, kDecodeStrideQkv, c.X) + kQkvWg * c.j + c.tid, S.hv[c.tid], ptag(A, l, 1));
    return true;
}

// ============================================================ B: attention ==
// Chunk j of the keys for the XCD's 4 query heads, in 64-key tiles:
//   scores   thread (key tid/8, part p = tid%8: dims 32i+4p..32i+4p+3 for
//            i < 4) holds its K slice in registers and reduces the 8 parts
//            of each head on DPP;
//   softmax  wave h < 4 owns head h (lane = key), online over the tiles;
//   P.V      v_mfma_f32_16x16x4_f32: the heads are the M rows (4 of 16
//            used), 16 dims per wave, 4 keys per step.
// The chunk's partial (o[128] unnormalised, m, l) of each head goes to the
// XCD's partial buffer.
__device__ __forceinline__ bool phase_attn(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                           uint32_t l, AttnPre& P) {
    const Ctx c = fresh(c0);
    const ModelDims& dm = A.dm;
    const AttnChunk k = attn_chunk(c);
    if (!k.active) return true;
    QH_MARK(1, 0);
    const uint32_t t0 = k.t0, t1 = k.t1, g = c.X / 2;
    const uint32_t tid = c.tid, wv = c.wv, lane = c.lane, pos = c.pos, ctx = c.ctx;
    // the XCD with the even index appends the new key and value (both XCDs
    // of a KV head compute the same ones)
    const bool holds = t0 <= pos && pos < t1 && (c.X & 1) == 0;
    const uint32_t tag_in = ptag(A, l, 1), tag = ptag(A, l, 2);
    float4(&kr)[4] = P.kr;
    float4(&vr)[4] = P.vr;
    const float2 cs = P.cs;
    // wave w < 4: query head w; wave 4: the new key; wave 5: the new value.
    // Lane l holds elements l and l + 64 (the rotated pair).
    const bool hasq = wv < kHX, hask = wv == kHX, hasv = wv == kHX + 1;
    bool ab = false;
    float qkv[2] = {0.f, 0.f};
    if (wv <= kHX + 1) {  // wave-uniform
        const uint32_t w0 = (hasq ? 128 * wv : hask ? 512 : 640) + lane;
        const uint32_t word[2] = {w0, w0 + 64};
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(lbuf(A.lqkv, kDecodeStrideQkv, c.X), kQkvX * 8);
        uint32_t need = 3, spins = 0;
        while (need != 0) {
            uint64_t w[2];
#pragma unroll
            for (uint32_t i = 0; i < 2; i++)
                if ((need >> i) & 1) w[i] = ld_word<kAuxL>(r, word[i]);
#pragma unroll
            for (uint32_t i = 0; i < 2; i++)
                if (((need >> i) & 1) && has_tag(w[i], tag_in)) {
                    qkv[i] = __uint_as_float((uint32_t)w[i]);
                    need &= ~(1u << i);
                }
            if (need == 0 || !keep_polling(A, spins, ab)) break;
        }
    }
    QH_MARK(1, 1);
    float* qs = S.big;               // [4][160]  normalised, rotated queries (the 16 dims of a part padded to 20)
    float* kn = qs + 4 * 160;        // [160]     new key, same layout
    float* vn = kn + 160;            // [128]     new value
    float* vs = vn + 128;            // [64][kTP] value tile
    float* ps = vs + kDTile * kTP;   // [4][kPP]  scores, then probabilities
    float* al = ps + 4 * kPP;        // [4]       rescale factor of each head for this tile
    float* ot = al + 4;              // [4][128]  output of the chunk
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
        // dim d belongs to part (d / 4) % 8, float4 d / 32 of it
        const uint32_t e = ((lane >> 2) & 7) * 20 + (lane & 3);
        dst[e + 4 * (lane >> 5)] = o0;
        dst[e + 4 * ((lane + 64) >> 5)] = o1;
        if (append) {  // KV append (model.rs:241-243)
            L.kcache[((size_t)g * ctx + pos) * 128 + lane] = o0;
            L.kcache[((size_t)g * ctx + pos) * 128 + lane + 64] = o1;
        }
    };
    if (hasq) norm_rope(qkv[0], qkv[1], P.qw0, P.qw1, qs + wv * 160, false);
    if (hask) norm_rope(qkv[0], qkv[1], P.kw0, P.kw1, kn, holds);
    if (hasv) {
        vn[lane] = qkv[0];
        vn[lane + 64] = qkv[1];
        if (holds) {
            L.vcache[((size_t)g * ctx + pos) * 128 + lane] = qkv[0];
            L.vcache[((size_t)g * ctx + pos) * 128 + lane + 64] = qkv[1];
        }
    }
    if (ab) S.abort = 1;
    __syncthreads();
    if (S.abort) return false;
    QH_MARK(1, 4);
    const float root = sqrtf(128.0f);
    const uint32_t part = tid & 7, kt = tid >> 3, grp = lane >> 4, col = lane & 15;
    float mh = -INFINITY, lh = 0.f;     // softmax state of head wv
    f4v oacc = {0.f, 0.f, 0.f, 0.f};    // O[head 4 grp + i][dim 16 wv + col] (grp 0 holds the 4 heads)
    for (uint32_t tt = t0; tt < t1; tt += kDTile) {
        const uint32_t nt = min(kDTile, t1 - tt);
        if (tt + kt == pos) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = reinterpret_cast<const float4*>(kn + part * 20)[i];
                vr[i] = *reinterpret_cast<const float4*>(vn + 32 * i + 4 * part);
            }
        }
        // scores: thread (key kt, part) holds its 16 dims of K in registers;
        // the 8 parts of each head reduce on DPP
        float mine = 0.f;
#pragma unroll
        for (uint32_t h = 0; h < kHX; h++) {
            float acc = 0.f;
            {
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
        {
            // the value tile; keys beyond nt as zero rows (probability 0, and a
            // zero row keeps P V finite)
            const bool in = kt < nt;
#pragma unroll
            for (int i = 0; i < 4; i++)
                *reinterpret_cast<float4*>(vs + kt * kTP + 32 * i + 4 * part) = in ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (in && part < kHX) ps[part * kPP + kt] = mine / root;
        }
        if (tt + kDTile < t1) kv_slice(kr, vr, L.kcache, L.vcache, g, ctx, tt + kDTile, t1, pos, tid);
        __syncthreads();
        QH_MARK(1, 5);
        if (wv < kHX) {  // wave-uniform: online softmax of head wv
            const float sv = lane < nt ? ps[wv * kPP + lane] : -INFINITY;
            const float M = fmaxf(mh, wave_max(sv));
            const float e = lane < nt ? expf(sv - M) : 0.f;
            const float alpha = expf(mh - M);  // 0 on the first tile
            lh = fmaf(lh, alpha, wave_sum(e));
            mh = M;
            ps[wv * kPP + lane] = e;
            if (lane == 0) al[wv] = alpha;
        }
        __syncthreads();
        QH_MARK(1, 6);
        // O[h][d] = alpha_h O[h][d] + sum_key P[h][key] V[key][d]: M = heads,
        // N = 16 dims per wave, K = 64 keys
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) oacc[i] *= grp == 0 ? al[i] : 0.f;
#pragma unroll 8
        for (uint32_t k4 = 0; k4 < kDTile / 4; k4++) {
            const uint32_t key = 4 * k4 + grp;
            const float pa = col < kHX ? ps[col * kPP + key] : 0.f;
            const float vb = vs[key * kTP + 16 * wv + col];
            oacc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vb, oacc, 0, 0, 0);
        }
        // the next tile rewrites vs and ps; after the last one the output
        // goes to ot, a region of its own
        if (tt + kDTile < t1) __syncthreads();
    }
    QH_MARK(1, 2);
    // O to LDS as [head][128]; wave h < 4 passes head h's partial on
    if (grp == 0) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) ot[i * 128 + 16 * wv + col] = oacc[i];
    }
    __syncthreads();
    if (wv < kHX) {
        uint64_t* dst = lbuf(A.lpart, kDecodeStridePart, c.X) + (size_t)(c.j * kHX + wv) * kPartWords;
        put_l(dst + lane, ot[wv * 128 + lane], tag);
        put_l(dst + 64 + lane, ot[wv * 128 + 64 + lane], tag);
        if (lane < 2) put_l(dst + 128 + lane, lane == 0 ? mh : lh, tag);
    }
    QH_MARK(1, 3);
    return true;
}

// Brings the scalar-cache lines of one layer descriptor (576 bytes, 64-byte
// aligned: nine lines) in with one s_load_dword per line and a single wait, so
// that the layer's own descriptor loads hit the scalar cache instead of each
// waiting for a line that the weight stream of the previous token evicted.
// The outputs are early-clobber: none may share a register with the base
// address, which the later loads of the block still read.
__device__ __forceinline__ void warm_layer(const LayerW* p) {
    static_assert(sizeof(LayerW) == 576, "nine 64-byte lines");
    uint32_t d0, d1, d2, d3, d4, d5, d6, d7, d8;
    asm volatile(
        "s_load_dword %0, %9, 0x0\n"
        "s_load_dword %1, %9, 0x40\n"
        "s_load_dword %2, %9, 0x80\n"
        "s_load_dword %3, %9, 0xc0\n"
        "s_load_dword %4, %9, 0x100\n"
        "s_load_dword %5, %9, 0x140\n"
        "s_load_dword %6, %9, 0x180\n"
        "s_load_dword %7, %9, 0x1c0\n"
        "s_load_dword %8, %9, 0x200\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7), "=&s"(d8)
        : "s"(p)
        : "memory");
}

// ============================================= C: merge + o-projection ==
// Every workgroup gathers the XCD's chunk partials and merges them:
// a = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M) for the 4 heads (the
// chunk weights by wave 0, lane = (head, chunk), then thread = (head, dim)).
// Then rows [64j, 64j+64) of the o-projection restricted to this XCD's 512
// attention columns (chunks 16X..16X+15): wave wv rows 64j + 8wv + rr + 4i
// (i < 2), lane = (rr lane/16, chunk lane%16).  The router fold
// F[e] . a over the same columns for experts 4j..4j+3 (two waves each).
template <uint32_t KO>
__device__ __forceinline__ bool phase_oproj(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                            uint32_t l) {
    const Ctx c = fresh(c0);
    const uint32_t rr = c.lane >> 4, cc = c.lane & 15, ch = 16 * c.X + cc;
    typename Fmt<KO>::Raw w[2];
#pragma unroll
    for (uint32_t i = 0; i < 2; i++)
        w[i] = Fmt<KO>::load(L.o.w + (size_t)(kRowsWg * c.j + 8 * c.wv + rr + 4 * i) * L.o.drb, L.o.geo, ch);
    const uint32_t fe = min(kExpWg * c.j + (c.tid >> 7), c.E - 1), fc = 512 * c.X + 4 * (c.tid & 127);
    const float4 f = gld<float4>(L.rfold + (size_t)fe * c.qd + fc);
    // the next layer's descriptor, while this phase waits for the partials
    if (l + 1 < A.l1) warm_layer(A.layers + l + 1);
    QH_MARK(2, 0);
    float* ps = S.big;             // [nch][4][130] chunk partials (padded layout; px(32*4*130 - 1) = 17679)
    float* xs = S.big + 17920;     // [512] merged attention output (padded layout)
    static_assert(17920 >= kMaxChunks * kHX * kPartWords + kMaxChunks * kHX * kPartWords / 64 * 4 &&
                      17920 + 512 + 512 / 64 * 4 <= kDSmem,
                  "the partials and the merged output in the phase scratch");
    const uint32_t nch = attn_chunk(c).nch;
    if (!gather_l(A, S, lbuf(A.lpart, kDecodeStridePart, c.X), nch * kHX * kPartWords, ptag(A, l, 2), ps, c.tid))
        return false;  // the chunk partials (phase B)
    QH_MARK(2, 1);
    {
        // every wave computes the merge weights (lane = (head, chunk ck), and
        // chunk ck + 16 in the same lane past 16 chunks) and reads its head's
        // from its own lanes: no hand-over through LDS
        const uint32_t h = c.lane >> 4, ck = c.lane & 15, pb0 = (ck * kHX + h) * kPartWords;
        const uint32_t hw = __builtin_amdgcn_readfirstlane(c.tid >> 7), d = c.tid & 127;  // head of this wave
        float a = 0.f;
        if (nch <= 16) {  // uniform
            const bool on = ck < nch;
            const float m = on ? ps[px(pb0 + 128)] : -INFINITY;
            float M = fmaxf(m, dpp_f<kDppXor1>(m));
            M = fmaxf(M, dpp_f<kDppXor2>(M));
            M = fmaxf(M, dpp_f<kDppHalfMirror>(M));
            M = fmaxf(M, dpp_f<kDppMirror>(M));  // max over the head's 16 lanes
            const float e = on ? expf(m - M) : 0.f;
            const float Ls = seg_sum(on ? ps[px(pb0 + 129)] * e : 0.f, 16);
            const float mw = e / Ls;
            for (uint32_t k = 0; k < nch; k++)
                a = fmaf(ps[px((k * kHX + hw) * kPartWords + d)],
                         __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(mw), hw * 16 + k)), a);
        } else {
            const uint32_t pb1 = ((ck + 16) * kHX + h) * kPartWords;
            const bool on1 = ck + 16 < nch;
            const float m0 = ps[px(pb0 + 128)], m1 = on1 ? ps[px(pb1 + 128)] : -INFINITY;
            float M = fmaxf(m0, m1);
            M = fmaxf(M, dpp_f<kDppXor1>(M));
            M = fmaxf(M, dpp_f<kDppXor2>(M));
            M = fmaxf(M, dpp_f<kDppHalfMirror>(M));
            M = fmaxf(M, dpp_f<kDppMirror>(M));  // max over the head's 16 lanes
            const float e0 = expf(m0 - M), e1 = on1 ? expf(m1 - M) : 0.f;
            const float Ls = seg_sum(ps[px(pb0 + 129)] * e0 + (on1 ? ps[px(pb1 + 129)] * e1 : 0.f), 16);
            const float mw0 = e0 / Ls, mw1 = e1 / Ls;
            for (uint32_t k = 0; k < 16; k++)
                a = fmaf(ps[px((k * kHX + hw) * kPartWords + d)],
                         __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(mw0), hw * 16 + k)), a);
            for (uint32_t k = 16; k < nch; k++)
                a = fmaf(ps[px((k * kHX + hw) * kPartWords + d)],
                         __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(mw1), hw * 16 + k - 16)),
                         a);
        }
        xs[px(c.tid)] = a;
    }
    __syncthreads();
    QH_MARK(2, 2);
    {
        float xa[16], xb[16], sa, sb;
        x_runs_p<KO>(xs, 0, cc, xa, xb, sa, sb);
#pragma unroll
        for (uint32_t i = 0; i < 2; i++) {
            const float acc = seg_sum(Fmt<KO>::dot(w[i], ch, xa, xb, sa, sb), 16);
            if (cc == 0) S.po[8 * c.wv + rr + 4 * i] = acc;
        }
    }
    {
        const float4 a = *reinterpret_cast<const float4*>(xs + px(4 * (c.tid & 127)));
        float fd = f.x * a.x;
        fd = fmaf(f.y, a.y, fd);
        fd = fmaf(f.z, a.z, fd);
        fd = fmaf(f.w, a.w, fd);
        fd = wave_sum(fd);
        if (c.lane == 0) S.red[c.wv] = fd;
    }
    __syncthreads();
    uint64_t* dst = lbuf(A.g1, kDecodeStrideG1, c.X);
    if (c.tid < kRowsWg) put_g(dst + kRowsWg * c.j + c.tid, S.po[c.tid], ptag(A, l, 3));  // one store instruction
    if (c.tid >= 64 && c.tid < 64 + kExpWg) {
        const uint32_t e = c.tid - 64;
        put_g(dst + c.H + kExpWg * c.j + e, S.ra[e] + (S.red[2 * e] + S.red[2 * e + 1]), ptag(A, l, 3));
    }
    return true;
}

// ======================================================== D: x' reduction ==
// Rows [64j, 64j+64) of x' = x + (p_0 + ... + p_7) and the unscaled router
// logits of experts 4j..4j+3 (sum of the XCDs' terms), from slice j of every
// XCD's partials; passed on to the XCD.
__device__ __forceinline__ bool phase_xr1(const DecodeArgs& A, DecodeLds& S, const Ctx& c0, uint32_t l) {
    const Ctx c = fresh(c0);
    constexpr uint32_t kPairsX = kRowsWg / 2 + kExpWg / 2;  // 34 pairs per XCD
    float* vals = S.big;  // [8][68]
    bool ab = false;
    if (c.tid < kNX * kPairsX) {
        const uint32_t k = c.tid / kPairsX, p = c.tid % kPairsX;
        const uint32_t w = p < kRowsWg / 2 ? kRowsWg * c.j + 2 * p : c.H + kExpWg * c.j + 2 * (p - kRowsWg / 2);
        const uint32_t word[1] = {k * kDecodeStrideG1 + w};
        float v[2];
        poll_pairs<kAuxG, 1>(A, buf_rsrc(A.g1, kNX * kDecodeStrideG1 * 8), word, 1u, 1u, ptag(A, l, 3), v, ab);
        vals[k * 68 + 2 * p] = v[0];
        vals[k * 68 + 2 * p + 1] = v[1];
    }
    if (ab) S.abort = 1;
    __syncthreads();
    if (S.abort) return false;
    QH_MARK(7, 0);
    uint64_t* dst = lbuf(A.lx1, kDecodeStrideX1, c.X);
    if (c.tid < kRowsWg + kExpWg) {
        float s = vals[c.tid];
#pragma unroll
        for (uint32_t k = 1; k < kNX; k++) s += vals[k * 68 + c.tid];
        if (c.tid < kRowsWg) {
            const float x1 = S.xo[c.tid] + s;  // residual (model.rs:246-248)
            S.x1[c.tid] = x1;
            put_l(dst + kRowsWg * c.j + c.tid, x1, ptag(A, l, 4));
        } else {
            put_l(dst + c.H + kExpWg * c.j + (c.tid - kRowsWg), s, ptag(A, l, 4));
        }
    }
    return true;
}

// The down rows of phase F, requested at the end of phase E by each wave as
// soon as its own gate/up dots are done (the expert is known and this wave's
// gate/up rows have arrived): KM or Q6_K chunks (one copy of phase E for both
// layer kinds).
template <uint32_t KM> struct DownPre {
    ChunkBox<KM> wd[kDownUnits];
};

// v (64-bit) of lane l of the wave, into scalar registers.
__device__ __forceinline__ long long readlane64(long long v, uint32_t l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
    return (long long)(((uint64_t)hi << 32) | lo);
}

// ============================================ E: routing, gate/up, SwiGLU ==
// Gathers x' and the unscaled router logits u; the ffn RMSNorm scale
// s = 1/sqrt(mean(x'^2) + eps) (ops.rs:3-15) gives logit e = s u_e.  Then
// the top-k in every workgroup, and this XCD's expert (rank X): gate/up rows
// 24j + 3wv + k (k < 3), lane = chunk.
template <uint32_t KG>
__device__ __forceinline__ bool phase_moe(const DecodeArgs& A, DecodeLds& S, const LayerW& L, const Ctx& c0,
                                          uint32_t l, DownPre<KG>& D) {
    const Ctx c = fresh(c0);
    const uint32_t E = c.E, top = c.top, H = c.H;
    const float4 fn = gld<float4>(L.ffn_norm + 4 * c.tid);
    QH_MARK(4, 0);
    float* xs = S.big;
    if (!gather_l(A, S, lbuf(A.lx1, kDecodeStrideX1, c.X), H + E, ptag(A, l, 4), xs, c.tid))
        return false;  // x' and u (phase D)
    float* x4 = xs + px(4 * c.tid);
    const float4 x1 = *reinterpret_cast<const float4*>(x4);
    const float s = 1.0f / sqrtf(dsum(sumsq4(x1), S.red) / (float)H + A.dm.eps);
    if (c.tid < E) S.lg[c.tid] = s * xs[px(H + c.tid)];  // router logits (model.rs:249-256)
    // xn = x' * (s * ffn_norm), in place (each thread rewrites its own float4;
    // the routing barriers below order it before the dots)
    x4[0] = x1.x * (s * fn.x);
    x4[1] = x1.y * (s * fn.y);
    x4[2] = x1.z * (s * fn.z);
    x4[3] = x1.w * (s * fn.w);
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
    if (c.tid == 0) S.s9 = -INFINITY;  // stays when every expert is routed
    __syncthreads();
    QH_MARK(4, 4);
    if (S.bad) {
        if (c.b == 0 && c.tid == 0) atomicOr(&A.a.st->err, kErrRouter);
        return false;  // every workgroup sees the same logits
    }
    {
        static_assert(kDW * 16 == 128, "eight waves rank 16 experts each");
        // wave wv ranks experts 16 wv .. 16 wv + 15: each lane holds keys lane
        // and lane + 64; expert i's key is read from its lane into scalar
        // registers, and its rank is the number of set bits of two ballots
        // "key above expert i's" (two LDS reads per lane, no LDS round trip
        // per expert); lane t < 16 then places expert 16 wv + t
        const long long k0 = S.ck[c.lane], k1 = S.ck[c.lane + 64];
        const long long kw = c.wv < kDW / 2 ? k0 : k1;  // keys 16 wv .. 16 wv + 15 sit in lanes 16 (wv % 4) + t
        uint32_t mine = 0;
#pragma unroll
        for (uint32_t t = 0; t < 16; t++) {
            const long long ki = readlane64(kw, 16 * (c.wv & 3) + t);
            const uint32_t rank = (uint32_t)(__popcll(__ballot(k0 > ki)) + __popcll(__ballot(k1 > ki)));
            mine = c.lane == t ? rank : mine;
        }
        const uint32_t i = 16 * c.wv + c.lane;
        if (c.lane < 16 && i < E && mine < top) {
            S.sid[mine] = i;
            S.sv[mine] = S.lg[i];
        }
        if (c.lane < 16 && i < E && mine == top) S.s9 = S.lg[i];
        if (c.lane < 16 && i < E && mine == E - 1) S.slast = S.lg[i];
    }
    __syncthreads();
    QH_MARK(4, 5);
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
    const uint32_t ex = S.sid[c.X];
    typename Fmt<KG>::Raw wg[3], wu[3];
#pragma unroll
    for (uint32_t k = 0; k < 3; k++) {
        const uint32_t rr = kFfWg * c.j + 3 * c.wv + k;
        wg[k] = Fmt<KG>::load(L.gate.w + (size_t)ex * L.gate.expert_stride + (size_t)rr * L.gate.drb, L.gate.geo, c.lane);
        wu[k] = Fmt<KG>::load(L.up.w + (size_t)ex * L.up.expert_stride + (size_t)rr * L.up.drb, L.up.geo, c.lane);
    }
    {
        float xa[16], xb[16], sa, sb;
        x_runs_p<KG>(xs, 0, c.lane, xa, xb, sa, sb);
#pragma unroll
        for (uint32_t k = 0; k < 3; k++) {
            float gv = Fmt<KG>::dot(wg[k], c.lane, xa, xb, sa, sb);
            float uv = Fmt<KG>::dot(wu[k], c.lane, xa, xb, sa, sb);
            gv = wave_sum(gv);
            uv = wave_sum(uv);
            if (c.lane == 0) {
#pragma clang fp contract(off)
                S.hv[3 * c.wv + k] = (gv / (1.f + expf(-gv))) * uv;  // SwiGLU (model.rs:272)
            }
        }
    }
    {
        // phase F's down rows of the same expert: row 64j + 8wv + lane/8,
        // chunks lane%8 + 8i (i < 3)
        const uint8_t* drow = L.down.w + (size_t)ex * L.down.expert_stride +
                              (size_t)(kRowsWg * c.j + 8 * c.wv + (c.lane >> 3)) * L.down.drb;
        if (L.down.kind == Q6_K) {
#pragma unroll
            for (uint32_t i = 0; i < kDownUnits; i++)
                D.wd[i].template put<Q6_K>(Fmt<Q6_K>::load(drow, L.down.geo, (c.lane & 7) + 8 * i));
        } else {
#pragma unroll
            for (uint32_t i = 0; i < kDownUnits; i++)
                D.wd[i].template put<KG>(Fmt<KG>::load(drow, L.down.geo, (c.lane & 7) + 8 * i));
        }
    }
    QH_MARK(4, 3);
    __syncthreads();  // S.hv complete; every wave is done with xn, which the next gather overwrites
    if (c.tid < kFfWg)  // one store instruction
        put_l(lbuf(A.lh, kDecodeStrideH, c.X) + kFfWg * c.j + c.tid, S.hv[c.tid], ptag(A, l, 5));
    return true;
}

// ========================================================= F: down projection ==
// Rows [64j, 64j+64) of expert rank X's down projection times its routing
// weight, passed across XCDs.
template <uint32_t KD, uint32_t KM>
__device__ __forceinline__ bool phase_down(const DecodeArgs& A, DecodeLds& S, const Ctx& c0, uint32_t l,
                                           const DownPre<KM>& D) {
    const Ctx c = fresh(c0);
    // the down rows (row 64j + 8wv + lane/8, chunks lane%8 + 8i, i < 3) were
    // requested at the end of phase E
    QH_MARK(5, 0);
    float* xs = S.big;
    if (!gather_l(A, S, lbuf(A.lh, kDecodeStrideH, c.X), c.ff, ptag(A, l, 5), xs, c.tid))
        return false;  // SwiGLU outputs (phase E)
    QH_MARK(5, 1);
    float acc = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < kDownUnits; i++) {
        const uint32_t chn = (c.lane & 7) + 8 * i;
        float xa[16], xb[16], sa, sb;
        x_runs_p<KD>(xs, 0, chn, xa, xb, sa, sb);
        acc += Fmt<KD>::dot(D.wd[i].template get<KD>(), chn, xa, xb, sa, sb);
    }
    acc = seg_sum(acc, 8);
    if ((c.lane & 7) == 0) S.po[8 * c.wv + (c.lane >> 3)] = S.wts[c.X] * acc;  // w * down (model.rs:281-284)
    __syncthreads();
    if (c.tid < kRowsWg)  // one store instruction
        put_g(lbuf(A.g2, kDecodeStrideG2, c.X) + kRowsWg * c.j + c.tid, S.po[c.tid], ptag(A, l, 6));
    return true;
}

// ======================================================== R: x'' reduction ==
// Rows [64j, 64j+64) of x'' = x' + moe, moe = ((0 + q_0) + q_1) + ... in rank
// order (model.rs:281-287), from slice j of every XCD's weighted down rows.
__device__ __forceinline__ bool phase_xr2(const DecodeArgs& A, DecodeLds& S, const Ctx& c0, uint32_t l, bool last) {
    const Ctx c = fresh(c0);
    float* vals = S.big;  // [8][64]
    bool ab = false;
    if (c.tid < kNX * kRowsWg / 2) {
        const uint32_t k = c.tid / (kRowsWg / 2), p = c.tid % (kRowsWg / 2);
        const uint32_t word[1] = {k * kDecodeStrideG2 + kRowsWg * c.j + 2 * p};
        float v[2];
        poll_pairs<kAuxG, 1>(A, buf_rsrc(A.g2, kNX * kDecodeStrideG2 * 8), word, 1u, 1u, ptag(A, l, 6), v, ab);
        vals[k * kRowsWg + 2 * p] = v[0];
        vals[k * kRowsWg + 2 * p + 1] = v[1];
    }
    if (ab) S.abort = 1;
    __syncthreads();
    if (S.abort) return false;
    QH_MARK(7, 1);
    if (c.tid < kRowsWg) {
        float moe = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < kNX; k++) moe += vals[k * kRowsWg + c.tid];
        const float x2 = S.x1[c.tid] + moe;
        S.xo[c.tid] = x2;
        put_l(lbuf(A.lx2, kDecodeStrideX2, c.X) + kRowsWg * c.j + c.tid, x2, ptag(A, l, 7));
        if (last && c.X == 0) A.a.x[kRowsWg * c.j + c.tid] = x2;  // x after the launch, for the host
    }
    // the routing of the layer, for the host (and the routing log)
    if (c.b == 0) {
        if (c.tid < c.top) {
            A.a.ids[c.tid] = S.ids[c.tid];
            A.a.wts[c.tid] = S.wts[c.tid];
            A.a.route_log[((size_t)c.pos * A.dm.layers + l) * c.top + c.tid] = S.ids[c.tid];
        }
        if (c.tid == 0)
            A.a.gap_log[(size_t)c.pos * A.dm.layers + l] =
                (S.sv[c.top - 1] - S.s9) / fmaxf(fabsf(S.sv[0]), fabsf(S.slast));
        if (c.tid < c.E) A.a.logits_r[c.tid] = S.lg[c.tid];
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
    const uint32_t tag = A.base + kDecodePhases * (A.l1 - A.l0) + 1;
    using Raw = typename Fmt<KV>::Raw;
    // unconditional loads (row and chunk clamped into the matrix; results of
    // clamped rows are dropped): the compiler then waits for exactly the group
    // it computes, not for the prefetched one behind it.  The rows are
    // wave-uniform: a row's byte offset goes in the buffer loads' scalar
    // offset, the lane's chunk offset (the same for every row) in the vector
    // one, so no per-lane 64-bit address arithmetic per load (the matrix is
    // below 4 GB: checked by persist_supported)
    const uint32_t ch = min(c.lane, cpr - 1);
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(mv.w, (uint32_t)((size_t)V * mv.drb));
    auto load_group = [&](Raw (&t)[kVocabRows], uint32_t gi) {
#pragma unroll
        for (uint32_t k = 0; k < kVocabRows; k++) {
            const uint32_t r = min(gi * kVocabRows + k, V - 1);
            t[k] = bload_u<KV>(vr, __builtin_amdgcn_readfirstlane(r * mv.drb), mv.geo, ch);
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
    QH_MARK(6, 0);
    float* xs = S.big;
    if (!gather_l_norm(A, S, lbuf(A.lx2, kDecodeStrideX2, c.X), c.H, ptag(A, A.l1 - 1, 7), A.onorm, xs, nullptr,
                       c.tid))
        return;  // x after the last layer, times the output norm's weights
    const float post = rms_scale(S, c.H, A.dm.eps);
    QH_MARK(6, 1);
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
            acc[k] = wave_sum(acc[k]) * post;
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
        put_g(A.tfin + 2 * c.b, __int_as_float(k0), tag);
        put_g(A.tfin + 2 * c.b + 1, __uint_as_float(i0), tag);
        if (S.bad) atomicOr(&a.st->err, kErrLogits);
    }
    QH_MARK(6, 4);
    if (c.b != 0) return;
    // workgroup 0: argmax over every workgroup's partial
    float* fin = S.big + 4096;  // clear of the padded x (px(2047) = 2171)
    {
        const uint32_t np = c.nwg;  // pairs (key, index)
        bool ab = false;
        if (c.tid < np) {
            const uint32_t word[1] = {2 * c.tid};
            float v[2];
            poll_pairs<kAuxG, 1>(A, buf_rsrc(A.tfin, np * 16), word, 1u, 1u, tag, v, ab);
            fin[2 * c.tid] = v[0];
            fin[2 * c.tid + 1] = v[1];
        }
        if (ab) S.abort = 1;
        __syncthreads();
        if (S.abort) return;
    }
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
// XCD of the calling wave (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xfu;
}

// Records the XCD of every workgroup of a launch shaped like k_decode's (the
// host checks the placement rule b % 8 before it selects the persistent step).
__global__ __launch_bounds__(kDT) void k_xcd_map(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

template <uint32_t KM>
__global__ __launch_bounds__(kDT) void k_decode(DecodeArgs A) {
    __shared__ __align__(16) DecodeLds S;
    Ctx c;
    c.b = blockIdx.x;
    c.nwg = gridDim.x;
    c.X = xcc_id();  // wave-uniform (a scalar register)
    c.j = c.b / kNX;
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
    if (A.l0 < A.l1) warm_layer(A.layers + A.l0);  // while the state loads are in flight
    {
        // the launch's arguments, likewise (seven 64-byte lines, read
        // throughout every layer)
        static_assert(sizeof(DecodeArgs) >= 0x1b4 + 4 && sizeof(DecodeArgs) <= 448,
                      "seven 64-byte lines, the last one holding offset 0x1b4");
        const auto* ka = (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
        uint32_t d0, d1, d2, d3, d4, d5, d6, d7;
        asm volatile(
            "s_load_dword %0, %8, 0x0\n"
            "s_load_dword %1, %8, 0x40\n"
            "s_load_dword %2, %8, 0x80\n"
            "s_load_dword %3, %8, 0xc0\n"
            "s_load_dword %4, %8, 0x100\n"
            "s_load_dword %5, %8, 0x140\n"
            "s_load_dword %6, %8, 0x180\n"
            "s_load_dword %7, %8, 0x1b4\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7)
            : "s"(ka)
            : "memory");
    }
    __syncthreads();
    if (c.pos >= dm.ctx || (err0 & kErrToken)) {
        if (c.b == 0 && c.tid == 0 && c.pos >= dm.ctx) atomicOr(&A.a.st->err, kErrContext);
        return;
    }
    c.tok = A.embed ? A.a.tokens[c.pos] : 0u;
    if (c.tok >= dm.vocab) {  // model.rs:222; every workgroup reads the same id
        if (c.b == 0 && c.tid == 0) atomicOr(&A.a.st->err, kErrToken);
        return;
    }
    if (ld_sys_u(A.abort_flag) != 0) {
        // a raised abort flag (a wait of an earlier step that gave up, or the
        // host's fault injection) fails this step before it starts
        if (c.b == 0 && c.tid == 0) atomicOr(&A.a.st->err, kErrSync);
        return;
    }
    if (c.X >= kNX) {
        // the exchanges assume 8 XCDs: give up, and make every other
        // workgroup's waits end
        if (c.tid == 0) {
            atomicOr(&A.a.st->err, kErrSync | kErrPlace);
            st_sys_u(A.abort_flag, 1u);
        }
        return;
    }
    c.T = c.pos + 1;
    c.H = dm.hidden;
    c.E = dm.experts;
    c.top = dm.top;
    c.ff = dm.ff;
    c.qd = dm.heads * 128;
    c.ctx = dm.ctx;
    for (uint32_t l = A.l0; l < A.l1; l++) {
        // read through the constant address space: scalar loads, which do
        // not wait behind this wave's outstanding vector loads and stores
        const LayerW& L = *(const LayerW*)((const __attribute__((address_space(4))) LayerW*)A.layers + l);
        bool ok = true;
        AttnPre P;
        ok = phase_qkv<KM>(A, S, L, c, l, P);
        if (!ok || !phase_attn(A, S, L, c, l, P)) return;
        if (!phase_oproj<KM>(A, S, L, c, l)) return;
        if (!phase_xr1(A, S, c, l)) return;
        DownPre<KM> D;
        ok = phase_moe<KM>(A, S, L, c, l, D);
        if (ok) QH_DISPATCH_KM(L.down.kind, KM, KD, ok = (phase_down<KD, KM>(A, S, c, l, D)));
        if (!ok || !phase_xr2(A, S, c, l, l + 1 == A.l1)) return;
    }
    if (A.vocab) QH_DISPATCH_BLOCK(A.out.kind, KV, phase_vocab<KV>(A, S, c));
}

template __global__ void k_decode<Q4_0>(DecodeArgs);
template __global__ void k_decode<Q8_0>(DecodeArgs);
template __global__ void k_decode<Q4_K>(DecodeArgs);
template __global__ void k_decode<Q5_K>(DecodeArgs);
template __global__ void k_decode<Q6_K>(DecodeArgs);

}  // namespace qh
