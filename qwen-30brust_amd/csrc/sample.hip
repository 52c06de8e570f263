// Device sampler: src/sampling.rs:26-63 (greedy, top-k, temperature, top-p
// and the seeded draw) over the logits in HBM, with the padding-vocab mask of
// src/main.rs:262-266 applied on the fly.  One workgroup of 1024 threads:
//
//   1. one pass over the masked logits: finiteness ("invalid logits") and the
//      first id under the sort of sampling.rs:31 (descending total order,
//      lowest index on ties); temperature 0 returns it (sampling.rs:32-35);
//   2. the candidate count P: K = top_k (or every id when top_k is 0 or
//      above the vocabulary) when K <= kSampleMax; otherwise the ids whose
//      probability exp((l - max) / T) is nonzero (the rest of the sorted list
//      adds exact zeros to every sum below), at most kSampleMax;
//   3. the composite key of rank P - 1 by radix selection (three digit passes
//      over the 32-bit total-order key, two over the index when the rank
//      falls inside a run of equal logits), the P candidates collected into
//      LDS and sorted there (bitonic, descending);
//   4. the probabilities in parallel, then one lane runs the sequential f32
//      folds of sampling.rs:44-62 (total, cumulative top-p cut, the draw
//      scaled by the kept mass, the walk) in the reference's order.
// The draw itself (rand's gen::<f32>()) comes from the host's ChaCha12
// stream and is passed in.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>

#include "kernels.hpp"
#include "qh_device.hpp"

namespace qh {

namespace {

constexpr uint32_t kST = 1024;         // threads of the sampling workgroup
constexpr uint32_t kSW = kST / 64;     // its waves
constexpr uint32_t kBins = 2048;       // widest digit: 11 bits

struct SampleLds {
    unsigned long long cand[kSampleMax];  // composite keys of the candidates
    float p[kSampleMax];                  // their probabilities, in sorted order
    uint32_t hist[kBins];
    uint32_t wsum[kSW];
    unsigned long long top;
    uint32_t ncand, digit, rank, count, bad, flag;
};

// Unsigned key with the order of f32::total_cmp.
__device__ __forceinline__ uint32_t ukey(float v) { return (uint32_t)total_key(v) ^ 0x80000000u; }
// Composite key: larger = earlier in the sampler's sort (key, then lower index).
__device__ __forceinline__ unsigned long long ckey(float v, uint32_t i) {
    return ((unsigned long long)ukey(v) << 32) | (uint32_t)~i;
}
__device__ __forceinline__ uint32_t ck_index(unsigned long long k) { return ~(uint32_t)k; }

__device__ __forceinline__ float masked(const float* lg, const uint8_t* valid, uint32_t i) {
    return (valid && !valid[i]) ? -FLT_MAX : lg[i];  // f32::MIN (main.rs:262-266)
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

// The bin holding rank `rr` when bins [0, nb) are walked from the top bin
// down (desc) or from bin 0 up: S.digit, and S.rank = rr minus the counts
// walked before it.  rr must be below the histogram's total.
__device__ void find_bin(SampleLds& S, uint32_t nb, uint32_t rr, bool desc) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t p0 = 2 * tid, p1 = 2 * tid + 1;
    const uint32_t b0 = desc ? nb - 1 - p0 : p0, b1 = desc ? nb - 1 - p1 : p1;
    const uint32_t c0 = p0 < nb ? S.hist[b0] : 0u, c1 = p1 < nb ? S.hist[b1] : 0u;
    const uint32_t s = c0 + c1, incl = wave_incl_scan(s, lane);
    if (lane == 63) S.wsum[wv] = incl;
    __syncthreads();
    if (wv == 0) {
        const uint32_t w = lane < kSW ? S.wsum[lane] : 0u;
        const uint32_t wi = wave_incl_scan(w, lane);
        if (lane < kSW) S.wsum[lane] = wi - w;
    }
    __syncthreads();
    const uint32_t excl = S.wsum[wv] + incl - s;
    if (rr >= excl && rr < excl + s) {
        if (rr < excl + c0) {
            S.digit = b0;
            S.rank = rr - excl;
        } else {
            S.digit = b1;
            S.rank = rr - excl - c0;
        }
    }
    __syncthreads();
}

// Composite key of the element of rank r (0 = first in the sampler's sort).
__device__ unsigned long long select_rank(SampleLds& S, const float* lg, const uint8_t* valid, uint32_t n,
                                          uint32_t r) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, pmask = 0, rr = r, neq = 0;
    // key digits, most significant first: bits 31..21, 20..10, 9..0
    const uint32_t shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
    for (int ps = 0; ps < 3; ps++) {
        const uint32_t sh = shifts[ps], nb = 1u << widths[ps];
        for (uint32_t b = tid; b < nb; b += kST) S.hist[b] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kST) {
            const uint32_t u = ukey(masked(lg, valid, i));
            if ((u & pmask) == prefix) atomicAdd(&S.hist[(u >> sh) & (nb - 1)], 1u);
        }
        __syncthreads();
        find_bin(S, nb, rr, true);
        neq = S.hist[S.digit];
        prefix |= S.digit << sh;
        pmask |= (nb - 1) << sh;
        rr = S.rank;
        __syncthreads();
    }
    // prefix is the key; rr ranks the run of equal keys by ascending index
    if (rr + 1 == neq) return (unsigned long long)prefix << 32;  // the whole run
    uint32_t iprefix = 0, imask = 0;
    const uint32_t ishift[2] = {10, 0};
    for (int ps = 0; ps < 2; ps++) {
        const uint32_t sh = ishift[ps], nb = 1024;
        for (uint32_t b = tid; b < nb; b += kST) S.hist[b] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kST)
            if (ukey(masked(lg, valid, i)) == prefix && (i & imask) == iprefix)
                atomicAdd(&S.hist[(i >> sh) & (nb - 1)], 1u);
        __syncthreads();
        find_bin(S, nb, rr, false);
        iprefix |= S.digit << sh;
        imask |= (nb - 1) << sh;
        rr = S.rank;
        __syncthreads();
    }
    return ((unsigned long long)prefix << 32) | (uint32_t)~iprefix;
}

__global__ __launch_bounds__(kST) void k_sample(SampleArgs a) {
    __shared__ SampleLds S;
    const uint32_t tid = threadIdx.x, n = a.n;
    const float* lg = a.logits;
    if (tid == 0) {
        S.top = 0;
        S.bad = 0;
        S.ncand = 0;
        S.count = 0;
        S.flag = 0;
    }
    __syncthreads();
    if (a.mode == kSampleModeRank) {  // the id of rank a.rank (the last kept id past the candidates)
        const unsigned long long k = select_rank(S, lg, a.valid, n, a.rank);
        if (tid == 0) {
            a.out[0] = ck_index(k);
            a.out[1] = 0;
        }
        return;
    }
    // 1. finiteness and the first id
    unsigned long long best = 0;
    bool bad = false;
    for (uint32_t i = tid; i < n; i += kST) {
        const float v = masked(lg, a.valid, i);
        bad |= !finite_f(v);
        const unsigned long long k = ckey(v, i);
        best = k > best ? k : best;
    }
    if (bad) S.bad = 1;
    atomicMax(&S.top, best);
    __syncthreads();
    if (S.bad || n == 0) {
        if (tid == 0) a.out[1] = kSampleBadLogits;
        return;
    }
    const uint32_t first = ck_index(S.top);
    if (a.temperature == 0.f) {
        if (tid == 0) {
            a.out[0] = first;
            a.out[1] = 0;
            a.out[2] = 1;
            a.out[3] = 1;
        }
        return;
    }
    const float T = a.temperature, mx = masked(lg, a.valid, first);
    const uint32_t K = (a.top_k > 0 && a.top_k < n) ? a.top_k : n;
    // 2. candidate count
    uint32_t P = K;
    if (K > kSampleMax) {
        uint32_t cnt = 0;
        for (uint32_t i = tid; i < n; i += kST) cnt += expf((masked(lg, a.valid, i) - mx) / T) > 0.f;
        atomicAdd(&S.count, cnt);
        __syncthreads();
        P = min(S.count, K);
        if (P > kSampleMax) {
            // the global path: the key of rank P - 1 bounds the candidates
            const unsigned long long theta = select_rank(S, lg, a.valid, n, P - 1);
            if (tid == 0) {
                a.out[1] = kSampleSupport;
                a.out[3] = P;
                a.out[4] = (uint32_t)theta;
                a.out[5] = (uint32_t)(theta >> 32);
            }
            return;
        }
    }
    // 3. the P first ids, sorted
    const unsigned long long theta = select_rank(S, lg, a.valid, n, P - 1);
    for (uint32_t i = tid; i < n; i += kST) {
        const unsigned long long k = ckey(masked(lg, a.valid, i), i);
        if (k >= theta) {
            const uint32_t slot = atomicAdd(&S.ncand, 1u);
            if (slot < kSampleMax) S.cand[slot] = k;
        }
    }
    uint32_t np = 1;
    while (np < P) np <<= 1;
    __syncthreads();
    if (S.ncand != P) {  // the selection must yield exactly the P first ids
        if (tid == 0) a.out[1] = kSampleInternal;
        return;
    }
    for (uint32_t i = P + tid; i < np; i += kST) S.cand[i] = 0;  // below every finite key
    __syncthreads();
    for (uint32_t k = 2; k <= np; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < np; i += kST) {
                const uint32_t l = i ^ j;
                if (l > i) {
                    const unsigned long long x = S.cand[i], y = S.cand[l];
                    const bool down = (i & k) == 0;  // descending runs first: overall descending
                    if (down ? x < y : x > y) {
                        S.cand[i] = y;
                        S.cand[l] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
    // 4. probabilities (sampling.rs:43-46), then the sequential folds
    for (uint32_t i = tid; i < P; i += kST) {
#pragma clang fp contract(off)
        S.p[i] = expf((masked(lg, a.valid, ck_index(S.cand[i])) - mx) / T);
    }
    __syncthreads();
    if (tid == 0) {
#pragma clang fp contract(off)
        float total = -0.0f;
        for (uint32_t i = 0; i < P; i++) total += S.p[i];
        float cumulative = 0.f;
        uint32_t m = K;
        for (uint32_t i = 0; i < P; i++) {
            cumulative += S.p[i] / total;
            if (cumulative >= a.top_p) {
                m = i + 1;
                break;
            }
        }
        const uint32_t mp = m < P ? m : P;
        float kept = -0.0f;
        for (uint32_t i = 0; i < mp; i++) kept += S.p[i];
        float draw = a.draw * kept;
        uint32_t pick = 0xffffffffu;
        for (uint32_t i = 0; i < mp; i++) {
            if (draw < S.p[i]) {
                pick = ck_index(S.cand[i]);
                break;
            }
            draw -= S.p[i];
        }
        if (pick == 0xffffffffu && m <= P) pick = ck_index(S.cand[m - 1]);  // ids.last()
        if (pick == 0xffffffffu) S.flag = m;  // the last kept id lies past the candidates
        a.out[0] = pick;
        a.out[1] = 0;
        a.out[2] = m;
        a.out[3] = P;
    }
    __syncthreads();
    if (S.flag) {  // rank m - 1 (= K - 1: every later probability is 0)
        const unsigned long long k = select_rank(S, lg, a.valid, n, S.flag - 1);
        if (tid == 0) a.out[0] = ck_index(k);
    }
}

// ------------------------------------------------- more than kSampleMax --
// cand[slot] = composite key of every id at or above theta (exactly P of
// them); cand[P, np) = 0, below every finite key.
__global__ __launch_bounds__(kBlock) void k_sample_collect(SampleArgs a, unsigned long long theta, uint32_t P,
                                                           uint32_t np, unsigned long long* cand, uint32_t* cnt) {
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < a.n; i += stride) {
        const unsigned long long k = ckey(masked(a.logits, a.valid, i), i);
        if (k >= theta) {
            const uint32_t slot = atomicAdd(cnt, 1u);
            if (slot < P) cand[slot] = k;
        }
    }
    for (uint32_t i = P + blockIdx.x * kBlock + threadIdx.x; i < np; i += stride) cand[i] = 0;
}

// One compare-exchange step (k, j) of a descending bitonic sort of cand[0, np).
__global__ __launch_bounds__(kBlock) void k_bitonic_step(unsigned long long* cand, uint32_t np, uint32_t k,
                                                         uint32_t j) {
    const uint32_t t = blockIdx.x * kBlock + threadIdx.x;  // pair index < np / 2
    if (t >= np / 2) return;
    const uint32_t i = 2 * t - (t & (j - 1)), l = i + j;  // i has bit j clear
    const unsigned long long x = cand[i], y = cand[l];
    const bool down = (i & k) == 0;
    if (down ? x < y : x > y) {
        cand[i] = y;
        cand[l] = x;
    }
}

// The steps with j < 2048 of stage k for every 4096-key block, in LDS.
__global__ __launch_bounds__(kST) void k_bitonic_local(unsigned long long* cand, uint32_t k, uint32_t j0) {
    __shared__ unsigned long long s[4096];
    const uint32_t base = blockIdx.x * 4096;
    for (uint32_t i = threadIdx.x; i < 4096; i += kST) s[i] = cand[base + i];
    __syncthreads();
    for (uint32_t j = j0; j > 0; j >>= 1) {
        for (uint32_t t = threadIdx.x; t < 2048; t += kST) {
            const uint32_t i = 2 * t - (t & (j - 1)), l = i + j;
            const unsigned long long x = s[i], y = s[l];
            const bool down = ((base + i) & k) == 0;
            if (down ? x < y : x > y) {
                s[i] = y;
                s[l] = x;
            }
        }
        __syncthreads();
    }
    for (uint32_t i = threadIdx.x; i < 4096; i += kST) cand[base + i] = s[i];
}

// The probabilities of the P sorted candidates (sampling.rs:43-46), then one
// lane runs the sequential folds of sampling.rs:47-62 in the reference's
// order, 4096 values at a time staged in LDS.
__global__ __launch_bounds__(kST) void k_sample_fold(SampleArgs a, const unsigned long long* cand, float* prob,
                                                     uint32_t P, uint32_t K) {
    __shared__ float sp[4096];
    __shared__ uint32_t m_sh;
    const uint32_t tid = threadIdx.x;
    const float T = a.temperature, mx = masked(a.logits, a.valid, ck_index(cand[0]));
    for (uint32_t i = tid; i < P; i += kST) {
#pragma clang fp contract(off)
        prob[i] = expf((masked(a.logits, a.valid, ck_index(cand[i])) - mx) / T);
    }
    __syncthreads();
    // total (sampling.rs:47)
    float total = -0.0f;
    for (uint32_t c0 = 0; c0 < P; c0 += 4096) {
        const uint32_t nc = min(4096u, P - c0);
        for (uint32_t i = tid; i < nc; i += kST) sp[i] = prob[c0 + i];
        __syncthreads();
        if (tid == 0) {
#pragma clang fp contract(off)
            for (uint32_t i = 0; i < nc; i++) total += sp[i];
        }
        __syncthreads();
    }
    // the top-p cut (sampling.rs:48-56); m = K when it is never reached
    float cumulative = 0.f;
    if (tid == 0) m_sh = K;
    bool done = false;  // thread 0's state
    for (uint32_t c0 = 0; c0 < P; c0 += 4096) {
        const uint32_t nc = min(4096u, P - c0);
        for (uint32_t i = tid; i < nc; i += kST) sp[i] = prob[c0 + i];
        __syncthreads();
        if (tid == 0 && !done) {
#pragma clang fp contract(off)
            for (uint32_t i = 0; i < nc; i++) {
                cumulative += sp[i] / total;
                if (cumulative >= a.top_p) {
                    m_sh = c0 + i + 1;
                    done = true;
                    break;
                }
            }
        }
        __syncthreads();
        if (m_sh != K) break;  // every thread reads the same word after the barrier
    }
    const uint32_t m = m_sh, mp = min(m, P);
    // kept mass, the draw scaled by it, the walk (sampling.rs:57-62)
    float kept = -0.0f;
    for (uint32_t c0 = 0; c0 < mp; c0 += 4096) {
        const uint32_t nc = min(4096u, mp - c0);
        for (uint32_t i = tid; i < nc; i += kST) sp[i] = prob[c0 + i];
        __syncthreads();
        if (tid == 0) {
#pragma clang fp contract(off)
            for (uint32_t i = 0; i < nc; i++) kept += sp[i];
        }
        __syncthreads();
    }
    float draw = a.draw * kept;  // thread 0's value
    uint32_t pick = 0xffffffffu;
    for (uint32_t c0 = 0; c0 < mp; c0 += 4096) {
        const uint32_t nc = min(4096u, mp - c0);
        for (uint32_t i = tid; i < nc; i += kST) sp[i] = prob[c0 + i];
        __syncthreads();
        if (tid == 0 && pick == 0xffffffffu) {
#pragma clang fp contract(off)
            for (uint32_t i = 0; i < nc; i++) {
                if (draw < sp[i]) {
                    pick = ck_index(cand[c0 + i]);
                    break;
                }
                draw -= sp[i];
            }
            m_sh = pick;
        }
        __syncthreads();
        if (m_sh != 0xffffffffu) break;
    }
    if (tid == 0) {
        uint32_t status = 0;
        if (pick == 0xffffffffu) {  // ids.last()
            if (m <= P) pick = ck_index(cand[m - 1]);
            else status = kSampleRank;  // rank m - 1 lies past the candidates (their probabilities are 0)
        }
        a.out[0] = pick;
        a.out[1] = status;
        a.out[2] = m;
        a.out[3] = P;
    }
}

}  // namespace

void launch_sample(const SampleArgs& a, hipStream_t s) { k_sample<<<1, kST, 0, s>>>(a); }

void launch_sample_collect(const SampleArgs& a, unsigned long long theta, uint32_t P, uint32_t np,
                           unsigned long long* cand, uint32_t* cnt, hipStream_t s) {
    const uint32_t grid = std::min<uint32_t>((std::max(a.n, np) + kBlock - 1) / kBlock, 1024);
    k_sample_collect<<<grid, kBlock, 0, s>>>(a, theta, P, np, cand, cnt);
}

// Descending bitonic sort of cand[0, np), np a power of two >= 4096: steps
// with j >= 2048 one launch each over the grid, the rest of a stage in LDS.
void launch_sample_sort(unsigned long long* cand, uint32_t np, hipStream_t s) {
    const uint32_t pairs_grid = (np / 2 + kBlock - 1) / kBlock;
    for (uint32_t k = 2; k <= np; k <<= 1) {
        uint32_t j = k >> 1;
        for (; j >= 2048; j >>= 1) k_bitonic_step<<<pairs_grid, kBlock, 0, s>>>(cand, np, k, j);
        k_bitonic_local<<<np / 4096, kST, 0, s>>>(cand, k, j);
    }
}

void launch_sample_fold(const SampleArgs& a, const unsigned long long* cand, float* prob, uint32_t P, uint32_t K,
                        hipStream_t s) {
    k_sample_fold<<<1, kST, 0, s>>>(a, cand, prob, P, K);
}

}  // namespace qh
