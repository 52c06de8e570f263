/*
 * Oracle: the stochastic sampler of src/sampling.rs:1-65 and the random
 * stream it draws from.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * The stream is `rand::rngs::StdRng` of rand 0.8.8 (Cargo.lock:1128-1129),
 * which is `rand_chacha::ChaCha12Rng` 0.3.1 (Cargo.lock:1149-1150); neither
 * crate is vendored in the reference, so their published algorithms are
 * restated here:
 *   - `SeedableRng::seed_from_u64` (rand_core 0.6.4): the 32-byte seed is
 *     filled 4 bytes at a time (little endian) with the output of a PCG32
 *     step: state = state * 6364136223846793005 + 11634580027462260723, then
 *     the XSH-RR output of the new state;
 *   - ChaCha with 12 rounds (6 double rounds), key = the seed as 8 LE words,
 *     64-bit block counter in words 12-13 starting at 0, stream id 0 in
 *     words 14-15; `next_u32` returns the keystream words in order;
 *   - `gen::<f32>()` (rand's `Standard` for f32): (next_u32 >> 8) * 2^-24.
 * The ChaCha core is pinned by the all-zero-key ChaCha20 keystream (the
 * rounds are a parameter); the seed expansion and the stream order have no
 * vector from the reference and stay "parity unpinned".
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

/* ------------------------------------------------------------ ChaCha -- */
static uint32_t rotl(uint32_t v, int n) { return (v << n) | (v >> (32 - n)); }

#define QR(a, b, c, d)                  \
    do {                                \
        a += b; d ^= a; d = rotl(d, 16); \
        c += d; b ^= c; b = rotl(b, 12); \
        a += b; d ^= a; d = rotl(d, 8);  \
        c += d; b ^= c; b = rotl(b, 7);  \
    } while (0)

void or_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = (uint32_t)stream;
    s[15] = (uint32_t)(stream >> 32);
    uint32_t x[16];
    memcpy(x, s, sizeof x);
    for (int r = 0; r < rounds; r += 2) {
        QR(x[0], x[4], x[8], x[12]);
        QR(x[1], x[5], x[9], x[13]);
        QR(x[2], x[6], x[10], x[14]);
        QR(x[3], x[7], x[11], x[15]);
        QR(x[0], x[5], x[10], x[15]);
        QR(x[1], x[6], x[11], x[12]);
        QR(x[2], x[7], x[8], x[13]);
        QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

void or_stdrng_seed(uint64_t seed, uint32_t key[8]) {
    uint64_t st = seed;
    for (int i = 0; i < 8; i++) {
        st = st * 6364136223846793005ull + 11634580027462260723ull;
        const uint32_t xs = (uint32_t)(((st >> 18) ^ st) >> 27);
        const uint32_t rot = (uint32_t)(st >> 59);
        key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
    }
}

/* word `i` of the ChaCha12 keystream of `key` */
static uint32_t stream_word(const uint32_t key[8], uint64_t i) {
    uint32_t blk[16];
    or_chacha_block(key, i / 16, 0, 12, blk);
    return blk[i % 16];
}

/* ----------------------------------------------------------- Sampler -- */
struct or_sampler {
    uint32_t key[8];
    uint64_t word;  /* next keystream word */
    float temperature, top_p;
    size_t top_k;
};

or_sampler *or_sampler_new(uint64_t seed, float temperature, size_t top_k, float top_p) {
    /* sampling.rs:10-25 */
    if (!(isfinite(temperature) && temperature >= 0.f && isfinite(top_p) && top_p > 0.f && top_p <= 1.f)) {
        or_fail("invalid sampling parameters");
        return NULL;
    }
    or_sampler *s = calloc(1, sizeof *s);
    or_stdrng_seed(seed, s->key);
    s->temperature = temperature;
    s->top_k = top_k;
    s->top_p = top_p;
    return s;
}

void or_sampler_free(or_sampler *s) { free(s); }

float or_sampler_draw(or_sampler *s) {
    const uint32_t w = stream_word(s->key, s->word++);
    return (float)(w >> 8) * (1.0f / 16777216.0f);
}

static const float *g_sort_logits;
/* descending total order, ascending index on ties (sampling.rs:31) */
static int cmp_desc(const void *a, const void *b) {
    const uint32_t i = *(const uint32_t *)a, j = *(const uint32_t *)b;
    const int c = or_total_cmp(g_sort_logits[j], g_sort_logits[i]);
    if (c) return c;
    return i < j ? -1 : (i > j);
}

/* sampling.rs:26-63 */
int or_sampler_sample(or_sampler *s, const float *logits, size_t n, uint32_t *out) {
    if (n == 0) return or_fail("invalid logits");
    for (size_t i = 0; i < n; i++)
        if (!or_isfinite(logits[i])) return or_fail("invalid logits");
    uint32_t *ids = malloc(n * sizeof *ids);
    for (size_t i = 0; i < n; i++) ids[i] = (uint32_t)i;
    g_sort_logits = logits;
    qsort(ids, n, sizeof *ids, cmp_desc);
    if (s->temperature == 0.f) {
        *out = ids[0];
        free(ids);
        return 0;
    }
    size_t k = n;
    if (s->top_k > 0 && s->top_k < n) k = s->top_k;
    const float max = logits[ids[0]];
    float *probs = malloc(k * sizeof *probs);
    for (size_t i = 0; i < k; i++) probs[i] = expf((logits[ids[i]] - max) / s->temperature);
    float total = -0.0f;
    for (size_t i = 0; i < k; i++) total += probs[i];
    float cumulative = 0.f;
    size_t m = k;
    for (size_t i = 0; i < k; i++) {
        cumulative += probs[i] / total;
        if (cumulative >= s->top_p) {
            m = i + 1;
            break;
        }
    }
    float sum = -0.0f;
    for (size_t i = 0; i < m; i++) sum += probs[i];
    float draw = or_sampler_draw(s) * sum;
    uint32_t pick = ids[m - 1];
    for (size_t i = 0; i < m; i++) {
        if (draw < probs[i]) {
            pick = ids[i];
            break;
        }
        draw -= probs[i];
    }
    *out = pick;
    free(probs);
    free(ids);
    return 0;
}
