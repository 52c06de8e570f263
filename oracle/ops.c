/*
 * Oracle: vector ops restated from src/ops.rs and the greedy branch of
 * src/sampling.rs.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

/* ops.rs:3-15.  scale = recip(sqrt(sum(v*v)/n + eps)); v *= scale * w. */
int or_rms(float *x, const float *w, size_t n, float eps) {
    if (n == 0 || !(eps > 0.f)) return or_fail("RMSNorm shape/epsilon invalid");
    float s = -0.0f; /* Rust float Sum starts at -0.0 */
    for (size_t i = 0; i < n; i++) s += x[i] * x[i];
    float scale = 1.0f / sqrtf(s / (float)n + eps);
    for (size_t i = 0; i < n; i++) x[i] *= scale * w[i];
    return 0;
}

/* ops.rs:17-28: NeoX split-half rotation of every head-sized chunk. */
void or_rope(float *x, size_t n, size_t head, size_t pos, float theta) {
    for (size_t h0 = 0; h0 + head <= n; h0 += head) {
        float *h = x + h0;
        for (size_t i = 0; i < head / 2; i++) {
            float e = -2.f * (float)i / (float)head;
            float angle = (float)pos * powf(theta, e);
            float s = sinf(angle), c = cosf(angle);
            float a = h[i], b = h[i + head / 2];
            h[i] = a * c - b * s;
            h[i + head / 2] = a * s + b * c;
        }
    }
}

/* ops.rs:29-44 */
int or_softmax(float *x, size_t n) {
    if (n == 0) return or_fail("invalid softmax logits");
    for (size_t i = 0; i < n; i++)
        if (!or_isfinite(x[i])) return or_fail("invalid softmax logits");
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
    return 0;
}

/* Descending by total order, ties to the lower index (ops.rs:51,
 * sampling.rs:33). */
static const float *g_sort_keys;
static int cmp_desc(const void *pa, const void *pb) {
    uint32_t a = *(const uint32_t *)pa, b = *(const uint32_t *)pb;
    int c = or_total_cmp(g_sort_keys[b], g_sort_keys[a]);
    if (c) return c;
    return (a > b) - (a < b);
}

/* ops.rs:45-56: top `top` ids by logit, then softmax over the chosen logits. */
int or_route(const float *logits, size_t n, size_t top, uint32_t *ids, float *w) {
    if (top == 0 || top > n) return or_fail("invalid MoE router");
    for (size_t i = 0; i < n; i++)
        if (!or_isfinite(logits[i])) return or_fail("invalid MoE router");
    uint32_t *all = malloc(n * sizeof *all);
    for (size_t i = 0; i < n; i++) all[i] = (uint32_t)i;
    g_sort_keys = logits; /* qsort has no context argument; single-threaded use */
    qsort(all, n, sizeof *all, cmp_desc);
    for (size_t i = 0; i < top; i++) {
        ids[i] = all[i];
        w[i] = logits[all[i]];
    }
    free(all);
    return or_softmax(w, top);
}

/* ops.rs:57-98.  KV time-major: element j of head kh at time t is at
 * (t*kvheads + kh)*d + j. */
int or_attention(const float *q, const float *k, const float *v, size_t klen, size_t heads,
                 size_t kvheads, size_t d, float *out) {
    if (!(kvheads > 0 && heads > 0 && d > 0 && heads % kvheads == 0 &&
          klen % (kvheads * d) == 0))
        return or_fail("attention shape mismatch");
    size_t time = klen / (kvheads * d);
    if (time == 0) return or_fail("empty KV cache");
    float *scores = malloc(time * sizeof *scores);
    float root = sqrtf((float)d);
    for (size_t i = 0; i < heads * d; i++) out[i] = 0.f;
    for (size_t h = 0; h < heads; h++) {
        size_t kh = h / (heads / kvheads);
        const float *qs = q + h * d;
        for (size_t t = 0; t < time; t++) {
            const float *kr = k + (t * kvheads + kh) * d;
            float s = -0.0f;
            for (size_t j = 0; j < d; j++) s += qs[j] * kr[j];
            scores[t] = s / root;
        }
        if (or_softmax(scores, time)) {
            free(scores);
            return -1;
        }
        for (size_t t = 0; t < time; t++)
            for (size_t j = 0; j < d; j++) out[h * d + j] += scores[t] * v[(t * kvheads + kh) * d + j];
    }
    free(scores);
    return 0;
}

/* sampling.rs:26-35 with temperature 0: argmax under total order, lowest
 * index on ties, after rejecting empty / non-finite logits. */
int or_greedy(const float *logits, size_t n, uint32_t *out) {
    if (n == 0) return or_fail("invalid logits");
    for (size_t i = 0; i < n; i++)
        if (!or_isfinite(logits[i])) return or_fail("invalid logits");
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (or_total_cmp(logits[i], logits[best]) > 0) best = i;
    *out = (uint32_t)best;
    return 0;
}
