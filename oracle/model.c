/*
 * Oracle: the CPU backend matvec (src/backend.rs:29-75) and the single-token
 * causal forward (src/model.rs).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_gguf.h"
#include "oracle_internal.h"

/* ------------------------------------------------------------------------ */
/* A small persistent thread pool: slice i of [0,n) goes to thread i.       */
/* ------------------------------------------------------------------------ */
typedef void (*job_fn)(void *arg, size_t begin, size_t end);
#define POOL_MAX 256
static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    int size;           /* worker threads started */
    unsigned gen;
    job_fn fn;
    void *arg;
    size_t n;
    int slices, remaining;
    pthread_t th[POOL_MAX];
} P = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};

static void *worker(void *p) {
    int id = (int)(intptr_t)p; /* slice index, >= 1 */
    unsigned seen = 0;
    pthread_mutex_lock(&P.mu);
    for (;;) {
        while (P.gen == seen) pthread_cond_wait(&P.go, &P.mu);
        seen = P.gen;
        if (id < P.slices) {
            job_fn fn = P.fn;
            void *arg = P.arg;
            size_t b = P.n * id / P.slices, e = P.n * (id + 1) / P.slices;
            pthread_mutex_unlock(&P.mu);
            fn(arg, b, e);
            pthread_mutex_lock(&P.mu);
            if (--P.remaining == 0) pthread_cond_signal(&P.done);
        }
    }
    return NULL;
}

static pthread_mutex_t g_run = PTHREAD_MUTEX_INITIALIZER; /* one parallel job at a time */

static void parallel_for(int threads, size_t n, job_fn fn, void *arg) {
    if (threads <= 1 || n < 2) {
        fn(arg, 0, n);
        return;
    }
    if (threads > POOL_MAX) threads = POOL_MAX;
    pthread_mutex_lock(&g_run);
    pthread_mutex_lock(&P.mu);
    while (P.size < threads - 1) {
        P.size++;
        pthread_create(&P.th[P.size], NULL, worker, (void *)(intptr_t)P.size);
    }
    P.fn = fn;
    P.arg = arg;
    P.n = n;
    P.slices = threads;
    P.remaining = threads - 1;
    P.gen++;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    fn(arg, 0, n / threads);
    pthread_mutex_lock(&P.mu);
    while (P.remaining) pthread_cond_wait(&P.done, &P.mu);
    pthread_mutex_unlock(&P.mu);
    pthread_mutex_unlock(&g_run);
}

/* ------------------------------------------------------------------------ */
/* backend.rs:29-52 (Cpu::matvec)                                           */
/* ------------------------------------------------------------------------ */
typedef struct {
    const uint8_t *data;
    uint32_t kind;
    size_t rb, cols;
    const float *x;
    float *y;
} mv_job;

/* Faithful loop of backend.rs:41-48: per-element quant::value, sequential
 * fold from -0.0. */
static void mv_faithful(void *a, size_t r0, size_t r1) {
    mv_job *j = a;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t *b = j->data + r * j->rb;
        float s = -0.0f;
        for (size_t i = 0; i < j->cols; i++) s += j->x[i] * or_value(b, j->kind, i);
        j->y[r] = s;
    }
}

/* Same values and the same per-row fold order, with each row decoded a block
 * at a time and four rows' folds interleaved (independent chains). */
static void mv_fast(void *a, size_t r0, size_t r1) {
    mv_job *j = a;
    size_t c = j->cols;
    float *w = malloc(4 * c * sizeof *w);
    size_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        for (int k = 0; k < 4; k++) or_decode_row_fast(j->data + (r + k) * j->rb, j->kind, c, w + k * c);
        float s0 = -0.0f, s1 = -0.0f, s2 = -0.0f, s3 = -0.0f;
        const float *x = j->x, *w0 = w, *w1 = w + c, *w2 = w + 2 * c, *w3 = w + 3 * c;
        for (size_t i = 0; i < c; i++) {
            s0 += x[i] * w0[i];
            s1 += x[i] * w1[i];
            s2 += x[i] * w2[i];
            s3 += x[i] * w3[i];
        }
        j->y[r] = s0;
        j->y[r + 1] = s1;
        j->y[r + 2] = s2;
        j->y[r + 3] = s3;
    }
    for (; r < r1; r++) {
        or_decode_row_fast(j->data + r * j->rb, j->kind, c, w);
        float s = -0.0f;
        for (size_t i = 0; i < c; i++) s += j->x[i] * w[i];
        j->y[r] = s;
    }
    free(w);
}

int or_packed_matvec(const uint8_t *data, size_t len, uint32_t kind, size_t rows, size_t cols,
                     const float *x, float *y, int threads) {
    size_t rb;
    if (or_row_bytes(kind, cols, &rb)) return -1;
    if (rows && rb > SIZE_MAX / rows) return or_fail("matrix overflow");
    if (len < rb * rows) return or_fail("packed matrix shorter than rows*row_bytes");
    mv_job j = {data, kind, rb, cols, x, y};
    if (threads <= 0)
        mv_faithful(&j, 0, rows);
    else
        parallel_for(threads, rows, mv_fast, &j);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* model.rs                                                                 */
/* ------------------------------------------------------------------------ */
typedef struct {
    float *k, *v;
    size_t len; /* floats used */
} kvbuf;

struct or_model {
    or_gguf *g;
    or_config c;
    kvbuf *cache;
    float *norms;       /* [layers][attn H | q_norm d | k_norm d | ffn H] */
    float *output_norm; /* [H] */
    size_t position, context;
    float *last_router; /* [layers][experts] */
    uint32_t *forced;   /* [layers][top] expert ids for the next step only, or NULL */
};

static size_t norm_stride(const or_config *c) { return 2 * c->hidden + 2 * c->head_dim; }

/* model.rs:21-90 */
static int config_from_gguf(const or_gguf *g, or_config *c) {
    const char *arch = or_gguf_str(g, "general.architecture");
    if (!arch || strcmp(arch, "qwen3moe")) return or_fail("only qwen3moe architecture is implemented");
    uint64_t v;
#define GET(key, dst)                                                      \
    do {                                                                   \
        if (or_gguf_uint(g, "qwen3moe." key, &v)) return -1;               \
        dst = v;                                                           \
    } while (0)
    GET("embedding_length", c->hidden);
    GET("attention.head_count", c->heads);
    GET("expert_used_count", c->top);
    uint64_t h = c->heads ? c->heads : 1;
    c->head_dim = or_gguf_uint(g, "qwen3moe.attention.key_length", &v) ? c->hidden / h : v;
    uint64_t vl = or_gguf_uint(g, "qwen3moe.attention.value_length", &v) ? c->head_dim : v;
    if (vl != c->head_dim) return or_fail("different key/value head sizes unsupported");
    GET("block_count", c->layers);
    GET("attention.head_count_kv", c->kvheads);
    GET("expert_count", c->experts);
    if (!or_gguf_uint(g, "qwen3moe.expert_feed_forward_length", &v)) {
        c->intermediate = v;
    } else {
        GET("feed_forward_length", c->intermediate);
        c->intermediate /= c->top ? c->top : 1;
    }
    const or_tensor *emb = or_gguf_find(g, "token_embd.weight");
    if (!emb) return or_fail("missing tensor token_embd.weight");
    if (emb->rank < 2) return or_fail("invalid embedding rank");
    c->vocab = emb->dims[1];
    GET("context_length", c->max_context);
#undef GET
    c->eps = or_gguf_float(g, "qwen3moe.attention.layer_norm_rms_epsilon", 1e-6f);
    c->theta = or_gguf_float(g, "qwen3moe.rope.freq_base", 1000000.f);
    if (!(c->hidden > 0 && c->layers > 0 && c->layers <= 256 && c->kvheads > 0 && c->heads > 0 &&
          c->heads % c->kvheads == 0 && c->head_dim > 0 && c->head_dim % 2 == 0 && c->top > 0 &&
          c->top <= c->experts && c->experts <= 1024 && c->intermediate > 0 && or_isfinite(c->eps) &&
          c->eps > 0.f && or_isfinite(c->theta) && c->theta > 0.f))
        return or_fail("invalid Qwen3 MoE config");
    uint64_t rd = or_gguf_uint(g, "qwen3moe.rope.dimension_count", &v) ? c->head_dim : v;
    if (rd != c->head_dim) return or_fail("partial rotary dimensions unsupported");
    const char *scaling = or_gguf_str(g, "qwen3moe.rope.scaling.type");
    if (scaling && strcmp(scaling, "none"))
        return or_fail("RoPE scaling is not implemented; use the original native-context model");
    return 0;
}

static int check_shape(const or_gguf *g, const char *name, int rank, uint64_t d0, uint64_t d1,
                       uint64_t d2) {
    const or_tensor *t = or_gguf_find(g, name);
    if (!t) return or_fail("missing tensor %s", name);
    uint64_t want[3] = {d0, d1, d2};
    if ((int)t->rank != rank) return or_fail("%s: unexpected shape", name);
    for (int k = 0; k < rank; k++)
        if (t->dims[k] != want[k]) return or_fail("%s: unexpected shape", name);
    return 0;
}

/* model.rs:91-149 */
static int validate_tensors(const or_config *c, const or_gguf *g) {
    char n[128];
    if (check_shape(g, "token_embd.weight", 2, c->hidden, c->vocab, 0)) return -1;
    if (check_shape(g, "output_norm.weight", 1, c->hidden, 0, 0)) return -1;
    if (or_gguf_find(g, "output.weight") && check_shape(g, "output.weight", 2, c->hidden, c->vocab, 0))
        return -1;
    for (uint64_t i = 0; i < c->layers; i++) {
#define CK(suffix, rank, a, b, e)                                          \
    snprintf(n, sizeof n, "blk.%llu." suffix ".weight", (unsigned long long)i); \
    if (check_shape(g, n, rank, a, b, e)) return -1;
        CK("attn_norm", 1, c->hidden, 0, 0);
        CK("ffn_norm", 1, c->hidden, 0, 0);
        CK("attn_q_norm", 1, c->head_dim, 0, 0);
        CK("attn_k_norm", 1, c->head_dim, 0, 0);
        CK("attn_q", 2, c->hidden, c->heads * c->head_dim, 0);
        CK("attn_k", 2, c->hidden, c->kvheads * c->head_dim, 0);
        CK("attn_v", 2, c->hidden, c->kvheads * c->head_dim, 0);
        CK("attn_output", 2, c->heads * c->head_dim, c->hidden, 0);
        CK("ffn_gate_inp", 2, c->hidden, c->experts, 0);
        CK("ffn_gate_exps", 3, c->hidden, c->intermediate, c->experts);
        CK("ffn_up_exps", 3, c->hidden, c->intermediate, c->experts);
        CK("ffn_down_exps", 3, c->intermediate, c->hidden, c->experts);
#undef CK
        char prefix[64];
        int pl = snprintf(prefix, sizeof prefix, "blk.%llu.", (unsigned long long)i);
        for (size_t t = 0; t < g->nt; t++) {
            const char *tn = g->t[t].name;
            size_t l = strlen(tn);
            if (!strncmp(tn, prefix, pl) && l >= 5 && !strcmp(tn + l - 5, ".bias"))
                return or_fail("unexpected bias tensors");
        }
    }
    return 0;
}

/* backend.rs:57-75 */
static int matrix(const or_gguf *g, const char *name, int64_t expert, const uint8_t **data,
                  uint32_t *kind, size_t *rows, size_t *cols) {
    const or_tensor *t = or_gguf_find(g, name);
    if (!t) return or_fail("missing tensor %s", name);
    if ((int)t->rank != (expert >= 0 ? 3 : 2)) return or_fail("matrix rank mismatch: %s", name);
    *cols = t->dims[0];
    *rows = t->dims[1];
    size_t rb;
    if (or_row_bytes(t->kind, *cols, &rb)) return -1;
    if (*rows && rb > SIZE_MAX / *rows) return or_fail("matrix overflow");
    size_t len = rb * *rows;
    size_t e = expert >= 0 ? (size_t)expert : 0;
    if (expert >= 0 && e >= t->dims[2]) return or_fail("expert out of bounds");
    *data = g->data + t->offset + e * len;
    *kind = t->kind;
    return 0;
}

static int bmatvec(or_model *m, const char *name, int64_t expert, const float *x, size_t n,
                   float *y, int threads) {
    const uint8_t *data;
    uint32_t kind;
    size_t rows, cols, rb;
    if (matrix(m->g, name, expert, &data, &kind, &rows, &cols)) return -1;
    if (cols != n) return or_fail("matvec shape mismatch %s", name);
    if (or_row_bytes(kind, cols, &rb)) return -1;
    return or_packed_matvec(data, rb * rows, kind, rows, cols, x, y, threads);
}

int or_model_matvec(or_model *m, const char *name, int64_t expert, const float *x, size_t cols,
                    float *y, size_t rows, int threads) {
    const uint8_t *data;
    uint32_t kind;
    size_t r, c;
    if (matrix(m->g, name, expert, &data, &kind, &r, &c)) return -1;
    if (c != cols) return or_fail("matvec shape mismatch %s", name);
    if (rows < r) return or_fail("output buffer too small");
    return bmatvec(m, name, expert, x, cols, y, threads);
}

or_model *or_model_new(or_gguf *g, size_t context) {
    or_config c;
    memset(&c, 0, sizeof c);
    if (config_from_gguf(g, &c) || validate_tensors(&c, g)) return NULL;
    if (!(context > 0 && context <= c.max_context)) {
        or_fail("context must be in 1..=%llu", (unsigned long long)c.max_context);
        return NULL;
    }
    or_model *m = calloc(1, sizeof *m);
    m->g = g;
    m->c = c;
    m->context = context;
    size_t ns = norm_stride(&c);
    m->norms = malloc(c.layers * ns * sizeof(float));
    m->output_norm = malloc(c.hidden * sizeof(float));
    m->last_router = calloc(c.layers * c.experts, sizeof(float));
    char n[128];
    for (uint64_t i = 0; i < c.layers; i++) {
        float *base = m->norms + i * ns;
        const char *names[4] = {"attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm"};
        float *dst[4] = {base, base + c.hidden, base + c.hidden + c.head_dim,
                         base + c.hidden + 2 * c.head_dim};
        size_t cnt[4] = {c.hidden, c.head_dim, c.head_dim, c.hidden};
        for (int k = 0; k < 4; k++) {
            snprintf(n, sizeof n, "blk.%llu.%s.weight", (unsigned long long)i, names[k]);
            if (or_gguf_row(g, n, 0, dst[k], cnt[k])) { or_model_free(m); return NULL; }
        }
    }
    if (or_gguf_row(g, "output_norm.weight", 0, m->output_norm, c.hidden)) {
        or_model_free(m);
        return NULL;
    }
    m->cache = calloc(c.layers, sizeof *m->cache);
    return m;
}

void or_model_free(or_model *m) {
    if (!m) return;
    if (m->cache)
        for (uint64_t i = 0; i < m->c.layers; i++) { free(m->cache[i].k); free(m->cache[i].v); }
    free(m->cache);
    free(m->norms);
    free(m->output_norm);
    free(m->last_router);
    free(m->forced);
    free(m);
}

int or_model_config(const or_model *m, or_config *c) {
    *c = m->c;
    return 0;
}

void or_model_reset(or_model *m) {
    for (uint64_t i = 0; i < m->c.layers; i++) m->cache[i].len = 0;
    m->position = 0;
}

size_t or_model_position(const or_model *m) { return m->position; }

static void kv_append(kvbuf *b, const float *k, const float *v, size_t n, size_t cap) {
    if (!b->k) {
        b->k = malloc(cap * sizeof(float));
        b->v = malloc(cap * sizeof(float));
    }
    memcpy(b->k + b->len, k, n * sizeof(float));
    memcpy(b->v + b->len, v, n * sizeof(float));
    b->len += n;
}

/* The body of the layer loop, model.rs:227-287, against an explicit KV
 * buffer (appended to) and position. */
static int layer_body(or_model *m, size_t i, float *x, size_t pos, kvbuf *kv, size_t kvcap,
                      uint32_t *ids_out, float *w_out, int threads) {
    const or_config *c = &m->c;
    size_t H = c->hidden, d = c->head_dim, nq = c->heads * d, nkv = c->kvheads * d;
    const float *nm = m->norms + i * norm_stride(c);
    char n[128];
    int rc = -1;
    float *xn = malloc(H * sizeof(float)), *q = malloc(nq * sizeof(float)),
          *k = malloc(nkv * sizeof(float)), *v = malloc(nkv * sizeof(float)),
          *a = malloc(nq * sizeof(float)), *o = malloc(H * sizeof(float)),
          *logits = malloc(c->experts * sizeof(float)), *moe = malloc(H * sizeof(float)),
          *gate = malloc(c->intermediate * sizeof(float)), *up = malloc(c->intermediate * sizeof(float)),
          *down = malloc(H * sizeof(float)), *w = malloc(c->top * sizeof(float));
    uint32_t *ids = malloc(c->top * sizeof(uint32_t));
    memcpy(xn, x, H * sizeof(float));
    if (or_rms(xn, nm, H, c->eps)) goto out;
#define MV(suffix, e, in, inlen, dst)                                              \
    snprintf(n, sizeof n, "blk.%zu." suffix ".weight", i);                         \
    if (bmatvec(m, n, e, in, inlen, dst, threads)) goto out;
    MV("attn_q", -1, xn, H, q);
    MV("attn_k", -1, xn, H, k);
    MV("attn_v", -1, xn, H, v);
    for (size_t h = 0; h < c->heads; h++)
        if (or_rms(q + h * d, nm + H, d, c->eps)) goto out;
    for (size_t h = 0; h < c->kvheads; h++)
        if (or_rms(k + h * d, nm + H + d, d, c->eps)) goto out;
    or_rope(q, nq, d, pos, c->theta);
    or_rope(k, nkv, d, pos, c->theta);
    kv_append(kv, k, v, nkv, kvcap);
    if (or_attention(q, kv->k, kv->v, kv->len, c->heads, c->kvheads, d, a)) goto out;
    MV("attn_output", -1, a, nq, o);
    for (size_t j = 0; j < H; j++) x[j] += o[j];
    memcpy(xn, x, H * sizeof(float));
    if (or_rms(xn, nm + H + 2 * d, H, c->eps)) goto out;
    MV("ffn_gate_inp", -1, xn, H, logits);
    memcpy(m->last_router + i * c->experts, logits, c->experts * sizeof(float));
    if (m->forced) {
        /* test hook: the caller's expert ids in the caller's rank order,
         * weighted by the softmax over this path's own logits at those ids
         * (the arithmetic of ops.rs:45-56 after its selection) */
        for (size_t s = 0; s < c->top; s++) {
            ids[s] = m->forced[i * c->top + s];
            w[s] = logits[ids[s]];
        }
        if (or_softmax(w, c->top)) goto out;
    } else if (or_route(logits, c->experts, c->top, ids, w)) {
        goto out;
    }
    for (size_t j = 0; j < H; j++) moe[j] = 0.f;
    for (size_t s = 0; s < c->top; s++) {
        MV("ffn_gate_exps", (int64_t)ids[s], xn, H, gate);
        MV("ffn_up_exps", (int64_t)ids[s], xn, H, up);
        for (size_t j = 0; j < c->intermediate; j++) gate[j] = (gate[j] / (1.f + expf(-gate[j]))) * up[j];
        MV("ffn_down_exps", (int64_t)ids[s], gate, c->intermediate, down);
        for (size_t j = 0; j < H; j++) moe[j] += w[s] * down[j];
    }
#undef MV
    for (size_t j = 0; j < H; j++) x[j] += moe[j];
    if (ids_out) memcpy(ids_out, ids, c->top * sizeof(uint32_t));
    if (w_out) memcpy(w_out, w, c->top * sizeof(float));
    rc = 0;
out:
    free(xn); free(q); free(k); free(v); free(a); free(o); free(logits); free(moe);
    free(gate); free(up); free(down); free(w); free(ids);
    return rc;
}

/* model.rs:217-302.  vocab = 0 stops after the last layer (a test's
 * shortcut for long prompts whose intermediate logits are not compared: no
 * final norm, vocab projection or finite check; the position still advances). */
static int forward_inner(or_model *m, uint32_t token, float *logits_out, int threads, int vocab) {
    const or_config *c = &m->c;
    if (!(m->position < m->context)) return or_fail("context limit %zu reached", m->context);
    if (!(token < c->vocab)) return or_fail("token outside vocabulary");
    size_t H = c->hidden;
    float *x = malloc(H * sizeof(float));
    float *logits = NULL;
    int rc = -1;
    if (or_gguf_row(m->g, "token_embd.weight", token, x, H)) goto out;
    size_t kvcap = m->context * c->kvheads * c->head_dim;
    for (size_t i = 0; i < c->layers; i++)
        if (layer_body(m, i, x, m->position, &m->cache[i], kvcap, NULL, NULL, threads)) goto out;
    if (!vocab) {
        m->position += 1;
        rc = 0;
        goto out;
    }
    if (or_rms(x, m->output_norm, H, c->eps)) goto out;
    const char *out = or_gguf_find(m->g, "output.weight") ? "output.weight" : "token_embd.weight";
    logits = malloc(c->vocab * sizeof(float));
    if (bmatvec(m, out, -1, x, H, logits, threads)) goto out;
    for (size_t j = 0; j < c->vocab; j++)
        if (!or_isfinite(logits[j])) { or_fail("nonfinite model output"); goto out; }
    m->position += 1;
    if (logits_out) memcpy(logits_out, logits, c->vocab * sizeof(float));
    rc = 0;
out:
    free(x);
    free(logits);
    return rc;
}

/* model.rs:209-216: roll back to a clean cache on any error */
static int forward_checked(or_model *m, uint32_t token, float *logits, int threads, int vocab) {
    int rc = forward_inner(m, token, logits, threads, vocab);
    free(m->forced); /* a forced routing holds for one step */
    m->forced = NULL;
    if (rc) {
        char saved[512];
        snprintf(saved, sizeof saved, "%s", or_last_error());
        or_model_reset(m);
        or_fail("%s", saved);
    }
    return rc;
}

int or_model_forward(or_model *m, uint32_t token, float *logits, int threads) {
    return forward_checked(m, token, logits, threads, 1);
}

int or_model_step(or_model *m, uint32_t token, int threads) {
    return forward_checked(m, token, NULL, threads, 0);
}

int or_layer_forward(or_model *m, size_t layer, float *x, size_t pos, const float *kprev,
                     const float *vprev, uint32_t *ids, float *w, int threads) {
    const or_config *c = &m->c;
    if (layer >= c->layers) return or_fail("layer out of range");
    size_t nkv = c->kvheads * c->head_dim;
    kvbuf kv = {0};
    size_t cap = (pos + 1) * nkv;
    kv.k = malloc(cap * sizeof(float));
    kv.v = malloc(cap * sizeof(float));
    if (pos) {
        memcpy(kv.k, kprev, pos * nkv * sizeof(float));
        memcpy(kv.v, vprev, pos * nkv * sizeof(float));
    }
    kv.len = pos * nkv;
    int rc = layer_body(m, layer, x, pos, &kv, cap, ids, w, threads);
    free(kv.k);
    free(kv.v);
    return rc;
}

int or_model_kv(const or_model *m, size_t layer, float *k, float *v, size_t cap) {
    if (layer >= m->c.layers) return or_fail("layer out of range");
    const kvbuf *b = &m->cache[layer];
    if (cap < b->len) return or_fail("buffer too small");
    if (b->len) {
        memcpy(k, b->k, b->len * sizeof(float));
        memcpy(v, b->v, b->len * sizeof(float));
    }
    return (int)0;
}

int or_model_force_routes(or_model *m, const uint32_t *ids, size_t n) {
    const or_config *c = &m->c;
    if (n != c->layers * c->top) return or_fail("forced routes need layers x top ids");
    for (size_t i = 0; i < c->layers; i++)
        for (size_t s = 0; s < c->top; s++) {
            uint32_t e = ids[i * c->top + s];
            if (e >= c->experts) return or_fail("forced expert out of range");
            for (size_t t = 0; t < s; t++)
                if (ids[i * c->top + t] == e) return or_fail("forced experts repeat");
        }
    free(m->forced);
    m->forced = malloc(n * sizeof(uint32_t));
    memcpy(m->forced, ids, n * sizeof(uint32_t));
    return 0;
}

int or_model_last_router(const or_model *m, size_t layer, float *out, size_t n) {
    if (layer >= m->c.layers || n < m->c.experts) return or_fail("bad arguments");
    memcpy(out, m->last_router + layer * m->c.experts, m->c.experts * sizeof(float));
    return 0;
}
