/*
 * Oracle: GGUF v2/v3 reader restated from src/gguf.rs (parse + validation;
 * the image is an in-memory buffer instead of a read-only mmap).  TEST
 * INFRASTRUCTURE ONLY (see oracle.h).
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"
#include "oracle_gguf.h"

typedef struct {
    const uint8_t *p;
    size_t len, pos;
    size_t budget; /* metadata byte budget, gguf.rs:107 */
} rd;

static int rd_bytes(rd *r, void *out, size_t n) {
    if (r->len - r->pos < n) return or_fail("failed to fill whole buffer");
    memcpy(out, r->p + r->pos, n);
    r->pos += n;
    return 0;
}
static int rd_u32(rd *r, uint32_t *v) { return rd_bytes(r, v, 4); }
static int rd_u64(rd *r, uint64_t *v) { return rd_bytes(r, v, 8); }
/* gguf.rs:44-48 */
static int rd_count(rd *r, uint64_t max, uint64_t *n) {
    if (rd_u64(r, n)) return -1;
    if (*n > max) return or_fail("GGUF count %llu exceeds limit %llu", (unsigned long long)*n,
                                 (unsigned long long)max);
    return 0;
}

static int utf8_valid(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        size_t k;
        uint32_t cp;
        if (c < 0x80) { i++; continue; }
        else if ((c & 0xe0) == 0xc0) { k = 1; cp = c & 0x1f; }
        else if ((c & 0xf0) == 0xe0) { k = 2; cp = c & 0x0f; }
        else if ((c & 0xf8) == 0xf0) { k = 3; cp = c & 0x07; }
        else return 0;
        if (n - i <= k) return 0;
        for (size_t j = 1; j <= k; j++) {
            if ((s[i + j] & 0xc0) != 0x80) return 0;
            cp = (cp << 6) | (s[i + j] & 0x3f);
        }
        if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) ||
            cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
            return 0;
        i += k + 1;
    }
    return 1;
}

/* gguf.rs:49-56 */
static int rd_string(rd *r, char **out) {
    uint64_t n;
    if (rd_count(r, 16u * 1024 * 1024, &n)) return -1;
    if (n > r->budget) return or_fail("GGUF metadata budget exceeded");
    r->budget -= n;
    if (r->len - r->pos < n) return or_fail("failed to fill whole buffer");
    if (!utf8_valid(r->p + r->pos, n)) return or_fail("invalid utf-8 sequence");
    if (out) {
        *out = malloc(n + 1);
        memcpy(*out, r->p + r->pos, n);
        (*out)[n] = 0;
    }
    r->pos += n;
    return 0;
}

static int finite64(double d) { return d - d == 0; }

/* gguf.rs:57-99.  Arrays are parsed (and budgeted) but not kept. */
static int rd_val(rd *r, uint32_t t, size_t depth, or_meta *m) {
    if (!(depth <= 4 && r->budget >= 8)) return or_fail("excessive metadata depth/size");
    r->budget -= 8;
    memset(m, 0, sizeof *m);
    uint8_t b1[1];
    uint16_t u16;
    uint32_t u32;
    uint64_t u64;
    switch (t) {
    case 0: if (rd_bytes(r, b1, 1)) return -1; m->tag = M_UINT; m->u = b1[0]; break;
    case 1: if (rd_bytes(r, b1, 1)) return -1; m->i = (int8_t)b1[0]; m->tag = m->i < 0 ? M_INT : M_UINT; m->u = (uint64_t)m->i; break;
    case 2: if (rd_bytes(r, &u16, 2)) return -1; m->tag = M_UINT; m->u = u16; break;
    case 3: if (rd_bytes(r, &u16, 2)) return -1; m->i = (int16_t)u16; m->tag = m->i < 0 ? M_INT : M_UINT; m->u = (uint64_t)m->i; break;
    case 4: if (rd_u32(r, &u32)) return -1; m->tag = M_UINT; m->u = u32; break;
    case 5: if (rd_u32(r, &u32)) return -1; m->i = (int32_t)u32; m->tag = m->i < 0 ? M_INT : M_UINT; m->u = (uint64_t)m->i; break;
    case 6: {
        float f;
        if (rd_bytes(r, &f, 4)) return -1;
        if (!or_isfinite(f)) return or_fail("nonfinite metadata");
        m->tag = M_FLOAT; m->f = f; break;
    }
    case 7:
        if (rd_bytes(r, b1, 1)) return -1;
        if (b1[0] > 1) return or_fail("invalid boolean");
        m->tag = M_BOOL; m->u = b1[0]; break;
    case 8: m->tag = M_STR; if (rd_string(r, &m->s)) return -1; break;
    case 9: {
        uint32_t ty;
        uint64_t n;
        if (rd_u32(r, &ty) || rd_count(r, 1000000, &n)) return -1;
        for (uint64_t i = 0; i < n; i++) {
            or_meta e;
            if (rd_val(r, ty, depth + 1, &e)) return -1;
            free(e.s);
        }
        m->tag = M_ARRAY; m->u = n; break;
    }
    case 10: if (rd_u64(r, &u64)) return -1; m->tag = M_UINT; m->u = u64; break;
    case 11: if (rd_u64(r, &u64)) return -1; m->i = (int64_t)u64; m->tag = m->i < 0 ? M_INT : M_UINT; m->u = u64; break;
    case 12: {
        double d;
        if (rd_bytes(r, &d, 8)) return -1;
        if (!finite64(d)) return or_fail("nonfinite metadata");
        m->tag = M_FLOAT; m->f = d; break;
    }
    default: return or_fail("unknown GGUF metadata type %u", t);
    }
    return 0;
}

static const or_meta *meta_get(const or_gguf *g, const char *key) {
    for (size_t i = 0; i < g->nmeta; i++)
        if (!strcmp(g->keys[i], key)) return &g->vals[i];
    return NULL;
}

const or_tensor *or_gguf_find(const or_gguf *g, const char *name) {
    for (size_t i = 0; i < g->nt; i++)
        if (!strcmp(g->t[i].name, name)) return &g->t[i];
    return NULL;
}

void or_gguf_free(or_gguf *g) {
    if (!g) return;
    for (size_t i = 0; i < g->nmeta; i++) { free(g->keys[i]); free(g->vals[i].s); }
    for (size_t i = 0; i < g->nt; i++) free(g->t[i].name);
    free(g->keys); free(g->vals); free(g->t); free(g);
}

static int cmp_name(const void *a, const void *b) {
    return strcmp(((const or_tensor *)a)->name, ((const or_tensor *)b)->name);
}
static int cmp_range(const void *a, const void *b) {
    const size_t *x = a, *y = b;
    if (x[0] != y[0]) return x[0] < y[0] ? -1 : 1;
    return (x[1] > y[1]) - (x[1] < y[1]);
}

/* gguf.rs:102-195 */
or_gguf *or_gguf_open(const uint8_t *data, size_t len) {
    rd r = {data, len, 0, 128u * 1024 * 1024};
    or_gguf *g = calloc(1, sizeof *g);
    g->data = data;
    g->len = len;
    char magic[4];
    uint32_t ver;
    uint64_t nt, nk;
    if (rd_bytes(&r, magic, 4)) goto fail;
    if (memcmp(magic, "GGUF", 4)) { or_fail("not a GGUF file"); goto fail; }
    if (rd_u32(&r, &ver)) goto fail;
    if (ver != 2 && ver != 3) { or_fail("GGUF version %u unsupported", ver); goto fail; }
    if (rd_count(&r, 100000, &nt) || rd_count(&r, 100000, &nk)) goto fail;
    g->keys = calloc(nk ? nk : 1, sizeof *g->keys);
    g->vals = calloc(nk ? nk : 1, sizeof *g->vals);
    for (uint64_t i = 0; i < nk; i++) {
        char *k;
        uint32_t t;
        if (rd_string(&r, &k)) goto fail;
        if (rd_u32(&r, &t)) { free(k); goto fail; }
        or_meta v;
        if (rd_val(&r, t, 0, &v)) { free(k); goto fail; }
        if (meta_get(g, k)) { free(k); free(v.s); or_fail("duplicate metadata key"); goto fail; }
        g->keys[g->nmeta] = k;
        g->vals[g->nmeta++] = v;
    }
    const or_meta *split = meta_get(g, "split.count");
    if (split && split->tag == M_UINT && split->u != 1) {
        or_fail("split GGUF not supported; merge shards first");
        goto fail;
    }
    g->t = calloc(nt ? nt : 1, sizeof *g->t);
    for (uint64_t i = 0; i < nt; i++) {
        or_tensor t;
        memset(&t, 0, sizeof t);
        uint32_t nd;
        if (rd_string(&r, &t.name)) goto fail;
        g->t[g->nt++] = t; /* owned from here on, for cleanup */
        or_tensor *tp = &g->t[g->nt - 1];
        if (rd_u32(&r, &nd)) goto fail;
        if (nd < 1 || nd > 3) { or_fail("unsupported tensor rank %u: %s", nd, tp->name); goto fail; }
        tp->rank = nd;
        for (uint32_t k = 0; k < nd; k++) {
            if (rd_u64(&r, &tp->dims[k])) goto fail;
            if (tp->dims[k] == 0) { or_fail("zero tensor dimension"); goto fail; }
        }
        uint64_t off;
        if (rd_u32(&r, &tp->kind) || rd_u64(&r, &off)) goto fail;
        tp->offset = off;
        size_t l;
        if (or_row_bytes(tp->kind, tp->dims[0], &l)) goto fail;
        for (uint32_t k = 1; k < nd; k++) {
            if (tp->dims[k] && l > SIZE_MAX / tp->dims[k]) { or_fail("tensor length overflow"); goto fail; }
            l *= tp->dims[k];
        }
        tp->len = l;
        for (size_t k = 0; k + 1 < g->nt; k++)
            if (!strcmp(g->t[k].name, tp->name)) { or_fail("duplicate tensor name"); goto fail; }
    }
    uint64_t alignment = 32;
    const or_meta *al = meta_get(g, "general.alignment");
    if (al && al->tag == M_UINT) alignment = al->u;
    if (!(alignment && !(alignment & (alignment - 1)) && alignment <= 4096)) {
        or_fail("invalid GGUF alignment");
        goto fail;
    }
    size_t start = (r.pos + alignment - 1) & ~(size_t)(alignment - 1);
    /* gguf.rs iterates a name-ordered map; keep that order for error parity */
    qsort(g->t, g->nt, sizeof *g->t, cmp_name);
    size_t *ranges = malloc(2 * (g->nt ? g->nt : 1) * sizeof(size_t));
    for (size_t i = 0; i < g->nt; i++) {
        or_tensor *t = &g->t[i];
        if (t->offset % alignment) { or_fail("unaligned tensor %s", t->name); free(ranges); goto fail; }
        if (t->offset > SIZE_MAX - start) { or_fail("tensor offset overflow"); free(ranges); goto fail; }
        t->offset += start;
        if (t->len > SIZE_MAX - t->offset) { or_fail("tensor end overflow"); free(ranges); goto fail; }
        size_t end = t->offset + t->len;
        if (end > len) { or_fail("truncated tensor %s", t->name); free(ranges); goto fail; }
        ranges[2 * i] = t->offset;
        ranges[2 * i + 1] = end;
    }
    qsort(ranges, g->nt, 2 * sizeof(size_t), cmp_range);
    for (size_t i = 1; i < g->nt; i++)
        if (ranges[2 * (i - 1) + 1] > ranges[2 * i]) { or_fail("overlapping tensors"); free(ranges); goto fail; }
    free(ranges);
    return g;
fail:
    or_gguf_free(g);
    return NULL;
}

size_t or_gguf_tensor_count(const or_gguf *g) { return g->nt; }

int or_gguf_tensor(const or_gguf *g, const char *name, uint32_t *kind, size_t *rank,
                   uint64_t dims[3], size_t *offset, size_t *len) {
    const or_tensor *t = or_gguf_find(g, name);
    if (!t) return or_fail("missing tensor %s", name);
    if (kind) *kind = t->kind;
    if (rank) *rank = t->rank;
    if (dims) for (int k = 0; k < 3; k++) dims[k] = k < (int)t->rank ? t->dims[k] : 0;
    if (offset) *offset = t->offset;
    if (len) *len = t->len;
    return 0;
}

/* gguf.rs:204-213 */
int or_gguf_row(const or_gguf *g, const char *name, size_t row, float *out, size_t n) {
    const or_tensor *t = or_gguf_find(g, name);
    if (!t) return or_fail("missing tensor %s", name);
    size_t size;
    if (or_row_bytes(t->kind, t->dims[0], &size)) return -1;
    if (row >= t->len / size) return or_fail("row out of bounds: %s", name);
    if (n < t->dims[0]) return or_fail("output buffer too small");
    return or_decode(g->data + t->offset + row * size, size, t->kind, t->dims[0], out);
}

/* gguf.rs:214-222: serde_json as_u64 accepts non-negative integers only */
int or_gguf_uint(const or_gguf *g, const char *key, uint64_t *out) {
    const or_meta *m = meta_get(g, key);
    if (!m || m->tag != M_UINT) return or_fail("missing integer %s", key);
    *out = m->u;
    return 0;
}

/* gguf.rs:223-229: as_f64 accepts any number */
float or_gguf_float(const or_gguf *g, const char *key, float dflt) {
    const or_meta *m = meta_get(g, key);
    if (!m) return dflt;
    if (m->tag == M_UINT) return (float)(double)m->u;
    if (m->tag == M_INT) return (float)(double)m->i;
    if (m->tag == M_FLOAT) return (float)m->f;
    return dflt;
}

const char *or_gguf_str(const or_gguf *g, const char *key) {
    const or_meta *m = meta_get(g, key);
    return m && m->tag == M_STR ? m->s : NULL;
}

uint64_t or_gguf_packed_bytes(const or_gguf *g) {
    uint64_t s = 0;
    for (size_t i = 0; i < g->nt; i++) s += g->t[i].len;
    return s;
}
