/*
 * CPU oracle for the Qwen3-MoE batch-1 token step.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU path (src/quant.rs, src/ops.rs, src/gguf.rs, src/model.rs,
 * src/backend.rs `Cpu`, src/sampling.rs with rand's StdRng restated).  It is what
 * the HIP engine is compared against; it is never linked into the engine and
 * nothing in the engine calls it.  Only tests/, __graft_entry__.smoke() and
 * bench.py's CPU-baseline leg load it.
 *
 * Numeric contract (what makes it bit-identical to the Rust CPU backend):
 *   - built with -O2 -ffp-contract=off, no -ffast-math: every product and sum
 *     is rounded separately, as Rust (which never contracts) does;
 *   - every reduction is a sequential left-to-right f32 fold; float `Sum`
 *     folds start at -0.0 (Rust's `impl Sum for f32`), explicit `0.` starts
 *     stay +0.0;
 *   - libm calls are the system's (expf, powf, sinf, cosf, sqrtf), which is
 *     what Rust std lowers f32::exp/powf/sin_cos/sqrt to on Linux.
 * Threading across matrix rows keeps each row's fold order, so the threaded
 * matvec is bit-identical to the single-threaded one.
 */
#ifndef QWEN_ORACLE_H
#define QWEN_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" if none). */
const char *or_last_error(void);

/* ---- quant.rs ---------------------------------------------------------- */
int or_layout(uint32_t kind, size_t *block, size_t *bytes);          /* quant.rs:5-11  */
int or_row_bytes(uint32_t kind, size_t cols, size_t *out);            /* quant.rs:12-21 */
float or_f16(uint16_t bits);                                          /* quant.rs:22-24 */
void or_kscale(const uint8_t *b12, size_t j, uint8_t *sc, uint8_t *m);/* quant.rs:25-34 */
float or_value(const uint8_t *row, uint32_t kind, size_t col);        /* quant.rs:36-80 */
int or_decode(const uint8_t *row, size_t len, uint32_t kind, size_t cols, float *out); /* quant.rs:81-84 */

/* ---- ops.rs ------------------------------------------------------------ */
int or_rms(float *x, const float *w, size_t n, float eps);            /* ops.rs:3-15  */
void or_rope(float *x, size_t n, size_t head, size_t pos, float theta); /* ops.rs:17-28 */
int or_softmax(float *x, size_t n);                                   /* ops.rs:29-44 */
int or_route(const float *logits, size_t n, size_t top, uint32_t *ids, float *w); /* ops.rs:45-56 */
int or_attention(const float *q, const float *k, const float *v, size_t klen,
                 size_t heads, size_t kvheads, size_t d, float *out); /* ops.rs:57-98 */

/* ---- sampling.rs (greedy branch) ---------------------------------------- */
int or_greedy(const float *logits, size_t n, uint32_t *out);          /* sampling.rs:26-35 */

/* ---- sampling.rs (stochastic branch) and rand's StdRng ------------------ */
/* ChaCha block function (djb layout: 64-bit counter in words 12-13, 64-bit
 * stream in 14-15), `rounds` = 20 for ChaCha20, 12 for StdRng. */
void or_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]);
/* rand_core 0.6.4 SeedableRng::seed_from_u64 seed expansion (PCG32). */
void or_stdrng_seed(uint64_t seed, uint32_t key[8]);
typedef struct or_sampler or_sampler;
or_sampler *or_sampler_new(uint64_t seed, float temperature, size_t top_k, float top_p); /* sampling.rs:10-25 */
void or_sampler_free(or_sampler *s);
float or_sampler_draw(or_sampler *s);                                 /* rng.gen::<f32>() */
int or_sampler_sample(or_sampler *s, const float *logits, size_t n, uint32_t *out); /* sampling.rs:26-63 */

/* ---- backend.rs Cpu::matvec on a packed matrix -------------------------- */
/* threads == 0: faithful path (per-element or_value, one thread), the
 * reference's backend.rs:41-48 loop.  threads >= 1: block decode per row,
 * rows spread over `threads` threads; bit-identical output. */
int or_packed_matvec(const uint8_t *data, size_t len, uint32_t kind, size_t rows,
                     size_t cols, const float *x, float *y, int threads);

/* ---- gguf.rs ----------------------------------------------------------- */
typedef struct or_gguf or_gguf;
/* Parses an in-memory GGUF image (the buffer is borrowed and must outlive the
 * handle); applies every check of gguf.rs:102-195. */
or_gguf *or_gguf_open(const uint8_t *data, size_t len);
void or_gguf_free(or_gguf *g);
size_t or_gguf_tensor_count(const or_gguf *g);
/* dims[0..3) and rank; offset is the absolute byte offset in the image. */
int or_gguf_tensor(const or_gguf *g, const char *name, uint32_t *kind, size_t *rank,
                   uint64_t dims[3], size_t *offset, size_t *len);
int or_gguf_row(const or_gguf *g, const char *name, size_t row, float *out, size_t n); /* gguf.rs:204-213 */
int or_gguf_uint(const or_gguf *g, const char *key, uint64_t *out);  /* gguf.rs:214-222 */
float or_gguf_float(const or_gguf *g, const char *key, float dflt);  /* gguf.rs:223-229 */
uint64_t or_gguf_packed_bytes(const or_gguf *g);                     /* main.rs:128 sum */

/* ---- model.rs ---------------------------------------------------------- */
typedef struct {
    uint64_t hidden, layers, heads, kvheads, head_dim, experts, top, intermediate,
        vocab, max_context;
    float eps, theta;
} or_config;

typedef struct or_model or_model;
or_model *or_model_new(or_gguf *g, size_t context);                 /* model.rs:173-201 */
void or_model_free(or_model *m);
int or_model_config(const or_model *m, or_config *c);
void or_model_reset(or_model *m);                                    /* model.rs:202-208 */
size_t or_model_position(const or_model *m);
/* Threads as in or_packed_matvec.  logits may be NULL. */
int or_model_forward(or_model *m, uint32_t token, float *logits, int threads); /* model.rs:209-302 */
/* The same step without the final norm and vocab projection (a test shortcut
 * for long prompts whose intermediate logits are not compared). */
int or_model_step(or_model *m, uint32_t token, int threads);
/* Backend::matvec surface: (name, expert) resolved as backend.rs:57-75. */
int or_model_matvec(or_model *m, const char *name, int64_t expert, const float *x,
                    size_t cols, float *y, size_t rows, int threads);
/* Layer-level entry (the loop body model.rs:227-287) for a single layer with a
 * caller-provided KV history: k/v are time-major [t][kvheads][head_dim] of
 * length `t` positions; the new token's k/v is appended inside, so the
 * history must hold exactly `pos` positions.  x is updated in place.
 * Optional diagnostics: ids/w receive the routed experts (top entries). */
int or_layer_forward(or_model *m, size_t layer, float *x, size_t pos,
                     const float *kprev, const float *vprev, uint32_t *ids, float *w,
                     int threads);
/* Read the model's KV cache for one layer (time-major), for tests. */
int or_model_kv(const or_model *m, size_t layer, float *k, float *v, size_t cap);
/* Test hook (no reference counterpart): the next forward/step routes
 * layer i to ids[i*top .. i*top+top) in that rank order instead of its own
 * top-k, with weights = softmax of its own router logits at those ids (the
 * arithmetic of ops.rs:45-56 after the selection).  Holds for one step. */
int or_model_force_routes(or_model *m, const uint32_t *ids, size_t n);
/* Router logits of the last forward (per layer, experts floats), for near-tie
 * diagnostics of end-to-end runs. */
int or_model_last_router(const or_model *m, size_t layer, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
