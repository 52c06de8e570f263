/*
 * qwen_hip.h -- C ABI of the MI355X (gfx950) Qwen3-MoE decode engine.
 *
 * This is the drop-in boundary for the reference's compute backend.  The
 * reference binds its backends through a Rust trait (src/backend.rs:14-23):
 *
 *     pub trait Backend {
 *         fn matvec(&mut self, model: &Gguf, name: &str, expert: Option<usize>,
 *                   x: &[f32]) -> Result<Vec<f32>>;
 *         fn stats(&self) -> &Stats;
 *     }
 *
 * and drives the token loop through `Model::forward` (src/model.rs:209-302).
 * Each entry point below names the reference interface it replaces.
 *
 * Conventions (all entry points):
 *   - return 0 on success, nonzero on failure; qh_last_error() then returns a
 *     message owned by the context (the anyhow message of the reference);
 *   - plain host pointers and sizes; caller-owned host buffers; the context
 *     owns every device allocation;
 *   - one context per host thread, calls block until host-visible outputs are
 *     ready (`&mut self` + blocking poll in the reference);
 *   - no silent CPU fallback: without a usable gfx950 device qh_create fails.
 */
#ifndef QWEN_HIP_H
#define QWEN_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qh_ctx qh_ctx;

/* == backend::Stats (src/backend.rs:7-13). */
typedef struct {
    uint64_t matvecs;        /* matvecs performed (a fused token step counts the
                                reference's 3 + 1 + 1 + 3*top per layer + 1)   */
    uint64_t uploaded_bytes; /* host->device bytes (weights at load, inputs)  */
    uint64_t cache_hits;     /* always 0: all weights stay resident in HBM    */
    double matvec_ms;        /* wall time spent in matvec / forward calls     */
} qh_stats_t;

/* == model::Config (src/model.rs:5-19). */
typedef struct {
    uint64_t hidden, layers, heads, kvheads, head_dim, experts, top, intermediate,
        vocab, max_context;
    float eps, theta;
} qh_config_t;

/* Creates a context on HIP device `device` (one HIP stream per context).
 * Replaces `Vulkan::new` (src/backend.rs:95-161) / `Compute::backend`
 * (src/main.rs:42-60).  Fails if the device is not gfx950. */
int qh_create(int device, qh_ctx **out);
void qh_destroy(qh_ctx *ctx);
/* Message of the last failure on this context (or of qh_create when ctx is
 * NULL). */
const char *qh_last_error(const qh_ctx *ctx);

/* Parses and validates a GGUF image held in host memory and uploads every
 * tensor to HBM once (no LRU cache, no buffer splitting).  Replaces
 * `Gguf::open` (src/gguf.rs:102-195) + `Model::new` (src/model.rs:173-201)
 * with the same checks and error behaviour; `context` is the `--ctx` limit.
 * A new load invalidates the previous model (src/backend.rs:357-361). */
int qh_load_model(qh_ctx *ctx, const void *gguf_image, size_t len, size_t context);
/* Same, reading the file at `path`. */
int qh_load_model_file(qh_ctx *ctx, const char *path, size_t context);
int qh_model_config(const qh_ctx *ctx, qh_config_t *out);
/* Number of models loaded into this context so far (no counterpart in the
 * reference, where each Model owns its weights): a caller that keeps a
 * handle to "the loaded model" compares it with the value seen at load time
 * to detect that a later load replaced it. */
int qh_model_generation(const qh_ctx *ctx, uint64_t *out);
/* == Gguf::tensor (src/gguf.rs:196-200): GGML kind, rank and dims of a
 * loaded tensor (dims[0] = columns); "missing tensor {name}" otherwise. */
int qh_tensor_info(const qh_ctx *ctx, const char *name, uint32_t *kind, size_t *rank,
                   uint64_t dims[3]);
/* Sum of tensor payload bytes (src/main.rs:128 packed_weight_bytes). */
int qh_packed_weight_bytes(const qh_ctx *ctx, uint64_t *out);

/* == the `inspect` command (src/main.rs:119-131): Gguf::open + Config::from_gguf
 * + validate_tensors + the context check ("invalid context") + Config::kv_bytes
 * (src/model.rs:150-156, "KV size overflow"), on the file at `path`, with no
 * device work and no context object.  On failure qh_last_error(NULL) holds
 * the message. */
typedef struct {
    qh_config_t config;
    uint64_t tensor_count;
    uint64_t packed_weight_bytes;
    uint64_t kv_f32_bytes_at_context;
} qh_inspect_t;
int qh_inspect(const char *path, size_t context, qh_inspect_t *out);

/* == `Vulkan::devices` (src/backend.rs:162-172) for HIP: number of devices and
 * a one-line description "name (arch, CUs, GiB)" of device `device`.  On
 * failure qh_last_error(NULL) holds the message. */
int qh_device_count(int *out);
int qh_device_name(int device, char *buf, size_t cap);

/* == Backend::matvec (src/backend.rs:14-23, resolution as `matrix`
 * src/backend.rs:57-75): y[rows] = W x for tensor `name`, expert slab
 * `expert` (-1 = None).  Errors: missing tensor, rank mismatch, expert out
 * of bounds, cols != len(x). */
int qh_matvec(qh_ctx *ctx, const char *name, int64_t expert, const float *x, size_t cols,
              float *y, size_t rows);
/* == Backend::stats (src/backend.rs:22). */
int qh_stats(const qh_ctx *ctx, qh_stats_t *out);

/* == Vulkan::packed_matvec test surface (src/backend.rs:173-182): packed
 * GGUF rows given directly.  kind is the GGML type id (0 F32, 1 F16, 2 Q4_0,
 * 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K). */
int qh_packed_matvec(qh_ctx *ctx, const void *data, size_t len, uint32_t kind, size_t rows,
                     size_t cols, const float *x, float *y);

/* The per-expert down projections of one MoE layer (the loop of
 * src/model.rs:274-284) as one streaming launch: y[b] = W_b x[b] for b < nvec
 * (1-8), data = the nvec matrices of rows x cols packed GGUF rows back to
 * back, x = nvec x cols floats, y = nvec x rows floats.  Block-quantised
 * formats only (kinds 2, 8, 12, 13, 14), rows of up to 8,192 columns and at
 * most 12,288 x floats in all; other shapes are refused with an error. */
int qh_packed_matvec_batch(qh_ctx *ctx, const void *data, size_t len, uint32_t kind, size_t rows,
                           size_t cols, size_t nvec, const float *x, float *y);

/* == quant::decode (src/quant.rs:81-84) on the device, for `rows` packed
 * rows: out[rows*cols].  Bit-exact with the reference decoder. */
int qh_dequant(qh_ctx *ctx, const void *data, size_t len, uint32_t kind, size_t rows, size_t cols,
               float *out);

/* == ops::route (src/ops.rs:45-56): top `top` expert ids (descending, total
 * order, lower index on ties) and softmax over the chosen logits. */
int qh_route(qh_ctx *ctx, const float *logits, size_t n, size_t top, uint32_t *ids, float *w);

/* == Sampler::sample with temperature 0 (src/sampling.rs:26-35). */
int qh_argmax(qh_ctx *ctx, const float *logits, size_t n, uint32_t *out);

/* == ops::attention (src/ops.rs:57-98); k/v time-major [t][kvheads][d],
 * klen = t*kvheads*d floats. */
int qh_attention(qh_ctx *ctx, const float *q, const float *k, const float *v, size_t klen,
                 size_t heads, size_t kvheads, size_t d, float *out);
/* qh_attention on device buffers that allocates nothing (no counterpart in
 * the reference; for callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  q, k, v
 * and out are device pointers in qh_attention's layouts; the kernel's chunk
 * partials and counters live in a fixed 1 MiB device array of the library
 * (one per GPU).  Both entry points cap the key chunks per KV head at what
 * the array holds (a chunk then takes several key tiles), so any history
 * length runs; a shape one chunk of whose partials alone exceeds it
 * (heads x (head_dim + 2) floats > 1 MiB) is refused with an error.  stream NULL:
 * the context's stream, and the call returns when out is written; otherwise
 * the work is enqueued on that HIP stream and the call returns at once.
 * Calls that overlap on one GPU share the array and race. */
int qh_attention_noalloc(qh_ctx *ctx, const float *q, const float *k, const float *v, size_t klen,
                         size_t heads, size_t kvheads, size_t d, float *out, void *stream);

/* == Model::forward (src/model.rs:209-216): one causal token step on the
 * device (embedding, every layer, KV append, final norm, vocab projection,
 * finite check).  logits (room for logits_cap floats; the model's vocab are
 * written) and argmax may be NULL; logits_cap below the vocabulary is an
 * error.  On error the KV cache and position are reset, as the reference
 * rolls back. */
int qh_forward(qh_ctx *ctx, uint32_t token, float *logits, size_t logits_cap, uint32_t *argmax);
/* Sequential prefill of `n_prompt` tokens followed by `n_new` greedy tokens,
 * all chained on the device with no per-token host round trip (the
 * src/main.rs:250-282 loop with temperature 0).  out_tokens receives the
 * n_new generated ids; logits_last (room for logits_cap floats, nullable)
 * the logits that produced the last generated token. */
int qh_generate(qh_ctx *ctx, const uint32_t *prompt, size_t n_prompt, size_t n_new,
                uint32_t *out_tokens, float *logits_last, size_t logits_cap);
/* == Sampler (src/sampling.rs:3-65) with its rand 0.8.8 StdRng stream
 * (ChaCha12 seeded by seed_from_u64), host-side state: qh_sampler_create
 * replaces Sampler::new (src/sampling.rs:10-25) with its check ("invalid
 * sampling parameters", message in qh_last_error(NULL)); top_k 0 = no
 * truncation.  qh_sampler_draw returns the stream's next rng.gen::<f32>(). */
typedef struct qh_sampler qh_sampler;
int qh_sampler_create(uint64_t seed, float temperature, size_t top_k, float top_p, qh_sampler **out);
void qh_sampler_destroy(qh_sampler *sampler);
int qh_sampler_draw(qh_sampler *sampler, float *out);
/* The padding-vocab mask of src/main.rs:262-266: ids with valid[id] == 0 read
 * as f32::MIN in qh_sample (vocab bytes; NULL clears it). */
int qh_set_valid_tokens(qh_ctx *ctx, const uint8_t *valid, size_t n);
/* == Sampler::sample (src/sampling.rs:26-63) on the logits of the last token
 * step, on the device: greedy at temperature 0, else top-k, temperature,
 * top-p and one draw from the stream (consumed only on success), over any
 * number of candidates (up to 4096 sorted in one workgroup's LDS, more in
 * HBM).  Errors: "invalid logits"; more than 1,048,576 logits. */
int qh_sample(qh_ctx *ctx, qh_sampler *sampler, uint32_t *out);
/* The same on n caller logits with an optional mask (valid may be NULL). */
int qh_sample_logits(qh_ctx *ctx, qh_sampler *sampler, const float *logits, const uint8_t *valid,
                     size_t n, uint32_t *out);
/* == Model::reset (src/model.rs:202-208). */
int qh_reset(qh_ctx *ctx);
/* == Model::position (src/model.rs:170). */
int qh_position(const qh_ctx *ctx, size_t *out);

/* Batched prefill of `n` prompt tokens from the current position: replaces
 * the sequential prompt loop of src/main.rs:250-256 (one Model::forward per
 * prompt token, src/model.rs:209-302) with layer-at-a-time fp16 matrix-core
 * GEMMs and a causal flash-attention pass, in chunks of up to 2048 tokens.
 * Fills the KV cache for those positions, writes the greedy id after the
 * last prompt token to the device token ring (so qh_forward / qh_generate
 * continue from it), advances the position by n.  logits (room for
 * logits_cap floats) and argmax (nullable) receive the last prompt token's
 * output.  Numerics: fp16
 * operands with fp32 accumulation (logits within about 1e-2 relative of the
 * FP32 path).  Models the batched path does not cover (head_dim != 128, more
 * than 8 query heads per KV head, more than 128 experts, widths that are not
 * whole 256-column super-blocks, projections that are not block-quantised)
 * run the prompt through the exact token step instead, one per token on the
 * device (the same bits as n qh_forward calls).  Errors as that loop of
 * forwards: the first prompt token at the context limit fails with "context
 * limit N reached", a token outside the vocabulary with "token outside
 * vocabulary" (src/model.rs:219-223), and every failure leaves a clean cache
 * at position 0 (src/model.rs:209-216). */
int qh_prefill(qh_ctx *ctx, const uint32_t *prompt, size_t n, float *logits, size_t logits_cap,
               uint32_t *argmax);
/* Prefill implementation (no counterpart in the reference, whose prompt loop
 * is one forward per token): *out = 1 when qh_prefill runs the loaded model's
 * prompts through the batched GEMM path, 0 when through the exact token step. */
int qh_prefill_batched(const qh_ctx *ctx, int *out);
/* Diagnostics (no reference counterpart): how many prompts the batched
 * prefill has run again through the exact token step in this context because
 * its fp16 operands could not hold them (an activation above 65504 in
 * magnitude after an RMSNorm, in q, k or v, or out of the SwiGLU) or its
 * router or output logits were not finite.  The rerun's results are the exact
 * step's (the same bits as n qh_forward calls). */
int qh_prefill_reruns(const qh_ctx *ctx, uint64_t *out);
/* Memory control (no counterpart in the reference, which holds one copy of
 * the weights): frees the batched prefill's device memory, the tile-layout
 * copy of every layer's projection matrices (as many bytes again as their
 * row layout) and the chunk buffers.  The KV cache, the position and the
 * token step's weights stay; the next batched prefill builds both again.
 * For callers that prefill once and then decode with the memory given back. */
int qh_prefill_release(qh_ctx *ctx);
/* Device bytes the batched prefill holds now (tile copies + chunk buffers);
 * 0 before the first batched prefill and after qh_prefill_release. */
int qh_prefill_bytes(const qh_ctx *ctx, uint64_t *out);

/* One decoder layer (the loop body src/model.rs:227-287) applied to x[hidden]
 * in place at position `pos`, with this layer's KV history replaced by
 * kprev/vprev (time-major, `pos` positions).  ids/w (nullable) receive the
 * routed experts.  Resets the model position to 0 afterwards. */
int qh_layer_forward(qh_ctx *ctx, size_t layer, float *x, size_t pos, const float *kprev,
                     const float *vprev, uint32_t *ids, float *w);

/* Token-step implementation (no counterpart in the reference, whose step is
 * host-driven): *out = 1 when qh_forward / qh_generate / qh_layer_forward run
 * the persistent single-launch step (one workgroup per CU, phases handed over
 * through memory), 0 when they run the per-phase kernels.  The persistent
 * step covers Qwen3-MoE shapes with block-quantised projections (one format
 * for q, k, o, gate and up, v and down in it or Q6_K); other models always
 * use the per-phase kernels. */
int qh_persistent(const qh_ctx *ctx, int *out);
/* Selects the implementation for the loaded model (enable = 0: per-phase
 * kernels).  Enabling fails when the model is not covered. */
int qh_set_persistent(qh_ctx *ctx, int enable);

/* Diagnostics of the token steps (no counterpart in the reference, whose
 * KV cache and routing are private to Model): qh_route_log copies the
 * routed experts recorded for positions [pos0, pos0 + n), ids[n][layers][top]
 * in rank order, as the last step that processed each position (qh_forward,
 * qh_generate, qh_prefill, either step implementation) chose them;
 * qh_read_kv copies layer `layer`'s K and V for those positions in the
 * reference's time-major layout [t][kvheads][head_dim] (src/ops.rs:84,93);
 * qh_route_gap_log copies, for the same steps, how close each routing
 * decision was: gaps[n][layers] = (top-th - (top+1)-th largest router logit)
 * / max |router logit| (+inf when every expert is routed), a decision with a
 * gap near 0 being one that rounding may turn either way. */
int qh_route_log(qh_ctx *ctx, size_t pos0, size_t n, uint32_t *ids);
int qh_route_gap_log(qh_ctx *ctx, size_t pos0, size_t n, float *gaps);
int qh_read_kv(qh_ctx *ctx, size_t layer, size_t pos0, size_t n, float *k, float *v);

/* Fault injection for tests of the failure paths (no counterpart in the
 * reference): QH_FAULT_ABORT raises the persistent step's abort flag, so the
 * next step's waits give up at once (every kernel still exits normally) and
 * the step fails with "device synchronisation timed out" and a reset. */
#define QH_FAULT_ABORT 1u
int qh_fault_inject(qh_ctx *ctx, uint32_t kind);

/* Persistent-step timing (no counterpart in the reference): `steps` decode
 * steps continuing from the current position, queued back to back, with HIP
 * events on the context's stream around each step's one k_decode launch;
 * ms_decode receives its mean milliseconds per token.  ms_embed receives the time between the
 * step's first event and that launch (the embedding row is computed inside
 * k_decode, so it is an empty interval).  Fails unless the persistent step is
 * selected. */
int qh_profile_decode(qh_ctx *ctx, size_t steps, double *ms_embed, double *ms_decode);

/* Benchmark surface: `warmup` untimed then `steps` timed greedy decode steps
 * continuing from the current position, timed with HIP events on the
 * context's stream.  ms_total receives the timed milliseconds. */
int qh_bench_decode(qh_ctx *ctx, size_t warmup, size_t steps, double *ms_total);

/* Per-kernel-class timing of `steps` decode steps launched one kernel at a
 * time with HIP events between kernels on the context's stream (continuing
 * from the current position).  ms_by_class[QH_NUM_KERNEL_CLASSES] receives
 * the mean GPU milliseconds per token of each class, in this order:
 * qkv (norm + q/k/v projections), attention (Q/K norm, RoPE, KV append,
 * attention), oproj (output projection, residual, router partials), gateup
 * (router top-k, gate/up projections, SwiGLU), down (down projections,
 * combine, residual), vocab (final norm, vocab projection), finish
 * (argmax, next token). */
#define QH_NUM_KERNEL_CLASSES 7
int qh_profile_step(qh_ctx *ctx, size_t steps, double *ms_by_class, size_t nclass);

/* Timing of one benchmarked matvec shape. */
typedef struct qh_matvec_timing {
    double mean_ms;   /* back-to-back launches rotating over the copies: elapsed / iters */
    double median_ms; /* median over iters launches, each between its own pair of events */
    double empty_ms;  /* back-to-back launches of an empty kernel: the launch floor */
} qh_matvec_timing_t;

/* Benchmark surface for matvecs with device-resident inputs (no reference
 * counterpart).  data holds nvec (1-8) matrices of rows x cols packed GGUF
 * rows back to back, x their nvec input vectors (nvec x cols floats): nvec = 1
 * is Backend::matvec's launch, nvec > 1 the streaming kernel's batched form
 * (one launch for the routed experts' down projections of a MoE layer).
 * `copies` copies of the matrices are uploaded so that successive launches
 * stream distinct HBM rather than the 256 MB MALL; `iters` launches rotate
 * over them.  Fails if an output is not finite. */
int qh_bench_matvec(qh_ctx *ctx, const void *data, size_t len, uint32_t kind, size_t rows,
                    size_t cols, size_t nvec, const float *x, size_t copies, size_t iters,
                    qh_matvec_timing_t *out);

/* Read-only stream ceiling (no reference counterpart): `bytes` of device
 * memory, `copies` copies rotated over, each 16-byte word loaded once per
 * launch by a plain streaming kernel; mean and median launch times as for
 * qh_bench_matvec (empty_ms is 0).  The matvec bandwidths are read against it. */
int qh_bench_read(qh_ctx *ctx, size_t bytes, size_t copies, size_t iters, qh_matvec_timing_t *out);

#ifdef __cplusplus
}
#endif
#endif
