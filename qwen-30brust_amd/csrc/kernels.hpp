// Kernel argument blocks and launch helpers shared by kernels.hip and the
// engine.  Every kernel here is hand-written for gfx950 (wave64, 256-thread
// workgroups = 4 waves).
#pragma once
#include <hip/hip_runtime.h>

#include "qh_format.hpp"

namespace qh {

constexpr int kBlock = 256;  // threads per workgroup (4 wavefronts)
constexpr int kWaves = kBlock / 64;

// One packed matrix (or a stack of expert matrices) resident in HBM.
struct DevMat {
    const uint8_t* w;   // device row layout
    uint32_t kind;
    uint32_t rows, cols;
    uint32_t drb;       // device row stride (bytes)
    RowGeo geo;
    size_t expert_stride;  // bytes between experts (rows * drb); 0 for 2-D
    // the batched-prefill GEMMs' copy of the same rows in the tile layout
    // (rows a multiple of 32, columns of 256; built on the first batched
    // prefill), or null.  Per expert, blocks (row group G of 32 rows,
    // 256-column super-block b) at G * tile_group_bytes + b *
    // tile_block_bytes(kind); expert e at e * expert_stride (the same size as
    // the row layout).
    const uint8_t* wt;
};

// The block-quantised formats (the token step's and the prefill GEMMs').
QH_HD bool block_kind(uint32_t k) { return k == Q4_0 || k == Q8_0 || k == Q4_K || k == Q5_K || k == Q6_K; }

// Bytes of one tile-layout block: 32 rows x one 256-column super-block
// (32 x the format's bytes per 256 columns).
//   Q4_K (4,608): headers [row][16]; quants [slice 4][lane 64][16], lane =
//                 32 g + row holding bytes 32 slice + 16 g .. of the row's
//                 128 quant bytes.
//   Q5_K (5,632): as Q4_K, then high bits [lane 64][16] (bytes 16 g .. of
//                 the row's 32).
//   Q6_K (6,720): low bits [half 2][part 2][lane 64][16] (bytes 64 half +
//                 32 part + 16 g ..); high bits [half 2][lane 64][16] (bytes
//                 32 half + 16 g ..); scales [slice 4][row][4]; d [row][2].
//   Q4_0 (4,608): d [row][8][2] (the eight 32-column blocks); quants
//                 [slice 4][part 2][row][16] (block 2 slice + part).
//   Q8_0 (8,704): d [row][8][2]; quants [slice 4][part 2][lane 64][16]
//                 (bytes 16 g .. of block 2 slice + part).
// A wave's load of one field for 32 rows is one contiguous run of 0.5-1 KB.
constexpr uint32_t kTileQ4K = 4608, kTileQ5K = 5632, kTileQ6K = 6720, kTileQ4_0 = 4608, kTileQ8_0 = 8704;
QH_HD uint32_t tile_block_bytes(uint32_t kind) {
    return kind == Q6_K ? kTileQ6K : kind == Q5_K ? kTileQ5K : kind == Q8_0 ? kTileQ8_0 : kind == Q4_0 ? kTileQ4_0 : kTileQ4K;
}
// Bytes of one row group (32 rows, all super-blocks) of a cols-wide matrix.
QH_HD size_t tile_group_bytes(uint32_t kind, uint32_t cols) { return (size_t)(cols / 256) * tile_block_bytes(kind); }

// Device-resident step state of one sequence.
struct DevState {
    uint32_t pos;      // position of the token being processed
    uint32_t n_given;  // tokens[0, n_given) come from the caller; later ones from argmax
    uint32_t err;      // error bits (kErr*)
    uint32_t argmax;   // greedy id of the last completed step
    uint32_t pad[4];
};

enum : uint32_t {
    kErrRouter = 1u,   // non-finite router logits (src/ops.rs:46-49)
    kErrLogits = 2u,   // non-finite output logits (src/model.rs:296-299)
    kErrToken = 4u,    // token outside vocabulary (src/model.rs:222)
    kErrContext = 8u,  // position beyond the allocated context
    kErrSync = 16u,    // a cross-workgroup wait of the persistent step timed out (or was abandoned)
    kErrPlace = 32u,   // a workgroup of the persistent step ran on an XCD beyond the eight it assumes
    kErrRange = 64u,   // a batched-prefill activation outside the fp16 range (the prompt reruns exactly)
};

struct LayerW {
    DevMat q, k, v, o, router, gate, up, down;
    const float* attn_norm;
    const float* q_norm;
    const float* k_norm;
    const float* ffn_norm;
    float* kcache;  // [kvheads][ctx][d]
    float* vcache;
    // persistent step only: F[e][k] = sum_j router[e][j] ffn_norm[j] attn_output[j][k]
    // ([experts][heads*d] f32), so that router logit e of x' = x + Wo a is
    // s (sum_j router[e][j] ffn_norm[j] x[j] + F[e] . a)
    const float* rfold;
    uint32_t index;  // layer number (the routing log's row)
};

struct ModelDims {
    uint32_t hidden, heads, kvheads, head_dim, experts, top, ff, vocab, ctx;
    float eps;
    uint32_t layers;
};

// Scratch activations of one step.
struct Acts {
    float* x;          // [H] residual stream
    float* q;          // [heads*d]   raw q projection
    float* k;          // [kvheads*d] raw k projection
    float* v;          // [kvheads*d] raw v projection
    float* attn;       // [heads*d] attention output
    float* rpart;      // [router parts][experts+1] router partial dots + sum of squares
    float* logits_r;   // [experts] router logits of the last layer run (diagnostics)
    uint32_t* ids;     // [top] routed experts of the current layer
    float* wts;        // [top] their renormalised weights
    float* h;          // [top][pad32(ff)] SwiGLU outputs
    float* logits;     // [vocab]
    float* part;       // attention partials [heads][max_chunks][d+2]
    uint32_t* attn_cnt;  // [kvheads] last-arrival counters of the attention combine
    uint32_t* fin_key;   // [final blocks] vocab argmax partial keys
    uint32_t* fin_idx;   // [final blocks]
    uint32_t* tokens;    // [ctx+2]
    uint32_t* route_log; // [ctx][layers][top] routed experts of every layer at every position (diagnostics)
    float* gap_log;      // [ctx][layers] (top-th - (top+1)-th router logit) / max |logit| (diagnostics)
    const float2* rope;  // [ctx][d/2] (cos, sin)
    DevState* st;
};

// Arguments of the split-T attention kernels (see kernels.hip).
struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    size_t sh, st;      // element (t, g, j) at k[g*sh + t*st + j]
    uint32_t heads, kvheads, d, tc, max_chunks;
    uint32_t span;      // keys per chunk (k_attention_api: whole tiles of tc)
    float* part;        // [heads][max_chunks][d+2]
    uint32_t* counter;  // [kvheads]
    float* out;         // [heads*d]
    uint32_t* err;      // nullable: error bits (kErrContext on a chunk overflow)
};

// Arguments of the persistent token-step kernel (decode.hip): layers
// [l0, l1) of one token, followed (vocab = 1) by the vocab projection, argmax
// and position advance.  Workgroups hand values to each other as tagged
// words: bits 63..32 carry the tag of the phase that wrote the value (base +
// phase number), bits 31..0 the value; a reader waits for its tag.  The l*
// buffers hold one region per XCD (used only by that XCD's workgroups, through
// its L2); the g* buffers are read across XCDs.  Region strides in words.
constexpr uint32_t kPartWords = 130;        // words per attention chunk partial: o[128], m, l
constexpr uint32_t kDecodePhases = 7;       // tagged hand-overs per layer
constexpr uint32_t kDecodeXcds = 8;         // XCDs of the device (workgroup b on XCD b % 8)
constexpr uint32_t kDecodeWgPerXcd = 32;    // workgroups per XCD
constexpr uint32_t kDecodeQkvX = 768;       // q|k|v rows per XCD: 4 query heads + one KV head
constexpr uint32_t kDecodeStrideQkv = 768;
constexpr uint32_t kDecodeStridePart = 32 * 4 * kPartWords;  // [chunk][head] partials, up to 32 chunks
constexpr uint32_t kDecodeStrideX1 = 2048 + 128;  // x' and the unscaled router logits
constexpr uint32_t kDecodeStrideH = 768;
constexpr uint32_t kDecodeStrideX2 = 2048;
constexpr uint32_t kDecodeStrideG1 = 2048 + 128;  // o-projection partial and router terms of an XCD
constexpr uint32_t kDecodeStrideG2 = 2048;        // weighted down rows of an XCD
struct DecodeArgs {
    const LayerW* layers;  // device array, one per layer
    DevMat emb, out;
    const float* onorm;
    Acts a;
    ModelDims dm;
    uint32_t* abort_flag;  // set when a wait times out; every wait then returns
    uint64_t* lqkv;        // [8][768]   q|k|v rows of the XCD
    uint64_t* lpart;       // [8][32][4][130] attention chunk partials (o, m, l)
    uint64_t* lx1;         // [8][2176]  x' and the unscaled router logits
    uint64_t* lh;          // [8][768]   SwiGLU outputs of the XCD's expert
    uint64_t* lx2;         // [8][2048]  x''
    uint64_t* g1;          // [8][2176]  o-projection partials + router terms
    uint64_t* g2;          // [8][2048]  weighted down partials
    uint64_t* tfin;        // [gridDim.x][2] vocab argmax partials (key, index)
    uint32_t base;         // tag before this launch's first phase
    uint32_t l0, l1, vocab;
    uint32_t embed;        // 1: x of layer l0 is the embedding row of tokens[pos]; 0: the x the host left
};

// Device sampler (sample.hip): src/sampling.rs:26-63 over n logits in HBM.
// Up to kSampleMax candidates are sorted in LDS by one workgroup; more go
// through a global buffer (collected, bitonic-sorted by grid-wide steps,
// folded by one workgroup).
constexpr uint32_t kSampleMax = 4096;  // largest candidate list sorted in LDS
enum : uint32_t {
    kSampleBadLogits = 1u,  // empty or non-finite logits ("invalid logits")
    kSampleSupport = 2u,    // more than kSampleMax candidates: out[3] = P, out[4..5] = key of rank P - 1
    kSampleInternal = 3u,   // the candidate selection did not yield the expected count
    kSampleRank = 4u,       // the pick is the id of rank out[2] - 1, beyond the candidates
};
enum : uint32_t { kSampleModeSample = 0u, kSampleModeRank = 1u };
struct SampleArgs {
    const float* logits;   // [n]
    const uint8_t* valid;  // [n] 0 = masked to f32::MIN, or null
    uint32_t n, top_k;     // top_k 0 = no truncation
    float temperature, top_p;
    float draw;            // rand's gen::<f32>() for this call (unused at temperature 0)
    uint32_t mode;         // kSampleModeRank: out[0] = the id of rank `rank` of the sort
    uint32_t rank;
    uint32_t* out;         // [8] id, status, kept count, candidate count, key of rank P - 1 (2 words)
};
void launch_sample(const SampleArgs& a, hipStream_t s);
// The candidates beyond kSampleMax: cand[0, np) = the P composite keys >=
// theta (in any order), then 0 (np a power of two >= P); cnt a zeroed
// counter.  Then sorted descending and folded (sampling.rs:43-62) into out.
void launch_sample_collect(const SampleArgs& a, unsigned long long theta, uint32_t P, uint32_t np,
                           unsigned long long* cand, uint32_t* cnt, hipStream_t s);
void launch_sample_sort(unsigned long long* cand, uint32_t np, hipStream_t s);
void launch_sample_fold(const SampleArgs& a, const unsigned long long* cand, float* prob, uint32_t P, uint32_t K,
                        hipStream_t s);

// Column splits of the batched prefill's router logits (prefill.hip:
// k_pf_router writes one partial sum per split, k_pf_topk adds them in split
// order).
constexpr uint32_t kPfRouterSplit = 8;

// Batched-prefill attention (prefill.hip: k_pf_attn): floats of the (O, m, l)
// hand-over slot of one workgroup (4 waves x 68 values x 64 lanes) when two
// workgroups share a query block's keys; two slots and a zeroed counter per
// block pair and KV head.
constexpr uint32_t kPfAttnSlot = 4 * 68 * 64;

// Expert work list of the batched-prefill grouped GEMMs (prefill.hip): tile
// y covers rows [tm, tm + 128) of expert te; the rows of expert e are
// [goff[e], goff[e+1]) of the assignments sorted by expert.
struct ExpertTiles {
    const uint32_t* goff;   // [E + 1]
    const uint32_t* tok;    // [n_asg] token of each sorted assignment
    const uint32_t* asg;    // [n_asg] assignment id (token * top + slot) of each sorted assignment
    const uint32_t* te;     // [max tiles] expert of tile y
    const uint32_t* tm;     // [max tiles] first row (within the expert) of tile y
    const uint32_t* ntile;  // [1] tiles in use
};

// Matrices of one dense-projection GEMM launch of the batched prefill
// (prefill.hip: k_gemm_dense): column tiles [tile_end[i-1], tile_end[i]) of
// the grid belong to W[i], whose output columns start at cofs[i].
struct DenseSegs {
    DevMat W[3];
    uint32_t tile_end[3];  // cumulative 128-row tiles
    uint32_t cofs[3];      // output column of row 0
    uint32_t n;
};

}  // namespace qh
