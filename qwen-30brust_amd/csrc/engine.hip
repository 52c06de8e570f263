// Host side of the decode engine: model upload, the captured token-step
// graph, and the C ABI declared in include/qwen_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fcntl.h>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <vector>

#include "../../include/qwen_hip.h"
#include "gguf.hpp"
#include "kernels.hpp"
#include "qh_rows.hpp"
#include "qh_tile.hpp"

namespace qh {
// Kernels (kernels.hip).
__global__ void k_repack(const uint8_t*, uint8_t*, uint32_t, uint32_t, size_t, size_t, size_t);
__global__ void k_dequant(DevMat, size_t, size_t, float*);
__global__ void k_fill_u32(uint32_t*, size_t, uint32_t);
__global__ void k_router_fold(DevMat, const float*, const float*, uint32_t, uint32_t, uint32_t, float*);
template <int R> __global__ void k_matvec(DevMat, const float*, float*, int);
__global__ void k_route(const float*, uint32_t, uint32_t, uint32_t*, float*, uint32_t*);
__global__ void k_argmax(const float*, uint32_t, int32_t*, uint32_t*, uint32_t*, uint32_t*, uint32_t*);
__global__ void k_attention_api(AttnArgs, uint32_t);
// Token-step kernels (step.hip).
// Template argument C: held chunk slots per lane (tile_slots), 0 = general.
template <int C> __global__ void k_qkv(LayerW, DevMat, Acts, ModelDims, int);
__global__ void k_attn(LayerW, AttnArgs, Acts, ModelDims);
__global__ void k_attn128(LayerW, AttnArgs, Acts, ModelDims);
template <int C> __global__ void k_oproj(LayerW, Acts, ModelDims);
template <int C> __global__ void k_gateup(LayerW, Acts, ModelDims, uint32_t);
template <int C> __global__ void k_down(LayerW, Acts, ModelDims);
template <int C> __global__ void k_vocab(DevMat, const float*, Acts, ModelDims);
__global__ void k_finish(Acts, ModelDims, uint32_t);
// Persistent token step (decode.hip).
template <uint32_t KM> __global__ void k_decode(DecodeArgs);
__global__ void k_xcd_map(uint32_t*);
// Streaming quantised matvec (matvec.hip).
bool launch_mv_stream(const DevMat&, const uint8_t* const*, uint32_t, const float*, float*, uint32_t, hipStream_t);
void launch_empty(hipStream_t);
void launch_read_stream(const void*, size_t, uint32_t*, uint32_t, hipStream_t);
// Batched prefill (prefill.hip).
template <uint32_t K>
__global__ void k_gemm_gateup(const _Float16*, uint32_t, ExpertTiles, DevMat, DevMat, _Float16*, uint32_t*);
template <uint32_t K> __global__ void k_gemm_down(const _Float16*, ExpertTiles, DevMat, float*);
__global__ void k_gemm_dense(const _Float16*, uint32_t, DenseSegs, float*, uint32_t, size_t);
__global__ void k_pf_embed(DevMat, const uint32_t*, uint32_t, uint32_t, float*, DevState*);
__global__ void k_tile_gemm(DevMat, uint32_t, uint8_t*);
__global__ void k_pf_norm(float*, const float*, uint32_t, float, _Float16*, float*, const float*, size_t, uint32_t*);
__global__ void k_pf_qkrope(const float*, const float*, const float*, const float2*, uint32_t, uint32_t, uint32_t,
                            uint32_t, uint32_t, float, _Float16*, float*, float*, _Float16*, _Float16*, uint32_t,
                            uint32_t*);
__global__ void k_pf_attn(const _Float16*, const _Float16*, const _Float16*, uint32_t, uint32_t, uint32_t, uint32_t,
                          uint32_t, uint32_t, _Float16*, float*, uint32_t*);
__global__ void k_pf_kvh(const float*, const float*, uint32_t, uint32_t, uint32_t, uint32_t, _Float16*, _Float16*);
__global__ void k_pf_router(const float*, DevMat, uint32_t, uint32_t, uint32_t, float*);
__global__ void k_pf_topk(const float*, uint32_t, uint32_t, uint32_t, uint32_t*, float*, DevState*, uint32_t*, float*,
                          uint32_t, uint32_t, uint32_t);
__global__ void k_pf_group(const uint32_t*, uint32_t, uint32_t, uint32_t, uint32_t*, uint32_t*, uint32_t*, uint32_t*,
                           uint32_t*, uint32_t*);
__global__ void k_pf_combine(float*, const float*, const float*, uint32_t, uint32_t, const float*, float, _Float16*,
                             uint32_t*);
}  // namespace qh

using namespace qh;

#define HIP_OK(expr)                                                                          \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) throw Error(std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

namespace {

constexpr uint32_t kMaxGrid = 2048;     // grid-stride cap for matvec-shaped kernels
constexpr uint32_t kRouterParts = 64;   // most k_oproj workgroups (router partial rows)
constexpr int kWideBlock = 512;         // k_oproj and k_gateup workgroup size

uint32_t pad32h(uint64_t n) { return (uint32_t)((n + 31) / 32 * 32); }

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
        return *this;
    }
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t bytes) {
        release();
        HIP_OK(hipMalloc(&p, std::max<size_t>(bytes, 256)));
        n = bytes;
    }
    // Grows (never shrinks) to at least `bytes`.
    void reserve(size_t bytes) {
        if (p && n >= bytes) return;
        alloc(bytes);
    }
    template <class T> T* as() const { return reinterpret_cast<T*>(p); }
};

struct HostPinned {
    void* p = nullptr;
    size_t n = 0;
    ~HostPinned() { if (p) (void)hipHostFree(p); }
    void reserve(size_t bytes) {
        if (p && n >= bytes) return;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        HIP_OK(hipHostMalloc(&p, bytes));
        n = bytes;
    }
};

struct ModelTensor {
    uint32_t kind = 0;
    std::vector<uint64_t> dims;
    DevBuf buf;
    DevMat mat{};   // rank >= 2 (per-expert view for rank 3 via expert_stride)
    DevBuf f32;     // rank 1: decoded f32 vector
};

DevMat make_mat(const uint8_t* w, uint32_t kind, uint64_t rows, uint64_t cols, uint64_t experts) {
    DevMat m{};
    m.w = w;
    m.kind = kind;
    m.rows = (uint32_t)rows;
    m.cols = (uint32_t)cols;
    m.drb = (uint32_t)dev_row_bytes(kind, cols);
    m.geo = row_geo(kind, cols);
    m.expert_stride = experts ? (size_t)rows * m.drb : 0;
    return m;
}

uint32_t blocks_for(uint64_t waves) {
    uint64_t b = (waves + kWaves - 1) / kWaves;
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(b, kMaxGrid));
}
uint64_t groups_host(uint64_t rows, uint64_t cols, int R) {
    int L = lanes_per_row((uint32_t)cols);
    uint64_t per = (uint64_t)R * (64 / L);
    return (rows + per - 1) / per;
}

}  // namespace

// ------------------------------------------------ no-allocation scratch --
// Device memory of qh_attention_noalloc: the chunk partials
// [heads][chunks][d+2] and the last-arrival counters [kvheads] of
// k_attention_api, at most kNoAllocScratchBytes.  Every GPU the library runs
// on holds its own copy for the life of the process; host code uses only the
// per-device address that hipGetSymbolAddress returns (the array's name is a
// host-side stand-in, not a device address).
namespace {
constexpr size_t kNoAllocScratchBytes = 1u << 20;
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mu;
std::array<void*, kNoAllocMaxDevices> g_scratch_ptr{};
}  // namespace
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Resolves this device's copy of `scratch` once per device (called by
// qh_create with the device current).
static void noalloc_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kNoAllocMaxDevices) throw Error("device index beyond the scratch table");
    if (g_scratch_ptr[device]) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
        throw Error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[device] = p;
}

struct qh_ctx {
    int device = 0;
    uint32_t num_cu = 0;  // compute units of the device
    hipStream_t s = nullptr;
    std::string err;
    qh_stats_t stats{};

    // model
    bool loaded = false;
    uint64_t generation = 0;  // models loaded so far (qh_model_generation)
    Config cfg{};
    ModelDims dm{};
    uint64_t packed = 0;
    std::map<std::string, ModelTensor> tensors;
    std::vector<LayerW> layers;
    std::vector<AttnArgs> attn;
    DevMat emb{}, out{};
    const float* onorm = nullptr;
    size_t context = 0, pos = 0;

    // activations / caches
    DevBuf acts_buf, kv, rope_buf;
    Acts acts{};
    uint32_t max_chunks = 0, tc = 32;
    bool attn128 = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;  // QH_NO_GRAPH=1: launch the step's kernels directly (profilers)

    // persistent token step (k_decode): one launch per token
    bool persist_ok = false;  // the model's formats and shapes are covered
    bool persist = false;     // and it is enabled (qh_set_persistent(0) disables it; QH_NO_PERSIST=1 at load leaves it out)
    uint32_t nwg = 0;         // workgroups of k_decode (one per CU)
    uint64_t prefill_reruns = 0;  // prompts the batched prefill handed to the exact step (numeric faults)
    const void* decode_fn = nullptr;  // k_decode<KM> for the model's main format KM
    uint32_t flag_base = 0;   // tag of the last phase launched
    DevBuf layers_dev, sync_buf;  // sync_buf: abort flag and tagged exchange words
    DevBuf rfold;                 // router folds of every layer ([layers][experts][heads*d])
    size_t sync_bytes = 0;
    DecodeArgs dargs{};

    // launch geometry of the step kernels; per layer the held chunk slots
    // (0 qkv, 1 oproj, 2 gateup, 3 down) and for the vocab projection
    uint32_t g_qkv = 1, g_o = 1, g_gu = 1, g_down = 1, g_vocab = 1;
    std::vector<std::array<int, 4>> slots;
    int vocab_slots = 0;
    size_t lds_h = 0, lds_attn = 0, lds_o = 0, lds_gu = 0, lds_down = 0;

    // batched prefill: buffers for chunks of up to pf_cap tokens
    struct Prefill {
        uint32_t cap = 0;
        DevBuf buf;
        float *X = nullptr, *Xn32 = nullptr, *QKV = nullptr, *LR = nullptr, *wts = nullptr, *Y = nullptr;
        _Float16 *Xn16 = nullptr, *Q16 = nullptr, *O16 = nullptr, *Hs = nullptr, *Kh = nullptr, *Vth = nullptr;
        uint32_t *ids = nullptr, *goff = nullptr, *tok = nullptr, *asg = nullptr, *te = nullptr, *tm = nullptr,
                 *ntile = nullptr;
        float* axw = nullptr;      // attention hand-over slots (kPfAttnSlot floats each)
        uint32_t* axc = nullptr;   // their arrival counters (zero between launches)
        uint32_t max_tiles = 0;
        // tile-layout copies of the GEMMs' matrices (DevMat::wt of q, k, v,
        // o, gate, up, down of every layer), built on the first batched
        // prefill: as many bytes again as those matrices' row layout
        DevBuf tiles;
        bool tiled = false;
    } pf;

    // scratch for the API surfaces
    DevBuf sa, sb, sc, sd;
    HostPinned pin;

    // sampler: the padding-vocab mask of the loaded model, host-logits upload
    // buffers and the result words
    DevBuf valid, samp_logits, samp_valid, samp_out, samp_big;
    size_t valid_n = 0;

    ~qh_ctx() {
        drop_model();
        if (s) (void)hipStreamDestroy(s);
    }

    void drop_model() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
        tensors.clear();
        layers.clear();
        attn.clear();
        acts_buf.release();
        pf.buf.release();
        pf.cap = 0;
        pf.tiles.release();
        pf.tiled = false;
        layers_dev.release();
        sync_buf.release();
        rfold.release();
        persist_ok = persist = false;
        kv.release();
        rope_buf.release();
        valid.release();
        valid_n = 0;
        loaded = false;
        pos = 0;
    }
};

namespace {

thread_local std::string g_create_err;

template <class F> int guarded(qh_ctx* c, F f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        if (c) c->err = e.what();
        return 1;
    }
}

void sync(qh_ctx* c) { HIP_OK(hipStreamSynchronize(c->s)); }

// Uploads `rows` packed GGUF rows (src) into device rows at dst, repacking on
// the device through a staging buffer.
void upload_rows(qh_ctx* c, const uint8_t* src, uint8_t* dst, uint32_t kind, uint64_t cols,
                 uint64_t rows) {
    const size_t src_rb = gguf_row_bytes(kind, cols), dst_rb = dev_row_bytes(kind, cols);
    const size_t stage = 256u << 20;
    const uint64_t per = std::max<uint64_t>(1, stage / std::max<size_t>(src_rb, 1));
    c->sa.reserve(std::min<uint64_t>(rows, per) * src_rb);
    HIP_OK(hipMemsetAsync(dst, 0, rows * dst_rb, c->s));
    for (uint64_t r = 0; r < rows; r += per) {
        uint64_t n = std::min(per, rows - r);
        HIP_OK(hipMemcpyAsync(c->sa.p, src + r * src_rb, n * src_rb, hipMemcpyHostToDevice, c->s));
        uint64_t total = n * src_rb;
        uint32_t grid = (uint32_t)std::min<uint64_t>((total + kBlock - 1) / kBlock, 65535);
        hipLaunchKernelGGL(k_repack, dim3(grid), dim3(kBlock), 0, c->s, c->sa.as<const uint8_t>(),
                           dst + r * dst_rb, kind, (uint32_t)cols, (size_t)n, src_rb, dst_rb);
        HIP_OK(hipGetLastError());
        HIP_OK(hipStreamSynchronize(c->s));  // staging buffer reused
    }
    c->stats.uploaded_bytes += rows * src_rb;
}

void launch_matvec(qh_ctx* c, const DevMat& m, const float* x, float* y, int R = 4) {
    // block-quantised rows of up to 8,192 columns: the streaming kernel
    const uint8_t* mats[1] = {m.w};
    if (launch_mv_stream(m, mats, 1, x, y, c->num_cu, c->s)) {
        HIP_OK(hipGetLastError());
        return;
    }
    const uint32_t np = pad32h(m.cols);
    const bool lds = np * 4 <= 65536;
    const size_t smem = lds ? np * 4 : 0;
    const uint32_t grid = blocks_for(groups_host(m.rows, m.cols, R));
    switch (R) {
    case 1: hipLaunchKernelGGL(k_matvec<1>, dim3(grid), dim3(kBlock), smem, c->s, m, x, y, (int)lds); break;
    case 2: hipLaunchKernelGGL(k_matvec<2>, dim3(grid), dim3(kBlock), smem, c->s, m, x, y, (int)lds); break;
    case 8: hipLaunchKernelGGL(k_matvec<8>, dim3(grid), dim3(kBlock), smem, c->s, m, x, y, (int)lds); break;
    default: hipLaunchKernelGGL(k_matvec<4>, dim3(grid), dim3(kBlock), smem, c->s, m, x, y, (int)lds); break;
    }
    HIP_OK(hipGetLastError());
}

// Row-parallel R heuristic: enough waves to cover the GPU, more rows per wave
// for tall matrices.
int pick_r(uint64_t rows, uint64_t cols) {
    for (int R : {8, 4, 2}) {
        if (groups_host(rows, cols, R) >= 2048) return R;
    }
    return 1;
}

// Upload host vector x (n floats) zero-padded to pad32.
const float* upload_x(qh_ctx* c, DevBuf& b, const float* x, size_t n) {
    size_t np = pad32h(n);
    b.reserve(np * 4);
    HIP_OK(hipMemsetAsync(b.p, 0, np * 4, c->s));
    if (n) HIP_OK(hipMemcpyAsync(b.p, x, n * 4, hipMemcpyHostToDevice, c->s));
    c->stats.uploaded_bytes += n * 4;
    return b.as<const float>();
}

// ---------------------------------------------------------------- model --
void build_rope(qh_ctx* c) {
    // (cos, sin) of angle = pos * theta^(-2i/d), computed as src/ops.rs:20-21
    // does (f32 powf, sin_cos), for every position of the context.
    const uint32_t d = c->dm.head_dim, half = d / 2;
    std::vector<float> tab((size_t)c->context * half * 2);
    std::vector<float> freq(half);
    for (uint32_t i = 0; i < half; i++) {
        volatile float e = -2.f * (float)i;
        e = e / (float)d;
        freq[i] = powf(c->cfg.theta, e);
    }
    for (size_t p = 0; p < c->context; p++)
        for (uint32_t i = 0; i < half; i++) {
            volatile float angle = (float)p * freq[i];
            tab[(p * half + i) * 2] = cosf(angle);
            tab[(p * half + i) * 2 + 1] = sinf(angle);
        }
    c->rope_buf.alloc(tab.size() * 4);
    HIP_OK(hipMemcpy(c->rope_buf.p, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
}

void alloc_acts(qh_ctx* c) {
    const ModelDims& d = c->dm;
    const uint64_t hp = pad32h(d.hidden), qd = pad32h((uint64_t)d.heads * d.head_dim),
                   kvd = pad32h((uint64_t)d.kvheads * d.head_dim), fp = pad32h(d.ff);
    Acts& a = c->acts;
    std::vector<std::pair<size_t, void**>> parts = {
        {hp * 4, (void**)&a.x},
        {qd * 4, (void**)&a.q},
        {kvd * 4, (void**)&a.k},
        {kvd * 4, (void**)&a.v},
        {qd * 4, (void**)&a.attn},
        {(uint64_t)kRouterParts * (d.experts + 1) * 4, (void**)&a.rpart},
        {pad32h(d.experts) * 4, (void**)&a.logits_r},
        {pad32h(d.top) * 4, (void**)&a.ids},
        {pad32h(d.top) * 4, (void**)&a.wts},
        {(uint64_t)d.top * fp * 4, (void**)&a.h},
        {pad32h(d.vocab) * 4, (void**)&a.logits},
        {(uint64_t)d.heads * c->max_chunks * (d.head_dim + 2) * 4, (void**)&a.part},
        {pad32h(d.kvheads) * 4, (void**)&a.attn_cnt},
        {kMaxGrid * 4, (void**)&a.fin_key},
        {kMaxGrid * 4, (void**)&a.fin_idx},
        {pad32h(c->context + 2) * 4, (void**)&a.tokens},
        {(uint64_t)c->context * d.layers * d.top * 4, (void**)&a.route_log},
        {(uint64_t)c->context * d.layers * 4, (void**)&a.gap_log},
        {256, (void**)&a.st},
    };
    size_t total = 0;
    for (auto& p : parts) total += (p.first + 255) / 256 * 256;
    c->acts_buf.alloc(total);
    HIP_OK(hipMemset(c->acts_buf.p, 0, total));
    size_t off = 0;
    for (auto& p : parts) {
        *p.second = c->acts_buf.as<uint8_t>() + off;
        off += (p.first + 255) / 256 * 256;
    }
    const size_t kv_layer = (size_t)d.kvheads * c->context * d.head_dim;
    c->kv.alloc(kv_layer * 2 * 4 * c->cfg.layers);
    HIP_OK(hipMemset(c->kv.p, 0, c->kv.n));
    build_rope(c);
    a.rope = c->rope_buf.as<const float2>();
}

// Attention geometry: up to 32 chunk workgroups per KV head (at least 32
// keys each), 32-key LDS tiles.  Fixes the partial buffer of the context.
constexpr uint32_t kAttnTile = 32, kAttnMaxChunks = 32;
void choose_attn_tile(qh_ctx* c) {
    const ModelDims& d = c->dm;
    const uint32_t G = d.heads / d.kvheads, hd = d.head_dim, T = kAttnTile;
    // head_dim 128 with up to 8 query heads per KV head: the register-slice
    // kernel (k_attn128); otherwise the general LDS-tiled one
    c->attn128 = hd == 128 && G >= 1 && G <= 8;
    if (c->attn128)
        c->lds_attn = (size_t)(8 * 160 + 160 + 128 + T * 128 + 8 * 36 + 8 + 16) * 4;
    else
        c->lds_attn = (size_t)(G * hd + 2 * hd + T * (hd + 1) + T * hd + G * T + G * hd + 3 * G) * 4;
    if (c->lds_attn > 64 * 1024) throw Error("attention shape exceeds the LDS budget");
    if (G > hd) throw Error("more query heads per KV head than head_dim is not supported");
    c->tc = T;
    c->max_chunks = (uint32_t)std::min<size_t>(kAttnMaxChunks, (c->context + 31) / 32);
}

void choose_geometry(qh_ctx* c) {
    const ModelDims& d = c->dm;
    const LayerW& L = c->layers[0];
    const size_t lds_cap = 64 * 1024;
    c->slots.clear();
    for (const LayerW& W : c->layers) {
        // held tiles need one block-quantised format per launch role
        const bool qkv_q = is_quant(W.q.kind) && is_quant(W.k.kind) && is_quant(W.v.kind);
        const bool gu_q = W.gate.kind == W.up.kind;
        c->slots.push_back({qkv_q ? tile_slots(W.q.kind, W.q.cols) : 0, tile_slots(W.o.kind, W.o.cols),
                            gu_q ? tile_slots(W.gate.kind, W.gate.cols) : 0, is_quant(W.down.kind) ? 1 : 0});
    }
    c->vocab_slots = tile_slots(c->out.kind, c->out.cols);
    c->lds_h = (size_t)pad32h(d.hidden) * 4;
    // k_qkv: one workgroup per 4 row groups (2 rows each), per matrix
    auto wgs = [](const DevMat& m) { return (groups_host(m.rows, m.cols, 2) + kWaves - 1) / kWaves; };
    const uint64_t gq = wgs(L.q) + wgs(L.k) + wgs(L.v);
    if (gq > 65535) throw Error("attention projections too large for one launch");
    c->g_qkv = (uint32_t)gq;
    c->g_o = std::min<uint32_t>(kRouterParts, d.hidden);
    c->lds_o = ((size_t)pad32h((uint64_t)d.heads * d.head_dim) + 2 * ((d.hidden + c->g_o - 1) / c->g_o)) * 4;
    {
        // k_gateup: per routed slot, enough workgroups that each wave owns one
        // group of 2 row pairs
        const uint64_t per_wg = (uint64_t)(kWideBlock / 64) * 2 * (64 / lanes_per_row(d.hidden));
        uint64_t wps = (d.ff + per_wg - 1) / per_wg;
        wps = std::max<uint64_t>(1, std::min<uint64_t>(wps, kMaxGrid / std::max<uint32_t>(1, d.top)));
        c->g_gu = (uint32_t)(d.top * wps);
    }
    // k_gateup folds the router partials of at most 64 workgroups for at most
    // 255 experts (two 128-expert passes of four threads each)
    if (d.experts + 1 > 256) throw Error("more than 255 experts is not supported by the routing kernel");
    if (c->g_o > 64) throw Error("too many router partial rows");
    c->lds_gu = ((size_t)pad32h(d.hidden) + d.experts + 1 + 2 * d.top + 4) * 4;
    c->g_down = blocks_for((d.hidden + 1) / 2);
    c->lds_down = ((size_t)d.top * pad32h(d.ff) + 2 * d.top) * 4;
    c->g_vocab = blocks_for(groups_host(c->out.rows, c->out.cols, 2));
    if (c->lds_h > lds_cap || c->lds_o > lds_cap || c->lds_gu > lds_cap)
        throw Error("hidden size exceeds the LDS budget of the device kernels");
    if (c->lds_down > lds_cap) throw Error("expert_used_count * expert FFN exceeds the LDS budget");
}

// Launches kern<C> for the held chunk slots C in {0, 1, 2}.
#define QH_LAUNCH_SLOTS(kern, C, ...)                                    \
    switch (C) {                                                         \
    case 1: hipLaunchKernelGGL(kern<1>, __VA_ARGS__); break;             \
    case 2: hipLaunchKernelGGL(kern<2>, __VA_ARGS__); break;             \
    default: hipLaunchKernelGGL(kern<0>, __VA_ARGS__); break;            \
    }

// Enqueues kernel k (0 qkv, 1 attention, 2 oproj, 3 gateup, 4 down) of
// layer l (first: the layer also embeds tokens[pos]).
void enqueue_kernel(qh_ctx* c, size_t l, bool first, int k) {
    const ModelDims& d = c->dm;
    const LayerW& L = c->layers[l];
    const auto& sl = c->slots[l];
    switch (k) {
    case 0: QH_LAUNCH_SLOTS(k_qkv, sl[0], dim3(c->g_qkv), dim3(kBlock), c->lds_h, c->s, L, c->emb, c->acts, d, (int)first); break;
    case 1:
        if (c->attn128)
            hipLaunchKernelGGL(k_attn128, dim3(d.kvheads, c->max_chunks), dim3(kBlock), c->lds_attn, c->s, L, c->attn[l], c->acts, d);
        else
            hipLaunchKernelGGL(k_attn, dim3(d.kvheads, c->max_chunks), dim3(kBlock), c->lds_attn, c->s, L, c->attn[l], c->acts, d);
        break;
    case 2: QH_LAUNCH_SLOTS(k_oproj, sl[1], dim3(c->g_o), dim3(kWideBlock), c->lds_o, c->s, L, c->acts, d); break;
    case 3: QH_LAUNCH_SLOTS(k_gateup, sl[2], dim3(c->g_gu), dim3(kWideBlock), c->lds_gu, c->s, L, c->acts, d, c->g_o); break;
    default:
        if (sl[3]) hipLaunchKernelGGL(k_down<1>, dim3(c->g_down), dim3(kBlock), c->lds_down, c->s, L, c->acts, d);
        else hipLaunchKernelGGL(k_down<0>, dim3(c->g_down), dim3(kBlock), c->lds_down, c->s, L, c->acts, d);
        break;
    }
}

void enqueue_vocab(qh_ctx* c) {
    QH_LAUNCH_SLOTS(k_vocab, c->vocab_slots, dim3(c->g_vocab), dim3(kBlock), c->lds_h, c->s, c->out, c->onorm, c->acts, c->dm);
}

void enqueue_layer(qh_ctx* c, size_t l, bool first) {
    for (int k = 0; k < 5; k++) enqueue_kernel(c, l, first, k);
}

void enqueue_tail(qh_ctx* c) {
    enqueue_vocab(c);
    hipLaunchKernelGGL(k_finish, dim3(1), dim3(kBlock), 0, c->s, c->acts, c->dm, c->g_vocab);
}

void enqueue_step(qh_ctx* c) {
    for (size_t l = 0; l < c->layers.size(); l++) enqueue_layer(c, l, l == 0);
    enqueue_tail(c);
}

void capture_graph(qh_ctx* c) {
    if (!c->use_graph) return;
    HIP_OK(hipStreamBeginCapture(c->s, hipStreamCaptureModeThreadLocal));
    enqueue_step(c);
    hipError_t e = hipStreamEndCapture(c->s, &c->graph);
    if (e != hipSuccess) throw Error(std::string("graph capture: ") + hipGetErrorString(e));
    HIP_OK(hipGraphInstantiate(&c->exec, c->graph, nullptr, nullptr, 0));
}

// Whether k_decode covers this model: the Qwen3-30B-A3B shapes (hidden
// 2048, 32 query / 4 KV heads of 128, up to 128 experts, top 8, expert FFN
// 768), one main block format KM (Q4_0, Q8_0, Q4_K, Q5_K or Q6_K) for q, k,
// o, gate and up with v and down in KM or Q6_K (llama.cpp's Q4_0, Q8_0,
// Q4_K_S/M, Q5_K_S/M and Q6_K files), a block-quantised vocab projection and
// an F32 router, and a device of 8 XCDs x 32 CUs running one 512-thread
// workgroup per CU.
bool persist_supported(const qh_ctx* c, uint32_t nwg) {
    const ModelDims& d = c->dm;
    auto block = block_kind;
    if (nwg != kDecodeXcds * kDecodeWgPerXcd) return false;
    if (!(d.hidden == 2048 && d.heads == 32 && d.kvheads == 4 && d.head_dim == 128)) return false;
    if (!(d.experts >= 8 && d.experts <= 128 && d.top == kDecodeXcds && d.ff == 768)) return false;
    if (!block(c->out.kind) || c->out.cols != d.hidden || c->layers.empty()) return false;
    if ((uint64_t)c->out.rows * c->out.drb >= (1ull << 32)) return false;  // 32-bit buffer offsets
    const uint32_t km = c->layers[0].q.kind;  // the main format
    if (!block(km)) return false;
    auto mv = [&](uint32_t k) { return k == km || k == Q6_K; };
    for (const LayerW& L : c->layers) {
        if (!(L.q.kind == km && L.k.kind == km && L.o.kind == km && L.gate.kind == km && L.up.kind == km &&
              mv(L.v.kind) && mv(L.down.kind) && L.router.kind == F32))
            return false;
    }
    return true;
}

// k_decode for the main format of the model (persist_supported holds).
const void* decode_kernel(uint32_t km) {
    switch (km) {
    case Q4_0: return reinterpret_cast<const void*>(k_decode<Q4_0>);
    case Q8_0: return reinterpret_cast<const void*>(k_decode<Q8_0>);
    case Q4_K: return reinterpret_cast<const void*>(k_decode<Q4_K>);
    case Q5_K: return reinterpret_cast<const void*>(k_decode<Q5_K>);
    default: return reinterpret_cast<const void*>(k_decode<Q6_K>);
    }
}

// Whether the workgroups of a 256-workgroup launch go to the XCDs in turn,
// workgroup b on XCD (b + s) % 8 for the launch's starting XCD s (read from the
// hardware register by a probe kernel): the persistent step takes a
// workgroup's place in its XCD, b / 8, from that order.
bool xcd_placement_ok(qh_ctx* c, uint32_t nwg) {
    DevBuf m;
    m.alloc(nwg * 4);
    uint32_t* out = m.as<uint32_t>();
    hipLaunchKernelGGL(k_xcd_map, dim3(nwg), dim3(512), 0, c->s, out);
    HIP_OK(hipGetLastError());
    std::vector<uint32_t> h(nwg);
    HIP_OK(hipMemcpyAsync(h.data(), m.p, nwg * 4, hipMemcpyDeviceToHost, c->s));
    HIP_OK(hipStreamSynchronize(c->s));
    const uint32_t s = h[0] % kDecodeXcds;
    for (uint32_t b = 0; b < nwg; b++)
        if (h[b] != (b + s) % kDecodeXcds) return false;
    return true;
}

void setup_persist(qh_ctx* c) {
    // QH_NO_PERSIST=1: no persistent step for this context (no placement
    // probe, no router folds)
    const char* np = std::getenv("QH_NO_PERSIST");
    if (np && np[0] == '1') {
        c->persist_ok = c->persist = false;
        return;
    }
    hipDeviceProp_t p;
    HIP_OK(hipGetDeviceProperties(&p, c->device));
    const uint32_t nwg = (uint32_t)p.multiProcessorCount;
    if (!persist_supported(c, nwg)) {
        c->persist_ok = c->persist = false;
        return;
    }
    c->decode_fn = decode_kernel(c->layers[0].q.kind);
    // one 512-thread workgroup per CU (nwg is the CU count), all resident at
    // once: the launch is an ordinary one (a cooperative launch adds nothing
    // here and left every profiled process failing in the profiler's exit
    // path), so residency is checked here -- at least one workgroup fits a
    // CU -- and at run time every wait of the step is bounded, so a
    // workgroup that is not resident ends the step with "device
    // synchronisation timed out" instead of a hang
    int per_cu = 0;
    HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, c->decode_fn, 512, 0));
    c->persist_ok = per_cu >= 1 && xcd_placement_ok(c, nwg);
    c->persist = c->persist_ok;
    if (!c->persist_ok) return;
    c->nwg = nwg;
    const ModelDims& d = c->dm;
    {
        // router folds: F = (router * ffn_norm) Wo per layer, from the
        // dequantised attn_output (one f32 copy of it at a time)
        const uint32_t H = d.hidden, qd = d.heads * 128, E = d.experts;
        const size_t per = (size_t)E * qd;
        c->rfold.alloc(c->layers.size() * per * 4);
        DevBuf wo;
        wo.alloc((size_t)H * qd * 4);
        for (size_t l = 0; l < c->layers.size(); l++) {
            LayerW& L = c->layers[l];
            hipLaunchKernelGGL(k_dequant, dim3(1024), dim3(kBlock), 0, c->s, L.o, (size_t)0, (size_t)H, wo.as<float>());
            hipLaunchKernelGGL(k_router_fold, dim3((qd + kBlock - 1) / kBlock, (E + 7) / 8), dim3(kBlock), 0, c->s,
                               L.router, L.ffn_norm, wo.as<const float>(), H, qd, E, c->rfold.as<float>() + l * per);
            HIP_OK(hipGetLastError());
            L.rfold = c->rfold.as<const float>() + l * per;
        }
        HIP_OK(hipStreamSynchronize(c->s));
    }
    c->layers_dev.alloc(c->layers.size() * sizeof(LayerW));
    HIP_OK(hipMemcpy(c->layers_dev.p, c->layers.data(), c->layers.size() * sizeof(LayerW), hipMemcpyHostToDevice));
    DecodeArgs& A = c->dargs;
    A = DecodeArgs{};
    A.layers = c->layers_dev.as<const LayerW>();
    A.emb = c->emb;
    A.out = c->out;
    A.onorm = c->onorm;
    A.a = c->acts;
    A.dm = c->dm;
    // abort flag | tagged words of each exchange; every region (and every
    // XCD's part of it) starts on a 256-byte boundary, so no cache line is
    // shared between XCDs
    const uint64_t X = kDecodeXcds;
    struct Region {
        uint64_t words;
        uint64_t** dst;
    } regions[] = {
        {X * kDecodeStrideQkv, &A.lqkv}, {X * kDecodeStridePart, &A.lpart},
        {X * kDecodeStrideX1, &A.lx1},   {X * kDecodeStrideH, &A.lh},       {X * kDecodeStrideX2, &A.lx2},
        {X * kDecodeStrideG1, &A.g1},    {X * kDecodeStrideG2, &A.g2},      {2ull * nwg, &A.tfin},
    };
    auto up256 = [](uint64_t b) { return (b + 255) / 256 * 256; };
    size_t total = 256;
    for (const Region& r : regions) total += up256(r.words * 8);
    c->sync_buf.alloc(total);
    c->sync_bytes = total;
    HIP_OK(hipMemset(c->sync_buf.p, 0, total));
    uint8_t* q = c->sync_buf.as<uint8_t>();
    A.abort_flag = reinterpret_cast<uint32_t*>(q);
    q += 256;
    for (const Region& r : regions) {
        *r.dst = reinterpret_cast<uint64_t*>(q);
        q += up256(r.words * 8);
    }
    c->flag_base = 0;
}

// Clears n bytes (a multiple of 4) of device memory with a fill kernel.
void clear_words(qh_ctx* c, void* p, size_t bytes) {
    hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)std::min<size_t>((bytes / 4 + kBlock - 1) / kBlock, 4096)),
                       dim3(kBlock), 0, c->s, static_cast<uint32_t*>(p), bytes / 4, 0u);
    HIP_OK(hipGetLastError());
}

// One launch of k_decode over layers [l0, l1) (one workgroup per CU, all
// resident: setup_persist checks it); vocab: also the final norm, vocab
// projection, argmax and position advance.
void launch_decode(qh_ctx* c, uint32_t l0, uint32_t l1, bool vocab, bool embed) {
    if (!(l0 < l1 && l1 <= c->layers.size())) throw Error("decode launch needs a non-empty layer range");
    const uint32_t phases = kDecodePhases * (l1 - l0) + (vocab ? 1 : 0);
    if (c->flag_base > 0xFFFFFFFFu - phases) {
        // tags would wrap: clear every tagged word (no launch is reading them:
        // this stream runs the launches in order) and start again from 0
        clear_words(c, c->sync_buf.p, c->sync_bytes);
        c->flag_base = 0;
    }
    DecodeArgs A = c->dargs;
    A.base = c->flag_base;
    A.l0 = l0;
    A.l1 = l1;
    A.vocab = vocab ? 1u : 0u;
    A.embed = embed ? 1u : 0u;
    c->flag_base += phases;
    void* args[] = {&A};
    HIP_OK(hipLaunchKernel(c->decode_fn, dim3(c->nwg), dim3(512), args, 0, c->s));
}

// One token step: the captured graph, or the same kernels launched directly.
void launch_step(qh_ctx* c) {
    if (c->persist) {
        launch_decode(c, 0, (uint32_t)c->layers.size(), true, true);
        return;
    }
    if (c->use_graph) {
        HIP_OK(hipGraphLaunch(c->exec, c->s));
    } else {
        enqueue_step(c);
        HIP_OK(hipGetLastError());
    }
}

// Read-only mapping of a whole file, unmapped when it goes out of scope.
struct MappedFile {
    const uint8_t* data = nullptr;
    size_t len = 0;
    explicit MappedFile(const char* path) {
        const int fd = open(path, O_RDONLY);
        if (fd < 0) throw Error(std::string("open ") + path);
        struct stat sb;
        if (fstat(fd, &sb) != 0) {
            close(fd);
            throw Error(std::string("stat ") + path);
        }
        len = (size_t)sb.st_size;
        void* m = len ? mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
        close(fd);
        if (len && m == MAP_FAILED) throw Error(std::string("mmap ") + path);
        data = static_cast<const uint8_t*>(m);
    }
    ~MappedFile() {
        if (len) munmap(const_cast<uint8_t*>(data), len);
    }
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
};

void load_image(qh_ctx* c, const uint8_t* data, size_t len, size_t context) {
    Gguf g = parse_gguf(data, len);
    Config cfg = config_from_gguf(g);
    validate_tensors(cfg, g);
    if (!(context > 0 && context <= cfg.max_context))
        throw Error("context must be in 1..=" + std::to_string(cfg.max_context));
    if (cfg.head_dim > 512) throw Error("head_dim above 512 is not supported by the device kernels");
    if (cfg.top > 1024) throw Error("expert_used_count above 1024 is not supported");
    c->drop_model();
    c->generation += 1;
    c->cfg = cfg;
    c->context = context;
    c->packed = g.packed_bytes();
    ModelDims& d = c->dm;
    d.hidden = (uint32_t)cfg.hidden; d.heads = (uint32_t)cfg.heads; d.kvheads = (uint32_t)cfg.kvheads;
    d.head_dim = (uint32_t)cfg.head_dim; d.experts = (uint32_t)cfg.experts; d.top = (uint32_t)cfg.top;
    d.ff = (uint32_t)cfg.intermediate; d.vocab = (uint32_t)cfg.vocab; d.ctx = (uint32_t)context;
    d.layers = (uint32_t)cfg.layers;
    d.eps = cfg.eps;
    // every tensor to HBM once, repacked into the device row layout
    for (auto& kv : g.tensors) {
        const Tensor& t = kv.second;
        ModelTensor mt;
        mt.kind = t.kind;
        mt.dims = t.dims;
        uint64_t cols = t.dims[0], rows = 1, experts = 0;
        for (size_t k = 1; k < t.dims.size(); k++) rows *= t.dims[k];
        if (t.dims.size() == 3) experts = t.dims[2];
        const size_t drb = dev_row_bytes(t.kind, cols);
        mt.buf.alloc(rows * drb + 64);
        upload_rows(c, data + t.offset, mt.buf.as<uint8_t>(), t.kind, cols, rows);
        if (t.dims.size() == 1) {
            DevMat m = make_mat(mt.buf.as<uint8_t>(), t.kind, 1, cols, 0);
            mt.f32.alloc(pad32h(cols) * 4);
            HIP_OK(hipMemsetAsync(mt.f32.p, 0, pad32h(cols) * 4, c->s));
            hipLaunchKernelGGL(k_dequant, dim3((uint32_t)std::min<uint64_t>((cols + 255) / 256, 1024)), dim3(kBlock), 0,
                               c->s, m, (size_t)0, (size_t)1, mt.f32.as<float>());
            HIP_OK(hipGetLastError());
        } else {
            mt.mat = make_mat(mt.buf.as<uint8_t>(), t.kind, t.dims[1], cols, experts);
        }
        c->tensors.emplace(kv.first, std::move(mt));
    }
    sync(c);
    auto mat = [&](const std::string& n) { return c->tensors.at(n).mat; };
    auto vec = [&](const std::string& n) { return c->tensors.at(n).f32.as<const float>(); };
    c->emb = mat("token_embd.weight");
    c->out = c->tensors.count("output.weight") ? mat("output.weight") : c->emb;
    c->onorm = vec("output_norm.weight");
    choose_attn_tile(c);
    alloc_acts(c);
    const size_t kv_layer = (size_t)d.kvheads * context * d.head_dim;
    for (uint64_t i = 0; i < cfg.layers; i++) {
        std::string p = "blk." + std::to_string(i) + ".";
        LayerW L{};
        L.index = (uint32_t)i;
        L.q = mat(p + "attn_q.weight");
        L.k = mat(p + "attn_k.weight");
        L.v = mat(p + "attn_v.weight");
        L.o = mat(p + "attn_output.weight");
        L.router = mat(p + "ffn_gate_inp.weight");
        L.gate = mat(p + "ffn_gate_exps.weight");
        L.up = mat(p + "ffn_up_exps.weight");
        L.down = mat(p + "ffn_down_exps.weight");
        L.attn_norm = vec(p + "attn_norm.weight");
        L.q_norm = vec(p + "attn_q_norm.weight");
        L.k_norm = vec(p + "attn_k_norm.weight");
        L.ffn_norm = vec(p + "ffn_norm.weight");
        L.kcache = c->kv.as<float>() + (2 * i) * kv_layer;
        L.vcache = c->kv.as<float>() + (2 * i + 1) * kv_layer;
        c->layers.push_back(L);
    }
    choose_geometry(c);
    for (uint64_t i = 0; i < cfg.layers; i++) {
        AttnArgs a{};
        a.q = c->acts.q;
        a.k = c->layers[i].kcache;
        a.v = c->layers[i].vcache;
        a.sh = (size_t)context * d.head_dim;
        a.st = d.head_dim;
        a.heads = d.heads;
        a.kvheads = d.kvheads;
        a.d = d.head_dim;
        a.tc = c->tc;
        a.max_chunks = c->max_chunks;
        a.part = c->acts.part;
        a.counter = c->acts.attn_cnt;
        a.out = c->acts.attn;
        a.err = &c->acts.st->err;
        c->attn.push_back(a);
    }
    capture_graph(c);
    setup_persist(c);
    c->loaded = true;
    c->pos = 0;
}

void need_model(qh_ctx* c) {
    if (!c->loaded) throw Error("no model loaded");
}

// A caller's logits buffer must hold the whole vocabulary of the loaded model.
void need_logits_room(const qh_ctx* c, const float* logits, size_t cap) {
    if (logits && cap < c->cfg.vocab)
        throw Error("logits buffer holds " + std::to_string(cap) + " floats, the model has a vocabulary of " +
                    std::to_string(c->cfg.vocab));
}

// Writes the device step state from the host mirror.
void put_state(qh_ctx* c, uint32_t pos, uint32_t n_given) {
    DevState st{};
    st.pos = pos;
    st.n_given = n_given;
    HIP_OK(hipMemcpyAsync(c->acts.st, &st, sizeof st, hipMemcpyHostToDevice, c->s));
}

DevState get_state(qh_ctx* c) {
    DevState st{};
    HIP_OK(hipMemcpyAsync(&st, c->acts.st, sizeof st, hipMemcpyDeviceToHost, c->s));
    sync(c);
    return st;
}

void reset_model(qh_ctx* c) {
    c->pos = 0;
    put_state(c, 0, 0);
    sync(c);
}

[[noreturn]] void fail_step(qh_ctx* c, uint32_t err) {
    // a persistent step that gave up leaves its abort flag raised (and
    // possibly tagged words of the abandoned phases): clear the flag before
    // anything else, so later steps do not abandon their waits
    if (err & (kErrSync | kErrPlace)) {
        if (c->persist_ok) clear_words(c, c->dargs.abort_flag, 4);
        clear_words(c, c->acts.attn_cnt, pad32h(c->dm.kvheads) * 4);
    }
    reset_model(c);
    if (err & kErrPlace) throw Error("persistent step: a workgroup ran on an unexpected XCD");
    if (err & kErrToken) throw Error("token outside vocabulary");
    if (err & kErrRouter) throw Error("invalid MoE router");
    if (err & kErrLogits) throw Error("nonfinite model output");
    if (err & kErrContext) throw Error("context limit " + std::to_string(c->context) + " reached");
    if (err & kErrSync) throw Error("device synchronisation timed out");
    throw Error("device step failed");
}

uint64_t matvecs_per_token(const qh_ctx* c) { return c->cfg.layers * (5 + 3 * c->cfg.top) + 1; }

// ------------------------------------------------------------ prefill --
constexpr uint32_t kPrefillChunk = 2048;  // most prompt tokens per batched pass

// Whether the batched prefill covers the model: head_dim 128 with at most 8
// query heads per KV head, at most 128 experts, F32 router, widths in whole
// 256-column super-blocks, and every projection block-quantised (gate and up
// in one format).  Empty when covered, else the first reason it is not.
std::string prefill_gap(const qh_ctx* c) {
    const ModelDims& d = c->dm;
    auto km = block_kind;
    if (d.head_dim != 128) return "head_dim " + std::to_string(d.head_dim) + " (needs 128)";
    if (d.heads % d.kvheads || d.heads / d.kvheads > 8) return "more than 8 query heads per KV head";
    if (d.experts > 128) return "more than 128 experts";
    if (d.hidden % 256 || d.ff % 256) return "hidden or expert width not a multiple of 256";
    // the o-projection runs as two column halves, each whole 256-column
    // super-blocks (and an even number of 64-column GEMM slices)
    if ((d.heads * 128) % 512) return "query width not a multiple of 512";
    for (const LayerW& L : c->layers) {
        if (!(km(L.q.kind) && km(L.k.kind) && km(L.v.kind) && km(L.o.kind) && km(L.gate.kind) &&
              L.up.kind == L.gate.kind && km(L.down.kind)))
            return "a projection is not block-quantised (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K)";
        if (L.router.kind != F32) return "router is not F32";
    }
    return "";
}

// The prefill GEMMs' tile-layout copies of every layer's q, k, v, o, gate,
// up and down (once per model; the row layout stays for the token step).
void prefill_tiles(qh_ctx* c) {
    auto& P = c->pf;
    if (P.tiled) return;
    auto mats = [](LayerW& L) { return std::array<DevMat*, 7>{&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down}; };
    auto bytes = [&](const DevMat& m) {
        return m.expert_stride ? (size_t)c->dm.experts * m.expert_stride : (size_t)m.rows * m.drb;
    };
    size_t total = 0;
    for (LayerW& L : c->layers)
        for (DevMat* m : mats(L)) {
            if (m->rows % 32 || m->cols % 256 || !block_kind(m->kind) ||
                (size_t)(m->rows / 32) * tile_group_bytes(m->kind, m->cols) > (size_t)m->rows * m->drb)
                throw Error("tile layout needs block-quantised rows in groups of 32, columns in groups of 256");
            total += (bytes(*m) + 255) / 256 * 256;
        }
    P.tiles.alloc(total);
    size_t off = 0;
    for (LayerW& L : c->layers)
        for (DevMat* m : mats(L)) {
            uint8_t* dst = P.tiles.as<uint8_t>() + off;
            const uint32_t experts = m->expert_stride ? c->dm.experts : 1;
            const size_t nblk = (size_t)experts * (m->rows / 32) * (m->cols / 256);
            hipLaunchKernelGGL(k_tile_gemm, dim3((uint32_t)std::min<size_t>(nblk, 65535)), dim3(kBlock), 0, c->s, *m,
                               experts, dst);
            HIP_OK(hipGetLastError());
            m->wt = dst;
            off += (bytes(*m) + 255) / 256 * 256;
        }
    P.tiled = true;
}


void prefill_alloc(qh_ctx* c, uint32_t cap) {
    auto& P = c->pf;
    if (P.cap >= cap) return;
    const ModelDims& d = c->dm;
    const uint64_t H = d.hidden, qd = (uint64_t)d.heads * 128, kvd = (uint64_t)d.kvheads * 128;
    const uint64_t n_asg = (uint64_t)cap * d.top;
    const uint32_t max_tiles = (uint32_t)((n_asg + 127) / 128 + d.experts);
    auto up = [](uint64_t b) { return (b + 255) / 256 * 256; };
    const uint64_t npair = ((cap + 15) / 16 + 1) / 2 * d.kvheads;  // attention block pairs
    struct R {
        uint64_t bytes;
        void** dst;
    } regs[] = {
        {cap * H * 4, (void**)&P.X},           {cap * H * 4, (void**)&P.Xn32},
        {cap * (qd + 2 * kvd) * 4, (void**)&P.QKV}, {(uint64_t)cap * d.experts * 4 * kPfRouterSplit, (void**)&P.LR},
        {n_asg * 4, (void**)&P.wts},           {std::max<uint64_t>(n_asg, 2ull * cap) * H * 4, (void**)&P.Y},
        {cap * H * 2, (void**)&P.Xn16},        {(uint64_t)d.heads * cap * 128 * 2, (void**)&P.Q16},
        {cap * qd * 2, (void**)&P.O16},        {n_asg * d.ff * 2, (void**)&P.Hs},
        {n_asg * 4, (void**)&P.ids},           {(uint64_t)(d.experts + 1) * 4, (void**)&P.goff},
        {n_asg * 4, (void**)&P.tok},           {n_asg * 4, (void**)&P.asg},
        {(uint64_t)max_tiles * 4, (void**)&P.te}, {(uint64_t)max_tiles * 4, (void**)&P.tm},
        {4, (void**)&P.ntile},
        {(uint64_t)d.kvheads * d.ctx * 128 * 2, (void**)&P.Kh},
        {(uint64_t)d.kvheads * 128 * ((d.ctx + 63) / 64 * 64) * 2, (void**)&P.Vth},
        {npair * 2 * kPfAttnSlot * 4, (void**)&P.axw}, {npair * 4, (void**)&P.axc},
    };
    uint64_t total = 0;
    for (const R& r : regs) total += up(r.bytes);
    P.buf.alloc(total);
    HIP_OK(hipMemset(P.buf.p, 0, total));
    uint8_t* q = P.buf.as<uint8_t>();
    for (const R& r : regs) {
        *r.dst = q;
        q += up(r.bytes);
    }
    P.cap = cap;
    P.max_tiles = max_tiles;
}

template <class F> void dispatch_km(uint32_t kind, F f) {
    switch (kind) {
    case Q4_0: f(std::integral_constant<uint32_t, Q4_0>{}); break;
    case Q8_0: f(std::integral_constant<uint32_t, Q8_0>{}); break;
    case Q4_K: f(std::integral_constant<uint32_t, Q4_K>{}); break;
    case Q5_K: f(std::integral_constant<uint32_t, Q5_K>{}); break;
    case Q6_K: f(std::integral_constant<uint32_t, Q6_K>{}); break;
    default: throw Error("prefill projection is not block-quantised");
    }
}

// C[t][cofs_i + n] = X16[t] . W_i[n] for t < S and each matrix i of `mats`
// (one launch; with `splits` > 1 the columns are split in equal parts, part z
// written to C + z * split_stride): the MFMA GEMM on the quantised rows
// (dequantised into the tiles).
void pf_dense(qh_ctx* c, std::initializer_list<std::pair<const DevMat*, uint32_t>> mats, const _Float16* X16,
              uint32_t S, float* C, uint32_t ldc, uint32_t splits = 1, size_t split_stride = 0) {
    DenseSegs G{};
    uint32_t tiles = 0;
    for (const auto& m : mats) {
        const DevMat& W = *m.first;
        if (!block_kind(W.kind)) throw Error("prefill projection is not block-quantised");
        if ((W.cols / splits) % 256 || W.cols % splits) throw Error("prefill projection width does not split");
        G.W[G.n] = W;
        tiles += (W.rows + 127) / 128;
        G.tile_end[G.n] = tiles;
        G.cofs[G.n] = m.second;
        G.n++;
    }
    for (uint32_t i = G.n; i < 3; i++) G.tile_end[i] = tiles;
    hipLaunchKernelGGL(k_gemm_dense, dim3(8 * ((S + 1023) / 1024) * tiles, 1, splits), dim3(256), 0, c->s, X16, S, G, C, ldc,
                       split_stride);
}

// One decoder layer (src/model.rs:227-287) for chunk tokens [0, S) at
// positions p0 + t.
void prefill_layer(qh_ctx* c, size_t l, uint32_t S, uint32_t p0) {
    auto& P = c->pf;
    const ModelDims& d = c->dm;
    const LayerW& L = c->layers[l];
    const uint32_t H = d.hidden, qd = d.heads * 128, kvd = d.kvheads * 128, row = qd + 2 * kvd;
    uint32_t* err = &c->acts.st->err;  // kErrRange: an fp16 operand out of range
    if (l == 0)  // later layers: written by the previous layer's combine
        hipLaunchKernelGGL(k_pf_norm, dim3(S), dim3(kBlock), 0, c->s, P.X, L.attn_norm, H, d.eps, P.Xn16,
                           (float*)nullptr, (const float*)nullptr, (size_t)0, err);
    // q | k | v: one launch over the three quantised matrices, QKV[t] = [q | k | v]
    pf_dense(c, {{&L.q, 0u}, {&L.k, qd}, {&L.v, qd + kvd}}, P.Xn16, S, P.QKV, row);
    const uint32_t vp = (d.ctx + 63) / 64 * 64;  // row pitch of the transposed V copy
    if (p0 > 0)  // fp16 copies of this layer's earlier positions
        hipLaunchKernelGGL(k_pf_kvh, dim3(p0), dim3(kBlock), 0, c->s, L.kcache, L.vcache, 0u, d.kvheads, d.ctx, vp,
                           P.Kh, P.Vth);
    hipLaunchKernelGGL(k_pf_qkrope, dim3(S), dim3(kBlock), 0, c->s, P.QKV, L.q_norm, L.k_norm, c->acts.rope, p0, S,
                       d.heads, d.kvheads, d.ctx, d.eps, P.Q16, L.kcache, L.vcache, P.Kh, P.Vth, vp, err);
    // two workgroups per pair of query blocks (the n-1-i-th and the i-th of n)
    const uint32_t npair = ((S + 15) / 16 + 1) / 2;
    hipLaunchKernelGGL(k_pf_attn, dim3(2 * npair * d.kvheads), dim3(256), 0, c->s, P.Q16, P.Kh, P.Vth, p0, S,
                       d.heads / d.kvheads, d.ctx, vp, qd, P.O16, P.axw, P.axc);
    // o in two column halves (twice the workgroups) into Y's space; the norm
    // adds both to the residual (model.rs:246-248) before normalising
    const size_t ostride = (size_t)S * H;
    pf_dense(c, {{&L.o, 0u}}, P.O16, S, P.Y, H, 2, ostride);
    hipLaunchKernelGGL(k_pf_norm, dim3(S), dim3(kBlock), 0, c->s, P.X, L.ffn_norm, H, d.eps, P.Xn16, P.Xn32,
                       (const float*)P.Y, ostride, err);
    hipLaunchKernelGGL(k_pf_router, dim3((S + 63) / 64, kPfRouterSplit), dim3(kBlock), 0, c->s, P.Xn32, L.router,
                       S, H, d.experts, P.LR);
    hipLaunchKernelGGL(k_pf_topk, dim3((S + kWaves - 1) / kWaves), dim3(kBlock), 0, c->s, P.LR, S,
                       d.experts, d.top, P.ids, P.wts, c->acts.st, c->acts.route_log, c->acts.gap_log, d.layers,
                       (uint32_t)l, p0);
    hipLaunchKernelGGL(k_pf_group, dim3(1), dim3(1024), 0, c->s, P.ids, S * d.top, d.top, d.experts, P.goff, P.tok,
                       P.asg, P.te, P.tm, P.ntile);
    const ExpertTiles T{P.goff, P.tok, P.asg, P.te, P.tm, P.ntile};
    const uint32_t tiles = (S * d.top + 127) / 128 + d.experts;
    dispatch_km(L.gate.kind, [&](auto K) {
        hipLaunchKernelGGL(k_gemm_gateup<decltype(K)::value>, dim3(8 * ((tiles + 7) / 8) * ((d.ff + 127) / 128)), dim3(256), 0, c->s,
                           P.Xn16, H, T, L.gate, L.up, P.Hs, err);
    });
    dispatch_km(L.down.kind, [&](auto K) {
        hipLaunchKernelGGL(k_gemm_down<decltype(K)::value>, dim3(8 * ((tiles + 7) / 8) * ((H + 127) / 128)), dim3(256), 0, c->s, P.Hs, T,
                           L.down, P.Y);
    });
    // + the next layer's attention RMSNorm (fp16 operand of its q|k|v GEMM)
    const float* next_norm = l + 1 < c->layers.size() ? c->layers[l + 1].attn_norm : nullptr;
    hipLaunchKernelGGL(k_pf_combine, dim3(S), dim3(kBlock), 0, c->s, P.X, P.Y, P.wts, H, d.top, next_norm, d.eps,
                       P.Xn16, err);
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

namespace {

// ============================================================ sampler RNG ==
// rand 0.8.8's StdRng (= rand_chacha 0.3.1 ChaCha12Rng) as src/sampling.rs:20
// seeds it with `StdRng::seed_from_u64` (rand_core 0.6.4): the 32-byte key is
// filled with PCG32 outputs (state advanced by the 64-bit LCG, then XSH-RR),
// the keystream is ChaCha with 12 rounds, 64-bit block counter from 0 and
// stream 0, read one 32-bit word at a time; `gen::<f32>()` is the word's top
// 24 bits times 2^-24.
struct ChaCha12Stream {
    uint32_t key[8];
    uint64_t word = 0;  // index of the next keystream word

    explicit ChaCha12Stream(uint64_t seed) {
        uint64_t st = seed;
        for (uint32_t& k : key) {
            st = st * 6364136223846793005ull + 11634580027462260723ull;
            const uint32_t xs = (uint32_t)(((st >> 18) ^ st) >> 27), rot = (uint32_t)(st >> 59);
            k = (xs >> rot) | (xs << ((32 - rot) & 31));
        }
    }
    static uint32_t rotl(uint32_t v, int n) { return (v << n) | (v >> (32 - n)); }
    static void quarter(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
        a += b, d = rotl(d ^ a, 16);
        c += d, b = rotl(b ^ c, 12);
        a += b, d = rotl(d ^ a, 8);
        c += d, b = rotl(b ^ c, 7);
    }
    uint32_t at(uint64_t i) const {
        const uint64_t blk = i / 16;
        const uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2],
                                 key[3],      key[4],      key[5],      key[6],      key[7], (uint32_t)blk,
                                 (uint32_t)(blk >> 32), 0u, 0u};
        uint32_t x[16];
        std::memcpy(x, in, sizeof x);
        for (int r = 0; r < 6; r++) {  // 12 rounds
            quarter(x[0], x[4], x[8], x[12]);
            quarter(x[1], x[5], x[9], x[13]);
            quarter(x[2], x[6], x[10], x[14]);
            quarter(x[3], x[7], x[11], x[15]);
            quarter(x[0], x[5], x[10], x[15]);
            quarter(x[1], x[6], x[11], x[12]);
            quarter(x[2], x[7], x[8], x[13]);
            quarter(x[3], x[4], x[9], x[14]);
        }
        return x[i % 16] + in[i % 16];
    }
    float peek_f32() const { return (float)(at(word) >> 8) * (1.0f / 16777216.0f); }
};

}  // namespace

struct qh_sampler {
    ChaCha12Stream rng;
    float temperature, top_p;
    size_t top_k;
};

namespace {

// Sampler::sample (src/sampling.rs:26-63) on device logits; the stream
// advances only when a draw was used (temperature > 0 and success).
uint32_t run_sample(qh_ctx* c, qh_sampler* sp, const float* dlogits, const uint8_t* dvalid, size_t n) {
    if (n == 0) throw Error("invalid logits");
    if (n > (1u << 20)) throw Error("the device sampler takes at most 1048576 logits");
    c->samp_out.reserve(32);
    c->pin.reserve(32);
    SampleArgs a{};
    a.logits = dlogits;
    a.valid = dvalid;
    a.n = (uint32_t)n;
    a.top_k = (uint32_t)std::min<size_t>(sp->top_k, 0xffffffffu);
    a.temperature = sp->temperature;
    a.top_p = sp->top_p;
    a.draw = sp->rng.peek_f32();
    a.mode = kSampleModeSample;
    a.out = c->samp_out.as<uint32_t>();
    HIP_OK(hipSetDevice(c->device));
    const uint32_t* r = static_cast<const uint32_t*>(c->pin.p);
    auto read_out = [&] {
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(c->pin.p, a.out, 32, hipMemcpyDeviceToHost, c->s));
        HIP_OK(hipStreamSynchronize(c->s));
    };
    launch_sample(a, c->s);
    read_out();
    if (r[1] == kSampleBadLogits) throw Error("invalid logits");
    if (r[1] == kSampleSupport) {
        // more candidates than one workgroup sorts in LDS: collect the P ids at
        // or above the key of rank P - 1 into HBM, sort them there, fold
        const uint32_t P = r[3];
        const unsigned long long theta = ((unsigned long long)r[5] << 32) | r[4];
        const uint32_t K = (a.top_k > 0 && a.top_k < a.n) ? a.top_k : a.n;
        uint32_t np = 4096;
        while (np < P) np <<= 1;
        c->samp_big.reserve((size_t)np * 8 + (size_t)P * 4 + 64);
        auto* cand = c->samp_big.as<unsigned long long>();
        float* prob = reinterpret_cast<float*>(cand + np);
        uint32_t* cnt = reinterpret_cast<uint32_t*>(prob + P);
        hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(kBlock), 0, c->s, cnt, (size_t)1, 0u);
        launch_sample_collect(a, theta, P, np, cand, cnt, c->s);
        launch_sample_sort(cand, np, c->s);
        launch_sample_fold(a, cand, prob, P, K, c->s);
        read_out();
        if (r[1] == kSampleRank) {  // ids.last() is the id of rank m - 1, past the candidates
            a.mode = kSampleModeRank;
            a.rank = r[2] - 1;
            launch_sample(a, c->s);
            read_out();
        }
    }
    if (r[1] != 0) throw Error("device sampler failed");
    if (sp->temperature != 0.f) sp->rng.word++;
    return r[0];
}

}  // namespace

// ===================================================================== C ABI ==
extern "C" {

int qh_create(int device, qh_ctx** out) {
    try {
        int n = 0;
        HIP_OK(hipGetDeviceCount(&n));
        if (device < 0 || device >= n) throw Error("HIP device " + std::to_string(device) + " not present");
        hipDeviceProp_t p;
        HIP_OK(hipGetDeviceProperties(&p, device));
        if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
            throw Error(std::string("device is ") + p.gcnArchName + ", this engine is built for gfx950");
        HIP_OK(hipSetDevice(device));
        noalloc_init(device);
        auto c = std::make_unique<qh_ctx>();
        c->device = device;
        c->num_cu = (uint32_t)p.multiProcessorCount;
        const char* ng = std::getenv("QH_NO_GRAPH");
        c->use_graph = !(ng && ng[0] == '1');
        HIP_OK(hipStreamCreateWithFlags(&c->s, hipStreamNonBlocking));
        *out = c.release();
        return 0;
    } catch (const std::exception& e) {
        g_create_err = e.what();
        return 1;
    }
}

void qh_destroy(qh_ctx* c) { delete c; }

const char* qh_last_error(const qh_ctx* c) { return c ? c->err.c_str() : g_create_err.c_str(); }

int qh_load_model(qh_ctx* c, const void* image, size_t len, size_t context) {
    return guarded(c, [&] {
        HIP_OK(hipSetDevice(c->device));
        load_image(c, static_cast<const uint8_t*>(image), len, context);
    });
}

int qh_load_model_file(qh_ctx* c, const char* path, size_t context) {
    return guarded(c, [&] {
        const MappedFile f(path);
        HIP_OK(hipSetDevice(c->device));
        load_image(c, f.data, f.len, context);
    });
}

int qh_inspect(const char* path, size_t context, qh_inspect_t* out) {
    try {
        const MappedFile f(path);
        const Gguf g = parse_gguf(f.data, f.len);
        const Config cfg = config_from_gguf(g);
        validate_tensors(cfg, g);
        if (!(context > 0 && context <= cfg.max_context)) throw Error("invalid context");
        // ctx * layers * kvheads * head_dim * 8 with overflow checks (src/model.rs:150-156)
        uint64_t kv = context;
        for (uint64_t m : {cfg.layers, cfg.kvheads, cfg.head_dim, (uint64_t)8})
            if (__builtin_mul_overflow(kv, m, &kv)) throw Error("KV size overflow");
        out->config = {cfg.hidden, cfg.layers, cfg.heads, cfg.kvheads, cfg.head_dim, cfg.experts, cfg.top,
                       cfg.intermediate, cfg.vocab, cfg.max_context, cfg.eps, cfg.theta};
        out->tensor_count = g.tensors.size();
        out->packed_weight_bytes = g.packed_bytes();
        out->kv_f32_bytes_at_context = kv;
        return 0;
    } catch (const std::exception& e) {
        g_create_err = e.what();
        return 1;
    }
}

int qh_sampler_create(uint64_t seed, float temperature, size_t top_k, float top_p, qh_sampler** out) {
    if (!(std::isfinite(temperature) && temperature >= 0.f && std::isfinite(top_p) && top_p > 0.f &&
          top_p <= 1.f)) {
        g_create_err = "invalid sampling parameters";
        return 1;
    }
    *out = new qh_sampler{ChaCha12Stream(seed), temperature, top_p, top_k};
    return 0;
}

void qh_sampler_destroy(qh_sampler* sp) { delete sp; }

int qh_sampler_draw(qh_sampler* sp, float* out) {
    *out = sp->rng.peek_f32();
    sp->rng.word++;
    return 0;
}

int qh_set_valid_tokens(qh_ctx* c, const uint8_t* valid, size_t n) {
    return guarded(c, [&] {
        need_model(c);
        if (!valid) {
            c->valid.release();
            c->valid_n = 0;
            return;
        }
        if (n != c->cfg.vocab) throw Error("valid-token mask length differs from the vocabulary");
        HIP_OK(hipSetDevice(c->device));
        c->valid.reserve(n);
        HIP_OK(hipMemcpyAsync(c->valid.p, valid, n, hipMemcpyHostToDevice, c->s));
        HIP_OK(hipStreamSynchronize(c->s));
        c->valid_n = n;
    });
}

int qh_sample(qh_ctx* c, qh_sampler* sp, uint32_t* out) {
    return guarded(c, [&] {
        need_model(c);
        if (c->pos == 0) throw Error("no logits: run a token step first");
        *out = run_sample(c, sp, c->acts.logits, c->valid_n ? c->valid.as<uint8_t>() : nullptr, c->cfg.vocab);
    });
}

int qh_sample_logits(qh_ctx* c, qh_sampler* sp, const float* logits, const uint8_t* valid, size_t n,
                     uint32_t* out) {
    return guarded(c, [&] {
        if (n == 0) throw Error("invalid logits");
        HIP_OK(hipSetDevice(c->device));
        c->samp_logits.reserve(n * 4);
        HIP_OK(hipMemcpyAsync(c->samp_logits.p, logits, n * 4, hipMemcpyHostToDevice, c->s));
        if (valid) {
            c->samp_valid.reserve(n);
            HIP_OK(hipMemcpyAsync(c->samp_valid.p, valid, n, hipMemcpyHostToDevice, c->s));
        }
        *out = run_sample(c, sp, c->samp_logits.as<float>(), valid ? c->samp_valid.as<uint8_t>() : nullptr, n);
    });
}

int qh_device_count(int* out) {
    try {
        int n = 0;
        HIP_OK(hipGetDeviceCount(&n));
        *out = n;
        return 0;
    } catch (const std::exception& e) {
        g_create_err = e.what();
        return 1;
    }
}

int qh_device_name(int device, char* buf, size_t cap) {
    try {
        int n = 0;
        HIP_OK(hipGetDeviceCount(&n));
        if (device < 0 || device >= n) throw Error("HIP device " + std::to_string(device) + " not present");
        hipDeviceProp_t p;
        HIP_OK(hipGetDeviceProperties(&p, device));
        char arch[sizeof(p.gcnArchName) + 1] = {};
        std::memcpy(arch, p.gcnArchName, sizeof(p.gcnArchName));
        if (char* colon = std::strchr(arch, ':')) *colon = 0;
        const std::string name = p.name[0] ? std::string(p.name) : "HIP device " + std::to_string(device);
        const std::string s = name + " (" + arch + ", " + std::to_string(p.multiProcessorCount) +
                              " CUs, " + std::to_string(p.totalGlobalMem >> 30) + " GiB)";
        if (cap == 0 || s.size() + 1 > cap) throw Error("device name buffer too small");
        std::memcpy(buf, s.c_str(), s.size() + 1);
        return 0;
    } catch (const std::exception& e) {
        g_create_err = e.what();
        return 1;
    }
}

int qh_model_config(const qh_ctx* c, qh_config_t* out) {
    return guarded(const_cast<qh_ctx*>(c), [&] {
        need_model(const_cast<qh_ctx*>(c));
        const Config& g = c->cfg;
        *out = {g.hidden, g.layers, g.heads, g.kvheads, g.head_dim, g.experts, g.top, g.intermediate,
                g.vocab, g.max_context, g.eps, g.theta};
    });
}

int qh_tensor_info(const qh_ctx* c, const char* name, uint32_t* kind, size_t* rank, uint64_t dims[3]) {
    return guarded(const_cast<qh_ctx*>(c), [&] {
        need_model(const_cast<qh_ctx*>(c));
        auto it = c->tensors.find(name);
        if (it == c->tensors.end()) throw Error(std::string("missing tensor ") + name);
        *kind = it->second.kind;
        *rank = it->second.dims.size();
        for (size_t k = 0; k < 3; k++) dims[k] = k < it->second.dims.size() ? it->second.dims[k] : 0;
    });
}

int qh_packed_weight_bytes(const qh_ctx* c, uint64_t* out) {
    return guarded(const_cast<qh_ctx*>(c), [&] {
        need_model(const_cast<qh_ctx*>(c));
        *out = c->packed;
    });
}

int qh_matvec(qh_ctx* c, const char* name, int64_t expert, const float* x, size_t cols, float* y,
              size_t rows) {
    return guarded(c, [&] {
        double t0 = now_ms();
        need_model(c);
        auto it = c->tensors.find(name);
        if (it == c->tensors.end()) throw Error(std::string("missing tensor ") + name);
        const ModelTensor& t = it->second;
        if (t.dims.size() != (expert >= 0 ? 3u : 2u)) throw Error(std::string("matrix rank mismatch: ") + name);
        if (expert >= 0 && (uint64_t)expert >= t.dims[2]) throw Error("expert out of bounds");
        if (cols != t.dims[0]) throw Error(std::string("matvec shape mismatch ") + name);
        if (rows < t.dims[1]) throw Error("output buffer too small");
        DevMat m = t.mat;
        if (expert >= 0) m.w += (size_t)expert * m.expert_stride;
        const float* xd = upload_x(c, c->sb, x, cols);
        c->sc.reserve((size_t)m.rows * 4);
        launch_matvec(c, m, xd, c->sc.as<float>(), pick_r(m.rows, m.cols));
        HIP_OK(hipMemcpyAsync(y, c->sc.p, (size_t)m.rows * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        c->stats.matvecs += 1;
        c->stats.matvec_ms += now_ms() - t0;
    });
}

int qh_stats(const qh_ctx* c, qh_stats_t* out) {
    *out = c->stats;
    return 0;
}

int qh_packed_matvec(qh_ctx* c, const void* data, size_t len, uint32_t kind, size_t rows, size_t cols,
                     const float* x, float* y) {
    return guarded(c, [&] {
        double t0 = now_ms();
        size_t rb = row_bytes_checked(kind, cols);
        if (!(rows > 0 && rows * rb == len)) throw Error("GPU matvec shape mismatch");
        if (rows > 0xffffffffull) throw Error("matrix too tall");
        const size_t drb = dev_row_bytes(kind, cols);
        c->sd.reserve(rows * drb + 64);
        upload_rows(c, static_cast<const uint8_t*>(data), c->sd.as<uint8_t>(), kind, cols, rows);
        DevMat m = make_mat(c->sd.as<uint8_t>(), kind, rows, cols, 0);
        const float* xd = upload_x(c, c->sb, x, cols);
        c->sc.reserve(rows * 4);
        launch_matvec(c, m, xd, c->sc.as<float>(), pick_r(rows, cols));
        HIP_OK(hipMemcpyAsync(y, c->sc.p, rows * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        c->stats.matvecs += 1;
        c->stats.matvec_ms += now_ms() - t0;
    });
}

int qh_packed_matvec_batch(qh_ctx* c, const void* data, size_t len, uint32_t kind, size_t rows, size_t cols,
                           size_t nvec, const float* x, float* y) {
    return guarded(c, [&] {
        double t0 = now_ms();
        size_t rb = row_bytes_checked(kind, cols);
        if (!(nvec >= 1 && nvec <= 8 && rows > 0 && nvec * rows * rb == len)) throw Error("GPU matvec shape mismatch");
        if (rows > 0xffffffffull) throw Error("matrix too tall");
        HIP_OK(hipSetDevice(c->device));
        const size_t drb = dev_row_bytes(kind, cols);
        c->sd.reserve(nvec * rows * drb + 64);
        upload_rows(c, static_cast<const uint8_t*>(data), c->sd.as<uint8_t>(), kind, cols, nvec * rows);
        const DevMat m = make_mat(c->sd.as<uint8_t>(), kind, rows, cols, 0);
        const uint8_t* mats[8];
        for (size_t b = 0; b < nvec; b++) mats[b] = c->sd.as<uint8_t>() + b * rows * drb;
        const float* xd = upload_x(c, c->sb, x, nvec * cols);
        c->sc.reserve(nvec * rows * 4);
        if (!launch_mv_stream(m, mats, (uint32_t)nvec, xd, c->sc.as<float>(), c->num_cu, c->s))
            throw Error("batched matvec shape not covered (block-quantised rows of <= 8192 columns, "
                        "<= 12288 x floats)");
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(y, c->sc.p, nvec * rows * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        c->stats.matvecs += nvec;
        c->stats.matvec_ms += now_ms() - t0;
    });
}

int qh_dequant(qh_ctx* c, const void* data, size_t len, uint32_t kind, size_t rows, size_t cols, float* out) {
    return guarded(c, [&] {
        size_t rb = row_bytes_checked(kind, cols);
        if (len < rows * rb) throw Error("truncated quantized row");
        if (rows == 0) return;
        const size_t drb = dev_row_bytes(kind, cols);
        c->sd.reserve(rows * drb + 64);
        upload_rows(c, static_cast<const uint8_t*>(data), c->sd.as<uint8_t>(), kind, cols, rows);
        DevMat m = make_mat(c->sd.as<uint8_t>(), kind, rows, cols, 0);
        c->sc.reserve(rows * cols * 4);
        uint32_t grid = (uint32_t)std::min<uint64_t>((rows * cols + kBlock - 1) / kBlock, 65535);
        hipLaunchKernelGGL(k_dequant, dim3(grid), dim3(kBlock), 0, c->s, m, (size_t)0, rows, c->sc.as<float>());
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(out, c->sc.p, rows * cols * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
    });
}

int qh_route(qh_ctx* c, const float* logits, size_t n, size_t top, uint32_t* ids, float* w) {
    return guarded(c, [&] {
        if (top == 0 || top > n) throw Error("invalid MoE router");
        if (n > 0xffffffffull) throw Error("invalid MoE router");
        const float* ld = upload_x(c, c->sb, logits, n);
        c->sc.reserve(pad32h(top) * 8 + 256);
        uint32_t* dids = c->sc.as<uint32_t>();
        float* dw = reinterpret_cast<float*>(dids + pad32h(top));
        uint32_t* derr = reinterpret_cast<uint32_t*>(dw + pad32h(top));
        HIP_OK(hipMemsetAsync(derr, 0, 4, c->s));
        hipLaunchKernelGGL(k_route, dim3(1), dim3(kBlock), top * 4, c->s, ld, (uint32_t)n, (uint32_t)top, dids, dw, derr);
        HIP_OK(hipGetLastError());
        uint32_t e = 0;
        HIP_OK(hipMemcpyAsync(&e, derr, 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        if (e) throw Error("invalid MoE router");
        HIP_OK(hipMemcpyAsync(ids, dids, top * 4, hipMemcpyDeviceToHost, c->s));
        HIP_OK(hipMemcpyAsync(w, dw, top * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
    });
}

int qh_argmax(qh_ctx* c, const float* logits, size_t n, uint32_t* out) {
    return guarded(c, [&] {
        if (n == 0 || n > 0xffffffffull) throw Error("invalid logits");
        const float* ld = upload_x(c, c->sb, logits, n);
        uint32_t grid = (uint32_t)std::min<uint64_t>((n + kBlock * 8 - 1) / (kBlock * 8), 1024);
        c->sc.reserve((2 * 1024 + 64) * 4);
        int32_t* pk = c->sc.as<int32_t>();
        uint32_t* pi = reinterpret_cast<uint32_t*>(pk + 1024);
        uint32_t* misc = pi + 1024;  // [0] counter, [1] out, [2] err
        HIP_OK(hipMemsetAsync(misc, 0, 16, c->s));
        hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(kBlock), 0, c->s, ld, (uint32_t)n, pk, pi, misc, misc + 1, misc + 2);
        HIP_OK(hipGetLastError());
        uint32_t h[3];
        HIP_OK(hipMemcpyAsync(h, misc, 12, hipMemcpyDeviceToHost, c->s));
        sync(c);
        if (h[2]) throw Error("invalid logits");
        *out = h[1];
    });
}

// Launch geometry of k_attention_api for `heads` query heads over T keys:
// keys per chunk tc (the LDS budget), chunks nch, dynamic LDS bytes.
constexpr size_t kAttnApiMaxChunks = 64;  // most key chunks per KV head of k_attention_api
struct AttnGeo {
    size_t T;
    uint32_t tc, nch, span;
    size_t lds;
};
AttnGeo attn_geometry(size_t klen, size_t heads, size_t kvheads, size_t d) {
    if (!(kvheads > 0 && heads > 0 && d > 0 && heads % kvheads == 0 && klen % (kvheads * d) == 0))
        throw Error("attention shape mismatch");
    AttnGeo g{};
    g.T = klen / (kvheads * d);
    if (g.T == 0) throw Error("empty KV cache");
    const uint32_t G = (uint32_t)(heads / kvheads);
    auto lds = [&](uint32_t tc) { return (size_t)(2 * G * d + tc * (d + 1) + tc * d + G * tc + 3 * G) * 4; };
    g.tc = 64;
    while (g.tc > 1 && lds(g.tc) > 60 * 1024) g.tc /= 2;
    if (lds(g.tc) > 64 * 1024) throw Error("attention shape exceeds the LDS budget");
    // at most kAttnApiMaxChunks chunks per KV head, fewer when one chunk's
    // partials of every head would not fit the no-allocation scratch that
    // many times: a chunk then takes several tiles (both entry points use
    // this geometry, so they give the same bits)
    const size_t tiles = (g.T + g.tc - 1) / g.tc, per_chunk = heads * (d + 2) * 4;
    const size_t fit = (kNoAllocScratchBytes - 4096) / per_chunk;
    const size_t cap = std::max<size_t>(1, std::min<size_t>(kAttnApiMaxChunks, fit));
    const size_t span_tiles = (tiles + std::min(tiles, cap) - 1) / std::min(tiles, cap);
    g.span = (uint32_t)(span_tiles * g.tc);
    g.nch = (uint32_t)((g.T + g.span - 1) / g.span);
    g.lds = lds(g.tc);
    return g;
}

int qh_attention(qh_ctx* c, const float* q, const float* k, const float* v, size_t klen, size_t heads,
                 size_t kvheads, size_t d, float* out) {
    return guarded(c, [&] {
        const AttnGeo geo = attn_geometry(klen, heads, kvheads, d);
        const size_t T = geo.T;
        const uint32_t tc = geo.tc, nch = geo.nch;
        auto lds = [&](uint32_t) { return geo.lds; };
        const float* qd = upload_x(c, c->sa, q, heads * d);
        c->sb.reserve(klen * 8 + 256);
        HIP_OK(hipMemcpyAsync(c->sb.p, k, klen * 4, hipMemcpyHostToDevice, c->s));
        HIP_OK(hipMemcpyAsync(c->sb.as<float>() + klen, v, klen * 4, hipMemcpyHostToDevice, c->s));
        c->stats.uploaded_bytes += klen * 8;
        const size_t part = heads * nch * (d + 2);
        c->sc.reserve((part + heads * d + kvheads + 64) * 4);
        float* dpart = c->sc.as<float>();
        float* dout = dpart + part;
        uint32_t* cnt = reinterpret_cast<uint32_t*>(dout + heads * d);
        HIP_OK(hipMemsetAsync(cnt, 0, kvheads * 4, c->s));
        AttnArgs a{};
        a.q = qd;
        a.k = c->sb.as<float>();
        a.v = c->sb.as<float>() + klen;
        a.sh = d;
        a.st = kvheads * d;
        a.heads = (uint32_t)heads;
        a.kvheads = (uint32_t)kvheads;
        a.d = (uint32_t)d;
        a.tc = tc;
        a.max_chunks = nch;
        a.span = geo.span;
        a.part = dpart;
        a.counter = cnt;
        a.out = dout;
        a.err = nullptr;
        hipLaunchKernelGGL(k_attention_api, dim3((uint32_t)kvheads, nch), dim3(kBlock), lds(tc), c->s, a, (uint32_t)T);
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(out, dout, heads * d * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
    });
}

int qh_attention_noalloc(qh_ctx* c, const float* q, const float* k, const float* v, size_t klen, size_t heads,
                         size_t kvheads, size_t d, float* out, void* stream) {
    return guarded(c, [&] {
        const AttnGeo geo = attn_geometry(klen, heads, kvheads, d);
        const size_t part_bytes = (heads * geo.nch * (d + 2) * 4 + 255) / 256 * 256;
        const size_t need = part_bytes + kvheads * 4;
        if (need > kNoAllocScratchBytes)
            throw Error("attention over " + std::to_string(geo.T) + " keys needs " + std::to_string(need) +
                        " bytes of scratch; the no-allocation entry point holds " +
                        std::to_string(kNoAllocScratchBytes));
        uint8_t* base = static_cast<uint8_t*>(g_scratch_ptr[c->device]);
        if (!base) throw Error("no-allocation scratch is not set up on this device");
        uint32_t* cnt = reinterpret_cast<uint32_t*>(base + part_bytes);
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->s;
        // the counters start at zero (a fill kernel, no memset node)
        hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(kBlock), 0, s, cnt, kvheads, 0u);
        AttnArgs a{};
        a.q = q;
        a.k = k;
        a.v = v;
        a.sh = d;
        a.st = kvheads * d;
        a.heads = (uint32_t)heads;
        a.kvheads = (uint32_t)kvheads;
        a.d = (uint32_t)d;
        a.tc = geo.tc;
        a.max_chunks = geo.nch;
        a.span = geo.span;
        a.part = reinterpret_cast<float*>(base);
        a.counter = cnt;
        a.out = out;
        a.err = nullptr;
        hipLaunchKernelGGL(k_attention_api, dim3((uint32_t)kvheads, geo.nch), dim3(kBlock), geo.lds, s, a,
                           (uint32_t)geo.T);
        HIP_OK(hipGetLastError());
        if (!stream) HIP_OK(hipStreamSynchronize(s));
    });
}

int qh_forward(qh_ctx* c, uint32_t token, float* logits, size_t logits_cap, uint32_t* argmax) {
    return guarded(c, [&] {
        double t0 = now_ms();
        need_model(c);
        need_logits_room(c, logits, logits_cap);
        if (!(c->pos < c->context)) {
            reset_model(c);
            throw Error("context limit " + std::to_string(c->context) + " reached");
        }
        if (!(token < c->cfg.vocab)) {
            reset_model(c);
            throw Error("token outside vocabulary");
        }
        HIP_OK(hipMemcpyAsync(c->acts.tokens + c->pos, &token, 4, hipMemcpyHostToDevice, c->s));
        put_state(c, (uint32_t)c->pos, (uint32_t)c->pos + 1);
        launch_step(c);
        if (logits)
            HIP_OK(hipMemcpyAsync(logits, c->acts.logits, c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->s));
        DevState st = get_state(c);
        if (st.err) fail_step(c, st.err);
        c->pos += 1;
        if (argmax) *argmax = st.argmax;
        c->stats.matvecs += matvecs_per_token(c);
        c->stats.matvec_ms += now_ms() - t0;
    });
}

int qh_generate(qh_ctx* c, const uint32_t* prompt, size_t n_prompt, size_t n_new, uint32_t* out_tokens,
                float* logits_last, size_t logits_cap) {
    return guarded(c, [&] {
        double t0 = now_ms();
        need_model(c);
        need_logits_room(c, logits_last, logits_cap);
        if (n_prompt == 0) throw Error("empty prompt");
        const size_t steps = n_prompt + (n_new ? n_new - 1 : 0);
        if (c->pos + steps > c->context) throw Error("prompt + max-tokens exceed --ctx");
        for (size_t i = 0; i < n_prompt; i++)
            if (prompt[i] >= c->cfg.vocab) throw Error("token outside vocabulary");
        HIP_OK(hipMemcpyAsync(c->acts.tokens + c->pos, prompt, n_prompt * 4, hipMemcpyHostToDevice, c->s));
        put_state(c, (uint32_t)c->pos, (uint32_t)(c->pos + n_prompt));
        for (size_t i = 0; i < steps; i++) launch_step(c);
        DevState st = get_state(c);
        if (st.err) fail_step(c, st.err);
        if (n_new)
            HIP_OK(hipMemcpyAsync(out_tokens, c->acts.tokens + c->pos + n_prompt, n_new * 4, hipMemcpyDeviceToHost, c->s));
        if (logits_last)
            HIP_OK(hipMemcpyAsync(logits_last, c->acts.logits, c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        c->pos += steps;
        c->stats.matvecs += matvecs_per_token(c) * steps;
        c->stats.matvec_ms += now_ms() - t0;
    });
}

static void prefill_body(qh_ctx* c, const uint32_t* prompt, size_t n, float* logits, size_t logits_cap,
                         uint32_t* argmax, double t0);

int qh_prefill(qh_ctx* c, const uint32_t* prompt, size_t n, float* logits, size_t logits_cap, uint32_t* argmax) {
    return guarded(c, [&] {
        double t0 = now_ms();
        need_model(c);
        // the reference's prompt loop is one Model::forward per token
        // (src/main.rs:250-256): the prompt fails at its first token that
        // fails forward's checks (src/model.rs:219-223: the context limit,
        // then the vocabulary), and any error leaves a clean cache
        // (src/model.rs:209-216), here whatever failed
        try {
            prefill_body(c, prompt, n, logits, logits_cap, argmax, t0);
        } catch (...) {
            try {
                reset_model(c);
            } catch (...) {
            }
            throw;
        }
    });
}

static void prefill_body(qh_ctx* c, const uint32_t* prompt, size_t n, float* logits, size_t logits_cap,
                         uint32_t* argmax, double t0) {
    {
        need_logits_room(c, logits, logits_cap);
        if (n == 0) throw Error("empty prompt");
        for (size_t i = 0; i < n; i++) {
            if (c->pos + i >= c->context) throw Error("context limit " + std::to_string(c->context) + " reached");
            if (prompt[i] >= c->cfg.vocab) throw Error("token outside vocabulary");
        }
        // the prompt through the exact token step, one per token, on the
        // device, as the reference's prompt loop does (src/main.rs:250-256)
        auto run_exact = [&] {
            HIP_OK(hipMemcpyAsync(c->acts.tokens + c->pos, prompt, n * 4, hipMemcpyHostToDevice, c->s));
            put_state(c, (uint32_t)c->pos, (uint32_t)(c->pos + n));
            for (size_t i = 0; i < n; i++) launch_step(c);
            DevState st = get_state(c);
            if (st.err) fail_step(c, st.err);
            if (logits) HIP_OK(hipMemcpyAsync(logits, c->acts.logits, c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->s));
            sync(c);
            if (argmax) *argmax = st.argmax;
            c->pos += n;
            c->stats.matvecs += matvecs_per_token(c) * n;
            c->stats.matvec_ms += now_ms() - t0;
        };
        if (!prefill_gap(c).empty()) {  // outside the batched path's coverage (formats, head_dim, ...)
            run_exact();
            return;
        }
        prefill_tiles(c);
        size_t chunk = kPrefillChunk;
        if (const char* e = std::getenv("QH_PREFILL_CHUNK")) chunk = std::max<long>(1, std::atol(e));
        const uint32_t cap = (uint32_t)std::min<size_t>({n, chunk, kPrefillChunk, c->context});
        prefill_alloc(c, cap);
        auto& P = c->pf;
        const ModelDims& d = c->dm;
        const uint32_t p_start = (uint32_t)c->pos;
        HIP_OK(hipMemcpyAsync(c->acts.tokens + p_start, prompt, n * 4, hipMemcpyHostToDevice, c->s));
        // the tail (vocab projection + argmax) runs as the step of the last
        // prompt token: tokens[pos + n] receives the greedy id
        put_state(c, (uint32_t)(p_start + n - 1), (uint32_t)(p_start + n - 1));
        uint32_t S = 0;
        for (size_t c0 = 0; c0 < n; c0 += cap) {
            S = (uint32_t)std::min<size_t>(cap, n - c0);
            const uint32_t p0 = p_start + (uint32_t)c0;
            hipLaunchKernelGGL(k_pf_embed, dim3(S), dim3(kBlock), 0, c->s, c->emb, c->acts.tokens + p0, d.hidden,
                               d.vocab, P.X, c->acts.st);
            for (size_t l = 0; l < c->layers.size(); l++) prefill_layer(c, l, S, p0);
        }
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(c->acts.x, P.X + (size_t)(S - 1) * d.hidden, d.hidden * 4, hipMemcpyDeviceToDevice,
                              c->s));
        enqueue_tail(c);
        HIP_OK(hipGetLastError());
        DevState st = get_state(c);
        if (st.err) {
            // the prompt's tokens and positions were checked above, so this is
            // numeric: an fp16 operand out of range (kErrRange), or router
            // logits or output logits that are not finite.  The exact FP32
            // step runs the prompt again from the same position (it rewrites
            // every KV row the batched pass wrote); its own errors are final.
            c->prefill_reruns++;
            run_exact();
            return;
        }
        if (logits) HIP_OK(hipMemcpyAsync(logits, c->acts.logits, c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        if (argmax) *argmax = st.argmax;
        c->pos += n;
        c->stats.matvecs += matvecs_per_token(c) * n;
        c->stats.matvec_ms += now_ms() - t0;
    }
}

int qh_prefill_reruns(const qh_ctx* c, uint64_t* out) {
    *out = c->prefill_reruns;
    return 0;
}

// Frees the batched prefill's device memory: the tile-layout copies of the
// projection matrices and the chunk buffers.  The next batched prefill builds
// both again (its fp16 K/V copies come from the KV cache, which stays).
int qh_prefill_release(qh_ctx* c) {
    return guarded(c, [&] {
        need_model(c);
        HIP_OK(hipStreamSynchronize(c->s));
        auto& P = c->pf;
        for (LayerW& L : c->layers)
            for (DevMat* m : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down}) m->wt = nullptr;
        P.tiles.release();
        P.tiled = false;
        P.buf.release();
        P.cap = 0;
        P.max_tiles = 0;
    });
}

int qh_prefill_bytes(const qh_ctx* c, uint64_t* out) {
    *out = (uint64_t)c->pf.tiles.n + (uint64_t)c->pf.buf.n;
    return 0;
}

int qh_reset(qh_ctx* c) {
    return guarded(c, [&] {
        need_model(c);
        reset_model(c);
    });
}

int qh_position(const qh_ctx* c, size_t* out) {
    *out = c->pos;
    return 0;
}

int qh_layer_forward(qh_ctx* c, size_t layer, float* x, size_t pos, const float* kprev, const float* vprev,
                     uint32_t* ids, float* w) {
    return guarded(c, [&] {
        need_model(c);
        if (layer >= c->layers.size()) throw Error("layer out of range");
        if (pos >= c->context) throw Error("context limit " + std::to_string(c->context) + " reached");
        const ModelDims& d = c->dm;
        const LayerW& L = c->layers[layer];
        HIP_OK(hipMemcpyAsync(c->acts.x, x, d.hidden * 4, hipMemcpyHostToDevice, c->s));
        if (pos) {
            // time-major host history -> head-major device cache
            const size_t kvd = (size_t)d.kvheads * d.head_dim;
            std::vector<float> hk(pos * kvd), hv(pos * kvd);
            for (size_t t = 0; t < pos; t++)
                for (uint32_t h = 0; h < d.kvheads; h++) {
                    std::memcpy(&hk[(h * pos + t) * d.head_dim], kprev + t * kvd + h * d.head_dim, d.head_dim * 4);
                    std::memcpy(&hv[(h * pos + t) * d.head_dim], vprev + t * kvd + h * d.head_dim, d.head_dim * 4);
                }
            for (uint32_t h = 0; h < d.kvheads; h++) {
                HIP_OK(hipMemcpyAsync(L.kcache + (size_t)h * c->context * d.head_dim, &hk[h * pos * d.head_dim],
                                      pos * d.head_dim * 4, hipMemcpyHostToDevice, c->s));
                HIP_OK(hipMemcpyAsync(L.vcache + (size_t)h * c->context * d.head_dim, &hv[h * pos * d.head_dim],
                                      pos * d.head_dim * 4, hipMemcpyHostToDevice, c->s));
            }
            c->stats.uploaded_bytes += 2 * pos * kvd * 4;
            sync(c);  // host staging vectors go out of scope
        }
        put_state(c, (uint32_t)pos, (uint32_t)pos + 1);
        if (c->persist)
            launch_decode(c, (uint32_t)layer, (uint32_t)layer + 1, false, false);
        else
            enqueue_layer(c, layer, false);
        HIP_OK(hipGetLastError());
        HIP_OK(hipMemcpyAsync(x, c->acts.x, d.hidden * 4, hipMemcpyDeviceToHost, c->s));
        if (ids) HIP_OK(hipMemcpyAsync(ids, c->acts.ids, d.top * 4, hipMemcpyDeviceToHost, c->s));
        if (w) HIP_OK(hipMemcpyAsync(w, c->acts.wts, d.top * 4, hipMemcpyDeviceToHost, c->s));
        DevState st = get_state(c);
        reset_model(c);
        if (st.err) fail_step(c, st.err);
    });
}

int qh_route_log(qh_ctx* c, size_t pos0, size_t n, uint32_t* ids) {
    return guarded(c, [&] {
        need_model(c);
        if (pos0 + n > c->context) throw Error("routing log range beyond the context");
        const size_t row = (size_t)c->dm.layers * c->dm.top;
        HIP_OK(hipMemcpyAsync(ids, c->acts.route_log + pos0 * row, n * row * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
    });
}

int qh_route_gap_log(qh_ctx* c, size_t pos0, size_t n, float* gaps) {
    return guarded(c, [&] {
        need_model(c);
        if (pos0 + n > c->context) throw Error("routing log range beyond the context");
        const size_t row = c->dm.layers;
        HIP_OK(hipMemcpyAsync(gaps, c->acts.gap_log + pos0 * row, n * row * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
    });
}

int qh_read_kv(qh_ctx* c, size_t layer, size_t pos0, size_t n, float* k, float* v) {
    return guarded(c, [&] {
        need_model(c);
        if (layer >= c->layers.size()) throw Error("layer out of range");
        if (pos0 + n > c->context) throw Error("KV range beyond the context");
        const ModelDims& d = c->dm;
        const LayerW& L = c->layers[layer];
        // device head-major [kvhead][ctx][d] -> time-major [t][kvhead][d]
        for (uint32_t h = 0; h < d.kvheads; h++) {
            const size_t src = ((size_t)h * c->context + pos0) * d.head_dim;
            HIP_OK(hipMemcpy2DAsync(k + (size_t)h * d.head_dim, (size_t)d.kvheads * d.head_dim * 4, L.kcache + src,
                                    d.head_dim * 4, d.head_dim * 4, n, hipMemcpyDeviceToHost, c->s));
            HIP_OK(hipMemcpy2DAsync(v + (size_t)h * d.head_dim, (size_t)d.kvheads * d.head_dim * 4, L.vcache + src,
                                    d.head_dim * 4, d.head_dim * 4, n, hipMemcpyDeviceToHost, c->s));
        }
        sync(c);
    });
}

int qh_model_generation(const qh_ctx* c, uint64_t* out) {
    *out = c->generation;
    return 0;
}

int qh_fault_inject(qh_ctx* c, uint32_t kind) {
    return guarded(c, [&] {
        need_model(c);
        if (kind != QH_FAULT_ABORT) throw Error("unknown fault kind " + std::to_string(kind));
        if (!c->persist) throw Error("the abort fault needs the persistent step");
        const uint32_t one = 1;
        HIP_OK(hipMemcpyAsync(c->dargs.abort_flag, &one, 4, hipMemcpyHostToDevice, c->s));
        sync(c);
    });
}

int qh_persistent(const qh_ctx* c, int* out) {
    return guarded(const_cast<qh_ctx*>(c), [&] {
        need_model(const_cast<qh_ctx*>(c));
        *out = c->persist ? 1 : 0;
    });
}

int qh_prefill_batched(const qh_ctx* c, int* out) {
    return guarded(const_cast<qh_ctx*>(c), [&] {
        need_model(const_cast<qh_ctx*>(c));
        *out = prefill_gap(c).empty() ? 1 : 0;
    });
}

int qh_set_persistent(qh_ctx* c, int enable) {
    return guarded(c, [&] {
        need_model(c);
        if (enable && !c->persist_ok) throw Error("the persistent step does not cover this model");
        c->persist = enable != 0;
    });
}

int qh_profile_decode(qh_ctx* c, size_t steps, double* ms_embed, double* ms_decode) {
    return guarded(c, [&] {
        need_model(c);
        if (!c->persist) throw Error("profile_decode times the persistent step: it is not selected");
        if (c->pos == 0) throw Error("profile_decode continues a sequence: run a prompt first");
        if (c->pos + steps > c->context) throw Error("prompt + max-tokens exceed --ctx");
        // the steps queued back to back, as the token loop runs them (a step
        // launched onto an idle queue would add the queue's wake-up to its
        // time); events before and after each launch, read at the end.  The
        // step is one launch (the embedding row included): the interval
        // between the two events before it is empty
        std::vector<hipEvent_t> ev(3 * steps);
        for (auto& e : ev) HIP_OK(hipEventCreate(&e));
        double acc[2] = {0.0, 0.0};
        put_state(c, (uint32_t)c->pos, (uint32_t)c->pos);
        for (size_t s = 0; s < steps; s++) {
            HIP_OK(hipEventRecord(ev[3 * s], c->s));
            HIP_OK(hipEventRecord(ev[3 * s + 1], c->s));
            launch_decode(c, 0, (uint32_t)c->layers.size(), true, true);
            HIP_OK(hipEventRecord(ev[3 * s + 2], c->s));
        }
        HIP_OK(hipEventSynchronize(ev[3 * steps - 1]));
        for (size_t s = 0; s < steps; s++)
            for (int k = 0; k < 2; k++) {
                float ms = 0;
                HIP_OK(hipEventElapsedTime(&ms, ev[3 * s + k], ev[3 * s + k + 1]));
                acc[k] += ms;
            }
        for (auto& e : ev) (void)hipEventDestroy(e);
        DevState st = get_state(c);
        if (st.err) fail_step(c, st.err);
        c->pos += steps;
        c->stats.matvecs += matvecs_per_token(c) * steps;
        *ms_embed = acc[0] / (double)steps;
        *ms_decode = acc[1] / (double)steps;
    });
}

int qh_bench_decode(qh_ctx* c, size_t warmup, size_t steps, double* ms_total) {
    return guarded(c, [&] {
        need_model(c);
        if (c->pos == 0) throw Error("bench_decode continues a sequence: run a prompt first");
        if (c->pos + warmup + steps > c->context) throw Error("prompt + max-tokens exceed --ctx");
        put_state(c, (uint32_t)c->pos, (uint32_t)c->pos);
        for (size_t i = 0; i < warmup; i++) launch_step(c);
        hipEvent_t e0, e1;
        HIP_OK(hipEventCreate(&e0));
        HIP_OK(hipEventCreate(&e1));
        HIP_OK(hipEventRecord(e0, c->s));
        for (size_t i = 0; i < steps; i++) launch_step(c);
        HIP_OK(hipEventRecord(e1, c->s));
        HIP_OK(hipEventSynchronize(e1));
        float ms = 0;
        HIP_OK(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        DevState st = get_state(c);
        if (st.err) fail_step(c, st.err);
        c->pos += warmup + steps;
        c->stats.matvecs += matvecs_per_token(c) * (warmup + steps);
        *ms_total = ms;
    });
}

int qh_profile_step(qh_ctx* c, size_t steps, double* ms_by_class, size_t nclass) {
    return guarded(c, [&] {
        need_model(c);
        if (nclass < QH_NUM_KERNEL_CLASSES) throw Error("ms_by_class needs QH_NUM_KERNEL_CLASSES entries");
        if (c->pos == 0) throw Error("profile_step continues a sequence: run a prompt first");
        if (c->pos + steps > c->context) throw Error("prompt + max-tokens exceed --ctx");
        const size_t L = c->layers.size();
        std::vector<hipEvent_t> ev(1 + 5 * L + 2);
        for (auto& e : ev) HIP_OK(hipEventCreate(&e));
        std::vector<double> acc(QH_NUM_KERNEL_CLASSES, 0.0);
        put_state(c, (uint32_t)c->pos, (uint32_t)c->pos);
        for (size_t s = 0; s < steps; s++) {
            size_t k = 0;
            HIP_OK(hipEventRecord(ev[k++], c->s));
            for (size_t l = 0; l < L; l++) {
                for (int kk = 0; kk < 5; kk++) {
                    enqueue_kernel(c, l, l == 0, kk);
                    HIP_OK(hipEventRecord(ev[k++], c->s));
                }
            }
            enqueue_vocab(c);
            HIP_OK(hipEventRecord(ev[k++], c->s));
            hipLaunchKernelGGL(k_finish, dim3(1), dim3(kBlock), 0, c->s, c->acts, c->dm, c->g_vocab);
            HIP_OK(hipEventRecord(ev[k++], c->s));
            HIP_OK(hipGetLastError());
            HIP_OK(hipEventSynchronize(ev[k - 1]));
            auto el = [&](size_t a) {
                float ms = 0;
                HIP_OK(hipEventElapsedTime(&ms, ev[a], ev[a + 1]));
                return (double)ms;
            };
            for (size_t l = 0; l < L; l++)
                for (size_t j = 0; j < 5; j++) acc[j] += el(5 * l + j);
            acc[5] += el(5 * L);
            acc[6] += el(5 * L + 1);
        }
        for (auto& e : ev) (void)hipEventDestroy(e);
        DevState st = get_state(c);
        if (st.err) fail_step(c, st.err);
        c->pos += steps;
        for (size_t j = 0; j < QH_NUM_KERNEL_CLASSES; j++) ms_by_class[j] = acc[j] / (double)steps;
    });
}

int qh_bench_read(qh_ctx* c, size_t bytes, size_t copies, size_t iters, qh_matvec_timing_t* out) {
    return guarded(c, [&] {
        if (bytes < 16 || copies == 0 || iters == 0) throw Error("bytes, copies and iters must be positive");
        HIP_OK(hipSetDevice(c->device));
        const size_t one = bytes / 16 * 16;
        DevBuf w, o;
        w.alloc(one * copies);
        o.alloc(64);
        HIP_OK(hipMemsetAsync(w.p, 0x5a, one * copies, c->s));
        const uint32_t grid = 4 * std::max(c->num_cu, 1u);
        auto launch = [&](size_t i) {
            launch_read_stream(w.as<uint8_t>() + (i % copies) * one, one, o.as<uint32_t>(), grid, c->s);
            HIP_OK(hipGetLastError());
        };
        for (size_t i = 0; i < std::min<size_t>(copies, 4); i++) launch(i);
        std::vector<hipEvent_t> ev(2 * iters + 2, nullptr);
        for (auto& e : ev) HIP_OK(hipEventCreate(&e));
        float ms = 0;
        HIP_OK(hipEventRecord(ev[0], c->s));
        for (size_t i = 0; i < iters; i++) launch(i);
        HIP_OK(hipEventRecord(ev[1], c->s));
        HIP_OK(hipEventSynchronize(ev[1]));
        HIP_OK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        out->mean_ms = ms / (double)iters;
        out->empty_ms = 0;
        for (size_t i = 0; i < iters; i++) {
            HIP_OK(hipEventRecord(ev[2 + 2 * i], c->s));
            launch(i);
            HIP_OK(hipEventRecord(ev[3 + 2 * i], c->s));
        }
        HIP_OK(hipEventSynchronize(ev[1 + 2 * iters]));
        std::vector<float> t(iters);
        for (size_t i = 0; i < iters; i++) HIP_OK(hipEventElapsedTime(&t[i], ev[2 + 2 * i], ev[3 + 2 * i]));
        for (auto& e : ev) (void)hipEventDestroy(e);
        std::sort(t.begin(), t.end());
        out->median_ms = iters % 2 ? t[iters / 2] : 0.5 * ((double)t[iters / 2 - 1] + t[iters / 2]);
        sync(c);
    });
}

int qh_bench_matvec(qh_ctx* c, const void* data, size_t len, uint32_t kind, size_t rows, size_t cols, size_t nvec,
                    const float* x, size_t copies, size_t iters, qh_matvec_timing_t* out) {
    return guarded(c, [&] {
        size_t rb = row_bytes_checked(kind, cols);
        if (!(nvec >= 1 && nvec <= 8 && rows > 0 && nvec * rows * rb == len)) throw Error("GPU matvec shape mismatch");
        if (rows > 0xffffffffull) throw Error("matrix too tall");
        if (copies == 0 || iters == 0) throw Error("copies and iters must be positive");
        HIP_OK(hipSetDevice(c->device));
        const size_t drb = dev_row_bytes(kind, cols), one = nvec * rows * drb;
        DevBuf w;
        w.alloc(one * copies + 64);
        upload_rows(c, static_cast<const uint8_t*>(data), w.as<uint8_t>(), kind, cols, nvec * rows);
        for (size_t i = 1; i < copies; i++)
            HIP_OK(hipMemcpyAsync(w.as<uint8_t>() + i * one, w.p, one, hipMemcpyDeviceToDevice, c->s));
        DevBuf xb, yb;
        xb.alloc(pad32h(nvec * cols) * 4);
        HIP_OK(hipMemsetAsync(xb.p, 0, pad32h(nvec * cols) * 4, c->s));
        HIP_OK(hipMemcpyAsync(xb.p, x, nvec * cols * 4, hipMemcpyHostToDevice, c->s));
        yb.alloc(nvec * rows * 4);
        const int R = pick_r(rows, cols);
        auto launch = [&](size_t i) {
            const uint8_t* base = w.as<uint8_t>() + (i % copies) * one;
            const DevMat m = make_mat(base, kind, rows, cols, 0);
            if (nvec == 1) {
                launch_matvec(c, m, xb.as<float>(), yb.as<float>(), R);
                return;
            }
            const uint8_t* mats[8];
            for (size_t b = 0; b < nvec; b++) mats[b] = base + b * rows * drb;
            if (!launch_mv_stream(m, mats, (uint32_t)nvec, xb.as<float>(), yb.as<float>(), c->num_cu, c->s))
                throw Error("batched matvec shape not covered by the streaming kernel");
            HIP_OK(hipGetLastError());
        };
        for (size_t i = 0; i < std::min<size_t>(copies, 8); i++) launch(i);
        std::vector<hipEvent_t> ev(2 * iters + 2, nullptr);
        for (auto& e : ev) HIP_OK(hipEventCreate(&e));
        float ms = 0;
        // back-to-back launches
        HIP_OK(hipEventRecord(ev[0], c->s));
        for (size_t i = 0; i < iters; i++) launch(i);
        HIP_OK(hipEventRecord(ev[1], c->s));
        HIP_OK(hipEventSynchronize(ev[1]));
        HIP_OK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        out->mean_ms = ms / (double)iters;
        // the empty kernel, back to back: the launch floor
        HIP_OK(hipEventRecord(ev[0], c->s));
        for (size_t i = 0; i < iters; i++) launch_empty(c->s);
        HIP_OK(hipEventRecord(ev[1], c->s));
        HIP_OK(hipEventSynchronize(ev[1]));
        HIP_OK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        out->empty_ms = ms / (double)iters;
        // each launch between its own pair of events
        for (size_t i = 0; i < iters; i++) {
            HIP_OK(hipEventRecord(ev[2 + 2 * i], c->s));
            launch(i);
            HIP_OK(hipEventRecord(ev[3 + 2 * i], c->s));
        }
        HIP_OK(hipEventSynchronize(ev[1 + 2 * iters]));
        std::vector<float> t(iters);
        for (size_t i = 0; i < iters; i++) HIP_OK(hipEventElapsedTime(&t[i], ev[2 + 2 * i], ev[3 + 2 * i]));
        for (auto& e : ev) (void)hipEventDestroy(e);
        std::sort(t.begin(), t.end());
        out->median_ms = iters % 2 ? t[iters / 2] : 0.5 * ((double)t[iters / 2 - 1] + t[iters / 2]);
        std::vector<float> y(nvec * rows);
        HIP_OK(hipMemcpyAsync(y.data(), yb.p, y.size() * 4, hipMemcpyDeviceToHost, c->s));
        sync(c);
        for (float v : y)
            if (!std::isfinite(v)) throw Error("benchmark matvec produced a non-finite value");
    });
}

}  // extern "C"
