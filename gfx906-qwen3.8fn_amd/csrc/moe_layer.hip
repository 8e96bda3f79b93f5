// Layer object and C ABI (include/moe_ffn.h) of the MI355X routed-MoE FFN.
//
// Boundary conventions follow the reference launchers (src/hip/linear.cuh:35-45,
// src/hip/session_ops.cuh:22-45): every argument is checked before the first
// HIP call, launchers only enqueue on the caller's stream, and only create /
// destroy / export, the diagnostics and the expert timing harness allocate or
// synchronise.
#include "moe_expf.h"
#include "moe_ffn.h"
#include "moe_internal.hpp"

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <new>

using moe::Act;
using moe::Item;
using moe::RouteOut;
using moe::Shape;

struct moe_ffn_layer {
    moe_ffn_config cfg{};
    int device = 0;
    Shape shape{};
    // Weight upload time (ExpertTiming::upload_ms): from the start of the
    // bank allocation until the repacked planes are complete.
    std::chrono::steady_clock::time_point create_start{};
    double upload_ms = 0.0;
    void *bank_mem = nullptr;
    size_t bank_bytes = 0;
    moe::Bank bank{};
    uint8_t *gate_codes = nullptr, *up_codes = nullptr, *down_codes = nullptr;
    uint16_t *gate_scales = nullptr, *up_scales = nullptr, *down_scales = nullptr;
    uint16_t *down_mins = nullptr;   // Q4_1 down matrices only
    bool down_q41 = false;
    void *ws_mem = nullptr;
    size_t ws_bytes = 0;
    Act xq{}, mq{};
    RouteOut routes{};
    float *contrib = nullptr;
    // Error word of the diagnostics (debug_last / last_stats re-group a
    // decode-path batch): never the caller's flag of a finished forward.
    int *diag_error = nullptr;
    // Smallest group routed to the MFMA path (0 = streaming only).  An MFMA
    // tile spends the same exact-order epilogue on 32 token columns however
    // many are filled; the streaming kernels do their integer dots on VALU at
    // about 3x the work per column, so from about 12 pairs a part-filled
    // tile is cheaper.  Measured on MI355X (us per layer at mfma_min 32 / 16
    // / 12 / 8): 4K Zipf(1.1) 1801 / 1552 / 1534 / 1537, 1032-token
    // Zipf(1.3) 662 / 608 / 580 / 579, 1032 uniform 1270 / 644 / 631 / 627,
    // 300 Zipf(1.3) 319 / 299 / 300 / 297, 256 uniform 358 / 355 / 348 / 354;
    // 16K uniform (all groups above 256) unaffected.
    int mfma_min = 12;
    // Batches of fewer routes (tokens x k) stream every group: below this the
    // MFMA items are too few to fill the chip and the streaming kernels win
    // (single-expert and 8-expert layers at 2048/512 and 2560/640: MFMA ahead
    // from about 1024 routes, streaming up to 3x ahead below 256).  An explicit
    // MOE_FFN_MFMA_MIN turns this off; MOE_FFN_MFMA_ROUTES sets it.
    int mfma_routes = 1024;
    int active_mfma_min = 12;   // mfma_min of the current / last forward
    int decode_mode = -1; // ungrouped decode path: -1 auto, 0 never, 1 whenever shapes allow
    bool last_decode = false;
    int cu_count = 256;   // compute units of the device
    int last_tokens = 0;
    // Inputs of the last forward (for moe_ffn_replay_stage).
    const float *last_x = nullptr, *last_weights = nullptr, *last_shared_gate = nullptr;
    const void *x_q8_in = nullptr;   // canonical Q8_1 input of the current / last forward_q8 (else nullptr)
    const int32_t *last_ids = nullptr;
    float *last_y = nullptr;
    int *last_error = nullptr;
    hipStream_t last_stream = nullptr;   // stream of the last forward (its side-stream work joins it)
    // Stage profiler (moe_ffn_profile): a ring of events, one set per forward.
    static constexpr int kStageMarks = MOE_STAGE_FOLD + 2;
    // Grouped forwards run the streaming items (small groups, bound by memory
    // latency) on `side` while the MFMA items (bound by VALU) run on the
    // caller's stream; fork/join events order them after grouping and before
    // the fold.
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool two_streams = true;
    hipEvent_t *prof_events = nullptr;
    int prof_capacity = 0, prof_used = 0;
};

namespace {

constexpr int kInvalid = hipErrorInvalidValue;

bool aligned(const void *p, size_t a) { return p && reinterpret_cast<uintptr_t>(p) % a == 0; }

bool config_ok(const moe_ffn_config *c) {
    return c && c->hidden >= 32 && c->hidden <= 16384 && c->hidden % 32 == 0 && c->intermediate >= 32 &&
           c->intermediate <= 16384 && c->intermediate % 32 == 0 && c->experts >= 1 && c->experts <= 4096 &&
           c->top_k >= 1 && c->top_k <= 32 && c->top_k <= c->experts && (c->has_shared == 0 || c->has_shared == 1) &&
           c->max_tokens >= 1 && c->max_tokens <= 65536 && c->hidden % 64 == 0 &&
           (c->down_type == MOE_DOWN_Q4_0 || c->down_type == MOE_DOWN_Q4_1);
}

Shape shape_of(const moe_ffn_config &c) {
    return Shape{c.hidden, c.intermediate, c.experts, c.experts + c.has_shared, c.top_k};
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t matrix_blocks(const Shape &s) { return static_cast<size_t>(s.H / 32) * s.I; }

// Canonical bytes of one matrix kind (m: 0 gate, 1 up, 2 down) of one expert,
// and of one expert: 18-byte Q4_0 blocks, 20-byte Q4_1 blocks for a Q4_1 down.
size_t matrix_bytes(const Shape &s, bool down_q41, int m) {
    return matrix_blocks(s) * (m == 2 && down_q41 ? 20 : 18);
}
size_t expert_bytes(const Shape &s, bool down_q41) {
    return matrix_bytes(s, down_q41, 0) + matrix_bytes(s, down_q41, 1) + matrix_bytes(s, down_q41, 2);
}

// Bank: code planes (16 B/block), scale planes (2 B/block), and for Q4_1
// down matrices a mins plane (2 B/block).
size_t bank_layout(const Shape &s, bool down_q41, size_t off[7]) {
    const size_t gb = static_cast<size_t>(s.Ep) * matrix_blocks(s);   // gate blocks == up blocks == down blocks
    size_t p = 0;
    for (int m = 0; m < 3; ++m) { off[m] = p; p = round_up(p + gb * 16, 256); }
    for (int m = 0; m < 3; ++m) { off[3 + m] = p; p = round_up(p + gb * 2, 256); }
    off[6] = p;
    if (down_q41) p = round_up(p + gb * 2, 256);
    return p;
}

struct WsLayout {
    size_t xq_codes, xq_heads, mq_codes, mq_heads, pair_token, pair_rank, pos_of, counts, offsets,
        stream_items, mfma_items, item_counts, bitmap, wprefix, contrib, diag_error, total;
};

size_t pairs_capacity(const Shape &s, int N) { return static_cast<size_t>(N) * s.k + (s.Ep > s.E ? N : 0); }

WsLayout ws_layout(const Shape &s, int N) {
    WsLayout w{};
    const size_t nbh = s.H / 32, nbi = s.I / 32, P = pairs_capacity(s, N);
    const size_t W = (static_cast<size_t>(N) + 31) / 32;
    size_t p = 0;
    auto take = [&](size_t bytes) { const size_t at = p; p = round_up(p + bytes, 256); return at; };
    w.xq_codes = take(static_cast<size_t>(N) * nbh * 32);
    w.xq_heads = take(static_cast<size_t>(N) * nbh * 4);
    w.mq_codes = take(P * nbi * 32);
    w.mq_heads = take(P * nbi * 4);
    w.pair_token = take(P * 4);
    w.pair_rank = take(P * 4);
    w.pos_of = take(static_cast<size_t>(N) * s.k * 4);
    w.counts = take(static_cast<size_t>(s.Ep) * 4);
    w.offsets = take((static_cast<size_t>(s.Ep) + 1) * 4);
    w.stream_items = take((P / moe::kStreamTokens + s.Ep + 1) * sizeof(Item));
    w.mfma_items = take((P / moe::kMfmaTile + s.Ep + 1) * sizeof(Item));
    w.item_counts = take(16);
    w.bitmap = take(W * s.Ep * 4);
    w.wprefix = take(W * s.Ep * 4);
    w.contrib = take(static_cast<size_t>(N) * (s.k + 1) * s.H * 4);
    w.diag_error = take(4);
    w.total = p;
    return w;
}

int finish_create(moe_ffn_layer *L) {
    // Workspace.
    const WsLayout w = ws_layout(L->shape, L->cfg.max_tokens);
    if (hipMalloc(&L->ws_mem, w.total) != hipSuccess) return hipErrorOutOfMemory;
    L->ws_bytes = w.total;
    auto *b = static_cast<uint8_t *>(L->ws_mem);
    L->xq = Act{b + w.xq_codes, reinterpret_cast<uint32_t *>(b + w.xq_heads)};
    L->mq = Act{b + w.mq_codes, reinterpret_cast<uint32_t *>(b + w.mq_heads)};
    L->routes.pair_token = reinterpret_cast<int32_t *>(b + w.pair_token);
    L->routes.pair_rank = reinterpret_cast<int32_t *>(b + w.pair_rank);
    L->routes.pos_of = reinterpret_cast<int32_t *>(b + w.pos_of);
    L->routes.counts = reinterpret_cast<int32_t *>(b + w.counts);
    L->routes.offsets = reinterpret_cast<int32_t *>(b + w.offsets);
    L->routes.stream_items = reinterpret_cast<Item *>(b + w.stream_items);
    L->routes.mfma_items = reinterpret_cast<Item *>(b + w.mfma_items);
    L->routes.item_counts = reinterpret_cast<int32_t *>(b + w.item_counts);
    L->routes.bitmap = reinterpret_cast<uint32_t *>(b + w.bitmap);
    L->routes.wprefix = reinterpret_cast<uint32_t *>(b + w.wprefix);
    L->contrib = reinterpret_cast<float *>(b + w.contrib);
    L->diag_error = reinterpret_cast<int *>(b + w.diag_error);
    if (hipMemset(L->ws_mem, 0, w.total) != hipSuccess) return hipErrorOutOfMemory;
    if (const char *env = std::getenv("MOE_FFN_MFMA_MIN")) {
        L->mfma_min = std::atoi(env);
        L->mfma_routes = 0;
    }
    if (const char *env = std::getenv("MOE_FFN_MFMA_ROUTES")) L->mfma_routes = std::atoi(env);
    if (const char *env = std::getenv("MOE_FFN_DECODE")) L->decode_mode = std::atoi(env) ? 1 : 0;
    if (const char *env = std::getenv("MOE_FFN_STREAMS")) L->two_streams = std::atoi(env) != 1;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, L->device) == hipSuccess && cus > 0)
        L->cu_count = cus;
    return hipDeviceSynchronize();
}

int alloc_bank(moe_ffn_layer *L) {
    size_t off[7];
    L->bank_bytes = bank_layout(L->shape, L->down_q41, off);
    if (hipMalloc(&L->bank_mem, L->bank_bytes) != hipSuccess) return hipErrorOutOfMemory;
    auto *b = static_cast<uint8_t *>(L->bank_mem);
    L->gate_codes = b + off[0];
    L->up_codes = b + off[1];
    L->down_codes = b + off[2];
    L->gate_scales = reinterpret_cast<uint16_t *>(b + off[3]);
    L->up_scales = reinterpret_cast<uint16_t *>(b + off[4]);
    L->down_scales = reinterpret_cast<uint16_t *>(b + off[5]);
    L->down_mins = L->down_q41 ? reinterpret_cast<uint16_t *>(b + off[6]) : nullptr;
    L->bank = moe::Bank{L->gate_codes, L->up_codes, L->down_codes, L->gate_scales, L->up_scales, L->down_scales,
                        L->down_mins};
    return hipSuccess;
}

// One matrix kind's planes: gate (m = 0), up (1), down (2).
struct Plane {
    uint8_t *codes;
    uint16_t *scales, *mins;   // mins: Q4_1 down only
    int blocks_per_row, group;
};

Plane plane(const moe_ffn_layer *L, int m) {
    const int nbh = L->shape.H / 32, nbi = L->shape.I / 32;
    if (m == 0) return Plane{L->gate_codes, L->gate_scales, nullptr, nbh, moe::kScaleGroupGateUp};
    if (m == 1) return Plane{L->up_codes, L->up_scales, nullptr, nbh, moe::kScaleGroupGateUp};
    return Plane{L->down_codes, L->down_scales, L->down_mins, nbi, moe::kScaleGroupDown};
}

// Repack `count` canonical experts starting at expert `first` from a device
// staging buffer into the planes.
int repack_experts(moe_ffn_layer *L, const uint8_t *staging, int first, int count) {
    const Shape &s = L->shape;
    const size_t mblocks = matrix_blocks(s);   // blocks per matrix
    for (int i = 0; i < count; ++i) {
        const size_t e = static_cast<size_t>(first + i);
        const uint8_t *src = staging + static_cast<size_t>(i) * expert_bytes(s, L->down_q41);
        for (int m = 0; m < 3; ++m) {
            const Plane pl = plane(L, m);
            const hipError_t r = moe::launch_repack_weights(src, pl.codes, pl.scales, pl.mins, mblocks, e * mblocks,
                                                            pl.blocks_per_row, pl.group, nullptr);
            if (r != hipSuccess) return r;
            src += matrix_bytes(s, L->down_q41, m);
        }
    }
    return hipSuccess;
}

// The layer's device must be current (the create entry points hold a
// DeviceScope around the whole creation).
int create_common(const moe_ffn_config *config, int device, moe_ffn_layer *&L) {
    L = new (std::nothrow) moe_ffn_layer();
    if (!L) return hipErrorOutOfMemory;
    L->cfg = *config;
    L->device = device;
    L->shape = shape_of(*config);
    L->down_q41 = config->down_type == MOE_DOWN_Q4_1;
    L->create_start = std::chrono::steady_clock::now();
    int r = alloc_bank(L);
    if (r == hipSuccess && (hipStreamCreateWithFlags(&L->side, hipStreamNonBlocking) != hipSuccess ||
                            hipEventCreateWithFlags(&L->fork, hipEventDisableTiming) != hipSuccess ||
                            hipEventCreateWithFlags(&L->join, hipEventDisableTiming) != hipSuccess))
        r = hipErrorOutOfMemory;
    if (r != hipSuccess) { moe_ffn_destroy(L); L = nullptr; return r; }
    return hipSuccess;
}


int upload(moe_ffn_layer *L, const void *experts, const void *shared, bool from_device) {
    const Shape &s = L->shape;
    const size_t ebytes = expert_bytes(s, L->down_q41);
    const int chunk = static_cast<int>(std::max<size_t>(1, (size_t{256} << 20) / ebytes));
    uint8_t *staging = nullptr;
    if (!from_device && hipMalloc(&staging, static_cast<size_t>(chunk) * ebytes) != hipSuccess)
        return hipErrorOutOfMemory;
    int r = hipSuccess;
    for (int first = 0; first < s.Ep && r == hipSuccess; first += chunk) {
        const int n = std::min(chunk, s.Ep - first);
        // Shared expert (index E) comes from its own pointer.
        const int routed = std::max(0, std::min(n, s.E - first));
        const uint8_t *src_routed = static_cast<const uint8_t *>(experts) + static_cast<size_t>(first) * ebytes;
        if (routed > 0) {
            if (from_device) r = repack_experts(L, src_routed, first, routed);
            else {
                r = hipMemcpy(staging, src_routed, routed * ebytes, hipMemcpyHostToDevice);
                if (r == hipSuccess) r = repack_experts(L, staging, first, routed);
                if (r == hipSuccess) r = hipDeviceSynchronize();
            }
        }
        if (r == hipSuccess && routed < n) {   // the shared expert
            if (from_device) r = repack_experts(L, static_cast<const uint8_t *>(shared), s.E, 1);
            else {
                r = hipMemcpy(staging, shared, ebytes, hipMemcpyHostToDevice);
                if (r == hipSuccess) r = repack_experts(L, staging, s.E, 1);
                if (r == hipSuccess) r = hipDeviceSynchronize();
            }
        }
    }
    if (r == hipSuccess) r = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    return r;
}

// Upload from three per-matrix host tensors [E][rows][blocks] (the GGUF
// routed-expert tensors) plus the shared expert's three matrices.  Each
// matrix's planes have the same expert-major order, so a chunk of experts is
// one copy and one repack launch.
int upload_tensors(moe_ffn_layer *L, const void *const routed[3], const void *const shared[3]) {
    const Shape &s = L->shape;
    const size_t mblocks = matrix_blocks(s);   // blocks per expert matrix
    const size_t max_bytes = matrix_bytes(s, L->down_q41, 2);
    const int chunk = static_cast<int>(std::max<size_t>(1, (size_t{256} << 20) / max_bytes));
    uint8_t *staging = nullptr;
    if (hipMalloc(&staging, static_cast<size_t>(chunk) * max_bytes) != hipSuccess) return hipErrorOutOfMemory;
    int r = hipSuccess;
    for (int m = 0; m < 3 && r == hipSuccess; ++m) {
        const Plane pl = plane(L, m);
        const size_t mbytes = matrix_bytes(s, L->down_q41, m);
        for (int first = 0; first < s.Ep && r == hipSuccess; first += chunk) {
            const int n = std::min(chunk, s.Ep - first);
            const int nr = std::max(0, std::min(n, s.E - first));   // routed experts in this chunk
            if (nr > 0)
                r = hipMemcpy(staging, static_cast<const uint8_t *>(routed[m]) + static_cast<size_t>(first) * mbytes,
                              static_cast<size_t>(nr) * mbytes, hipMemcpyHostToDevice);
            if (r == hipSuccess && nr < n)   // the shared expert follows the routed ones
                r = hipMemcpy(staging + static_cast<size_t>(nr) * mbytes, shared[m], mbytes, hipMemcpyHostToDevice);
            if (r == hipSuccess)
                r = moe::launch_repack_weights(staging, pl.codes, pl.scales, pl.mins, static_cast<size_t>(n) * mblocks,
                                               static_cast<size_t>(first) * mblocks, pl.blocks_per_row, pl.group,
                                               nullptr);
            if (r == hipSuccess) r = hipDeviceSynchronize();
        }
    }
    (void)hipFree(staging);
    return r;
}

void profile_free(moe_ffn_layer *L) {
    for (int i = 0; i < L->prof_capacity * moe_ffn_layer::kStageMarks; ++i) (void)hipEventDestroy(L->prof_events[i]);
    delete[] L->prof_events;
    L->prof_events = nullptr;
    L->prof_capacity = L->prof_used = 0;
}

void mark_uploaded(moe_ffn_layer *L) {
    L->upload_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - L->create_start).count();
}

// Validates a create call before any HIP call, makes `device` current for
// the creation (restoring the caller's device afterwards), and runs
// `fill(L)` to put the weights into a new layer's planes.
template<class Fill>
int create_layer(const moe_ffn_config *config, int device, moe_ffn_layer **layer, Fill &&fill) {
    if (!config_ok(config) || !layer) return kInvalid;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return kInvalid;
    moe::DeviceScope scope(device);
    if (!scope.ok()) return kInvalid;
    moe_ffn_layer *L = nullptr;
    int r = create_common(config, device, L);
    if (r != hipSuccess) return r;
    r = fill(L);
    mark_uploaded(L);
    if (r == hipSuccess) r = finish_create(L);
    if (r != hipSuccess) { moe_ffn_destroy(L); return r; }
    *layer = L;
    return hipSuccess;
}

moe::FfnArgs base_args(moe_ffn_layer *L, int tokens, int *error) {
    moe::FfnArgs a{};
    a.shape = L->shape;
    a.bank = L->bank;
    a.xq = L->xq;
    a.mq = L->mq;
    a.routes = L->routes;
    a.out = L->contrib;
    a.out_stride_k = L->shape.k + 1;
    a.tokens = tokens;
    a.pairs_bound = static_cast<int>(pairs_capacity(L->shape, tokens));
    a.mfma_min = L->active_mfma_min;
    a.error = error;
    a.cu_count = L->cu_count;
    return a;
}

}  // namespace

extern "C" {

int moe_ffn_memory_bytes(const moe_ffn_config *config, size_t *weight_bytes, size_t *workspace_bytes) {
    if (!config_ok(config) || !weight_bytes || !workspace_bytes) return kInvalid;
    size_t off[7];
    const Shape s = shape_of(*config);
    *weight_bytes = bank_layout(s, config->down_type == MOE_DOWN_Q4_1, off);
    *workspace_bytes = ws_layout(s, config->max_tokens).total;
    return hipSuccess;
}

int moe_ffn_create(const moe_ffn_config *config, const void *experts_q4, const void *shared_q4, int device,
                   moe_ffn_layer **layer) {
    if (!experts_q4 || (config && config->has_shared && !shared_q4)) return kInvalid;
    return create_layer(config, device, layer,
                        [&](moe_ffn_layer *L) { return upload(L, experts_q4, shared_q4, false); });
}

int moe_ffn_create_from_device(const moe_ffn_config *config, const void *experts_q4_device,
                               const void *shared_q4_device, int device, moe_ffn_layer **layer) {
    if (!experts_q4_device || !aligned(experts_q4_device, 2) ||
        (config && config->has_shared && !aligned(shared_q4_device, 2)))
        return kInvalid;
    return create_layer(config, device, layer,
                        [&](moe_ffn_layer *L) { return upload(L, experts_q4_device, shared_q4_device, true); });
}

int moe_ffn_create_tensors(const moe_ffn_config *config, const void *gate_exps, const void *up_exps,
                           const void *down_exps, const void *shared_gate, const void *shared_up,
                           const void *shared_down, int device, moe_ffn_layer **layer) {
    if (!gate_exps || !up_exps || !down_exps) return kInvalid;
    if (config && config->has_shared && (!shared_gate || !shared_up || !shared_down)) return kInvalid;
    const void *const routed[3] = {gate_exps, up_exps, down_exps};
    const void *const shared[3] = {shared_gate, shared_up, shared_down};
    return create_layer(config, device, layer, [&](moe_ffn_layer *L) { return upload_tensors(L, routed, shared); });
}

int moe_ffn_create_synthetic(const moe_ffn_config *config, uint64_t seed, int device, moe_ffn_layer **layer) {
    return create_layer(config, device, layer, [&](moe_ffn_layer *L) {
        const size_t blocks = static_cast<size_t>(L->shape.Ep) * L->shape.I * (L->shape.H / 32);
        int r = hipSuccess;
        for (int m = 0; m < 3 && r == hipSuccess; ++m) {
            const Plane pl = plane(L, m);
            r = moe::launch_synthetic_weights(pl.codes, pl.scales, pl.mins, blocks, static_cast<size_t>(m) * blocks,
                                              pl.blocks_per_row, pl.group, seed, nullptr);
        }
        return r == hipSuccess ? static_cast<int>(hipDeviceSynchronize()) : r;
    });
}

int moe_ffn_destroy(moe_ffn_layer *L) {
    if (!L) return kInvalid;
    moe::DeviceScope scope(L->device);
    (void)hipDeviceSynchronize();
    profile_free(L);
    if (L->join) (void)hipEventDestroy(L->join);
    if (L->fork) (void)hipEventDestroy(L->fork);
    if (L->side) (void)hipStreamDestroy(L->side);
    if (L->bank_mem) (void)hipFree(L->bank_mem);
    if (L->ws_mem) (void)hipFree(L->ws_mem);
    delete L;
    return hipSuccess;
}

int moe_ffn_export_expert(moe_ffn_layer *L, int expert, void *host_q4) {
    if (!L || !host_q4 || expert < 0 || expert >= L->shape.Ep) return kInvalid;
    const Shape &s = L->shape;
    const size_t mblocks = matrix_blocks(s);
    const size_t ebytes = expert_bytes(s, L->down_q41);
    uint8_t *staging = nullptr;
    moe::DeviceScope scope(L->device);
    if (!scope.ok()) return kInvalid;
    if (hipMalloc(&staging, ebytes) != hipSuccess) return hipErrorOutOfMemory;
    const size_t e = static_cast<size_t>(expert);
    int r = hipSuccess;
    uint8_t *dst = staging;
    for (int m = 0; m < 3 && r == hipSuccess; ++m) {
        const Plane pl = plane(L, m);
        r = moe::launch_unpack_weights(pl.codes, pl.scales, pl.mins, dst, mblocks, e * mblocks, pl.blocks_per_row,
                                       pl.group, nullptr);
        dst += matrix_bytes(s, L->down_q41, m);
    }
    if (r == hipSuccess) r = hipMemcpy(host_q4, staging, ebytes, hipMemcpyDeviceToHost);
    (void)hipFree(staging);
    return r;
}

namespace {
// The ungrouped decode path: shapes its kernels cover, and (in auto mode)
// few enough routes per expert that re-reading an expert shared by two tokens
// costs less than grouping (tokens * k <= E / 4), or few routes in all
// (tokens * k <= 16: a single expert's first 16 tokens, whose re-reads hit L2).
bool use_decode(const moe_ffn_layer *L, int tokens) {
    const Shape &sh = L->shape;
    const int P1 = sh.k + (sh.Ep > sh.E ? 1 : 0);
    const bool fits = sh.H / 32 <= moe::kDecodeMaxBlocksH && sh.I / 32 <= moe::kDecodeMaxBlocksI &&
                      P1 <= moe::kDecodeMaxPairs;
    if (!fits || L->decode_mode == 0) return false;
    const long routes = static_cast<long>(tokens) * sh.k;
    return L->decode_mode == 1 || routes * 4 <= sh.E || routes <= 16;
}

int run_stage(moe_ffn_layer *L, int stage, const float *x, const int32_t *ids, const float *weights, int tokens,
              const float *shared_gate, float *y, int *error, hipStream_t s, bool decode) {
    const Shape &sh = L->shape;
    moe::FfnArgs a = base_args(L, tokens, error);
    hipError_t r = hipSuccess;
    if (decode) {
        const moe::DecodeArgs d{a, x, ids, weights, shared_gate, y, L->x_q8_in};
        if (stage == MOE_STAGE_GATE_UP) return moe::launch_decode_gate_up(d, s);
        if (stage == MOE_STAGE_DOWN) return moe::launch_decode_down_fold(d, s);
        return stage >= MOE_STAGE_PREPARE && stage <= MOE_STAGE_FOLD ? hipSuccess : kInvalid;
    }
    switch (stage) {
    case MOE_STAGE_PREPARE:
        if (L->x_q8_in) {   // grouping only, then the given Q8 rows into the activation planes
            if ((r = moe::launch_prepare(nullptr, ids, weights, tokens, sh, L->xq, L->routes, L->active_mfma_min, error, s)) !=
                hipSuccess)
                return r;
            return moe::launch_canonical_to_planes(L->x_q8_in, L->xq, tokens * (sh.H / 32), s);
        }
        return moe::launch_prepare(x, ids, weights, tokens, sh, L->xq, L->routes, L->active_mfma_min, error, s);
    // With mfma_min == 1 every nonempty group is an MFMA item and the
    // streaming launch would only start empty workgroups.
    case MOE_STAGE_GATE_UP:
        if (a.mfma_min != 1 && (r = moe::launch_gate_up(a, false, s)) != hipSuccess) return r;
        if (a.mfma_min > 0) r = moe::launch_gate_up(a, true, s);
        return r;
    case MOE_STAGE_DOWN:
        if (a.mfma_min != 1 && (r = moe::launch_down(a, false, s)) != hipSuccess) return r;
        if (a.mfma_min > 0) r = moe::launch_down(a, true, s);
        return r;
    case MOE_STAGE_FOLD: {
        const size_t stride = static_cast<size_t>(sh.k + 1) * sh.H;
        return moe::launch_fold(L->contrib, stride, weights, sh.k, L->routes.pos_of,
                                sh.Ep > sh.E ? L->contrib + static_cast<size_t>(sh.k) * sh.H : nullptr, stride,
                                shared_gate, tokens, sh.H, y, error, s);
    }
    default:
        return kInvalid;
    }
}
}  // namespace

namespace {
int forward_impl(moe_ffn_layer *L, const float *x, const void *x_q8, const int32_t *ids, const float *weights,
                 int tokens, const float *shared_gate, float *y, int *error, void *stream) {
    if (!L || !(x_q8 ? aligned(x_q8, 4) : aligned(x, 4)) || !aligned(ids, 4) || !aligned(weights, 4) ||
        !aligned(y, 4) || !aligned(error, 4) || tokens < 1 || tokens > L->cfg.max_tokens ||
        (shared_gate && !aligned(shared_gate, 4)))
        return kInvalid;
    L->x_q8_in = x_q8;
    const auto s = static_cast<hipStream_t>(stream);
    const bool decode = use_decode(L, tokens);
    L->active_mfma_min = static_cast<long>(tokens) * L->shape.k < L->mfma_routes ? 0 : L->mfma_min;
    hipEvent_t *marks = nullptr;
    if (L->prof_used < L->prof_capacity) marks = L->prof_events + (L->prof_used++) * moe_ffn_layer::kStageMarks;
    if (!decode && !marks && L->two_streams && L->active_mfma_min >= 2) {
        // Both item kinds can exist: streaming chain on the side stream, MFMA
        // chain here, joined before the fold (the two chains touch disjoint
        // middle and contribution rows).
        int r = run_stage(L, MOE_STAGE_PREPARE, x, ids, weights, tokens, shared_gate, y, error, s, false);
        if (r != hipSuccess) return r;
        if ((r = hipEventRecord(L->fork, s)) != hipSuccess || (r = hipStreamWaitEvent(L->side, L->fork, 0)) != hipSuccess)
            return r;
        const moe::FfnArgs a = base_args(L, tokens, error);
        if ((r = moe::launch_gate_up(a, false, L->side)) != hipSuccess || (r = moe::launch_down(a, false, L->side)) != hipSuccess ||
            (r = moe::launch_gate_up(a, true, s)) != hipSuccess || (r = moe::launch_down(a, true, s)) != hipSuccess)
            return r;
        if ((r = hipEventRecord(L->join, L->side)) != hipSuccess || (r = hipStreamWaitEvent(s, L->join, 0)) != hipSuccess)
            return r;
        if ((r = run_stage(L, MOE_STAGE_FOLD, x, ids, weights, tokens, shared_gate, y, error, s, false)) != hipSuccess)
            return r;
    } else {
        if (marks && hipEventRecord(marks[0], s) != hipSuccess) return kInvalid;
        for (int stage = MOE_STAGE_PREPARE; stage <= MOE_STAGE_FOLD; ++stage) {
            const int r = run_stage(L, stage, x, ids, weights, tokens, shared_gate, y, error, s, decode);
            if (r != hipSuccess) return r;
            if (marks && hipEventRecord(marks[stage + 1], s) != hipSuccess) return kInvalid;
        }
    }
    L->last_decode = decode;
    L->last_tokens = tokens;
    L->last_x = x;
    L->last_ids = ids;
    L->last_weights = weights;
    L->last_shared_gate = shared_gate;
    L->last_y = y;
    L->last_error = error;
    L->last_stream = s;
    return hipSuccess;
}
}  // namespace

int moe_ffn_forward(moe_ffn_layer *L, const float *x, const int32_t *ids, const float *weights, int tokens,
                    const float *shared_gate, float *y, int *error, void *stream) {
    return forward_impl(L, x, nullptr, ids, weights, tokens, shared_gate, y, error, stream);
}

int moe_ffn_forward_q8(moe_ffn_layer *L, const void *x_q8, const int32_t *ids, const float *weights, int tokens,
                       const float *shared_gate, float *y, int *error, void *stream) {
    return forward_impl(L, nullptr, x_q8, ids, weights, tokens, shared_gate, y, error, stream);
}

int moe_ffn_profile(moe_ffn_layer *L, int forwards) {
    if (!L || forwards < 0 || forwards > 65536) return kInvalid;
    profile_free(L);
    if (forwards == 0) return hipSuccess;
    const int n = forwards * moe_ffn_layer::kStageMarks;
    L->prof_events = new (std::nothrow) hipEvent_t[n]();
    if (!L->prof_events) return hipErrorOutOfMemory;
    for (int i = 0; i < n; ++i) {
        // Timing markers without the system-scope release of a default event,
        // so recording them does not add cache writebacks between stages.
        if (hipEventCreateWithFlags(&L->prof_events[i], hipEventDisableSystemFence) != hipSuccess) {
            for (int j = 0; j < i; ++j) (void)hipEventDestroy(L->prof_events[j]);
            delete[] L->prof_events;
            L->prof_events = nullptr;
            return hipErrorOutOfMemory;
        }
    }
    L->prof_capacity = forwards;
    L->prof_used = 0;
    return hipSuccess;
}

int moe_ffn_profile_read(moe_ffn_layer *L, double *stage_ms, int *forwards) {
    if (!L || !stage_ms || !forwards) return kInvalid;
    for (int st = 0; st <= MOE_STAGE_FOLD; ++st) stage_ms[st] = 0.0;
    *forwards = L->prof_used;
    if (L->prof_used == 0) return hipSuccess;
    hipEvent_t *last = L->prof_events + (L->prof_used - 1) * moe_ffn_layer::kStageMarks;
    hipError_t r = hipEventSynchronize(last[moe_ffn_layer::kStageMarks - 1]);
    for (int f = 0; f < L->prof_used && r == hipSuccess; ++f) {
        hipEvent_t *m = L->prof_events + f * moe_ffn_layer::kStageMarks;
        for (int st = 0; st <= MOE_STAGE_FOLD && r == hipSuccess; ++st) {
            float ms = 0.0f;
            r = hipEventElapsedTime(&ms, m[st], m[st + 1]);
            stage_ms[st] += ms;
        }
    }
    L->prof_used = 0;
    return r;
}

int moe_ffn_replay_stage(moe_ffn_layer *L, int stage, void *stream) {
    if (!L || L->last_tokens < 1 || stage < MOE_STAGE_PREPARE || stage > MOE_STAGE_FOLD) return kInvalid;
    return run_stage(L, stage, L->last_x, L->last_ids, L->last_weights, L->last_tokens, L->last_shared_gate,
                     L->last_y, L->last_error, static_cast<hipStream_t>(stream), L->last_decode);
}

int moe_quantize_q8_1(const float *x, void *q8, int width, int columns, int *error, void *stream) {
    if (!aligned(x, 4) || !aligned(q8, 4) || !aligned(error, 4) || width < 32 || width > 16384 || width % 32 ||
        columns < 1 || columns > 65536)
        return kInvalid;
    return moe::launch_quantize_canonical(x, q8, width, columns, error, static_cast<hipStream_t>(stream));
}

int moe_ffn_group_routes(moe_ffn_layer *L, const int32_t *ids, const float *weights, int tokens, int32_t *counts,
                         int32_t *offsets, int32_t *route_token, int32_t *route_rank, int *error, void *stream) {
    if (!L || !aligned(ids, 4) || !aligned(weights, 4) || !aligned(counts, 4) || !aligned(offsets, 4) ||
        !aligned(route_token, 4) || !aligned(route_rank, 4) || !aligned(error, 4) || tokens < 1 ||
        tokens > L->cfg.max_tokens)
        return kInvalid;
    const auto s = static_cast<hipStream_t>(stream);
    const Shape &sh = L->shape;
    hipError_t r = moe::launch_prepare(nullptr, ids, weights, tokens, sh, L->xq, L->routes, 0, error, s);
    if (r != hipSuccess) return r;
    const size_t P = static_cast<size_t>(tokens) * sh.k;
    if ((r = hipMemcpyAsync(counts, L->routes.counts, sh.E * 4, hipMemcpyDeviceToDevice, s)) != hipSuccess) return r;
    if ((r = hipMemcpyAsync(offsets, L->routes.offsets, (sh.E + 1) * 4, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return r;
    if ((r = hipMemcpyAsync(route_token, L->routes.pair_token, P * 4, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return r;
    return hipMemcpyAsync(route_rank, L->routes.pair_rank, P * 4, hipMemcpyDeviceToDevice, s);
}

int moe_ffn_expert_gate_up(moe_ffn_layer *L, int expert, const void *x_q8, int columns, float *middle,
                           void *middle_q8, int32_t *gate_dots, int32_t *up_dots, int path, int *error,
                           void *stream) {
    if (!L || expert < 0 || expert >= L->shape.Ep || !aligned(x_q8, 4) || !aligned(middle_q8, 4) ||
        !aligned(error, 4) || columns < 1 || columns > L->cfg.max_tokens || (middle && !aligned(middle, 4)) ||
        (gate_dots && !aligned(gate_dots, 4)) || (up_dots && !aligned(up_dots, 4)) || path < 0 || path > 2)
        return kInvalid;
    const bool mfma = path != MOE_PATH_STREAM;
    const auto s = static_cast<hipStream_t>(stream);
    const Shape &sh = L->shape;
    hipError_t r = moe::launch_canonical_to_planes(x_q8, L->xq, columns * (sh.H / 32), s);
    if (r != hipSuccess) return r;
    if ((r = moe::launch_single_expert_items(sh, L->routes, expert, columns, mfma, s)) != hipSuccess) return r;
    moe::FfnArgs a = base_args(L, columns, error);
    a.pairs_bound = columns;
    a.mfma_min = mfma ? 1 : 0;   // the single group is an MFMA item or streaming items
    a.middle_f32 = middle;
    a.gate_dots = gate_dots;
    a.up_dots = up_dots;
    if ((r = moe::launch_gate_up(a, mfma, s)) != hipSuccess) return r;
    return moe::launch_planes_to_canonical(L->mq, middle_q8, columns * (sh.I / 32), s);
}

int moe_ffn_expert_down(moe_ffn_layer *L, int expert, const void *middle_q8, int columns, float *y,
                        int32_t *down_dots, int path, int *error, void *stream) {
    if (!L || expert < 0 || expert >= L->shape.Ep || !aligned(middle_q8, 4) || !aligned(y, 4) ||
        !aligned(error, 4) || columns < 1 || columns > L->cfg.max_tokens || (down_dots && !aligned(down_dots, 4)) ||
        path < 0 || path > 2)
        return kInvalid;
    const bool mfma = path != MOE_PATH_STREAM;
    if (mfma && !aligned(y, 16)) return kInvalid;   // the MFMA down kernel stores float4 rows
    const auto s = static_cast<hipStream_t>(stream);
    const Shape &sh = L->shape;
    hipError_t r = moe::launch_canonical_to_planes(middle_q8, L->mq, columns * (sh.I / 32), s);
    if (r != hipSuccess) return r;
    if ((r = moe::launch_single_expert_items(sh, L->routes, expert, columns, mfma, s)) != hipSuccess) return r;
    moe::FfnArgs a = base_args(L, columns, error);
    a.pairs_bound = columns;
    a.mfma_min = mfma ? 1 : 0;   // the single group is an MFMA item or streaming items
    a.out = y;
    a.out_stride_k = 1;
    a.down_dots = down_dots;
    return moe::launch_down(a, mfma, s);
}

int moe_ffn_expert_run(moe_ffn_layer *L, int expert, const float *x, int columns, float *y, int repeats, int path,
                       int *flags, moe_expert_timing *timing, void *stream) {
    if (!L || expert < 0 || expert >= L->shape.Ep || !x || !y || !flags || !timing || columns < 1 ||
        columns > L->cfg.max_tokens || repeats < 1 || repeats > 10000 || path < 0 || path > 2)
        return kInvalid;
    using Clock = std::chrono::steady_clock;
    const Shape &sh = L->shape;
    bool mfma = path == MOE_PATH_MFMA;
    if (path == MOE_PATH_AUTO) {   // forward()'s rule for one group of `columns` pairs
        const int active = columns < L->mfma_routes ? 0 : L->mfma_min;
        mfma = active > 0 && columns >= active;
    }
    // x and y live in the contribution buffer (>= 2 * max_tokens rows of H
    // floats); y starts a whole number of 128-byte rows in, as the MFMA down
    // kernel's float4 stores need.
    const size_t elems = static_cast<size_t>(columns) * sh.H;
    float *xd = L->contrib, *yd = L->contrib + elems;
    int *err = L->diag_error;
    const auto s = static_cast<hipStream_t>(stream);
    moe::DeviceScope scope(L->device);
    if (!scope.ok()) return kInvalid;
    // One forward: quantize x, gate/up + SiLU*up + Q8, down (the work list
    // of the single group is built once, before the warm-up).
    auto pass = [&]() -> hipError_t {
        hipError_t r = moe::launch_quantize_planes(xd, L->xq, sh.H, columns, err, s);
        moe::FfnArgs a = base_args(L, columns, err);
        a.pairs_bound = columns;
        a.mfma_min = mfma ? 1 : 0;
        a.out = yd;
        a.out_stride_k = 1;
        if (r == hipSuccess) r = moe::launch_gate_up(a, mfma, s);
        if (r == hipSuccess) r = moe::launch_down(a, mfma, s);
        return r;
    };
    auto read_flags = [&](int *value) -> hipError_t {
        hipError_t r = hipMemcpyAsync(value, err, sizeof(int), hipMemcpyDeviceToHost, s);
        return r == hipSuccess ? hipStreamSynchronize(s) : r;
    };
    hipError_t r = moe::launch_fill_u32(reinterpret_cast<uint32_t *>(err), 0u, 1, s);
    if (r == hipSuccess) r = moe::launch_single_expert_items(sh, L->routes, expert, columns, mfma, s);
    if (r == hipSuccess) r = hipMemcpyAsync(xd, x, elems * sizeof(float), hipMemcpyHostToDevice, s);
    if (r == hipSuccess) r = pass();   // warm-up outside the timing
    int value = 0;
    if (r == hipSuccess) r = read_flags(&value);
    if (r != hipSuccess) return r;
    *flags = value;
    if (value) return hipSuccess;
    hipEvent_t begin = nullptr, end = nullptr;
    if (hipEventCreate(&begin) != hipSuccess) return hipErrorOutOfMemory;
    if (hipEventCreate(&end) != hipSuccess) { (void)hipEventDestroy(begin); return hipErrorOutOfMemory; }
    const auto start = Clock::now();
    r = hipEventRecord(begin, s);
    for (int i = 0; i < repeats && r == hipSuccess; ++i) r = pass();
    if (r == hipSuccess) r = hipEventRecord(end, s);
    float ms = 0.0f;
    if (r == hipSuccess) r = hipEventSynchronize(end);
    if (r == hipSuccess) r = hipEventElapsedTime(&ms, begin, end);
    if (r == hipSuccess) r = hipMemcpyAsync(&value, err, sizeof(int), hipMemcpyDeviceToHost, s);
    if (r == hipSuccess) r = hipMemcpyAsync(y, yd, elems * sizeof(float), hipMemcpyDeviceToHost, s);
    if (r == hipSuccess) r = hipStreamSynchronize(s);
    const double wall = std::chrono::duration<double, std::milli>(Clock::now() - start).count();
    (void)hipEventDestroy(begin);
    (void)hipEventDestroy(end);
    if (r != hipSuccess) return r;
    *flags = value;
    *timing = moe_expert_timing{L->upload_ms, static_cast<double>(ms) / repeats, wall / repeats};
    return hipSuccess;
}

int moe_combine(const float *contributions, const float *weights, const float *shared, const float *shared_gate,
                int tokens, int top_k, int hidden, float *y, int *error, void *stream) {
    if (!aligned(contributions, 4) || !aligned(weights, 4) || !aligned(y, 4) || !aligned(error, 4) || tokens < 1 ||
        top_k < 1 || top_k > 32 || hidden < 1 || (shared && !aligned(shared, 4)) ||
        (shared_gate && !aligned(shared_gate, 4)))
        return kInvalid;
    return moe::launch_fold(contributions, static_cast<size_t>(top_k) * hidden, weights, top_k, nullptr, shared,
                            static_cast<size_t>(hidden), shared ? shared_gate : nullptr, tokens, hidden, y, error,
                            static_cast<hipStream_t>(stream));
}

int moe_ffn_debug_last(moe_ffn_layer *L, void *x_q8, void *middle_q8, int32_t *route_token, int32_t *route_rank,
                       void *stream) {
    if (!L || L->last_tokens < 1) return kInvalid;
    const auto s = static_cast<hipStream_t>(stream);
    const Shape &sh = L->shape;
    const int N = L->last_tokens;
    hipError_t r = hipSuccess;
    if (x_q8 && (r = moe::launch_planes_to_canonical(L->xq, x_q8, N * (sh.H / 32), s)) != hipSuccess) return r;
    const int P = static_cast<int>(pairs_capacity(sh, N));
    if (L->last_decode) {
        // The decode path does not group: group the same routes now (the last
        // inputs must still be valid) and reorder its middle rows to match.
        if ((r = moe::launch_prepare(nullptr, L->last_ids, L->last_weights, N, sh, L->xq, L->routes, L->active_mfma_min,
                                     L->diag_error, s)) != hipSuccess)
            return r;
        if (middle_q8 && (r = moe::launch_decode_middle_grouped(L->mq, L->routes, sh, N, middle_q8, s)) != hipSuccess)
            return r;
    } else if (middle_q8 && (r = moe::launch_planes_to_canonical(L->mq, middle_q8, P * (sh.I / 32), s)) != hipSuccess)
        return r;
    const size_t routed = static_cast<size_t>(N) * sh.k * 4;
    if (route_token &&
        (r = hipMemcpyAsync(route_token, L->routes.pair_token, routed, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return r;
    if (route_rank &&
        (r = hipMemcpyAsync(route_rank, L->routes.pair_rank, routed, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return r;
    return hipSuccess;
}

int moe_ffn_last_stats(moe_ffn_layer *L, int32_t *stream_items, int32_t *mfma_items, int32_t *active_experts) {
    if (!L) return kInvalid;
    int32_t c[4] = {0, 0, 0, 0};
    moe::DeviceScope scope(L->device);
    if (!scope.ok()) return kInvalid;
    // Synchronous diagnostic: wait for the last forward's stream (its
    // streaming chain on the side stream joins that stream before the fold),
    // so the counts are that forward's; other streams keep running.
    const hipStream_t s = L->last_stream;
    if (hipStreamSynchronize(s) != hipSuccess) return kInvalid;
    if (L->last_decode && L->last_tokens > 0) {   // group the last batch's routes (not done by the decode path)
        const hipError_t g = moe::launch_prepare(nullptr, L->last_ids, L->last_weights, L->last_tokens, L->shape,
                                                 L->xq, L->routes, L->active_mfma_min, L->diag_error, s);
        if (g != hipSuccess) return g;
    }
    hipError_t r = hipMemcpyAsync(c, L->routes.item_counts, sizeof(c), hipMemcpyDeviceToHost, s);
    if (r == hipSuccess) r = hipStreamSynchronize(s);
    if (r != hipSuccess) return r;
    if (stream_items) *stream_items = c[0];
    if (mfma_items) *mfma_items = c[1];
    if (active_experts) *active_experts = c[2];
    return hipSuccess;
}

int moe_expf_device(const float *x, float *y, int n, void *stream) {
    if (!aligned(x, 4) || !aligned(y, 4) || n < 1) return kInvalid;
    return moe::launch_expf(x, y, n, static_cast<hipStream_t>(stream));
}

int moe_router_select(const float *logits, int tokens, int experts, int top_k, float *probabilities,
                      int32_t *ids, float *weights, int *error, void *stream) {
    if (!aligned(logits, 4) || !aligned(ids, 4) || !aligned(weights, 4) || !aligned(error, 4) ||
        (probabilities && !aligned(probabilities, 4)) || tokens < 1 || experts < 32 || experts > 1024 ||
        experts % 32 != 0 || top_k < 1 || top_k > 32 || top_k > experts)
        return kInvalid;
    return moe::launch_router(logits, tokens, experts, top_k, probabilities, ids, weights, error,
                              static_cast<hipStream_t>(stream));
}

int moe_read_probe(const void *buffer, size_t bytes, void *sink, void *stream) {
    if (!aligned(buffer, 16) || !aligned(sink, 4) || bytes < 16 || bytes % 16 != 0) return kInvalid;
    return moe::launch_read_probe(buffer, bytes, static_cast<uint32_t *>(sink), static_cast<hipStream_t>(stream));
}

int moe_expf_host(const float *x, float *y, size_t n) {
    if (!x || !y) return kInvalid;
    for (size_t i = 0; i < n; ++i) y[i] = moe_expf(x[i]);
    return hipSuccess;
}

}  // extern "C"
