// Routed-MoE Q4_0 x Q8_1 expert FFN kernels for MI355X (gfx950, CDNA4, wave64).
//
// Arithmetic contract (reference 0FL01/gfx906-qwen3.8fn):
//   Q8_1 quantization  src/quant.cpp:275-325, GPU form src/hip/linear.hip:99-150
//   Q4_0 block dot     src/quant.cpp:48-55   (unsigned nibbles x signed codes)
//   block scaling      src/quant.cpp:88-93   d4 * (I*d8 - 8*s8)
//   SiLU(gate)*up      src/hip/linear.hip:106-120 (sanitised; expf with the host libm bits, moe_expf.h)
//   rank-order fold    src/hip/session_ops.hip:307-324, shared add :375-391
// The per-block int32 dots and the Q8 codes are bit-exact with the reference;
// the fp32 accumulation order across blocks is this implementation's own.
#include "moe_device.hpp"

#include <algorithm>
#include <climits>

#pragma clang fp contract(off)

namespace moe {
namespace {

// ------------------------------------------------------------ quantizers ---
// One thread per element; 32-lane groups are whole Q8 blocks.
template<bool Canonical>
__global__ __launch_bounds__(256) void k_quantize(const float *__restrict__ x, uint8_t *codes,
                                                  uint32_t *heads, size_t elements, int *error) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= elements) return;   // elements is a multiple of 32: whole groups exit together
    const Q8Lane q = quantize32(x[i]);
    const size_t block = i >> 5;
    const int lane = static_cast<int>(i & 31);
    if constexpr (Canonical) {
        codes[block * 36 + 4 + lane] = static_cast<uint8_t>(q.code);
        if (lane == 0) *reinterpret_cast<uint32_t *>(codes + block * 36) = q.head;
    } else {
        codes[block * 32 + lane] = static_cast<uint8_t>(q.code);
        if (lane == 0) heads[block] = q.head;
    }
    if (lane == 0 && q.flags) atomicOr(error, q.flags);
}

__global__ __launch_bounds__(256) void k_canonical_to_planes(const uint8_t *q8, uint8_t *codes,
                                                             uint32_t *heads, size_t blocks) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= blocks * 9) return;
    const size_t b = i / 9, w = i % 9;
    const uint32_t v = reinterpret_cast<const uint32_t *>(q8)[i];
    if (w == 0) heads[b] = v;
    else reinterpret_cast<uint32_t *>(codes)[b * 8 + (w - 1)] = v;
}

__global__ __launch_bounds__(256) void k_planes_to_canonical(const uint8_t *codes, const uint32_t *heads,
                                                             uint8_t *q8, size_t blocks) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= blocks * 9) return;
    const size_t b = i / 9, w = i % 9;
    const uint32_t v = w == 0 ? heads[b] : reinterpret_cast<const uint32_t *>(codes)[b * 8 + (w - 1)];
    reinterpret_cast<uint32_t *>(q8)[i] = v;
}

// ---------------------------------------------------------- weight planes ---
// Canonical blocks are 18 bytes with 2-byte alignment: read them as 9 u16.
// Canonical blocks -> planes.  mins == nullptr: 18-byte Q4_0 blocks {d, qs};
// else 20-byte Q4_1 blocks {d, m, qs}, m going to its own plane (same order
// as the scales).
__global__ __launch_bounds__(256) void k_repack(const uint16_t *canonical, uint32_t *codes,
                                                uint16_t *scales, uint16_t *mins, size_t blocks, size_t block0,
                                                int nb, int group) {
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const size_t g = block0 + b;
    const uint16_t *src = canonical + b * (mins ? 10 : 9);
    const size_t si = scale_index(g / nb, static_cast<int>(g % nb), nb, group);
    scales[si] = src[0];
    if (mins) {
        mins[si] = src[1];
        ++src;
    }
    uint4 c;
    c.x = src[1] | (static_cast<uint32_t>(src[2]) << 16);
    c.y = src[3] | (static_cast<uint32_t>(src[4]) << 16);
    c.z = src[5] | (static_cast<uint32_t>(src[6]) << 16);
    c.w = src[7] | (static_cast<uint32_t>(src[8]) << 16);
    reinterpret_cast<uint4 *>(codes)[g] = c;
}

__global__ __launch_bounds__(256) void k_unpack(const uint32_t *codes, const uint16_t *scales,
                                                const uint16_t *mins, uint16_t *canonical, size_t blocks,
                                                size_t block0, int nb, int group) {
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const size_t g = block0 + b;
    const uint4 c = reinterpret_cast<const uint4 *>(codes)[g];
    uint16_t *dst = canonical + b * (mins ? 10 : 9);
    const size_t si = scale_index(g / nb, static_cast<int>(g % nb), nb, group);
    dst[0] = scales[si];
    if (mins) {
        dst[1] = mins[si];
        ++dst;
    }
    dst[1] = c.x & 0xffffu; dst[2] = c.x >> 16;
    dst[3] = c.y & 0xffffu; dst[4] = c.y >> 16;
    dst[5] = c.z & 0xffffu; dst[6] = c.z >> 16;
    dst[7] = c.w & 0xffffu; dst[8] = c.w >> 16;
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Synthetic Q4_0 blocks: codes uniform 0..15 (16 random bytes), d =
// half(|N(0, 0.02)|) by Box-Muller, all from a counter hash of (seed, block).
// With a mins plane (Q4_1): m = half(-8 d (0.75 + 0.5 u)), values centred as
// in Q4_0.
__global__ __launch_bounds__(256) void k_synthetic(uint32_t *codes, uint16_t *scales, uint16_t *mins, size_t blocks,
                                                   size_t hash0, int nb, int group, uint64_t seed) {
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const uint64_t g = hash0 + b;
    const uint64_t h0 = mix64(seed ^ mix64(4 * g + 0)), h1 = mix64(seed ^ mix64(4 * g + 1));
    const uint64_t h2 = mix64(seed ^ mix64(4 * g + 2));
    uint4 c;
    c.x = static_cast<uint32_t>(h0); c.y = static_cast<uint32_t>(h0 >> 32);
    c.z = static_cast<uint32_t>(h1); c.w = static_cast<uint32_t>(h1 >> 32);
    reinterpret_cast<uint4 *>(codes)[b] = c;
    const float u1 = (static_cast<float>(h2 >> 40) + 1.0f) * 0x1p-24f;          // (0, 1]
    const float u2 = static_cast<float>((h2 >> 16) & 0xffffffu) * 0x1p-24f;      // [0, 1)
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    const float d = h2f(f2h(fabsf(z) * 0.02f));
    const size_t si = scale_index(b / nb, static_cast<int>(b % nb), nb, group);
    scales[si] = static_cast<uint16_t>(f2h(d));
    if (mins) {
        const float u3 = static_cast<float>(h2 & 0xffffu) * 0x1p-16f;             // [0, 1)
        mins[si] = static_cast<uint16_t>(f2h(-8.0f * d * (0.75f + 0.5f * u3)));
    }
}

// Plain streaming read of n 16-byte words, one contiguous chunk per
// workgroup, eight loads in flight per thread; the XOR of the words is kept
// only so that the loads cannot be dropped (written when it equals `never`).
// It measures how fast this device streams a buffer of a given size from HBM,
// the practical ceiling the decode kernels are compared with.
__global__ __launch_bounds__(512) void k_read_probe(const uint4 *__restrict__ p, size_t n, size_t chunk,
                                                    uint32_t never, uint32_t *sink) {
    const size_t b = static_cast<size_t>(blockIdx.x) * chunk;
    const size_t e = b + chunk < n ? b + chunk : n;
    uint32_t acc = 0;
    for (size_t i = b + threadIdx.x; i < e; i += static_cast<size_t>(blockDim.x) * 8) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t j = i + static_cast<size_t>(u) * blockDim.x;
            v[u] = j < e ? p[j] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == never) sink[0] = acc;
}

// The kernels' expf as the epilogues use it (table in lane registers, every
// lane taking part even past n), so special-case inputs mixed into one wave
// are covered.
__global__ __launch_bounds__(256) void k_expf(const float *x, float *y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const LaneExpfTable table{expf_table_word(threadIdx.x & 63)};
    const float v = moe_expf_with(i < n ? x[i] : 0.0f, table);
    if (i < n) y[i] = v;
}

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t *p, uint32_t v, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ------------------------------------------------------------- grouping ----
// Grouping replaces RouteGroups::prepare (src/routes.cpp:59-115): groups
// ascend by expert, within a group by token then rank.  Each expert keeps a
// token bitmap; a pair's position is offset[e] + (popcount of the expert's
// bits for earlier tokens), which is the stable counting-sort position,
// computed without any ordering between threads.  The shared expert is group
// E, holding every token once (rank = k).

// Block-wide exclusive scan of n ints (any n) by a 1024-thread block.
__device__ int block_exclusive_scan(const int32_t *in, int32_t *out, int n, int32_t *tmp) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int per = (n + blockDim.x - 1) / blockDim.x;
    const int lo = min(n, tid * per), hi = min(n, lo + per);
    int local = 0;
    for (int i = lo; i < hi; ++i) local += in[i];
    int incl = local;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
    }
    if (lane == 63) tmp[wave] = incl;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int w = 0; w < nw; ++w) { const int v = tmp[w]; tmp[w] = run; run += v; }
        tmp[nw] = run;
    }
    __syncthreads();
    int run = tmp[wave] + incl - local;
    for (int i = lo; i < hi; ++i) { const int v = in[i]; out[i] = run; run += v; }
    const int total = tmp[nw];
    __syncthreads();
    return total;
}

struct GroupParams {
    const int32_t *ids;
    const float *weights;
    int tokens;
    Shape shape;
    RouteOut r;
    int mfma_min;
    int *error;
};

// Items from group counts/offsets: groups below mfma_min (or all groups when
// mfma_min == 0) become streaming items of <= kStreamTokens pairs, larger
// groups become MFMA items of <= kMfmaTile pairs.  cnt/off may live in LDS.
// With fill, the grouped pair arrays are already written (by this block) and
// streaming items get their tokens and ranks inline.
__device__ void build_items(const GroupParams &p, const int32_t *cnt, const int32_t *off, int32_t *ns,
                            int32_t *nm, int32_t *tmp, bool fill) {
    const int Ep = p.shape.Ep;
    for (int e = threadIdx.x; e < Ep; e += blockDim.x) {
        const int n = cnt[e];
        const bool big = p.mfma_min > 0 && n >= p.mfma_min;
        ns[e] = (n > 0 && !big) ? (n + kStreamTokens - 1) / kStreamTokens : 0;
        nm[e] = big ? (n + kMfmaTile - 1) / kMfmaTile : 0;
    }
    __syncthreads();
    const int total_s = block_exclusive_scan(ns, ns, Ep, tmp);
    const int total_m = block_exclusive_scan(nm, nm, Ep, tmp);
    // One thread per item.  Item i of a path belongs to the last group e with
    // first_item[e] <= i (groups without items of that path share the next
    // group's first index, so the last such e is the owner).
    for (int i = threadIdx.x; i < total_s + total_m; i += blockDim.x) {
        const bool big = i >= total_s;
        const int li = big ? i - total_s : i;
        const int32_t *first = big ? nm : ns;
        int lo = 0, hi = Ep;   // first e with first[e] > li
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (first[mid] <= li) lo = mid + 1; else hi = mid;
        }
        const int e = lo - 1;
        const int size = big ? kMfmaTile : kStreamTokens;
        const int f = (li - first[e]) * size;
        Item it;
        it.expert = e; it.first = off[e] + f; it.ncols = min(size, cnt[e] - f); it.pad = 0;
        for (int j = 0; j < kStreamTokens; ++j) {
            const bool in = fill && !big && j < it.ncols;
            it.token[j] = in ? p.r.pair_token[it.first + j] : 0;
            it.rank[j] = in ? p.r.pair_rank[it.first + j] : 0;
        }
        (big ? p.r.mfma_items : p.r.stream_items)[li] = it;
    }
    // Active groups: counted with one LDS atomic per nonempty group.
    if (threadIdx.x == 0) tmp[0] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < Ep; e += blockDim.x)
        if (cnt[e] > 0) atomicAdd(&tmp[0], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        p.r.item_counts[0] = total_s;
        p.r.item_counts[1] = total_m;
        p.r.item_counts[2] = tmp[0];
        p.r.item_counts[3] = off[Ep];   // grouped pairs incl. shared
    }
}

// Small path: block 0 groups (bitmaps in LDS), blocks 1.. quantize x.
__global__ __launch_bounds__(1024) void k_prepare_small(GroupParams p, const float *__restrict__ x,
                                                        Act xq, size_t q_elements) {
    extern __shared__ uint32_t lds[];
    if (blockIdx.x > 0) {
        const size_t i = static_cast<size_t>(blockIdx.x - 1) * blockDim.x + threadIdx.x;
        if (i >= q_elements) return;
        const Q8Lane q = quantize32(x[i]);
        const size_t block = i >> 5;
        const int lane = static_cast<int>(i & 31);
        xq.codes[block * 32 + lane] = static_cast<uint8_t>(q.code);
        if (lane == 0) {
            xq.heads[block] = q.head;
            if (q.flags) atomicOr(p.error, q.flags);
        }
        return;
    }
    const int N = p.tokens, k = p.shape.k, E = p.shape.E, Ep = p.shape.Ep;
    const int W = (N + 31) / 32;
    uint32_t *bits = lds;                                               // [E][W]
    uint32_t *wpre = bits + E * W;                                      // [E][W]
    int32_t *cnt = reinterpret_cast<int32_t *>(wpre + E * W);           // [Ep]
    int32_t *off = cnt + Ep;                                            // [Ep+1]
    int32_t *ns = off + Ep + 1;                                         // [Ep]
    int32_t *nm = ns + Ep;                                              // [Ep]
    int32_t *tmp = nm + Ep;                                             // [17]
    int32_t *eid = tmp + 17;                                            // [N*k] expert or -1
    for (int i = threadIdx.x; i < E * W; i += blockDim.x) bits[i] = 0;
    for (int i = threadIdx.x; i < N * k; i += blockDim.x) eid[i] = p.ids[i];
    __syncthreads();
    // Validate (src/routes.cpp:76-90) from LDS.  Thread tid owns entries
    // tid + m*blockDim (m < 32, N*k <= 32*blockDim); bit m of `valid` records
    // entry m's validity for the scatter below.
    int flags = 0;
    uint32_t valid = 0;
    for (int i = threadIdx.x, m = 0; i < N * k; i += blockDim.x, ++m) {
        const int t = i / k, r = i % k, e = eid[i];
        const float w = p.weights[i];
        if (!isfinite(w) || w < 0.0f) flags |= 1;
        bool ok = e >= 0 && e < E;
        for (int q = 0; ok && q < r; ++q) ok = eid[t * k + q] != e;
        if (!ok) { flags |= 1; continue; }
        valid |= 1u << m;
        atomicOr(&bits[e * W + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    for (int e = threadIdx.x; e < Ep; e += blockDim.x) {
        if (e >= E) { cnt[e] = N; continue; }   // shared expert: every token
        int run = 0;
        for (int w = 0; w < W; ++w) { wpre[e * W + w] = run; run += __popc(bits[e * W + w]); }
        cnt[e] = run;
    }
    __syncthreads();
    const int total = block_exclusive_scan(cnt, off, Ep, tmp);
    if (threadIdx.x == 0) off[Ep] = total;
    __syncthreads();
    for (int i = threadIdx.x, m = 0; i < N * k; i += blockDim.x, ++m) {
        const int t = i / k, r = i % k, e = eid[i];
        int pos = -1;
        if (valid & (1u << m)) {
            const uint32_t word = bits[e * W + (t >> 5)];
            pos = off[e] + static_cast<int>(wpre[e * W + (t >> 5)]) + __popc(word & ((1u << (t & 31)) - 1u));
            p.r.pair_token[pos] = t;
            p.r.pair_rank[pos] = r;
        }
        p.r.pos_of[i] = pos;
    }
    if (Ep > E)
        for (int t = threadIdx.x; t < N; t += blockDim.x) { p.r.pair_token[off[E] + t] = t; p.r.pair_rank[off[E] + t] = k; }
    for (int e = threadIdx.x; e < Ep; e += blockDim.x) { p.r.counts[e] = cnt[e]; p.r.offsets[e] = off[e]; }
    if (threadIdx.x == 0) p.r.offsets[Ep] = off[Ep];
    __syncthreads();   // pair arrays complete before build_items copies them into items
    build_items(p, cnt, off, ns, nm, tmp, true);
    if (flags) atomicOr(p.error, flags);
}

// Large path.  Mark and scatter blocks take 256 tokens each and stage their
// ids in LDS ([256][k] ints, dynamic), so the duplicate checks of
// src/routes.cpp:76-90 read LDS rather than chains of global loads.
// Validates entry (t, r) (src/routes.cpp:76-90) and returns its expert, or
// -1 when it cannot be grouped (bad id, duplicate of an earlier rank); bad
// ids, duplicates and negative or nonfinite weights set flag bit 1.
__device__ __forceinline__ int staged_entry(const int32_t *sid, int tl, int r, int k, int E, int &flags) {
    const int e = sid[tl * k + r];
    if (e < 0 || e >= E) { flags |= 1; return -1; }
    for (int q = 0; q < r; ++q)
        if (sid[tl * k + q] == e) { flags |= 1; return -1; }
    return e;
}

// The ids of tokens t0 .. t0 + 255 into LDS: up to 16 rounds with every
// load issued before the first LDS write (a strided loop would wait for each
// load in turn), a plain loop for the rest (k > 16).
__device__ void stage_ids(const GroupParams &p, int t0, int32_t *sid) {
    const int k = p.shape.k;
    const int n = min(256, p.tokens - t0) * k;
    const int32_t *src = p.ids + static_cast<size_t>(t0) * k;
    constexpr int kRounds = 16;
    const int step = static_cast<int>(blockDim.x);
    int v[kRounds];
#pragma unroll
    for (int u = 0; u < kRounds; ++u) {
        const int i = static_cast<int>(threadIdx.x) + u * step;
        if (i < n) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < kRounds; ++u) {
        const int i = static_cast<int>(threadIdx.x) + u * step;
        if (i < n) sid[i] = v[u];
    }
    for (int i = static_cast<int>(threadIdx.x) + kRounds * step; i < n; i += step) sid[i] = src[i];
    __syncthreads();
}

// Bit 1 for a negative or nonfinite routing weight of tokens t0 .. t0 + 255,
// each weight read once, coalesced, with the loads issued together.
__device__ int weight_flags(const GroupParams &p, int t0) {
    const int k = p.shape.k;
    const int n = min(256, p.tokens - t0) * k;
    const float *src = p.weights + static_cast<size_t>(t0) * k;
    constexpr int kRounds = 16;
    const int step = static_cast<int>(blockDim.x);
    int flags = 0;
    for (int i0 = 0; i0 < n; i0 += kRounds * step) {
        float v[kRounds];
#pragma unroll
        for (int u = 0; u < kRounds; ++u) {
            const int i = i0 + static_cast<int>(threadIdx.x) + u * step;
            v[u] = i < n ? src[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kRounds; ++u)
            if (!isfinite(v[u]) || v[u] < 0.0f) flags |= 1;
    }
    return flags;
}

constexpr int kQuantPer = 8;   // quantized elements per thread in k_mark_quantize

// Step 1: blocks [0, mark_blocks) set bitmap bits (one thread per token),
// the rest quantize x.  The bitmap is [W][Ep] (word-major) so the
// per-expert prefix kernel reads it coalesced.
__global__ __launch_bounds__(256) void k_mark_quantize(GroupParams p, int mark_blocks,
                                                       const float *__restrict__ x, Act xq,
                                                       size_t q_elements) {
    extern __shared__ uint32_t lds[];
    if (static_cast<int>(blockIdx.x) < mark_blocks) {
        int32_t *sid = reinterpret_cast<int32_t *>(lds);
        const int t0 = blockIdx.x * 256;
        stage_ids(p, t0, sid);
        int flags = weight_flags(p, t0);
        const int t = t0 + threadIdx.x;
        if (t < p.tokens)
            for (int r = 0; r < p.shape.k; ++r) {
                const int e = staged_entry(sid, threadIdx.x, r, p.shape.k, p.shape.E, flags);
                if (e >= 0) atomicOr(&p.r.bitmap[static_cast<size_t>(t >> 5) * p.shape.Ep + e], 1u << (t & 31));
            }
        if (flags) atomicOr(p.error, flags);
        return;
    }
    // A workgroup quantizes 64 blocks (2048 consecutive floats): wave w takes
    // blocks 16w .. 16w + 15, lane l elements 8 (l / 16) .. + 7 of block
    // 16w + l % 16 (two 16-byte loads, one 8-byte code store), reduced by
    // quantize_part<4> (aligned subtrees of the reference's butterfly, the same
    // bytes as quantize32).  q_elements is a multiple of 32, so the bound check
    // keeps or drops whole blocks; every lane takes part in the shuffles.
    static_assert(kQuantPer == 8, "k_mark_quantize: 8 elements per lane");
    const int lane = static_cast<int>(threadIdx.x & 63), wave = static_cast<int>(threadIdx.x >> 6);
    const int part = lane >> 4;
    const size_t blk0 = static_cast<size_t>(blockIdx.x - mark_blocks) * 64;
    const size_t block = blk0 + 16 * wave + (lane & 15);
    const bool in = block * 32 < q_elements;
    // The workgroup's 8 KB through one buffer descriptor (x needs only
    // 4-byte alignment; past q_elements the loads read zeros).
    const size_t left = q_elements - blk0 * 32;
    const auto xr = buffer_rsrc(x + blk0 * 32, static_cast<uint32_t>(std::min<size_t>(left, 2048) * 4));
    const uint32_t off = static_cast<uint32_t>((16 * wave + (lane & 15)) * 128 + 32 * part);
    const uint4 a = buffer_load16(xr, off, 0), b = buffer_load16(xr, off, 16);
    float v[kQuantPer] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w),
                          __uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w)};
    const Q8Part<4> q = quantize_part<4>(v);
    if (in) {
        *reinterpret_cast<uint2 *>(xq.codes + block * 32 + 8 * part) = make_uint2(q.codes[0], q.codes[1]);
        if (part == 0) {
            xq.heads[block] = q.head;
            if (q.flags) atomicOr(p.error, q.flags);
        }
    }
}

// Step 2: one wave per routed expert: exclusive popcount prefix over words.
__global__ __launch_bounds__(256) void k_word_prefix(GroupParams p) {
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (e >= p.shape.E) return;
    const int W = (p.tokens + 31) / 32, Ep = p.shape.Ep;
    int carry = 0;
    for (int w0 = 0; w0 < W; w0 += 64) {
        const int w = w0 + lane;
        const int c = w < W ? __popc(p.r.bitmap[static_cast<size_t>(w) * Ep + e]) : 0;
        int incl = c;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int v = __shfl_up(incl, d, 64);
            if (lane >= d) incl += v;
        }
        if (w < W) p.r.wprefix[static_cast<size_t>(w) * Ep + e] = static_cast<uint32_t>(carry + incl - c);
        carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) p.r.counts[e] = carry;
}

// Step 3 (single block): offsets, shared group, items.
__global__ __launch_bounds__(1024) void k_offsets_items(GroupParams p) {
    extern __shared__ uint32_t lds[];
    const int Ep = p.shape.Ep;
    int32_t *cnt = reinterpret_cast<int32_t *>(lds);
    int32_t *off = cnt + Ep;
    int32_t *ns = off + Ep + 1;
    int32_t *nm = ns + Ep;
    int32_t *tmp = nm + Ep;
    for (int e = threadIdx.x; e < Ep; e += blockDim.x) cnt[e] = e < p.shape.E ? p.r.counts[e] : p.tokens;
    __syncthreads();
    const int total = block_exclusive_scan(cnt, off, Ep, tmp);
    if (threadIdx.x == 0) off[Ep] = total;
    __syncthreads();
    for (int e = threadIdx.x; e < Ep; e += blockDim.x) { p.r.counts[e] = cnt[e]; p.r.offsets[e] = off[e]; }
    if (threadIdx.x == 0) p.r.offsets[Ep] = off[Ep];
    build_items(p, cnt, off, ns, nm, tmp, false);   // tokens filled by k_item_tokens
}

// Step 4: one thread per token places its pairs.
__global__ __launch_bounds__(256) void k_scatter_pairs(GroupParams p) {
    extern __shared__ uint32_t lds[];
    int32_t *sid = reinterpret_cast<int32_t *>(lds);
    const int t0 = blockIdx.x * 256;
    stage_ids(p, t0, sid);
    const int t = t0 + threadIdx.x;
    if (t >= p.tokens) return;
    const int k = p.shape.k, E = p.shape.E, Ep = p.shape.Ep;
    // Ranks in chunks of kChunk: the chunk's offset, prefix and bitmap loads
    // are issued before any is used (one round trip per chunk, not per rank).
    constexpr int kChunk = 8;
    for (int r0 = 0; r0 < k; r0 += kChunk) {
        int ev[kChunk], off[kChunk];
        uint32_t pre[kChunk], bits[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            int dummy = 0;
            ev[u] = r0 + u < k ? staged_entry(sid, threadIdx.x, r0 + u, k, E, dummy) : -1;
            if (ev[u] >= 0) {
                const size_t wi = static_cast<size_t>(t >> 5) * Ep + ev[u];
                off[u] = p.r.offsets[ev[u]];
                pre[u] = p.r.wprefix[wi];
                bits[u] = p.r.bitmap[wi];
            }
        }
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const int r = r0 + u;
            if (r >= k) break;
            int pos = -1;
            if (ev[u] >= 0) {
                pos = off[u] + static_cast<int>(pre[u]) + __popc(bits[u] & ((1u << (t & 31)) - 1u));
                p.r.pair_token[pos] = t;
                p.r.pair_rank[pos] = r;
            }
            p.r.pos_of[static_cast<size_t>(t) * k + r] = pos;
        }
    }
    if (Ep > E) {
        const int s = p.r.offsets[E] + t;
        p.r.pair_token[s] = t;
        p.r.pair_rank[s] = k;
    }
}

// Copies each streaming item's pair tokens and ranks into the item (runs
// after the grouped pair arrays are complete).
__global__ __launch_bounds__(256) void k_item_tokens(RouteOut r) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= r.item_counts[0]) return;
    Item &it = r.stream_items[i];
    for (int j = 0; j < it.ncols; ++j) {
        it.token[j] = r.pair_token[it.first + j];
        it.rank[j] = r.pair_rank[it.first + j];
    }
}

// Single-expert stage setup (one block).
__global__ void k_single_items(Shape shape, RouteOut r, int expert, int columns, int use_mfma) {
    for (int j = threadIdx.x; j < columns; j += blockDim.x) { r.pair_token[j] = j; r.pair_rank[j] = 0; }
    if (threadIdx.x == 0) {
        const int size = use_mfma ? kMfmaTile : kStreamTokens;
        Item *dst = use_mfma ? r.mfma_items : r.stream_items;
        int c = 0;
        for (int f = 0; f < columns; f += size, ++c) {
            Item it;
            it.expert = expert; it.first = f; it.ncols = min(size, columns - f); it.pad = 0;
            for (int j = 0; j < kStreamTokens; ++j) { it.token[j] = f + j; it.rank[j] = 0; }
            dst[c] = it;
        }
        r.item_counts[0] = use_mfma ? 0 : c;
        r.item_counts[1] = use_mfma ? c : 0;
        r.item_counts[2] = 1;
        r.item_counts[3] = columns;
        (void)shape;
    }
}

// ------------------------------------------------ streaming (decode) path ---
// gate/up + SiLU + Q8.  One work unit = (item, slice of 32 intermediate rows).
// 8 waves: waves 0-3 take gate rows slice*32 + 8w .. +7, waves 4-7 the same
// up rows.  Lane l takes blocks l, l+64, ... (NBL of them): each row is one
// coalesced 16-byte-per-lane wave load of the code plane, held in registers
// while the item's tokens are processed one at a time.  For H > 2048 a lane
// holds several blocks, and each token's rows follow the reference's fp32
// order (src/cpu_expert.cpp:156-213): the lane keeps one accumulator per row
// and fragment, acc = fma(d4, fma(float(I_f), d8, -4 s8), acc) over its
// blocks in ascending order, and fold_rows8 reduces them as the reference's
// 128-lane fold does.  The 64 row sums go through LDS, and wave j quantizes
// token j's 32 SiLU(g)*u values into one Q8_1 block.
template<int NBL, bool Dbg>
__global__ __launch_bounds__(512) void k_gate_up_stream(FfnArgs a) {
    constexpr int T = kStreamTokens;
    __shared__ float gu[2][32][T];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t expf_word = expf_table_word(lane);
    const int H = a.shape.H, I = a.shape.I, nbh = H / 32, nbi = I / 32, S = I / 32;
    const int units = a.routes.item_counts[0] * S;
    const int mat = wave >> 2;
    const int rho = 4 * ((lane >> 5) & 1) + 2 * (lane & 1) + ((lane >> 1) & 1);   // row fold_rows8 leaves here
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const Item it = a.routes.stream_items[u / S];
        const int s = u % S;
        const int row0 = s * 32 + (wave & 3) * 8;
        const size_t mrow = static_cast<size_t>(it.expert) * I + row0;
        const uint8_t *codes = (mat ? a.bank.up_codes : a.bank.gate_codes) + mrow * nbh * 16;
        const uint16_t *scales = mat ? a.bank.up_scales : a.bank.gate_scales;
        // NBL <= 2: the item's weight rows stay in registers across its
        // tokens.  NBL == 0 (H > 4096): rows are re-read per token (L1/L2 hits).
        constexpr int HOLD = NBL > 0 ? NBL : 1;
        uint4 w[HOLD][8];
        float d4[HOLD][8];
#pragma unroll
        for (int nb = 0; nb < NBL; ++nb) {
            const int kb = lane + 64 * nb;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                if (kb < nbh) {
                    w[nb][r] = *reinterpret_cast<const uint4 *>(codes + (static_cast<size_t>(r) * nbh + kb) * 16);
                    d4[nb][r] = h2f(scales[scale_index(mrow + r, kb, nbh, kScaleGroupGateUp)]);
                } else {
                    w[nb][r] = make_uint4(0, 0, 0, 0);
                    d4[nb][r] = 0.0f;
                }
            }
        }
#pragma unroll 1
        for (int j = 0; j < it.ncols; ++j) {
            const int tok = a.routes.pair_token[it.first + j];
            float acc[8][2];
#pragma unroll
            for (int r = 0; r < 8; ++r) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
            for (int nb = 0; nb < (NBL > 0 ? NBL : 1); ++nb)
            for (int kb = lane + 64 * nb; kb < nbh; kb += (NBL > 0 ? nbh : 64)) {
                if constexpr (NBL == 0) {
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        w[0][r] = *reinterpret_cast<const uint4 *>(codes + (static_cast<size_t>(r) * nbh + kb) * 16);
                        d4[0][r] = h2f(scales[scale_index(mrow + r, kb, nbh, kScaleGroupGateUp)]);
                    }
                }
                const size_t xb = static_cast<size_t>(tok) * nbh + kb;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(a.xq.codes + xb * 32);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(a.xq.codes + xb * 32 + 16);
                const uint32_t hd = a.xq.heads[xb];
                const float d8 = h2f(hd), c4 = -4.0f * h2f(hd >> 16);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    int f0, f1;
                    fragment_dots(w[nb][r], x0, x1, f0, f1);
                    if constexpr (Dbg) {
                        int32_t *dots = mat ? a.up_dots : a.gate_dots;
                        if (dots) dots[(static_cast<size_t>(it.first + j) * I + row0 + r) * nbh + kb] = f0 + f1;
                    }
                    acc[r][0] = fmaf(d4[nb][r], fmaf(static_cast<float>(f0), d8, c4), acc[r][0]);
                    acc[r][1] = fmaf(d4[nb][r], fmaf(static_cast<float>(f1), d8, c4), acc[r][1]);
                }
            }
            const float v = fold_rows8(acc, lane);
            if ((lane & 28) == 0) gu[mat][(wave & 3) * 8 + rho][j] = v;
        }
        __syncthreads();
        if (wave < it.ncols) {
            const int j = wave, i = lane & 31;
            int flags = 0;
            const float m = silu_mul(gu[0][i][j], gu[1][i][j], flags, LaneExpfTable{expf_word});
            const Q8Lane q = quantize32(m);
            if (lane < 32) {
                const size_t pair = static_cast<size_t>(it.first + j);
                const size_t mb = pair * nbi + s;
                a.mq.codes[mb * 32 + i] = static_cast<uint8_t>(q.code);
                if (i == 0) a.mq.heads[mb] = q.head;
                if (Dbg && a.middle_f32) a.middle_f32[pair * I + s * 32 + i] = m;
                const int f = flags | (i == 0 ? q.flags : 0);
                if (f) atomicOr(a.error, f);
            }
        }
        __syncthreads();
    }
}

// High-occupancy form of k_gate_up_stream for H <= 2048 (one block per lane,
// one unit per workgroup).  Decode streaming is bound by bytes in flight per
// CU: each wave keeps its 8 weight rows (8 KB) in flight with a small register
// footprint, so 4 workgroups (32 waves, 256 KB of loads) fit on a CU.  Grid =
// item bound x I/32 slices; same arithmetic and outputs as k_gate_up_stream.
// Full: H/32 == 64, every lane holds a block.  Two: H/32 in 65..128, lane
// j also holds block j + 64 (rows8_exact2, the reference lane's FMA chain).
// One unit (item, slice) of k_gate_up_lean; false once the item is past the
// stream item count (which it stores in `count`).
// Spread (H/32 in 65..80, the reference model's 2560: 80): the second
// slot's 8 x (H/32 - 64) chunks go over the lanes as in k_decode_gate_up's
// spread form (lane 16k + j: rows k and k + 4 of block 64 + j) and each
// token's t values reach their rows' lanes by ds_bpermute (rows8_exact2t).
template<bool Full, bool Two, bool Dbg, bool Spread = false>
__device__ __forceinline__ bool gate_up_lean_unit(const FfnArgs &a, int uid, int &count,
                                                  float (&gu)[2][32][kStreamTokens]) {
    constexpr int T = kStreamTokens;
    // The wave index is uniform: as a scalar it keeps row bases in SGPRs.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t expf_word = expf_table_word(lane);
    const int H = a.shape.H, I = a.shape.I, nbh = H / 32, nbi = I / 32;
    // Workgroup id = item * I/32 + slice: with I/32 a multiple of 8 each
    // slice stays on one XCD (id % 8), so consecutive items of one expert
    // find its rows in that XCD's L2.
    const int S = I / 32;
    const int item = uid / S, s = uid % S;
    // Item header, its tokens and the item count are independent loads
    // (the item is below the grid's item bound, or below the count the
    // workgroup's previous unit read), issued together.
    const int4 hdr = *reinterpret_cast<const int4 *>(a.routes.stream_items + item);
    const int4 tok = *reinterpret_cast<const int4 *>(a.routes.stream_items[item].token);
    count = a.routes.item_counts[0];
    // Keeps the compiler from deferring the item loads behind the count check.
    asm volatile("" ::"s"(hdr.x), "s"(hdr.y), "s"(hdr.z), "s"(tok.x), "s"(tok.y), "s"(tok.z), "s"(tok.w), "s"(count));
    if (item >= count) return false;   // uniform per workgroup
    const int expert = hdr.x, first = hdr.y, ncols = hdr.z;
    const int mat = wave >> 2;
    const int row0 = s * 32 + (wave & 3) * 8;
    // Lanes past the row end (H < 2048) read block 0 and drop their products:
    // every load is unconditional, so a wave's 8 row loads are all in flight
    // at once (a guarded load would be waited for before the next is issued).
    const bool has = lane < nbh;
    const int kb = has ? lane : 0;
    // The wave's 8 rows are one buffer (uniform base, per-row SGPR offset, one
    // lane-offset VGPR); the lane's 8 scales (rows row0..row0+7 of its block)
    // are one 16-byte load.
    const size_t mrow = static_cast<size_t>(expert) * I + row0;    // row0 % 8 == 0
    const uint32_t row_bytes = static_cast<uint32_t>(nbh) * 16u;
    const auto wr = buffer_rsrc((mat ? a.bank.up_codes : a.bank.gate_codes) + mrow * row_bytes, 8 * row_bytes);
    const auto sr = buffer_rsrc((mat ? a.bank.up_scales : a.bank.gate_scales) + mrow * nbh, row_bytes);
    const uint32_t lane_off = static_cast<uint32_t>(kb) * 16u;
    const int rho = 4 * ((lane >> 5) & 1) + 2 * (lane & 1) + ((lane >> 1) & 1);   // row rows8_exact leaves in this lane
    // The weights are loaded once per item and held for its tokens (reloading
    // them per token relied on L2 hits that a busy XCD L2 does not give).
    uint4 w[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) w[r] = buffer_load16(wr, lane_off, r * row_bytes);
    const uint4 d4p = buffer_load16(sr, lane_off, 0);
    const bool has2 = Two && lane + 64 < nbh;
    const uint32_t lane_off2 = has2 ? static_cast<uint32_t>(lane + 64) * 16u : 0u;
    // Spread: this lane's chunks, rows xk and xk + 4 of block 64 + xj.
    const int xk = lane >> 4, xj = lane & 15;
    const bool xhas = Spread && xj < nbh - 64;
    const uint32_t x_off2 = xhas ? static_cast<uint32_t>(64 + xj) * 16u : 0u;
    uint4 w2[Spread ? 2 : 8];
    uint4 d4p2 = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (Spread) {
        w2[0] = buffer_load16(wr, x_off2 + static_cast<uint32_t>(xk) * row_bytes, 0);
        w2[1] = buffer_load16(wr, x_off2 + static_cast<uint32_t>(xk + 4) * row_bytes, 0);
        d4p2 = buffer_load16(sr, lane_off2, 0);
    } else if constexpr (Two) {
#pragma unroll
        for (int r = 0; r < 8; ++r) w2[r] = buffer_load16(wr, lane_off2, r * row_bytes);
        d4p2 = buffer_load16(sr, lane_off2, 0);
    }
    // A token's activations (the lane's one or two blocks) are loaded while
    // the previous token computes.
    const int toks[T] = {tok.x, tok.y, tok.z, tok.w};
    struct Xb {
        uint4 x0, x1, y0, y1;
        uint32_t hx, hy;
    };
    auto load_x = [&](int j, Xb &b) {
        const size_t xrow = static_cast<size_t>(toks[j < ncols ? j : 0]) * nbh;
        const auto xr = buffer_rsrc(a.xq.codes + xrow * 32, static_cast<uint32_t>(nbh) * 32u);
        const auto hr = buffer_rsrc(a.xq.heads + xrow, static_cast<uint32_t>(nbh) * 4u);
        b.x0 = buffer_load16(xr, 2 * lane_off, 0);
        b.x1 = buffer_load16(xr, 2 * lane_off, 16);
        b.hx = buffer_load4(hr, lane_off / 4, 0);
        if constexpr (Two) {
            // Spread: the block of this lane's chunks (64 + xj); else block lane + 64.
            const uint32_t o2 = Spread ? x_off2 : lane_off2;
            b.y0 = buffer_load16(xr, 2 * o2, 0);
            b.y1 = buffer_load16(xr, 2 * o2, 16);
            b.hy = buffer_load4(hr, o2 / 4, 0);
        }
    };
    Xb cur;
    load_x(0, cur);
#pragma unroll
    for (int j = 0; j < T; ++j) {
        if (j < ncols) {   // uniform per workgroup
            Xb nxt = cur;
            if (j + 1 < T && j + 1 < ncols) load_x(j + 1, nxt);
            if constexpr (Dbg) {
                int32_t *dots = mat ? a.up_dots : a.gate_dots;
                if (dots && has)
#pragma unroll
                    for (int r = 0; r < 8; ++r)
                        dots[(static_cast<size_t>(first + j) * I + row0 + r) * nbh + lane] = dot_block(w[r], cur.x0, cur.x1);
                if (Two && dots && has2)
#pragma unroll
                    for (int r = 0; r < 8; ++r)
                        dots[(static_cast<size_t>(first + j) * I + row0 + r) * nbh + lane + 64] =
                            dot_block(w2[r], cur.y0, cur.y1);
            }
            float v;
            if constexpr (Spread) {
                const float e8 = h2f(cur.hy), e4 = -4.0f * h2f(cur.hy >> 16);
                float tx[2][2];
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    int g0, g1;
                    fragment_dots(w2[c], cur.y0, cur.y1, g0, g1);
                    tx[c][0] = fmaf(static_cast<float>(g0), e8, e4);
                    tx[c][1] = fmaf(static_cast<float>(g1), e8, e4);
                }
                // Row q of block 64 + j sits in lane j + 16 (q % 4), chunk q / 4.
                float t2[8][2];
#pragma unroll
                for (int q = 0; q < 8; ++q)
#pragma unroll
                    for (int f = 0; f < 2; ++f)
                        t2[q][f] = (q & 3) == 0 ? tx[q >> 2][f]
                                                : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                                      4 * ((lane & 15) + 16 * (q & 3)), __float_as_int(tx[q >> 2][f])));
                v = rows8_exact2t(w, d4p, cur.x0, cur.x1, cur.hx, d4p2, t2, has2, lane);
            } else if constexpr (Two) {
                v = rows8_exact2(w, d4p, cur.x0, cur.x1, cur.hx, w2, d4p2, cur.y0, cur.y1, cur.hy, has2, lane);
            } else {
                v = rows8_exact<Full>(w, d4p, cur.x0, cur.x1, cur.hx, has, lane);
            }
            if ((lane & 28) == 0) gu[mat][(wave & 3) * 8 + rho][j] = v;
            cur = nxt;
        }
    }
    __syncthreads();
    if (wave < ncols) {
        const int j = wave, i = lane & 31;
        int flags = 0;
        const float m = silu_mul(gu[0][i][j], gu[1][i][j], flags, LaneExpfTable{expf_word});
        const Q8Lane q = quantize32(m);
        if (lane < 32) {
            const size_t pair = static_cast<size_t>(first + j);
            const size_t mb = pair * nbi + s;
            a.mq.codes[mb * 32 + i] = static_cast<uint8_t>(q.code);
            if (i == 0) a.mq.heads[mb] = q.head;
            if (Dbg && a.middle_f32) a.middle_f32[pair * I + s * 32 + i] = m;
            const int f = flags | (i == 0 ? q.flags : 0);
            if (f) atomicOr(a.error, f);
        }
    }
    __syncthreads();   // gu is free for the workgroup's next unit
    return true;
}

// Units id, id + grid, ...: the grid is capped (kLeanGridCap), a multiple of
// 8 and of I/32, so a workgroup keeps its XCD and slice and a batch with no
// streaming items starts few workgroups.
template<bool Full, bool Two, bool Dbg, bool Spread = false>
__global__ __launch_bounds__(512, Two && !Spread ? 2 : 3) void k_gate_up_lean(FfnArgs a) {
    __shared__ float gu[2][32][kStreamTokens];
    const int S = a.shape.I / 32;
    int count = INT_MAX;
    for (int u = static_cast<int>(blockIdx.x); u / S < count; u += static_cast<int>(gridDim.x))
        if (!gate_up_lean_unit<Full, Two, Dbg, Spread>(a, u, count, gu)) break;
}

// Down projection, streaming path, for rows of more than 32 blocks (I >
// 1024).  Work unit = (item, slice of 32 output rows); 8 waves x 4 rows (8
// rows a wave spilled: two accumulators per row and token).  A row spans the
// wave: lane j holds blocks j, j + 64, ... and keeps one
// accumulator per fragment over them in ascending order, as the reference's
// lane 2 (k % 64) + f does (src/cpu_expert.cpp:156-213):
//   Q4_0: acc = fma(d4, fma(float(I_f), d8, -4 s8), acc)
//   Q4_1: acc = acc + fma(float(I_f), half(d4 d8), half(m4 s8) / 2)
// then the reference's fold: lane j + lane j ^ 32 per fragment, the two
// fragments, XOR 1 .. 16.  Unweighted results go to the contribution row
// (token * out_stride_k + rank) like the reference's scatter
// (src/hip/session_ops.hip:357-373).
template<bool Q41, bool Dbg>
__global__ __launch_bounds__(512) void k_down_stream(FfnArgs a) {
    constexpr int T = kStreamTokens, R = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.shape.H, I = a.shape.I, nbi = I / 32, S = H / 32;
    const int units = a.routes.item_counts[0] * S;
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const Item it = a.routes.stream_items[u / S];
        const int row0 = (u % S) * 32 + wave * R;
        const size_t mrow = static_cast<size_t>(it.expert) * H + row0;
        const uint8_t *codes = a.bank.down_codes + mrow * nbi * 16;
        const uint16_t *scales = a.bank.down_scales, *mins = a.bank.down_mins;
        float acc[R][T][2];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < T; ++j) acc[r][j][0] = acc[r][j][1] = 0.0f;
        for (int kb = lane; kb < nbi; kb += 64) {
            uint4 w[R];
            float d4[R], m4[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                w[r] = *reinterpret_cast<const uint4 *>(codes + (static_cast<size_t>(r) * nbi + kb) * 16);
                const size_t si = scale_index(mrow + r, kb, nbi, kScaleGroupDown);
                d4[r] = h2f(scales[si]);
                m4[r] = Q41 ? h2f(mins[si]) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < T; ++j) {
                if (j >= it.ncols) break;
                const size_t xb = static_cast<size_t>(it.first + j) * nbi + kb;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(a.mq.codes + xb * 32);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(a.mq.codes + xb * 32 + 16);
                const uint32_t hd = a.mq.heads[xb];
                const float d8 = h2f(hd), s8 = h2f(hd >> 16), c4 = -4.0f * s8;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    int f[2];
                    fragment_dots(w[r], x0, x1, f[0], f[1]);
                    if constexpr (Dbg) {
                        if (a.down_dots)
                            a.down_dots[(static_cast<size_t>(it.first + j) * H + row0 + r) * nbi + kb] = f[0] + f[1];
                    }
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        if constexpr (Q41) {
                            const float dd = h2f(f2h(d4[r] * d8)), hm = h2f(f2h(m4[r] * s8)) * 0.5f;
                            acc[r][j][q] = acc[r][j][q] + fmaf(static_cast<float>(f[q]), dd, hm);
                        } else {
                            acc[r][j][q] = fmaf(d4[r], fmaf(static_cast<float>(f[q]), d8, c4), acc[r][j][q]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < T; ++j) {
            if (j >= it.ncols) break;
            const int pair = it.first + j;
            const size_t orow = static_cast<size_t>(a.routes.pair_token[pair]) * a.out_stride_k +
                                a.routes.pair_rank[pair];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v0 = xor_sum<32>(acc[r][j][0]), v1 = xor_sum<32>(acc[r][j][1]);
                float v = v0 + v1;
                v = xor_sum<1>(v);
                v = xor_sum<2>(v);
                v = xor_sum<4>(v);
                v = xor_sum<8>(v);
                v = xor_sum<16>(v);
                if (lane == 0) a.out[orow * H + row0 + r] = v;
            }
        }
    }
}

// High-occupancy streaming down projection for I <= 512 (a row of I/32 <= 16
// blocks is <= 256 code bytes, 16 lanes; one wave load covers 4 rows).  Work
// unit = (item, slice of 64 output rows), grid = item bound x H/64; a 2-wave
// workgroup gives each wave 32 rows = 8 independent 16-byte loads per lane in
// flight.  Row sums of the item's pairs are written unweighted to their
// contribution rows (token * out_stride_k + rank), like the reference's
// scatter (src/hip/session_ops.hip:357-373).
// NBI = 16 specialises I = 512 (every lane holds a block); NBI = 0 reads
// I/32 <= 16 at run time.  Q41: Q4_1 blocks (mins plane in the scales' order).
// Two: I/32 in 17..32, lane kl also holds block kl + 16; the row is (tree over
// blocks 0..15) + (tree over blocks 16..31), the last stage of the reference's
// fold.
// One unit (item, slice of 64 rows) of k_down_lean; false once the item is
// past the stream item count (stored in `count`).
// Spread (I/32 in 17..20): the second tree's chunks go two to a lane as in
// k_decode_down_fold's spread form, the weights held across the item's pairs.
template<int NBI, bool Q41, bool Two, bool Dbg, bool Spread = false>
__device__ __forceinline__ bool down_lean_unit(const FfnArgs &a, int uid, int &count) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shape.H, nbi = NBI ? NBI : a.shape.I / 32;
    // Unit id = item * H/64 + slice (one XCD per slice, as in k_gate_up_lean).
    const int S = H / 64;
    const int item = uid / S, slice = uid % S;
    const int4 hdr = *reinterpret_cast<const int4 *>(a.routes.stream_items + item);
    const int4 tok = *reinterpret_cast<const int4 *>(a.routes.stream_items[item].token);
    const int4 rnk = *reinterpret_cast<const int4 *>(a.routes.stream_items[item].rank);
    count = a.routes.item_counts[0];
    asm volatile("" ::"s"(hdr.x), "s"(hdr.y), "s"(hdr.z), "s"(tok.x), "s"(tok.y), "s"(tok.z), "s"(tok.w),
                 "s"(rnk.x), "s"(rnk.y), "s"(rnk.z), "s"(rnk.w), "s"(count));
    if (item >= count) return false;   // uniform per workgroup
    const int expert = hdr.x, first = hdr.y, ncols = hdr.z;
    const int row0 = slice * 64 + wave * 32;
    const int sub = lane >> 4, kl = lane & 15;
    // Lanes past the row end (I < 512) read block 0 and drop their products,
    // so all loads are unconditional and in flight together.
    const bool has = NBI == 16 || kl < nbi;
    const int kb = has ? kl : 0;
    // The wave's 32 rows are one buffer (per-load SGPR offset, one lane-offset
    // VGPR); the lane's 8 scales (rows row0 + sub + 4l of its block) are one
    // 16-byte load.
    const size_t mrow = static_cast<size_t>(expert) * H + row0;     // row0 % 32 == 0
    const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
    const auto wr = buffer_rsrc(a.bank.down_codes + mrow * row_bytes, 32 * row_bytes);
    const auto sr = buffer_rsrc(a.bank.down_scales + mrow * nbi, 4 * row_bytes);
    const uint32_t lane_off = static_cast<uint32_t>(sub * nbi + kb) * 16u;
    // Transposing reduction over the 16 lanes of a row: xor 8/4/2 halve the
    // 8 load-rows, xor 1 finishes; lane ends with load-row lr(lane).
    const int lr = 4 * (lane & 1) + 2 * ((lane >> 1) & 1) + ((lane >> 2) & 1);   // row rows8_down_exact leaves here
    // The weights are loaded once per item and held for its pairs.
    uint4 w[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) w[l] = buffer_load16(wr, lane_off, 4 * l * row_bytes);
    const uint4 d4p = buffer_load16(sr, static_cast<uint32_t>(kb * 32 + sub * 8) * 2u, 0);
    uint4 m4p = make_uint4(0u, 0u, 0u, 0u);
    const auto mr = buffer_rsrc(Q41 ? a.bank.down_mins + mrow * nbi : a.bank.down_scales, 4 * row_bytes);
    if constexpr (Q41) m4p = buffer_load16(mr, static_cast<uint32_t>(kb * 32 + sub * 8) * 2u, 0);
    const bool has2 = Two && kl + 16 < nbi;
    const int kb2 = has2 ? kl + 16 : 0;
    // Spread: this lane's chunks, block 16 + (lane & 3) of rows lane / 4 and
    // 16 + lane / 4 of the wave's 32.
    const int sj = lane & 3;
    const bool shas = Spread && 16 + sj < nbi;
    const int skb = shas ? 16 + sj : 0;
    uint4 w2[Spread ? 2 : 8];
    uint32_t sdh[2] = {0u, 0u}, smh[2] = {0u, 0u};
    uint4 d4p2 = make_uint4(0u, 0u, 0u, 0u), m4p2 = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (Spread) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int rr = 16 * u + (lane >> 2);
            w2[u] = buffer_load16(wr, static_cast<uint32_t>(rr) * row_bytes + static_cast<uint32_t>(skb) * 16u, 0);
            // Scale plane: [32-row group][block][32 halves], row r at half (r & 3) * 8 + r / 4.
            const uint32_t hi = static_cast<uint32_t>(skb * 32 + (rr & 3) * 8 + (rr >> 2));
            const uint32_t dw = buffer_load4(sr, (hi >> 1) * 4u, 0);
            sdh[u] = (hi & 1) ? dw >> 16 : dw & 0xffffu;
            if constexpr (Q41) {
                const uint32_t mw = buffer_load4(mr, (hi >> 1) * 4u, 0);
                smh[u] = (hi & 1) ? mw >> 16 : mw & 0xffffu;
            }
        }
    } else if constexpr (Two) {
        const uint32_t lane_off2 = static_cast<uint32_t>(sub * nbi + kb2) * 16u;
#pragma unroll
        for (int l = 0; l < 8; ++l) w2[l] = buffer_load16(wr, lane_off2, 4 * l * row_bytes);
        d4p2 = buffer_load16(sr, static_cast<uint32_t>(kb2 * 32 + sub * 8) * 2u, 0);
        if constexpr (Q41) m4p2 = buffer_load16(mr, static_cast<uint32_t>(kb2 * 32 + sub * 8) * 2u, 0);
    }
    // A pair's middle row (the lane's one or two blocks) is loaded while the
    // previous pair computes.
    struct Xb {
        uint4 x0, x1, y0, y1;
        uint32_t hx, hy;
    };
    auto load_x = [&](int j, Xb &b) {
        const size_t xrow = static_cast<size_t>(first + (j < ncols ? j : 0)) * nbi;
        const auto xr = buffer_rsrc(a.mq.codes + xrow * 32, static_cast<uint32_t>(nbi) * 32u);
        const auto hr = buffer_rsrc(a.mq.heads + xrow, static_cast<uint32_t>(nbi) * 4u);
        b.x0 = buffer_load16(xr, static_cast<uint32_t>(kb) * 32u, 0);
        b.x1 = buffer_load16(xr, static_cast<uint32_t>(kb) * 32u, 16);
        b.hx = buffer_load4(hr, static_cast<uint32_t>(kb) * 4u, 0);
        if constexpr (Two) {
            // Spread: the block of this lane's chunks (16 + lane % 4); else block kl + 16.
            const uint32_t b2 = static_cast<uint32_t>(Spread ? skb : kb2);
            b.y0 = buffer_load16(xr, b2 * 32u, 0);
            b.y1 = buffer_load16(xr, b2 * 32u, 16);
            b.hy = buffer_load4(hr, b2 * 4u, 0);
        }
    };
    const int toks[kStreamTokens] = {tok.x, tok.y, tok.z, tok.w};
    const int rnks[kStreamTokens] = {rnk.x, rnk.y, rnk.z, rnk.w};
    Xb cur;
    load_x(0, cur);
#pragma unroll
    for (int j = 0; j < kStreamTokens; ++j) {
        if (j < ncols) {   // uniform per workgroup
            Xb nxt = cur;
            if (j + 1 < kStreamTokens && j + 1 < ncols) load_x(j + 1, nxt);
            if constexpr (Dbg) {
                if (a.down_dots && has)
#pragma unroll
                    for (int l = 0; l < 8; ++l)
                        a.down_dots[(static_cast<size_t>(first + j) * H + row0 + 4 * l + sub) * nbi + kl] =
                            dot_block(w[l], cur.x0, cur.x1);
                if (Two && a.down_dots && has2)
#pragma unroll
                    for (int l = 0; l < 8; ++l)
                        a.down_dots[(static_cast<size_t>(first + j) * H + row0 + 4 * l + sub) * nbi + kl + 16] =
                            dot_block(w2[l], cur.y0, cur.y1);
            }
            float v = rows8_down_exact<Q41>(w, d4p, m4p, cur.x0, cur.x1, cur.hx, has, lane);
            if constexpr (Spread) {
                // ((n16 + n17) + (n18 + n19)) per row in its lane quad, then to
                // the lane holding the row's first tree (row 4 lr + sub).
                float sq[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    float n = down_chunk<Q41>(w2[u], sdh[u], smh[u], cur.y0, cur.y1, cur.hy, shas);
                    n = n + lane_xor<1>(n);
                    sq[u] = n + lane_xor<2>(n);
                }
                const int row = 4 * lr + sub, src = 4 * (row & 15);
                const float a0 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src, __float_as_int(sq[0])));
                const float a1 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src, __float_as_int(sq[1])));
                v = v + ((row >> 4) ? a1 : a0);
            } else if constexpr (Two) {
                v = v + rows8_down_exact<Q41>(w2, d4p2, m4p2, cur.y0, cur.y1, cur.hy, has2, lane);
            }
            if ((lane & 8) == 0) {
                const size_t orow = static_cast<size_t>(toks[j]) * a.out_stride_k + rnks[j];
                a.out[orow * H + row0 + 4 * lr + sub] = v;
            }
            cur = nxt;
        }
    }
    return true;
}

// Units id, id + grid, ... over a capped grid (a multiple of 8 and of H/64,
// as in k_gate_up_lean).
template<int NBI, bool Q41, bool Two, bool Dbg, bool Spread = false>
__global__ __launch_bounds__(128, Two ? (Spread ? 3 : 2) : 4) void k_down_lean(FfnArgs a) {
    const int S = a.shape.H / 64;
    int count = INT_MAX;
    for (int u = static_cast<int>(blockIdx.x); u / S < count; u += static_cast<int>(gridDim.x))
        if (!down_lean_unit<NBI, Q41, Two, Dbg, Spread>(a, u, count)) break;
}

// ----------------------------------------------------- ungrouped decode ---
// Route (t, r) of a decode batch, validated as RouteGroups::prepare does
// (src/routes.cpp:76-90): returns the expert (E = shared for r == k) or -1
// for a bad id or a duplicate of an earlier rank.  `flags` gets bit 1 for a
// bad id, a duplicate, or a negative / nonfinite weight.  Every lane of the
// wave calls it with the same (t, r): lane j < k reads id j of the row, so
// the row arrives in one round trip and the duplicate test is a ballot, not
// a chain of dependent loads in front of the weight address.
__device__ __forceinline__ int decode_route(const DecodeArgs &d, int t, int r, int &flags) {
    const int k = d.f.shape.k, E = d.f.shape.E;
    if (r == k) return E;
    const int lane = threadIdx.x & 63;
    const size_t base = static_cast<size_t>(t) * k;
    const int mine = lane < k ? d.ids[base + lane] : -1;
    const float w = d.weights[base + r];
    const int e = __builtin_amdgcn_readlane(mine, r);
    if (!isfinite(w) || w < 0.0f) flags |= 1;
    const bool dup = __builtin_amdgcn_ballot_w64(lane < r && mine == e) != 0;
    if (e < 0 || e >= E || dup) { flags |= 1; return -1; }
    return e;
}

// gate/up + SiLU + Q8 for one (token, rank) pair and one slice of 32
// intermediate rows; grid = (k + shared, tokens, I/32).  The 8 waves take
// 8 gate / up rows each as in k_gate_up_lean.  The token's x row is quantized
// by the whole workgroup into LDS (the same quantize32 as the quantize
// kernels) while the weight loads are in flight.
// Q8In: the token rows come as canonical Q8_1 blocks (d.x_q8) and waves 0-3
// copy them into LDS instead of quantizing x.  Full: H/32 == 64, every lane
// holds a block.  Two: H/32 in 65..128 (the reference model's 2560: 80
// blocks), lane j holds blocks j and j + 64, and all 8 waves take part in
// quantizing the row.
// Spread (Two, H/32 in 65..80: the reference model's 2560): the 8 x nx
// second-slot chunks of a wave's rows (nx = H/32 - 64 <= 16) are spread over
// the lanes instead of every lane holding 8: lane 16k + j loads rows k and
// k + 4 of block 64 + j and forms their t = fma(float(I_f), d8', -4 s8'),
// which ds_bpermute hands to lane j (rows8_exact2t).  Each lane keeps 2
// chunks instead of 8, so more waves fit (73 VGPRs against 98): the 2560/640
// B8 gate/up stage 40.4 -> 32.1 us.
template<bool Q8In, bool Full, bool Two, bool Spread = false>
__global__ __launch_bounds__(512, Two ? (Spread ? 6 : 4) : 8) void k_decode_gate_up(DecodeArgs d) {
    __shared__ uint32_t xs[kDecodeMaxBlocksH * 8];   // Q8 codes of the token, [blocks][32 B]
    __shared__ uint32_t xh[kDecodeMaxBlocksH];       // heads
    __shared__ float gu[2][32];
    const FfnArgs &a = d.f;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t expf_word = expf_table_word(lane);
    const int H = a.shape.H, I = a.shape.I, nbh = H / 32, nbi = I / 32;
    // XCD-aware order: workgroup id i runs on XCD i % 8.  Ids are laid out so
    // that the tokens of one (rank, slice) are consecutive on one XCD: the
    // shared expert's rows of a slice (and an expert two tokens share, at the
    // same rank) are then fetched from HBM once into that XCD's L2.
    const int N = a.tokens, P1 = a.shape.k + (a.shape.Ep > a.shape.E ? 1 : 0), S = I / 32;
    const int id = blockIdx.x, j = id >> 3;
    const int t = j % N, r = (j / N) % P1, s = (id & 7) + 8 * (j / (N * P1));
    if (s >= S) return;
    int flags = 0;
    const int expert = decode_route(d, t, r, flags);
    if (s == 0 && flags && threadIdx.x == 0) atomicOr(a.error, flags);
    // Rank 0 / slice 0 reports the token's input flags and writes its x Q8,
    // so it quantizes even when its own route is invalid.
    const bool report = r == 0 && s == 0;
    if (expert < 0 && !report) return;   // uniform per workgroup
    // Waves 0-3 quantize the token row, 4 lanes per block (wave w, lane l:
    // block 16w + l % 16, elements 8 * (l / 16) .. +7).  They issue their x
    // loads before their weight loads, so waiting for x never waits behind
    // the weights.
    const bool quant_wave = Two || wave < 4;
    const int qblk = wave * 16 + (lane & 15), qpart = lane >> 4;
    float xv[8];
    uint2 qin = make_uint2(0u, 0u);   // Q8In: codes 8 * qpart .. +7 of block qblk
    uint32_t qhead = 0;
    if (Q8In && quant_wave && qblk < nbh) {
        const auto qr = buffer_rsrc(static_cast<const uint8_t *>(d.x_q8) + static_cast<size_t>(t) * nbh * 36,
                                    static_cast<uint32_t>(nbh) * 36u);
        const uint32_t off = static_cast<uint32_t>(qblk) * 36u, part = off + 4u + 8u * static_cast<uint32_t>(qpart);
        qin = make_uint2(buffer_load4(qr, part, 0), buffer_load4(qr, part, 4));
        qhead = buffer_load4(qr, off, 0);
    }
    if (!Q8In && quant_wave) {
        const auto xr = buffer_rsrc(d.x + static_cast<size_t>(t) * H, static_cast<uint32_t>(H) * 4u);
        const uint32_t off = static_cast<uint32_t>(qblk * 32 + qpart * 8) * 4u;   // past H: reads 0
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint4 v = buffer_load16(xr, off, q * 16);
            xv[4 * q] = __uint_as_float(v.x); xv[4 * q + 1] = __uint_as_float(v.y);
            xv[4 * q + 2] = __uint_as_float(v.z); xv[4 * q + 3] = __uint_as_float(v.w);
        }
    }
    // Weights of this wave's 8 rows (as k_gate_up_lean).
    const int mat = wave >> 2;
    const int row0 = s * 32 + (wave & 3) * 8;
    const bool has = lane < nbh;
    const int kb = has ? lane : 0;
    const size_t mrow = static_cast<size_t>(expert < 0 ? 0 : expert) * I + row0;
    const uint32_t row_bytes = static_cast<uint32_t>(nbh) * 16u;
    const auto wr = buffer_rsrc((mat ? a.bank.up_codes : a.bank.gate_codes) + mrow * row_bytes, 8 * row_bytes);
    const auto sr = buffer_rsrc((mat ? a.bank.up_scales : a.bank.gate_scales) + mrow * nbh, row_bytes);
    const uint32_t lane_off = static_cast<uint32_t>(kb) * 16u;
    uint4 w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = buffer_load16_nt(wr, lane_off, q * row_bytes);
    const uint4 d4p = buffer_load16(sr, lane_off, 0);
    // Two: the lane's second block, lane + 64 (block 0 when past the row end).
    const bool has2 = Two && lane + 64 < nbh;
    const uint32_t lane_off2 = has2 ? static_cast<uint32_t>(lane + 64) * 16u : 0u;
    uint4 w2[Spread ? 1 : 8];
    uint4 d4p2 = make_uint4(0u, 0u, 0u, 0u);
    // Spread: this lane's chunks, rows xk and xk + 4 of block 64 + xj.  Lanes
    // without one point past the row buffer: zeros, no memory access.
    const int xk = lane >> 4, xj = lane & 15;
    const bool xhas = Spread && xj < nbh - 64;
    uint4 wx[2];
    if constexpr (Spread) {
        const uint32_t xoff = xhas ? static_cast<uint32_t>(64 + xj) * 16u + static_cast<uint32_t>(xk) * row_bytes
                                   : 8u * row_bytes;
        wx[0] = buffer_load16_nt(wr, xoff, 0);
        wx[1] = buffer_load16_nt(wr, xoff, 4u * row_bytes);
        d4p2 = buffer_load16(sr, lane_off2, 0);
        __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (Two) {
#pragma unroll
        for (int q = 0; q < 8; ++q) w2[q] = buffer_load16_nt(wr, lane_off2, q * row_bytes);
        d4p2 = buffer_load16(sr, lane_off2, 0);
        // Every load is issued before the quantisation waits on x (the
        // scheduler would otherwise sink half of them behind that wait).
        __builtin_amdgcn_sched_barrier(0);
    }
    if (Q8In && quant_wave && qblk < nbh) {
        reinterpret_cast<uint2 *>(xs)[qblk * 4 + qpart] = qin;
        if (qpart == 0) xh[qblk] = qhead;
        if (report) {
            const size_t gb = static_cast<size_t>(t) * nbh + qblk;
            reinterpret_cast<uint2 *>(a.xq.codes)[gb * 4 + qpart] = qin;
            if (qpart == 0) a.xq.heads[gb] = qhead;
        }
    }
    if (!Q8In && quant_wave) {
        const Q8Part<4> qp = quantize_part<4>(xv);
        if (qblk < nbh) {
            reinterpret_cast<uint2 *>(xs)[qblk * 4 + qpart] = make_uint2(qp.codes[0], qp.codes[1]);
            if (qpart == 0) xh[qblk] = qp.head;
            if (report) {
                const size_t gb = static_cast<size_t>(t) * nbh + qblk;
                reinterpret_cast<uint2 *>(a.xq.codes)[gb * 4 + qpart] = make_uint2(qp.codes[0], qp.codes[1]);
                if (qpart == 0) {
                    a.xq.heads[gb] = qp.head;
                    if (qp.flags) atomicOr(a.error, qp.flags);
                }
            }
        }
    }
    if (expert < 0) return;   // the reporting workgroup of an invalid route
    __syncthreads();
    const uint4 x0 = reinterpret_cast<const uint4 *>(xs)[kb * 2];
    const uint4 x1 = reinterpret_cast<const uint4 *>(xs)[kb * 2 + 1];
    float v;
    if constexpr (Spread) {
        const int eb = 64 + (xhas ? xj : 0);
        const uint4 e0 = reinterpret_cast<const uint4 *>(xs)[eb * 2];
        const uint4 e1 = reinterpret_cast<const uint4 *>(xs)[eb * 2 + 1];
        const uint32_t eh = xh[eb];
        const float e8 = h2f(eh), e4 = -4.0f * h2f(eh >> 16);
        float tx[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            int g0, g1;
            fragment_dots(wx[c], e0, e1, g0, g1);
            tx[c][0] = fmaf(static_cast<float>(g0), e8, e4);
            tx[c][1] = fmaf(static_cast<float>(g1), e8, e4);
        }
        // Row q of block 64 + j sits in lane j + 16 (q % 4), chunk q / 4.
        float t2[8][2];
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int f = 0; f < 2; ++f)
                t2[q][f] = (q & 3) == 0 ? tx[q >> 2][f]
                                        : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                              4 * ((lane & 15) + 16 * (q & 3)), __float_as_int(tx[q >> 2][f])));
        v = rows8_exact2t(w, d4p, x0, x1, xh[kb], d4p2, t2, has2, lane);
    } else if constexpr (Two) {
        const int kb2 = has2 ? lane + 64 : 0;
        const uint4 y0 = reinterpret_cast<const uint4 *>(xs)[kb2 * 2];
        const uint4 y1 = reinterpret_cast<const uint4 *>(xs)[kb2 * 2 + 1];
        v = rows8_exact2(w, d4p, x0, x1, xh[kb], w2, d4p2, y0, y1, xh[kb2], has2, lane);
    } else {
        v = rows8_exact<Full>(w, d4p, x0, x1, xh[kb], has, lane);
    }
    const int rho = 4 * ((lane >> 5) & 1) + 2 * (lane & 1) + ((lane >> 1) & 1);
    if ((lane & 28) == 0) gu[mat][(wave & 3) * 8 + rho] = v;
    __syncthreads();
    if (wave == 0) {
        const int i = lane & 31;
        int f = 0;
        const float m = silu_mul(gu[0][i], gu[1][i], f, LaneExpfTable{expf_word});
        const Q8Lane q = quantize32(m);
        if (lane < 32) {
            const size_t mb = (static_cast<size_t>(t) * P1 + r) * nbi + s;
            a.mq.codes[mb * 32 + i] = static_cast<uint8_t>(q.code);
            if (i == 0) a.mq.heads[mb] = q.head;
            f |= i == 0 ? q.flags : 0;
            if (f) atomicOr(a.error, f);
        }
    }
}

// down + fold for one token and 32 output rows; grid = (tokens, H/32), one
// wave per rank (block = 64 * (k + shared) threads).  Wave r computes the 32
// unweighted row sums of its pair (lane (sub, kb): rows sub + 4l, l < 8, as in
// k_down_lean), then 32 threads fold the ranks in order and add the shared
// expert -- the separately rounded fold of k_fold, with no contribution
// buffer and no second kernel.  Q41: Q4_1 down blocks.
// Two: I/32 in 17..32 (the reference model's 640: 20 blocks); lane kl also
// takes block kl + 16.  The reference's fold pairs blocks k and k ^ 16 last,
// so the row is (tree over blocks 0..15) + (tree over blocks 16..31), each
// tree as rows8_down_exact sums it.
// Spread (I/32 in 17..20, the reference model's 640: 20): the second tree
// holds at most blocks 16..19, i.e. ((n16 + n17) + (n18 + n19)) with n the
// chunks of rows8_down_exact (its other lanes add +0).  The wave's 32 rows x
// 4 second-slot chunks go two to a lane instead of 8 rows per lane: lane l
// takes block 16 + (l & 3) of rows l / 4 and 16 + l / 4, the lane quad sums
// a row's four chunks in that order (XOR 1, then 2), and ds_bpermute brings
// each row's sum to the lane that holds the row's first tree.
template<bool Q41, bool Two, bool Spread = false>
__global__ __launch_bounds__(1024) void k_decode_down_fold(DecodeArgs d) {
    __shared__ float part[kDecodeMaxPairs][32];
    __shared__ int valid[kDecodeMaxPairs];
    __shared__ float wt[kDecodeMaxPairs];   // the token's routing weights, then its shared gate
    const FfnArgs &a = d.f;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shape.H, nbi = a.shape.I / 32, k = a.shape.k;
    const int P1 = blockDim.x >> 6;
    // XCD-aware order (workgroup i runs on XCD i % 8): the tokens of one row
    // slice are consecutive on one XCD, so the rows of the shared expert (and
    // of an expert two tokens share) are fetched from HBM once per slice.
    const int N = a.tokens, S = H / 32;
    const int id = blockIdx.x, j = id >> 3;
    const int t = j % N, slice = (id & 7) + 8 * (j / N);
    if (slice >= S) return;
    const int row0 = slice * 32, r = wave;
    // The fold's operands into LDS now: after the barrier it reads no
    // global memory (the weights were one dependent round trip per rank).
    if (threadIdx.x < static_cast<unsigned>(k)) wt[threadIdx.x] = d.weights[static_cast<size_t>(t) * k + threadIdx.x];
    if (threadIdx.x == static_cast<unsigned>(k) && P1 > k && d.shared_gate) wt[k] = d.shared_gate[t];
    int dummy = 0;
    const int expert = decode_route(d, t, r, dummy);
    if (lane == 0) valid[r] = expert >= 0;
    if (expert >= 0) {
        const int sub = lane >> 4, kl = lane & 15;
        const bool has = kl < nbi;
        const int kb = has ? kl : 0;
        const size_t mrow = static_cast<size_t>(expert) * H + row0;     // row0 % 32 == 0
        const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
        const auto wr = buffer_rsrc(a.bank.down_codes + mrow * row_bytes, 32 * row_bytes);
        const auto sr = buffer_rsrc(a.bank.down_scales + mrow * nbi, 4 * row_bytes);
        const uint32_t lane_off = static_cast<uint32_t>(sub * nbi + kb) * 16u;
        const size_t xrow = (static_cast<size_t>(t) * P1 + r) * nbi;
        const auto xr = buffer_rsrc(a.mq.codes + xrow * 32, static_cast<uint32_t>(nbi) * 32u);
        const auto hr = buffer_rsrc(a.mq.heads + xrow, static_cast<uint32_t>(nbi) * 4u);
        uint4 w[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) w[l] = buffer_load16_nt(wr, lane_off, 4 * l * row_bytes);
        const uint4 d4p = buffer_load16(sr, static_cast<uint32_t>(kb * 32 + sub * 8) * 2u, 0);
        uint4 m4p = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (Q41) {
            const auto mr = buffer_rsrc(a.bank.down_mins + mrow * nbi, 4 * row_bytes);
            m4p = buffer_load16(mr, static_cast<uint32_t>(kb * 32 + sub * 8) * 2u, 0);
        }
        const uint4 x0 = buffer_load16(xr, static_cast<uint32_t>(kb) * 32u, 0);
        const uint4 x1 = buffer_load16(xr, static_cast<uint32_t>(kb) * 32u, 16);
        const uint32_t hx = buffer_load4(hr, static_cast<uint32_t>(kb) * 4u, 0);
        float v = rows8_down_exact<Q41>(w, d4p, m4p, x0, x1, hx, has, lane);
        if constexpr (Spread) {
            const int j = lane & 3, kb2 = 16 + j;
            const bool has2 = kb2 < nbi;
            const int kk = has2 ? kb2 : 0;
            float sr2[2];
            const uint4 y0 = buffer_load16(xr, static_cast<uint32_t>(kk) * 32u, 0);
            const uint4 y1 = buffer_load16(xr, static_cast<uint32_t>(kk) * 32u, 16);
            const uint32_t hy = buffer_load4(hr, static_cast<uint32_t>(kk) * 4u, 0);
            uint4 wc[2];
            uint32_t dh[2], mh[2] = {0u, 0u};
            const auto mr = buffer_rsrc(Q41 ? a.bank.down_mins + mrow * nbi : a.bank.down_scales, 4 * row_bytes);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int rr = 16 * u + (lane >> 2);   // row within the slice
                wc[u] = buffer_load16_nt(wr, static_cast<uint32_t>(rr) * row_bytes + static_cast<uint32_t>(kk) * 16u, 0);
                // Scale plane: [32-row group][block][32 halves], row r at half (r & 3) * 8 + r / 4.
                const uint32_t hi = static_cast<uint32_t>(kk * 32 + (rr & 3) * 8 + (rr >> 2));
                const uint32_t dw = buffer_load4(sr, (hi >> 1) * 4u, 0);
                dh[u] = (hi & 1) ? dw >> 16 : dw & 0xffffu;
                if constexpr (Q41) {
                    const uint32_t mw = buffer_load4(mr, (hi >> 1) * 4u, 0);
                    mh[u] = (hi & 1) ? mw >> 16 : mw & 0xffffu;
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                float n = down_chunk<Q41>(wc[u], dh[u], mh[u], y0, y1, hy, has2);
                n = n + lane_xor<1>(n);
                sr2[u] = n + lane_xor<2>(n);
            }
            // This lane's first-tree row (meaningful where lane & 8 == 0): 4 lr + sub.
            const int lr = 4 * (lane & 1) + 2 * ((lane >> 1) & 1) + ((lane >> 2) & 1);
            const int row = 4 * lr + (lane >> 4);
            const int src = 4 * (row & 15);
            const float a0 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src, __float_as_int(sr2[0])));
            const float a1 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src, __float_as_int(sr2[1])));
            v = v + ((row >> 4) ? a1 : a0);
        } else if constexpr (Two) {
            const bool has2 = kl + 16 < nbi;
            const int kb2 = has2 ? kl + 16 : 0;
            const uint32_t lane_off2 = static_cast<uint32_t>(sub * nbi + kb2) * 16u;
            uint4 w2[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) w2[l] = buffer_load16_nt(wr, lane_off2, 4 * l * row_bytes);
            const uint4 d4p2 = buffer_load16(sr, static_cast<uint32_t>(kb2 * 32 + sub * 8) * 2u, 0);
            uint4 m4p2 = make_uint4(0u, 0u, 0u, 0u);
            if constexpr (Q41) {
                const auto mr = buffer_rsrc(a.bank.down_mins + mrow * nbi, 4 * row_bytes);
                m4p2 = buffer_load16(mr, static_cast<uint32_t>(kb2 * 32 + sub * 8) * 2u, 0);
            }
            const uint4 y0 = buffer_load16(xr, static_cast<uint32_t>(kb2) * 32u, 0);
            const uint4 y1 = buffer_load16(xr, static_cast<uint32_t>(kb2) * 32u, 16);
            const uint32_t hy = buffer_load4(hr, static_cast<uint32_t>(kb2) * 4u, 0);
            v = v + rows8_down_exact<Q41>(w2, d4p2, m4p2, y0, y1, hy, has2, lane);
        }
        const int lr = 4 * (lane & 1) + 2 * ((lane >> 1) & 1) + ((lane >> 2) & 1);
        if ((lane & 8) == 0) part[r][4 * lr + sub] = v;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int row = threadIdx.x;
        int flags = 0;
        float v = 0.0f;
        for (int q = 0; q < k; ++q) {
            if (!valid[q]) continue;
            float x = part[q][row];
            float s = wt[q];
            if (!isfinite(x)) { flags |= 1; x = 0.0f; }
            if (!isfinite(s)) { flags |= 1; s = 0.0f; }
            float p = s * x;
            if (!isfinite(p)) { flags |= 2; p = 0.0f; }
            v = v + p;
            if (!isfinite(v)) { flags |= 2; v = 0.0f; }
        }
        // The routed fold writes 0 on a flag, and the shared add starts from
        // that value with flags of its own (two kernels in the reference).
        if (flags) v = 0.0f;
        int sflags = 0;
        if (P1 > k) {
            float x = part[k][row];
            if (!isfinite(x)) { sflags |= 1; x = 0.0f; }
            float scale = 1.0f;
            if (d.shared_gate) {
                float g = wt[k];
                if (!isfinite(g)) { sflags |= 1; g = 0.0f; }
                scale = 1.0f / (1.0f + moe_expf(-g));
                if (!isfinite(scale)) { sflags |= 2; scale = 0.0f; }
            }
            float p = scale * x;
            if (!isfinite(p)) { sflags |= 2; p = 0.0f; }
            v = v + p;
            if (!isfinite(v)) { sflags |= 2; v = 0.0f; }
        }
        d.y[static_cast<size_t>(t) * H + row0 + row] = sflags ? 0.0f : v;
        if (flags | sflags) atomicOr(a.error, flags | sflags);
    }
}

// One thread per (pair, block, word): canonical Q8_1 block words of decode
// row t * P1 + r written at the pair's grouped position.
__global__ __launch_bounds__(256) void k_decode_middle_grouped(Act mq, RouteOut routes, Shape sh, int tokens,
                                                               uint32_t *q8) {
    const int P1 = sh.k + (sh.Ep > sh.E ? 1 : 0), nbi = sh.I / 32;
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(tokens) * P1 * nbi * 9) return;
    const size_t word = i % 9, blk = (i / 9) % nbi, pair = i / 9 / nbi;
    const int t = static_cast<int>(pair / P1), r = static_cast<int>(pair % P1);
    const int pos = r < sh.k ? routes.pos_of[static_cast<size_t>(t) * sh.k + r] : routes.offsets[sh.E] + t;
    if (pos < 0) return;
    const size_t src = pair * nbi + blk;
    const uint32_t v = word == 0 ? mq.heads[src] : reinterpret_cast<const uint32_t *>(mq.codes)[src * 8 + word - 1];
    q8[(static_cast<size_t>(pos) * nbi + blk) * 9 + word] = v;
}

// ------------------------------------------------------------------ fold ---
// y = +0; y = y + (w_r * c_r) for r = 0..k-1 (separately rounded, rank
// order); then y = y + scale * shared with scale = 1/(1+expf(-g)) or 1 (moe_expf).
// Nonfinite operands set bit 1, nonfinite results bit 2; the routed fold's
// flags zero its value (src/hip/session_ops.hip:307-324) before the shared
// add, whose own flags zero the output (:375-391).  Pairs that could not
// be grouped (pos_of < 0: bad id / duplicate, already flagged) contribute 0.
// V consecutive elements per thread (V = 4: 16-byte loads when every row is
// 16-byte aligned); each element is folded on its own, exactly as above.
template<int V>
__global__ __launch_bounds__(256) void k_fold(const float *__restrict__ c, size_t token_stride,
                                              const float *__restrict__ w, int k, const int32_t *pos_of,
                                              const float *__restrict__ shared, size_t shared_stride,
                                              const float *__restrict__ shared_gate, int tokens, int H,
                                              float *__restrict__ y, int *error) {
    const size_t i = (static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x) * V;
    if (i >= static_cast<size_t>(tokens) * H) return;
    const size_t t = i / H, h = i % H;   // H % V == 0: the V elements share a token
    auto load = [](const float *p, float (&out)[V]) {
        if constexpr (V == 4) {
            // Each contribution is read once: nontemporal loads (16K layer
            // 338 -> 288 us for this kernel).
            typedef float f4v __attribute__((ext_vector_type(4)));
            const f4v q = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
            out[0] = q[0]; out[1] = q[1]; out[2] = q[2]; out[3] = q[3];
        } else {
            out[0] = *p;
        }
    };
    int flags[V] = {};
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = 0.0f;
    // Ranks are taken 8 at a time: all loads of a chunk are issued before the
    // sequential (rank-order) accumulation.  Rows of ungrouped pairs are read
    // but not used.
    for (int r0 = 0; r0 < k; r0 += 8) {
        float xs[8][V], ws[8];
        bool use[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = r0 + q;
            const bool in = r < k;
            use[q] = in && (!pos_of || pos_of[t * k + r] >= 0);
            if (in) load(c + t * token_stride + static_cast<size_t>(r) * H + h, xs[q]);
            ws[q] = in ? w[t * k + r] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (!use[q]) continue;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                float x = xs[q][e], s = ws[q];
                if (!isfinite(x)) { flags[e] |= 1; x = 0.0f; }
                if (!isfinite(s)) { flags[e] |= 1; s = 0.0f; }
                float p = s * x;
                if (!isfinite(p)) { flags[e] |= 2; p = 0.0f; }
                v[e] = v[e] + p;
                if (!isfinite(v[e])) { flags[e] |= 2; v[e] = 0.0f; }
            }
        }
    }
    // The routed fold's value is 0 where it raised a flag; the shared add
    // starts from it with flags of its own and zeroes only on those (the
    // reference runs these as two kernels).
    int sflags[V] = {};
#pragma unroll
    for (int e = 0; e < V; ++e)
        if (flags[e]) v[e] = 0.0f;
    if (shared) {
        float xsh[V];
        load(shared + t * shared_stride + h, xsh);
        float scale = 1.0f;
        int gflags = 0;
        if (shared_gate) {
            float g = shared_gate[t];
            if (!isfinite(g)) { gflags |= 1; g = 0.0f; }
            scale = 1.0f / (1.0f + moe_expf(-g));
            if (!isfinite(scale)) { gflags |= 2; scale = 0.0f; }
        }
#pragma unroll
        for (int e = 0; e < V; ++e) {
            float x = xsh[e];
            sflags[e] |= gflags;
            if (!isfinite(x)) { sflags[e] |= 1; x = 0.0f; }
            float p = scale * x;
            if (!isfinite(p)) { sflags[e] |= 2; p = 0.0f; }
            v[e] = v[e] + p;
            if (!isfinite(v[e])) { sflags[e] |= 2; v[e] = 0.0f; }
        }
    }
    int any = 0;
#pragma unroll
    for (int e = 0; e < V; ++e) {
        y[i + e] = sflags[e] ? 0.0f : v[e];
        any |= flags[e] | sflags[e];
    }
    if (any) atomicOr(error, any);
}

// ---------------------------------------------------------------- router ---
// One token row per wave (a 64-thread workgroup), no barriers: lane L holds
// the logits of experts L + 64 j, j < J = ceil(E / 64).
//
// Softmax as router_softmax (src/hip/session_ops.hip:401-434), whose 32 lanes
// hold logits l + 32k: nonfinite inputs count as 0 with bit 1; row max (any
// order gives the same max); e = expf(x - max); reference lane l's total is
// the left sum from +0 of e[l + 32k] over k, then an ascending XOR butterfly
// 1..16 across the 32 totals; reciprocal and multiply; any flag zeroes the
// row.  Entry l + 32k sits on lane l (k even, j = k / 2) or lane l + 32 (k
// odd), so a permlane32 swap hands lane l < 32 every entry of its reference
// lane and it adds them in the reference's order.  The reference checks every
// partial sum; its addends are finite and >= 0 (sanitised exponentials), so
// partial sums only grow and the last one is nonfinite exactly when one of
// them is: checking the lane total raises the same bit.  e * (1 / total)
// cannot become nonfinite when no flag is set (e <= 1 <= total), and any flag
// zeroes the row, so that check adds nothing.
//
// Selection as select_routes (src/session.hip:666-687): the top_k largest
// probabilities, ties to the lower id.  Entry i's key is the integer
// bits(p) * 1024 + (1023 - i) held in a double (below 2^40, so exact): p >= +0
// makes bits(p) order like p, so larger keys are larger p, then lower id, and
// the keys of a row are distinct.  A key's rank is the number of larger keys,
// counted from the sign of the exact difference key_i - key_j (no
// compare-and-carry chain through VCC).  Bound: the lanes' largest keys are
// ranked among themselves; the one of rank top_k - 1 has top_k keys (the
// larger lane maxima and itself) at or above it, so the row's top_k all lie
// at or above it, and only the keys at or above it (at most top_k * J) are
// ranked among themselves.  Then, in rank order, bucket id % 32 accumulates p
// from +0, an ascending XOR butterfly, denominator max(bucket 0, 1/16384),
// weight = p * (1 / denominator).  expf is moe_expf (the host C library's
// bits).
constexpr int kRouterMaxTopK = 32;
constexpr int kRouterMaxJ = 16;      // experts <= 1024
constexpr int kRouterBatch = 16;     // keys read from LDS per round trip

// Branch-free (selects, no exec-mask branches on the router's serial path).
__device__ __forceinline__ float router_check(float x, int &flags, int bit) {
    const bool bad = !isfinite(x);
    flags |= bad ? bit : 0;
    return bad ? 0.0f : x;
}

__device__ __forceinline__ double router_key(float p, int id) {
    return static_cast<double>(__float_as_uint(p)) * 1024.0 + static_cast<double>(1023 - id);
}
// 1 when key j > key i: the sign bit of the exact difference (x - x = +0).
__device__ __forceinline__ uint32_t router_larger(double ki, double kj) {
    return static_cast<uint32_t>(__double_as_longlong(ki - kj) >> 32) >> 31;
}

// How many of the n keys at `keys` (LDS, 16-byte aligned; the entries up to
// the next multiple of B are readable and hold -1) are larger than k: B keys
// per LDS round trip.
template<int B>
__device__ __forceinline__ int router_rank(double k, const double *keys, int n) {
    uint32_t c = 0;
#pragma unroll 1
    for (int j = 0; j < n; j += B) {
        double v[B];
#pragma unroll
        for (int i = 0; i < B; ++i) v[i] = keys[j + i];
#pragma unroll
        for (int i = 0; i < B; i += 2) c += router_larger(k, v[i]) + router_larger(k, v[i + 1]);
    }
    return static_cast<int>(c);
}

// Lanes below this one in a wave mask.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// LDS fence between a wave's own writes and its reads of other lanes' values.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// SPREAD: one workgroup of J waves per token row; wave w evaluates the
// exponentials of experts 64 w + lane (one each), then wave 0 alone
// continues with all of them (latency: small batches).  Otherwise one wave
// per row evaluates all J per lane, every table read issued together
// (throughput: large batches).  FULL: E == 64 J, every lane holds J entries
// (no per-lane guards).  K > 0: top_k == K (the loops over ranks end at K).
template<int J, bool FULL, bool SPREAD, int K>
__global__ __launch_bounds__(SPREAD ? 64 * J : 64) void k_router(const float *__restrict__ logits, int E, int top_k,
                                                                float *__restrict__ prob, int32_t *__restrict__ ids,
                                                                float *__restrict__ weights, int *error) {
    constexpr int KT = K > 0 ? K : kRouterMaxTopK;                       // ranks the bucket loop visits
    constexpr int NS = kRouterMaxTopK * 2 * J + kRouterBatch;            // survivor slots (+ padding)
    __shared__ uint64_t etab[32];                                        // moe_expf's table
    __shared__ float e_lds[SPREAD ? 64 * J : 1];
    __shared__ int wflags[SPREAD ? J : 1];
    __shared__ __align__(16) double lmax[32];
    __shared__ __align__(16) double surv[NS];
    __shared__ __align__(16) float top_p[kRouterMaxTopK];
    __shared__ __align__(16) int top_id[kRouterMaxTopK];
    const int t = blockIdx.x, L = threadIdx.x & 63;
    const int wave = SPREAD ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) : 0;
    const float *row = logits + static_cast<size_t>(t) * E;
    // Every wave reads the whole row (its max and input flags), lane L the
    // entries L + 64 j.
    float x[J];
#pragma unroll
    for (int j = 0; j < J; ++j) x[j] = (FULL || L + 64 * j < E) ? row[L + 64 * j] : 0.0f;
    if (wave == 0 && L < 32) etab[L] = moe_expf_table(L);
    if (wave == 0 && L >= top_k && L < kRouterMaxTopK) top_p[L] = 0.0f;   // unused ranks add +0 to the buckets
    int flags = 0;
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool has = (FULL || L + 64 * j < E);
        int f = 0;
        x[j] = router_check(x[j], f, 1);
        flags |= has ? f : 0;
        m = has ? fmaxf(m, x[j]) : m;
    }
    m = fmaxf(m, lane_xor<1>(m));
    m = fmaxf(m, lane_xor<2>(m));
    m = fmaxf(m, lane_xor<4>(m));
    m = fmaxf(m, lane_xor<8>(m));
    m = fmaxf(m, lane_xor<16>(m));
    m = fmaxf(m, lane_xor<32>(m));
    float e[J];
    if constexpr (SPREAD) {
        // This wave's entry: x[wave] without indexing the register array by
        // a runtime value.
        float xw = x[0];
#pragma unroll
        for (int j = 1; j < J; ++j) xw = wave == j ? x[j] : xw;
        const bool has = FULL || L + 64 * wave < E;
        int f = 0;
        const float shifted = router_check(has ? xw - m : 0.0f, f, 2);
        const MoeExpfReduced red = moe_expf_reduce(shifted);
        __syncthreads();   // etab
        const float ew = router_check(moe_expf_finish(shifted, red, etab[moe_expf_index(red)]), f, 2);
        flags |= has ? f : 0;
        e_lds[L + 64 * wave] = has ? ew : 0.0f;
        const bool b1 = __ballot(flags & 1) != 0, b2 = __ballot(flags & 2) != 0;
        if (L == 0) wflags[wave] = (b1 ? 1 : 0) | (b2 ? 2 : 0);
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int j = 0; j < J; ++j) e[j] = e_lds[L + 64 * j];
        flags = 0;
#pragma unroll
        for (int j = 0; j < J; ++j) flags |= wflags[j];
    } else {
        float sh[J];
        MoeExpfReduced red[J];
        uint64_t ent[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool has = (FULL || L + 64 * j < E);
            int f = 0;
            sh[j] = router_check(has ? x[j] - m : 0.0f, f, 2);
            flags |= has ? f : 0;
            red[j] = moe_expf_reduce(sh[j]);
        }
        wave_lds_sync();   // etab
#pragma unroll
        for (int j = 0; j < J; ++j) ent[j] = etab[moe_expf_index(red[j])];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool has = (FULL || L + 64 * j < E);
            int f = 0;
            e[j] = router_check(moe_expf_finish(sh[j], red[j], ent[j]), f, 2);
            flags |= has ? f : 0;
            e[j] = has ? e[j] : 0.0f;
        }
    }
    // Reference lane l = L & 31 (lanes >= 32 repeat it): left sum of
    // e[l + 32k] over k < E / 32; odd k come from lane l + 32.
    float total = 0.0f;
    {
        float o[J];
#pragma unroll
        for (int j = 0; j < J; ++j) o[j] = lane_xor<32>(e[j]);
        const bool lo = L < 32;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            total = total + (lo ? e[j] : o[j]);                                          // k = 2j
            if (FULL || 32 * (2 * j + 1) < E) total = total + (lo ? o[j] : e[j]);   // k = 2j + 1
        }
    }
    total = router_check(total, flags, 2);
    total = total + lane_xor<1>(total);
    total = total + lane_xor<2>(total);
    total = total + lane_xor<4>(total);
    total = total + lane_xor<8>(total);
    total = total + lane_xor<16>(total);
    total = router_check(total, flags, 2);
    if (!(total > 0.0f)) flags |= 2;
    const float inverse = total > 0.0f ? router_check(1.0f / total, flags, 2) : 0.0f;
    const int rflags = (__ballot(flags & 1) != 0 ? 1 : 0) | (__ballot(flags & 2) != 0 ? 2 : 0);
    double key[J];
    double kmax = -1.0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = L + 64 * j;
        const bool has = FULL || i < E;
        const float p = rflags ? 0.0f : e[j] * inverse;
        if (prob && has) prob[static_cast<size_t>(t) * E + i] = p;
        key[j] = has ? router_key(p, i) : -1.0;
        kmax = fmax(kmax, key[j]);
    }
    // The bound: the largest key of lanes 2g, 2g + 1 is ranked among the 32
    // pair maxima; the one of rank top_k - 1 has top_k keys (the larger pair
    // maxima and itself) at or above it, so the row's top_k all lie at or
    // above it.  With fewer than top_k nonempty pairs every key is kept.
    kmax = fmax(kmax, __hiloint2double(lane_xor<1>(__double2hiint(kmax)), lane_xor<1>(__double2loint(kmax))));
    if ((L & 1) == 0) lmax[L >> 1] = kmax;
    wave_lds_sync();
    double bound = -0.5;
    if (FULL || (min(E, 64) + 1) / 2 >= top_k) {   // uniform
        const int r = router_rank<32>(kmax, lmax, 32);
        const uint64_t at = __ballot((L & 1) == 0 && kmax >= 0.0 && r == top_k - 1);
        const int src = static_cast<int>(__builtin_ctzll(at));
        const int blo = __builtin_amdgcn_readlane(__double2loint(kmax), src);
        const int bhi = __builtin_amdgcn_readlane(__double2hiint(kmax), src);
        bound = __hiloint2double(bhi, blo);
    }
    // Survivors (the keys at or above the bound: at most 2 J per selected
    // pair) into surv[0..ns); other lanes write to the last padding slot.
    int ns = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint64_t keep = __ballot(key[j] >= bound);
        surv[((keep >> L) & 1) ? ns + lanes_below(keep) : NS - 1] = key[j];
        ns += __popcll(keep);
    }
    wave_lds_sync();
    if (L < kRouterBatch) surv[ns + L] = -1.0;   // padding of the last batch
    wave_lds_sync();
    for (int c0 = 0; c0 < ns; c0 += 64) {
        const double k = surv[min(c0 + L, ns + kRouterBatch - 1)];   // lanes past ns read padding
        const int r = router_rank<kRouterBatch>(k, surv, ns);
        if (c0 + L < ns && r < top_k) {
            const int64_t bits = static_cast<int64_t>(k);
            top_p[r] = __uint_as_float(static_cast<uint32_t>(bits >> 10));
            top_id[r] = 1023 - static_cast<int>(bits & 1023);
        }
    }
    wave_lds_sync();
    // Bucket l of select_routes: p of the ids with id % 32 == l, in rank
    // order from +0 (another bucket's entry, or an unused rank, whose p is
    // +0, adds +0, which changes nothing).
    const int l = L & 31;
    float tp[KT];
    int ti[KT];
#pragma unroll
    for (int i = 0; i < KT; ++i) {
        tp[i] = top_p[i];
        ti[i] = top_id[i];
    }
    const float my_p = top_p[min(L, kRouterMaxTopK - 1)];
    const int my_id = top_id[min(L, kRouterMaxTopK - 1)];
    float bucket = 0.0f;
#pragma unroll
    for (int i = 0; i < KT; ++i) bucket = bucket + ((ti[i] & 31) == l ? tp[i] : 0.0f);
    bucket = bucket + lane_xor<1>(bucket);
    bucket = bucket + lane_xor<2>(bucket);
    bucket = bucket + lane_xor<4>(bucket);
    bucket = bucket + lane_xor<8>(bucket);
    bucket = bucket + lane_xor<16>(bucket);
    bucket = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__float_as_int(bucket)));   // bucket 0
    const float lowest = 1.0f / 16384.0f;
    const float denominator = bucket < lowest ? lowest : bucket;
    const int dflags = (!(denominator > 0.0f) || !isfinite(denominator)) ? 2 : 0;
    const float dinv = dflags ? 0.0f : 1.0f / denominator;
    if (L < top_k) {
        const size_t o = static_cast<size_t>(t) * top_k + L;
        ids[o] = my_id;
        weights[o] = my_p * dinv;
    }
    if (L == 0 && (rflags | dflags)) atomicOr(error, rflags | dflags);
}

// Batches of at most kRouterSpreadTokens rows spread each row's
// exponentials over J waves (lower latency); larger batches run one wave per
// row (more rows resident).  Measured on MI355X (graph replays, E = 512,
// top-10), spread against one wave per row: 256 rows 3.99 vs 4.49 us (257),
// 512 rows 4.49 vs 4.67 us, 1024 rows 5.35 vs 4.95 us, 4096 rows 13.2 vs
// 7.8 us.
constexpr int kRouterSpreadTokens = 512;

template<int J>
void router_launch(const float *logits, int tokens, int experts, int top_k, float *prob, int32_t *ids,
                   float *weights, int *error, hipStream_t s) {
    const bool spread = tokens <= kRouterSpreadTokens;
    if constexpr (J == 8) {
        if (experts == 512 && top_k == 10) {   // the model's router: 512 experts, top-10
            if (spread) k_router<8, true, true, 10><<<tokens, 512, 0, s>>>(logits, experts, top_k, prob, ids, weights, error);
            else k_router<8, true, false, 10><<<tokens, 64, 0, s>>>(logits, experts, top_k, prob, ids, weights, error);
            return;
        }
    }
    if (spread) k_router<J, false, true, 0><<<tokens, 64 * J, 0, s>>>(logits, experts, top_k, prob, ids, weights, error);
    else k_router<J, false, false, 0><<<tokens, 64, 0, s>>>(logits, experts, top_k, prob, ids, weights, error);
}

inline unsigned blocks_for(size_t n, unsigned per) { return static_cast<unsigned>((n + per - 1) / per); }

}  // namespace

// -------------------------------------------------------------- launchers ---
hipError_t launch_quantize_canonical(const float *x, void *q8, int width, int columns, int *error,
                                     hipStream_t s) {
    const size_t n = static_cast<size_t>(width) * columns;
    k_quantize<true><<<blocks_for(n, 256), 256, 0, s>>>(x, static_cast<uint8_t *>(q8), nullptr, n, error);
    return hipGetLastError();
}

hipError_t launch_quantize_planes(const float *x, Act out, int width, int columns, int *error,
                                  hipStream_t s) {
    const size_t n = static_cast<size_t>(width) * columns;
    k_quantize<false><<<blocks_for(n, 256), 256, 0, s>>>(x, out.codes, out.heads, n, error);
    return hipGetLastError();
}

hipError_t launch_canonical_to_planes(const void *q8, Act out, int blocks, hipStream_t s) {
    const size_t n = static_cast<size_t>(blocks) * 9;
    k_canonical_to_planes<<<blocks_for(n, 256), 256, 0, s>>>(static_cast<const uint8_t *>(q8), out.codes,
                                                              out.heads, static_cast<size_t>(blocks));
    return hipGetLastError();
}

hipError_t launch_planes_to_canonical(Act in, void *q8, int blocks, hipStream_t s) {
    const size_t n = static_cast<size_t>(blocks) * 9;
    k_planes_to_canonical<<<blocks_for(n, 256), 256, 0, s>>>(in.codes, in.heads, static_cast<uint8_t *>(q8),
                                                              static_cast<size_t>(blocks));
    return hipGetLastError();
}

hipError_t launch_repack_weights(const uint8_t *canonical, uint8_t *codes, uint16_t *scales, uint16_t *mins,
                                 size_t blocks,
                                 size_t block0, int blocks_per_row, int group, hipStream_t s) {
    k_repack<<<blocks_for(blocks, 256), 256, 0, s>>>(reinterpret_cast<const uint16_t *>(canonical),
                                                      reinterpret_cast<uint32_t *>(codes), scales, mins, blocks,
                                                      block0, blocks_per_row, group);
    return hipGetLastError();
}

hipError_t launch_unpack_weights(const uint8_t *codes, const uint16_t *scales, const uint16_t *mins,
                                 uint8_t *canonical, size_t blocks,
                                 size_t block0, int blocks_per_row, int group, hipStream_t s) {
    k_unpack<<<blocks_for(blocks, 256), 256, 0, s>>>(reinterpret_cast<const uint32_t *>(codes), scales, mins,
                                                      reinterpret_cast<uint16_t *>(canonical), blocks, block0,
                                                      blocks_per_row, group);
    return hipGetLastError();
}

hipError_t launch_synthetic_weights(uint8_t *codes, uint16_t *scales, uint16_t *mins, size_t blocks, size_t hash0,
                                    int blocks_per_row, int group, uint64_t seed, hipStream_t s) {
    k_synthetic<<<blocks_for(blocks, 256), 256, 0, s>>>(reinterpret_cast<uint32_t *>(codes), scales, mins, blocks,
                                                         hash0, blocks_per_row, group, seed);
    return hipGetLastError();
}

hipError_t launch_read_probe(const void *p, size_t bytes, uint32_t *sink, hipStream_t s) {
    const size_t n = bytes / 16;
    const unsigned grid = 4096;   // best of 256..8192 for 45-180 MiB on MI355X
    const size_t chunk = (n + grid - 1) / grid;
    k_read_probe<<<grid, 512, 0, s>>>(static_cast<const uint4 *>(p), n, chunk, 0x9e3779b9u, sink);
    return hipGetLastError();
}

hipError_t launch_expf(const float *x, float *y, int n, hipStream_t s) {
    k_expf<<<blocks_for(static_cast<size_t>(n), 256), 256, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t *p, uint32_t value, size_t count, hipStream_t s) {
    if (count == 0) return hipSuccess;
    k_fill_u32<<<blocks_for(count, 256), 256, 0, s>>>(p, value, count);
    return hipGetLastError();
}

hipError_t launch_prepare(const float *x, const int32_t *ids, const float *weights, int tokens, Shape shape,
                          Act xq, RouteOut routes, int mfma_min, int *error, hipStream_t s) {
    GroupParams p{ids, weights, tokens, shape, routes, mfma_min, error};
    // Grouping alone (x == nullptr, as moe_ffn_group_routes calls it) launches
    // no quantization blocks: they would read x.
    const size_t q_elements = x ? static_cast<size_t>(tokens) * shape.H : 0;
    const int W = (tokens + 31) / 32;
    const size_t small_lds = (static_cast<size_t>(shape.E) * W * 2 + static_cast<size_t>(shape.Ep) * 4 + 1 + 17 +
                              static_cast<size_t>(tokens) * shape.k) * 4;
    if (tokens <= kSmallGroupTokens && small_lds <= 60 * 1024 && tokens * shape.k <= 32 * 1024) {
        k_prepare_small<<<1 + blocks_for(q_elements, 1024), 1024, small_lds, s>>>(p, x, xq, q_elements);
        return hipGetLastError();
    }
    hipError_t e = launch_fill_u32(routes.bitmap, 0u, static_cast<size_t>(W) * shape.Ep, s);
    if (e != hipSuccess) return e;
    const int mark_blocks = static_cast<int>(blocks_for(static_cast<size_t>(tokens), 256));
    const size_t id_lds = static_cast<size_t>(256) * shape.k * 4;
    k_mark_quantize<<<mark_blocks + blocks_for(q_elements, 256 * kQuantPer), 256, id_lds, s>>>(p, mark_blocks, x, xq,
                                                                                           q_elements);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    k_word_prefix<<<blocks_for(static_cast<size_t>(shape.E), 4), 256, 0, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t lds = (static_cast<size_t>(shape.Ep) * 4 + 1 + 17) * 4;
    k_offsets_items<<<1, 1024, lds, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    k_scatter_pairs<<<blocks_for(static_cast<size_t>(tokens), 256), 256, id_lds, s>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t pairs = static_cast<size_t>(tokens) * (shape.k + (shape.Ep > shape.E ? 1 : 0));
    const size_t item_bound = pairs / kStreamTokens + std::min<size_t>(pairs, shape.Ep);
    k_item_tokens<<<blocks_for(item_bound, 256), 256, 0, s>>>(routes);
    return hipGetLastError();
}

hipError_t launch_single_expert_items(Shape shape, RouteOut routes, int expert, int columns, int use_mfma,
                                      hipStream_t s) {
    k_single_items<<<1, 256, 0, s>>>(shape, routes, expert, columns, use_mfma);
    return hipGetLastError();
}

namespace {
// Upper bound on streaming items (the size the item array is allocated for):
// one partial item per nonempty group plus full items.
// Upper bound on the streaming items the device can produce: a group of n
// pairs gives ceil(n / 4) items, so at most one partial item per nonempty
// group plus full items; with mfma_min >= 2 only groups of < mfma_min pairs
// stream, each giving at most ceil((mfma_min - 1) / 4) items.
unsigned stream_item_bound(const FfnArgs &a) {
    const size_t P = static_cast<size_t>(a.pairs_bound);
    const size_t G = std::min(P, static_cast<size_t>(a.shape.Ep));
    size_t b = P / kStreamTokens + G;
    if (a.mfma_min >= 2) b = std::min(b, G * ((a.mfma_min - 1 + kStreamTokens - 1) / kStreamTokens));
    return static_cast<unsigned>(std::max<size_t>(b, 1));
}

// Grid of a lean streaming launch (k_gate_up_lean, k_down_lean): one
// workgroup per unit of the item bound, capped at kLeanGridCap rounded down to
// a multiple of 8 x slices (the kernels loop over units id, id + grid, ...).
// The bound holds for any grouping, so a batch whose groups all go to MFMA
// would otherwise start up to ~10^5 workgroups that find no item.  Measured
// per layer (2048/512, 512 experts), cap 8192 / 16384 / 32768 / none, us:
// 1032 uniform tokens 1160 / 1125 / 1090 / 1105, 1032 Zipf(1.3) 680 / 684 /
// 705 / 755, 4K Zipf(1.1) 1867 / 1856 / 1867 / 1926, 16K uniform 5338 /
// 5334 / 5338 / 5436.
constexpr unsigned kLeanGridCap = 16384;
unsigned lean_grid(unsigned item_bound, unsigned slices) {
    const size_t units = static_cast<size_t>(item_bound) * slices;
    const unsigned step = 8u * slices;
    const unsigned cap = std::max(step, kLeanGridCap / step * step);
    return units < cap ? static_cast<unsigned>(units) : cap;
}

unsigned stream_grid(const FfnArgs &a, int slices) {
    // The persistent loop covers whatever the device produced.
    const size_t units = static_cast<size_t>(stream_item_bound(a)) * slices;
    return static_cast<unsigned>(std::min<size_t>(units, 4096));
}
}  // namespace

template<int NBL>
void gate_up_stream(const FfnArgs &a, bool dbg, unsigned grid, hipStream_t s) {
    if (dbg) k_gate_up_stream<NBL, true><<<grid, 512, 0, s>>>(a);
    else k_gate_up_stream<NBL, false><<<grid, 512, 0, s>>>(a);
}

hipError_t launch_gate_up(const FfnArgs &a, bool mfma, hipStream_t s) {
    if (mfma) return launch_gate_up_mfma(a, s);
    const bool dbg = a.middle_f32 || a.gate_dots || a.up_dots;
    const unsigned grid = stream_grid(a, a.shape.I / 32);
    const int nbl = (a.shape.H / 32 + 63) / 64;
    if (nbl <= 2) {
        // One unit per workgroup; grid = item bound x slices, extra items exit.
        const unsigned lgrid = lean_grid(stream_item_bound(a), static_cast<unsigned>(a.shape.I / 32));
        if (nbl == 2) {
            if (dbg) k_gate_up_lean<false, true, true><<<lgrid, 512, 0, s>>>(a);
            else if (a.shape.H <= 80 * 32) k_gate_up_lean<false, true, false, true><<<lgrid, 512, 0, s>>>(a);
            else k_gate_up_lean<false, true, false><<<lgrid, 512, 0, s>>>(a);
        } else if (dbg) k_gate_up_lean<false, false, true><<<lgrid, 512, 0, s>>>(a);
        else if (a.shape.H == 2048) k_gate_up_lean<true, false, false><<<lgrid, 512, 0, s>>>(a);
        else k_gate_up_lean<false, false, false><<<lgrid, 512, 0, s>>>(a);
    } else gate_up_stream<0>(a, dbg, grid, s);
    return hipGetLastError();
}

// Grids cover 8 XCD lanes x ceil(slices / 8) x the other dimensions (the
// kernels map a linear id to (token, rank, slice) and skip slices past the end).
hipError_t launch_decode_gate_up(const DecodeArgs &d, hipStream_t s) {
    const Shape &sh = d.f.shape;
    const int P1 = sh.k + (sh.Ep > sh.E ? 1 : 0);
    const unsigned groups = static_cast<unsigned>((sh.I / 32 + 7) / 8);
    const unsigned grid = 8u * groups * P1 * d.f.tokens;
    const bool full = sh.H == 2048, two = sh.H > 2048, spread = two && sh.H <= 80 * 32;
    if (d.x_q8) {
        if (spread) k_decode_gate_up<true, false, true, true><<<grid, 512, 0, s>>>(d);
        else if (two) k_decode_gate_up<true, false, true><<<grid, 512, 0, s>>>(d);
        else if (full) k_decode_gate_up<true, true, false><<<grid, 512, 0, s>>>(d);
        else k_decode_gate_up<true, false, false><<<grid, 512, 0, s>>>(d);
    } else {
        if (spread) k_decode_gate_up<false, false, true, true><<<grid, 512, 0, s>>>(d);
        else if (two) k_decode_gate_up<false, false, true><<<grid, 512, 0, s>>>(d);
        else if (full) k_decode_gate_up<false, true, false><<<grid, 512, 0, s>>>(d);
        else k_decode_gate_up<false, false, false><<<grid, 512, 0, s>>>(d);
    }
    return hipGetLastError();
}

hipError_t launch_decode_down_fold(const DecodeArgs &d, hipStream_t s) {
    const Shape &sh = d.f.shape;
    const int P1 = sh.k + (sh.Ep > sh.E ? 1 : 0);
    const unsigned groups = static_cast<unsigned>((sh.H / 32 + 7) / 8);
    const dim3 grid(8u * groups * d.f.tokens), block(64 * P1);
    const bool two = sh.I > 512, spread = two && sh.I <= 20 * 32;
    if (d.f.bank.down_mins) {
        if (spread) k_decode_down_fold<true, true, true><<<grid, block, 0, s>>>(d);
        else if (two) k_decode_down_fold<true, true><<<grid, block, 0, s>>>(d);
        else k_decode_down_fold<true, false><<<grid, block, 0, s>>>(d);
    } else {
        if (spread) k_decode_down_fold<false, true, true><<<grid, block, 0, s>>>(d);
        else if (two) k_decode_down_fold<false, true><<<grid, block, 0, s>>>(d);
        else k_decode_down_fold<false, false><<<grid, block, 0, s>>>(d);
    }
    return hipGetLastError();
}

hipError_t launch_decode_middle_grouped(Act mq, RouteOut routes, Shape shape, int tokens, void *q8, hipStream_t s) {
    const int P1 = shape.k + (shape.Ep > shape.E ? 1 : 0);
    const size_t n = static_cast<size_t>(tokens) * P1 * (shape.I / 32) * 9;
    k_decode_middle_grouped<<<blocks_for(n, 256), 256, 0, s>>>(mq, routes, shape, tokens, static_cast<uint32_t *>(q8));
    return hipGetLastError();
}

hipError_t launch_down(const FfnArgs &a, bool mfma, hipStream_t s) {
    if (mfma) return launch_down_mfma(a, s);   // Q4_0 and Q4_1 down rows
    const int nbi = a.shape.I / 32;
    const unsigned grid = stream_grid(a, a.shape.H / 32);   // k_down_stream's units: 32-row slices
    const bool dbg = a.down_dots != nullptr, q41 = a.bank.down_mins != nullptr;
    if (nbi <= 16) {
        const unsigned g = lean_grid(stream_item_bound(a), static_cast<unsigned>(a.shape.H / 64));
        if (q41) {
            if (dbg) k_down_lean<0, true, false, true><<<g, 128, 0, s>>>(a);
            else if (nbi == 16) k_down_lean<16, true, false, false><<<g, 128, 0, s>>>(a);
            else k_down_lean<0, true, false, false><<<g, 128, 0, s>>>(a);
        } else {
            if (dbg) k_down_lean<0, false, false, true><<<g, 128, 0, s>>>(a);
            else if (nbi == 16) k_down_lean<16, false, false, false><<<g, 128, 0, s>>>(a);
            else k_down_lean<0, false, false, false><<<g, 128, 0, s>>>(a);
        }
    } else if (nbi <= 32) {
        const unsigned g = lean_grid(stream_item_bound(a), static_cast<unsigned>(a.shape.H / 64));
        const bool spread = nbi <= 20;
        if (q41) {
            if (dbg) k_down_lean<0, true, true, true><<<g, 128, 0, s>>>(a);
            else if (spread) k_down_lean<0, true, true, false, true><<<g, 128, 0, s>>>(a);
            else k_down_lean<0, true, true, false><<<g, 128, 0, s>>>(a);
        } else {
            if (dbg) k_down_lean<0, false, true, true><<<g, 128, 0, s>>>(a);
            else if (spread) k_down_lean<0, false, true, false, true><<<g, 128, 0, s>>>(a);
            else k_down_lean<0, false, true, false><<<g, 128, 0, s>>>(a);
        }
    } else if (q41) {
        if (dbg) k_down_stream<true, true><<<grid, 512, 0, s>>>(a);
        else k_down_stream<true, false><<<grid, 512, 0, s>>>(a);
    } else {
        if (dbg) k_down_stream<false, true><<<grid, 512, 0, s>>>(a);
        else k_down_stream<false, false><<<grid, 512, 0, s>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_router(const float *logits, int tokens, int experts, int top_k, float *prob, int32_t *ids,
                         float *weights, int *error, hipStream_t s) {
    using Launch = void (*)(const float *, int, int, int, float *, int32_t *, float *, int *, hipStream_t);
    static constexpr Launch table[kRouterMaxJ] = {
        router_launch<1>, router_launch<2>, router_launch<3>, router_launch<4>, router_launch<5>, router_launch<6>,
        router_launch<7>, router_launch<8>, router_launch<9>, router_launch<10>, router_launch<11>,
        router_launch<12>, router_launch<13>, router_launch<14>, router_launch<15>, router_launch<16>};
    if (top_k > kRouterMaxTopK || experts > 64 * kRouterMaxJ) return hipErrorInvalidValue;
    table[(experts + 63) / 64 - 1](logits, tokens, experts, top_k, prob, ids, weights, error, s);
    return hipGetLastError();
}

hipError_t launch_fold(const float *contributions, size_t token_stride, const float *weights, int k,
                       const int32_t *pos_of, const float *shared, size_t shared_stride,
                       const float *shared_gate, int tokens, int H, float *y, int *error, hipStream_t s) {
    const size_t n = static_cast<size_t>(tokens) * H;
    const auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (H % 4 == 0 && token_stride % 4 == 0 && shared_stride % 4 == 0 && a16(contributions) &&
        (!shared || a16(shared)))
        k_fold<4><<<blocks_for(n / 4, 256), 256, 0, s>>>(contributions, token_stride, weights, k, pos_of, shared,
                                                         shared_stride, shared_gate, tokens, H, y, error);
    else
        k_fold<1><<<blocks_for(n, 256), 256, 0, s>>>(contributions, token_stride, weights, k, pos_of, shared,
                                                     shared_stride, shared_gate, tokens, H, y, error);
    return hipGetLastError();
}

}  // namespace moe
