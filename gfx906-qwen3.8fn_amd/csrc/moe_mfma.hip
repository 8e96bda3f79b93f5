// Int8-MFMA grouped expert projections for prefill-width groups (gfx950).
//
// Replaces the reference's MMQ path (src/hip/mmq.hip:139-381, mmq<Q4_0,J>) and
// the Session's MMVQ expert projections for wide groups
// (src/hip/linear.hip:156-490), with the same arithmetic contract:
//   per-block int32 dot  I = sum (qs&15)*c[i] + (qs>>4)*c[i+16]  src/quant.cpp:48-55
//   block value          d4 * (I*d8 - 8*s8)                       src/quant.cpp:88-93
//   SiLU(g)*u + Q8_1     src/hip/linear.hip:99-150, :509-525
//
// One v_mfma_i32_32x32x32_i8 is one Q4_0 block (K = 32) of a 32-row x
// 32-token tile, so its int32 results are exactly the reference's per-block
// dots.  The per-block scaling cannot be chained through the MFMA, so every
// result needs a vector epilogue; it is kept to two VALU instructions:
//   * the MFMA accumulates onto the constant 0x4B400000 (1.5 * 2^23), so the
//     result bits read as the float F = 12582912 + I exactly (|I| <= 61440);
//   * t = fma(F, d8, -12582912*d8) = round(I*d8)  (12582912*d8 is exact: d8 is
//     an fp16 value, 3*2^22 times it needs at most 13 significand bits);
//   * acc = fma(d4, t, acc) with d4 taken straight from its fp16 plane
//     (v_fma_mix_f32).
// The -8*d4*s8 terms form a [rows x blocks] x [blocks x tokens] product of
// fp16 values; one v_mfma_f32_32x32x16_f16 covers 16 blocks of it (fp16
// products are exact in fp32), and it seeds the accumulators.
//
// Work unit = (MFMA item of <= 128 grouped pairs of one expert, row slice),
// ordered item-major and dealt to the XCDs in chunks (see mfma_unit).
#include "moe_device.hpp"

#include <algorithm>
#include <type_traits>

#pragma clang fp contract(off)

namespace moe {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kSub = 32;                   // tokens per MFMA tile (N)
constexpr int kSubs = kMfmaTile / kSub;    // tiles per item
constexpr int kMagic = 0x4B400000;         // bits of 12582912.0f
constexpr float kMagicF = 12582912.0f;
constexpr uint32_t kNibbles = 0x0f0f0f0fu;

struct Unit {
    int item, slice;
    bool ok;
};

// blockIdx -> (item, slice).  Workgroup i runs on XCD i % 8; XCD x takes
// chunks of kUnitChunk consecutive units round-robin (chunk c goes to XCD
// c % 8), so the units of one item slice share an XCD while the work of the
// popular experts is spread over all XCDs.
constexpr int kUnitChunk = 4;

// The dealing permutes each round of 8 * kUnitChunk consecutive ids.  Within
// an XCD the dispatcher hands consecutive workgroups to its four shader
// engines in turn (measured: a workgroup's engine follows its position
// modulo 4 in the XCD's sequence for three quarters of them), so the unit
// at position p of chunk k is unit (p + k) % 4 of that chunk: the gate/up
// kernel's token tile `sub` (empty for the tail tiles of small items) then
// visits every engine instead of pinning the working tiles to one.
__device__ __forceinline__ int dealt_unit(int id) {
    const int n = id >> 3, x = id & 7, k = n / kUnitChunk;
    return (k * 8 + x) * kUnitChunk + (n + k) % kUnitChunk;
}

// Chunks of kGuChunkRows row slices per XCD (the gate/up kernel): the
// item-major sequence of (item, row slice) pairs is cut into chunks of
// kGuChunkRows, chunk c runs on XCD c % 8, and the activations of an item's
// token tiles, read by every row slice, are fetched into fewer L2s.  Within a
// chunk, row slice r's token tiles are rotated by r + c over the four
// positions so each engine sees every tile index.  Chunk rows, layer ms
// (2048/512, two runs each): 1 (one row slice): 4K 1.47-1.49, 16K 4.61,
// stack 26.65; 4: 1.47-1.48, 4.53-4.55, 26.56; 8: 1.46-1.47, 4.51-4.56,
// 26.90; 16 (whole items): 1.48-1.50, 4.52, 27.7 (items dealt whole leave
// the XCDs unevenly loaded on the stack's 1,032-token layers).
constexpr int kGuChunkRows = 4;
constexpr int kGuChunk = kGuChunkRows * kSubs;

__device__ __forceinline__ Unit row_chunk_unit(int count, int slices) {
    const int id = static_cast<int>(blockIdx.x);
    const int n = id >> 3, x = id & 7, k = n / kGuChunk, p = n - k * kGuChunk;
    const int rl = p / kSubs;
    const int u = (k * 8 + x) * kGuChunk + rl * kSubs + (p + rl + k) % kSubs;
    Unit r;
    r.ok = u < count * slices;
    r.item = r.ok ? u / slices : 0;
    r.slice = r.ok ? u % slices : 0;
    return r;
}

__device__ __forceinline__ Unit mfma_unit(int count, int slices) {
    const int units = count * slices;
    const int u = dealt_unit(static_cast<int>(blockIdx.x));
    Unit r;
    r.ok = u < units;
    r.item = r.ok ? u / slices : 0;
    r.slice = r.ok ? u % slices : 0;
    return r;
}

__device__ __forceinline__ float half_lo(uint32_t w) { return h2f(w); }
__device__ __forceinline__ float half_hi(uint32_t w) { return h2f(w >> 16); }

// 8 fp16 values as an MFMA operand.
__device__ __forceinline__ v8h pack8(const uint32_t (&w)[4]) {
    v4i v = {static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]), static_cast<int>(w[3])};
    return __builtin_bit_cast(v8h, v);
}

// The fp16 hi halves (s of a Q8_1 head) of 8 heads, zero for blocks >= nb.
__device__ __forceinline__ v8h head_sums(uint4 h0, uint4 h1, int kb0, int nb) {
    const uint32_t hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = kb0 + 2 * e < nb ? hv[2 * e] >> 16 : 0u;
        const uint32_t hi = kb0 + 2 * e + 1 < nb ? hv[2 * e + 1] & 0xffff0000u : 0u;
        w[e] = lo | hi;
    }
    return pack8(w);
}

// fp16 -> fp32 conversions the compiler cannot fold into v_fma_mix_f32.  On
// gfx950 v_fma_mix_f32 issues at about the rate of a conversion (measured:
// 0.5 wave-instructions per SIMD per ns against 0.9 for v_fma_f32, v_mul_f32
// and v_add_f32), so a scale used by several products is converted once and
// the products are plain fp32 fmas.  (Same values: fp16 -> fp32 is exact.)
__device__ __forceinline__ float cvt_half_lo(uint32_t w) {
    float r;
    asm("v_cvt_f32_f16 %0, %1" : "=v"(r) : "v"(w));
    return r;
}
__device__ __forceinline__ float cvt_half_hi(uint32_t w) {
    float r;
    asm("v_cvt_f32_f16_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1" : "=v"(r) : "v"(w));
    return r;
}

// As scale_block below, with the 16 row scales already in fp32.
__device__ __forceinline__ void scale_block_f32(float (&acc)[16], v16i r, uint32_t head, const float (&d4)[16]) {
    const v16f f = __builtin_bit_cast(v16f, r);
    const float d8 = cvt_half_lo(head);
    const float nk = -kMagicF * d8;
    // Eight independent products, then their eight accumulations: at two
    // waves per SIMD back-to-back dependent fmas issue at about 60 % of the
    // rate of independent ones (measured).
#pragma unroll
    for (int g = 0; g < 16; g += 8) {
        float t[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) t[v] = fmaf(f[g + v], d8, nk);
#pragma unroll
        for (int v = 0; v < 8; ++v) acc[g + v] = fmaf(d4[g + v], t[v], acc[g + v]);
    }
}

// acc[v] += d4[v] * round(I[v] * d8) for one MFMA result (see the file comment).
__device__ __forceinline__ void scale_block(float (&acc)[16], v16i r, uint32_t head, const uint32_t (&d4)[8]) {
    const v16f f = __builtin_bit_cast(v16f, r);
    const float d8 = half_lo(head);
    const float nk = -kMagicF * d8;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float t = fmaf(f[v], d8, nk);
        const float s = (v & 1) ? half_hi(d4[v >> 1]) : half_lo(d4[v >> 1]);
        acc[v] = fmaf(s, t, acc[v]);
    }
}

// Q4_1 blocks {d4, m4, codes}: the reference's per-fragment value is
// fma(float(I_f), half(d4*d8), half(m4*s8) / 2) (src/cpu_expert.cpp:167-194),
// i.e. per block half(d4*d8) * I + half(m4*s8) with both products rounded to
// fp16 (d4*d8 and m4*s8 are exact in fp32: fp16 times fp16).  Here, per
// block: acc = fma(I, dd, acc) + ms with the same two fp16 roundings; only
// the fp32 summation order is this kernel's own.
__device__ __forceinline__ void scale_block_q41(float (&acc)[16], v16i r, uint32_t head, const uint32_t (&d4)[8],
                                                const uint32_t (&m4)[8]) {
    const v16f f = __builtin_bit_cast(v16f, r);
    const float d8 = half_lo(head), s8 = half_hi(head);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float I = f[v] - kMagicF;   // exact: F = 12582912 + I
        const float d = (v & 1) ? half_hi(d4[v >> 1]) : half_lo(d4[v >> 1]);
        const float mn = (v & 1) ? half_hi(m4[v >> 1]) : half_lo(m4[v >> 1]);
        const float dd = h2f(f2h(d * d8)), ms = h2f(f2h(mn * s8));
        acc[v] = fmaf(I, dd, acc[v]) + ms;
    }
}

// What one wave needs to project its 32 weight rows against up to kSubs
// token tiles.  Offsets are per lane; per-block steps are uniform.
struct TileArgs {
    __amdgpu_buffer_rsrc_t wr, sr, xr, hr;   // weight codes, weight scales, activation codes, activation heads
    __amdgpu_buffer_rsrc_t mr;               // Q4_1: weight mins (the scales' layout); unused for Q4_0
    uint32_t w_off;                          // lane's A row (block b at + 16 b)
    uint32_t s_off0, s_off1, s_step;         // lane's two 16-byte scale groups (block b at + b s_step)
    uint32_t x_off[kSubs], h_off[kSubs];     // lane's token rows (block b at + 32 b / + 4 b)
    const uint16_t *cscale;                  // lane's A-row scale of block kb at cscale[kb * cstride]
    int cstride;
    int nb;                                  // blocks per row (K / 32)
    int shift;                               // 0: low nibbles (lane half 0), 4: high nibbles
    int32_t *dots;                           // debug: per-block dots [pair][rows][nb] or null
    size_t dot_rows;                         // rows per pair in `dots`
    int dot_row0, dot_pair0, ncols, m, h;
};

// Debug-dot row of accumulator register v in lane half h.
template<bool Down>
__device__ __forceinline__ int acc_row(int v, int h) {
    return Down ? 4 * (v & 7) + 2 * h + (v >> 3) : 16 * h + v;
}

struct Loads {
    uint4 w, d0, d1, m0, m1;
    uint4 x[kSubs];
    uint32_t hd[kSubs];
};

template<int NS, bool Q41 = false>
__device__ __forceinline__ Loads tile_loads(const TileArgs &t, int b) {
    Loads l;
    const uint32_t ub = static_cast<uint32_t>(b);
    l.w = buffer_load16(t.wr, t.w_off, ub * 16u);
    l.d0 = buffer_load16(t.sr, t.s_off0, ub * t.s_step);
    l.d1 = buffer_load16(t.sr, t.s_off1, ub * t.s_step);
    if constexpr (Q41) {
        l.m0 = buffer_load16(t.mr, t.s_off0, ub * t.s_step);
        l.m1 = buffer_load16(t.mr, t.s_off1, ub * t.s_step);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        l.x[s] = buffer_load16(t.xr, t.x_off[s], ub * 32u);
        l.hd[s] = buffer_load4(t.hr, t.h_off[s], ub * 4u);
    }
    return l;
}

// acc[s] = -8 * sum_b d4 s8 + sum_b d4 round(I d8) for the NS token tiles
// (Q41: sum_b of scale_block_q41's terms from +0).
// The loads of block b + 1 are issued before block b is computed.
template<int NS, bool Dbg, bool Down, bool Q41 = false>
__device__ __forceinline__ void tile_project(const TileArgs &t, float (&acc)[kSubs][16]) {
    v16f corr[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) corr[s] = v16f{};
    for (int c = 0; c < (Q41 ? 0 : t.nb); c += 16) {
        const int kb0 = c + 8 * t.h;
        uint32_t dw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k0 = kb0 + 2 * e, k1 = k0 + 1;
            const uint32_t lo = t.cscale[std::min(k0, t.nb - 1) * t.cstride];
            const uint32_t hi = t.cscale[std::min(k1, t.nb - 1) * t.cstride];
            dw[e] = (k0 < t.nb ? lo : 0u) | (k1 < t.nb ? hi << 16 : 0u);
        }
        const v8h da = pack8(dw);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint4 h0 = buffer_load16(t.hr, t.h_off[s] + 4u * kb0, 0);
            const uint4 h1 = buffer_load16(t.hr, t.h_off[s] + 4u * kb0, 16);
            corr[s] = __builtin_amdgcn_mfma_f32_32x32x16_f16(da, head_sums(h0, h1, kb0, t.nb), corr[s], 0, 0, 0);
        }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[s][v] = Q41 ? 0.0f : -8.0f * corr[s][v];

    v16i magic;
#pragma unroll
    for (int v = 0; v < 16; ++v) magic[v] = kMagic;
    Loads cur = tile_loads<NS, Q41>(t, 0);
#pragma unroll 1
    for (int b = 0; b < t.nb; ++b) {
        const Loads nxt = tile_loads<NS, Q41>(t, std::min(b + 1, t.nb - 1));
        const uint32_t d4[8] = {cur.d0.x, cur.d0.y, cur.d0.z, cur.d0.w, cur.d1.x, cur.d1.y, cur.d1.z, cur.d1.w};
        const uint32_t m4[8] = {cur.m0.x, cur.m0.y, cur.m0.z, cur.m0.w, cur.m1.x, cur.m1.y, cur.m1.z, cur.m1.w};
        const v4i A = {static_cast<int>((cur.w.x >> t.shift) & kNibbles), static_cast<int>((cur.w.y >> t.shift) & kNibbles),
                       static_cast<int>((cur.w.z >> t.shift) & kNibbles), static_cast<int>((cur.w.w >> t.shift) & kNibbles)};
        v16i r[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const v4i B = {static_cast<int>(cur.x[s].x), static_cast<int>(cur.x[s].y), static_cast<int>(cur.x[s].z),
                           static_cast<int>(cur.x[s].w)};
            r[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, magic, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if constexpr (Q41) scale_block_q41(acc[s], r[s], cur.hd[s], d4, m4);
            else scale_block(acc[s], r[s], cur.hd[s], d4);
            if constexpr (Dbg) {
                const int j = kSub * s + t.m;
                if (t.dots && j < t.ncols)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        t.dots[(static_cast<size_t>(t.dot_pair0 + j) * t.dot_rows + t.dot_row0 + acc_row<Down>(v, t.h)) *
                                   t.nb + b] = r[s][v] - kMagic;
            }
        }
        cur = nxt;
    }
}

template<bool Dbg, bool Down, bool Q41 = false>
__device__ __forceinline__ void tile_dispatch(const TileArgs &t, int nsub, float (&acc)[kSubs][16]) {
    switch (nsub) {
    case 1: tile_project<1, Dbg, Down, Q41>(t, acc); break;
    case 2: tile_project<2, Dbg, Down, Q41>(t, acc); break;
    case 3: tile_project<3, Dbg, Down, Q41>(t, acc); break;
    default: tile_project<4, Dbg, Down, Q41>(t, acc); break;
    }
}

// ------------------------------------------------------------- gate / up ---
// The gate and up projections feed SiLU and the middle Q8, and one middle
// code that rounds differently moves its token's output by ~1e-2 rms, so they
// reproduce the reference's fp32 arithmetic exactly (cpu_expert's
// matrix_gpu_order, src/cpu_expert.cpp:156-213, the order of the gfx906
// MMVQ kernel src/hip/linear.hip:156-281):
//   fragment f of block k: bytes 8f..8f+7 of the code chunk, i.e. elements
//     8f..8f+7 (low nibbles) and 16+8f..16+8f+7 (high nibbles);
//   lane L = 2*(k%64) + f:  acc[L] = fma(d4, fma(float(I_f), d8, -4*s8), acc[L])
//     over k = L/2, L/2 + 64, ... in increasing k;
//   u_f(k') = acc[2k'+f] + acc[2(k'+32)+f],  v(k') = u_0(k') + u_1(k')  (k' < 32);
//   result = pairwise tree of v(0..31) in index order (XOR butterfly 1..32).
// Every add and fma is the same IEEE fp32 operation, so the gate and up
// values are bit-identical to the reference's, and with moe_expf so is the
// middle.  Fragment dots come from two MFMAs per block whose A operands keep
// only that fragment's bytes (the other half zero); both MFMAs start from 0.

// acc[v] = fma(d4[v], fma(float(I[v]), d8, c4), acc[v]); d4 read as fp16 by
// v_fma_mix_f32 (lo / hi half of each word).
__device__ __forceinline__ float fma_mix_lo(uint32_t h2, float t, float acc) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(t), "v"(acc));
    return r;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t h2, float t, float acc) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(t), "v"(acc));
    return r;
}

__device__ __forceinline__ void fragment_scale(float (&acc)[16], v16i I, float d8, float c4, const uint32_t (&d4)[8]) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float t = fmaf(static_cast<float>(I[v]), d8, c4);
        acc[v] = (v & 1) ? fma_mix_hi(d4[v >> 1], t, acc[v]) : fma_mix_lo(d4[v >> 1], t, acc[v]);
    }
}

struct GuTile {
    __amdgpu_buffer_rsrc_t wr, sr, xr, hr;
    uint32_t w_off, s_off0, s_off1, x_off, h_off;   // token block b at x_off + b XStride / h_off + b HStride
    int nb, shift;
    int32_t *dots;     // debug: [pair][I][nb] or null
    size_t dot_base;   // dots index of (pair of this lane, row R0 + 16h, block 0)
    bool dot_ok;
};

// Per-block steps of a token's codes and head: split planes (32 / 4 bytes),
// or canonical 36-byte Q8_1 blocks read in place (Canon).
template<bool Canon> constexpr uint32_t XStride = Canon ? 36u : 32u;
template<bool Canon> constexpr uint32_t HStride = Canon ? 36u : 4u;

struct BlockLoads {
    uint4 w, d0, d1, x;
    uint32_t hd;
};

template<bool Canon = false>
__device__ __forceinline__ BlockLoads block_loads(const GuTile &t, int b) {
    const uint32_t ub = static_cast<uint32_t>(b);
    BlockLoads l;
    l.w = buffer_load16(t.wr, t.w_off, ub * 16u);
    l.d0 = buffer_load16(t.sr, t.s_off0, ub * 16u);
    l.d1 = buffer_load16(t.sr, t.s_off1, ub * 16u);
    l.x = buffer_load16(t.xr, t.x_off, ub * XStride<Canon>);
    l.hd = buffer_load4(t.hr, t.h_off, ub * HStride<Canon>);
    return l;
}

// Fragment f's dots of one block for the wave's 32 rows x 32 tokens.
template<int F>
__device__ __forceinline__ v16i fragment_dots(const GuTile &t, const BlockLoads &l) {
    const v16i zero = {};
    const v4i B = {static_cast<int>(l.x.x), static_cast<int>(l.x.y), static_cast<int>(l.x.z), static_cast<int>(l.x.w)};
    const v4i A = F == 0 ? v4i{static_cast<int>((l.w.x >> t.shift) & kNibbles), static_cast<int>((l.w.y >> t.shift) & kNibbles), 0, 0}
                         : v4i{0, 0, static_cast<int>((l.w.z >> t.shift) & kNibbles), static_cast<int>((l.w.w >> t.shift) & kNibbles)};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, zero, 0, 0, 0);
}

template<bool Dbg>
__device__ __forceinline__ void store_dots(const GuTile &t, int b, v16i I0, v16i I1) {
    if constexpr (Dbg) {
        if (t.dot_ok)
#pragma unroll
            for (int v = 0; v < 16; ++v) t.dots[t.dot_base + static_cast<size_t>(v) * t.nb + b] = I0[v] + I1[v];
    }
}

// ---- H <= 2048 (one block per reference lane): staged scales and heads,
// weights and activations prefetched one leaf pair ahead.
constexpr int kGuMaxBlocks = 64;

struct GuStage {
    const uint32_t *d4;   // LDS [nb][32 halfs] of this wave's rows (row 16h + v at half 16h + v)
    const uint32_t *hd;   // unused
};

struct Blk {
    uint4 w, x;           // code chunk of the lane's A row, Q8 codes of its token (16 bytes each)
};

template<bool Canon = false>
__device__ __forceinline__ Blk blk_load(const GuTile &t, int b) {
    const uint32_t ub = static_cast<uint32_t>(b);
    return Blk{buffer_load16(t.wr, t.w_off, ub * 16u), buffer_load16(t.xr, t.x_off, ub * XStride<Canon>)};
}

// Fragment F's dots of one block with v_mfma_i32_32x32x16_i8 (K = 16 = one
// fragment): lane half h supplies the fragment's 8 nibbles of elements
// 16h + 8F .. +7 and the same 8 Q8 codes.
template<int F>
__device__ __forceinline__ v16i frag_mfma(const Blk &k, int shift) {
    const uint32_t w0 = F ? k.w.z : k.w.x, w1 = F ? k.w.w : k.w.y;
    const uint32_t x0 = F ? k.x.z : k.x.x, x1 = F ? k.x.w : k.x.y;
    const long A = static_cast<long>((static_cast<uint64_t>((w1 >> shift) & kNibbles) << 32) | ((w0 >> shift) & kNibbles));
    const long B = static_cast<long>((static_cast<uint64_t>(x1) << 32) | x0);
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B, v16i{}, 0, 0, 0);
}

// fma(d4[v], fma(float(I), d8, c4), +0): the reference's lane value of one
// block and fragment for output register v.
__device__ __forceinline__ float frag_value(int I, float d8, float c4, const uint32_t (&d4)[8], int v) {
    const float t = fmaf(static_cast<float>(I), d8, c4);
    return (v & 1) ? mul_half_hi(d4[v >> 1], t) : mul_half_lo(d4[v >> 1], t);
}

// v(k') = (acc[2k'] + acc[2(k'+32)]) + (acc[2k'+1] + acc[2(k'+32)+1]) with
// acc[2j+f] the fragment-f value of block j (+0 past nb).  Full: nb == 64.
// Blocks k' and k'+32 are loaded here; the fragment-0 pair is finished before
// the fragment-1 MFMAs so only two MFMA results are live.
template<bool Full, bool Dbg, bool Canon = false>
__device__ __forceinline__ void leaf_staged(const GuTile &t, const GuStage &g, int kp, int m, int h, float (&v)[16]) {
    const int jb = kp + 32;
    const bool has_a = Full || kp < t.nb, has_b = Full || jb < t.nb;   // uniform
    const int ja = has_a ? kp : 0, jc = has_b ? jb : 0;
    const Blk ka = blk_load<Canon>(t, ja), kb = blk_load<Canon>(t, jc);
    const uint32_t ha = buffer_load4(t.hr, t.h_off, static_cast<uint32_t>(ja) * HStride<Canon>);
    const uint32_t hb = buffer_load4(t.hr, t.h_off, static_cast<uint32_t>(jc) * HStride<Canon>);
    const uint4 *da4 = reinterpret_cast<const uint4 *>(g.d4 + ja * 16 + 8 * h);
    const uint4 *db4 = reinterpret_cast<const uint4 *>(g.d4 + jc * 16 + 8 * h);
    const uint4 a0 = da4[0], a1 = da4[1], b0 = db4[0], b1 = db4[1];
    const uint32_t da[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const uint32_t db[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float d8a = cvt_half_lo(ha), c4a = -4.0f * cvt_half_hi(ha);
    const float d8b = cvt_half_lo(hb), c4b = -4.0f * cvt_half_hi(hb);
    float u0[16];
    v16i keep_a0, keep_b0;
    {
        const v16i Ia = frag_mfma<0>(ka, t.shift), Ib = frag_mfma<0>(kb, t.shift);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float za = frag_value(Ia[i], d8a, c4a, da, i), zb = frag_value(Ib[i], d8b, c4b, db, i);
            if (!Full) { za = has_a ? za : 0.0f; zb = has_b ? zb : 0.0f; }
            u0[i] = za + zb;
        }
        if constexpr (Dbg) { keep_a0 = Ia; keep_b0 = Ib; }
    }
    {
        const v16i Ia = frag_mfma<1>(ka, t.shift), Ib = frag_mfma<1>(kb, t.shift);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float za = frag_value(Ia[i], d8a, c4a, da, i), zb = frag_value(Ib[i], d8b, c4b, db, i);
            if (!Full) { za = has_a ? za : 0.0f; zb = has_b ? zb : 0.0f; }
            v[i] = u0[i] + (za + zb);
        }
        if constexpr (Dbg) {
            if (has_a) store_dots<Dbg>(t, kp, keep_a0, Ia);
            if (has_b) store_dots<Dbg>(t, jb, keep_b0, Ib);
        }
    }
    // One leaf at a time: hoisting the next leaf's loads and MFMAs above this
    // point multiplies the live registers.
    __builtin_amdgcn_sched_barrier(0);
}

// Leaves 2p and 2p+1 and their merge into the pairwise tree over v(0..31):
// leaves are taken two at a time (a level-1 node) and merged upward like a
// binary counter, so each level holds at most one pending left operand.
// Levels 1-2 stay in registers; levels 3-4 (touched every 8, 16 leaves) wait
// in LDS (`park`, 2 x 16 floats per lane of this wave).
template<bool Full, bool Dbg>
__device__ __forceinline__ void tree_step(const GuTile &t, const GuStage &g, float (*park)[16][64], int lane, int p,
                                          float (&l1)[16], float (&l2)[16], float (&res)[16]) {
    const int m = lane & 31, h = lane >> 5;
    float w[16], x[16];
    leaf_staged<Full, Dbg>(t, g, 2 * p, m, h, w);
    leaf_staged<Full, Dbg>(t, g, 2 * p + 1, m, h, x);
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = w[i] + x[i];
    if ((p & 1) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l1[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = l1[i] + w[i];
    if ((p & 2) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l2[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = l2[i] + w[i];
    int lvl = 0;
    for (; lvl < 2; ++lvl) {
        if (((p >> (lvl + 2)) & 1) == 0) break;
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = park[lvl][i][lane] + w[i];
    }
    if (lvl < 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) park[lvl][i][lane] = w[i];
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) res[i] = w[i];
    }
}

template<bool Full, bool Dbg>
__device__ __forceinline__ void fold_tree_staged(const GuTile &t, const GuStage &g, float (*park)[16][64], int lane,
                                                 float (&res)[16]) {
    float l1[16], l2[16];
#pragma unroll 1
    for (int p = 0; p < 16; ++p) tree_step<Full, Dbg>(t, g, park, lane, p, l1, l2, res);
}

// ---- H == 2048 (64 blocks): loads in groups of four leaves that use whole
// cache lines.  Group g covers blocks 4g..4g+3 and 4g+32..4g+35, loaded half
// (two leaves) at a time.  Lane half h of row m reads contiguous bytes of its
// row (blocks 4g+32h+i); a v_permlane32_swap of the low- and high-nibble
// words then gives, per leaf, the MFMA operand of block 4g+i (low nibbles in
// lanes < 32, high in lanes >= 32) and of block 4g+32+i.  Lane half h of
// token n reads bytes 16h..16h+15 of consecutive 32-byte Q8 blocks, so the
// two halves of a token use the same lines.
struct HalfGroup {
    uint4 w[2];           // A row: blocks 4g+2q+i (h = 0) / 4g+32+2q+i (h = 1)
    uint4 xa[2], xb[2];   // token codes, half h: blocks 4g+2q+i / 4g+32+2q+i
    uint2 ha, hb;         // token heads of blocks 4g+2q, +1 / 4g+32+2q, +1
};

// The operands of level-1 node p = 2g + q (leaves 4g + 2q and 4g + 2q + 1).
// Loading half a line group at a time keeps the kernel at three waves per
// SIMD (a whole group in registers needed 211 VGPRs: two waves).  The weight
// half (8 VGPRs) of node p + 1 is loaded while node p computes (157 VGPRs;
// 16K layer 5.42 -> 5.35 ms); the activation half as well would need 177
// VGPRs, two waves per SIMD.
__device__ __forceinline__ void half_load_w(const GuTile &t, uint32_t w_off, int p, uint4 (&w)[2]) {
    const uint32_t b0 = static_cast<uint32_t>(4 * (p >> 1) + 2 * (p & 1));
#pragma unroll
    for (int i = 0; i < 2; ++i) w[i] = buffer_load16(t.wr, w_off, (b0 + i) * 16u);
}
template<bool Canon = false>
__device__ __forceinline__ void half_load_x(const GuTile &t, int p, HalfGroup &G) {
    constexpr uint32_t xs = XStride<Canon>, hs = HStride<Canon>;
    const uint32_t b0 = static_cast<uint32_t>(4 * (p >> 1) + 2 * (p & 1));
#pragma unroll
    for (int i = 0; i < 2; ++i) G.xa[i] = buffer_load16(t.xr, t.x_off, (b0 + i) * xs);
#pragma unroll
    for (int i = 0; i < 2; ++i) G.xb[i] = buffer_load16(t.xr, t.x_off, (b0 + 32 + i) * xs);
    if constexpr (Canon) {
        G.ha = make_uint2(buffer_load4(t.hr, t.h_off, b0 * hs), buffer_load4(t.hr, t.h_off, (b0 + 1) * hs));
        G.hb = make_uint2(buffer_load4(t.hr, t.h_off, (b0 + 32) * hs), buffer_load4(t.hr, t.h_off, (b0 + 33) * hs));
    } else {   // head plane: the two heads are adjacent
        const auto a = __builtin_amdgcn_raw_buffer_load_b64(t.hr, t.h_off, b0 * hs, 0);
        const auto b = __builtin_amdgcn_raw_buffer_load_b64(t.hr, t.h_off, (b0 + 32) * hs, 0);
        G.ha = make_uint2(a[0], a[1]);
        G.hb = make_uint2(b[0], b[1]);
    }
}

__device__ __forceinline__ v16i frag_mfma2(uint32_t a0, uint32_t a1, uint32_t x0, uint32_t x1) {
    const long A = static_cast<long>((static_cast<uint64_t>(a1) << 32) | a0);
    const long B = static_cast<long>((static_cast<uint64_t>(x1) << 32) | x0);
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B, v16i{}, 0, 0, 0);
}

// Rows of 65..96 blocks in the grouped form (the reference model's 2560:
// 80 blocks).  Reference lane j also holds block j + 64 when j + 64 < nb, and
// its accumulator continues with fma(d4, t, acc) over that block; lane j + 32
// holds no second block (j + 96 >= nb).  So leaf kp's chain A gets one more
// block, kp + 64, for kp < nb - 64.  Its operands per node (leaves 2p, 2p+1):
// the lane's row chunk of the block, the token's half block and its head.
struct ExtraBlk {
    uint4 w[2], x[2];
    uint32_t hd[2];
};

template<bool Canon = false>
__device__ __forceinline__ void extra_load(const GuTile &t, int p, ExtraBlk &E) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t e = static_cast<uint32_t>(std::min(64 + 2 * p + i, t.nb - 1));   // past nb: unused
        E.w[i] = buffer_load16(t.wr, t.w_off, e * 16u);
        E.x[i] = buffer_load16(t.xr, t.x_off, e * XStride<Canon>);
        E.hd[i] = buffer_load4(t.hr, t.h_off, e * HStride<Canon>);
    }
}

// acc[v] = fma(d4[v], fma(float(I[v]), d8, c4), acc[v]) for block kp + 64's
// fragment F, after block kp's value (the chain of reference lane kp).
template<int F>
__device__ __forceinline__ v16i extra_dots(const ExtraBlk &E, int i, int shift) {
    return frag_mfma<F>(Blk{E.w[i], E.x[i]}, shift);
}
__device__ __forceinline__ void extra_scale(const GuStage &g, const ExtraBlk &E, int i, int blk, int h, v16i I,
                                            float (&acc)[16]) {
    const uint4 *de4 = reinterpret_cast<const uint4 *>(g.d4 + blk * 16 + 8 * h);
    const uint4 e0 = de4[0], e1 = de4[1];
    const uint32_t de[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
    const float d8 = cvt_half_lo(E.hd[i]), c4 = -4.0f * cvt_half_hi(E.hd[i]);
    fragment_scale(acc, I, d8, c4, de);
}

// Leaf kp with block kp + 64 in chain A: v = (A0 + B0) + (A1 + B1), with
// A_f = fma(d4', t', fma(d4, t, +0)) over blocks kp, kp + 64 and B_f block
// kp + 32's value, as leaf_grouped without the extra block.
template<bool Dbg>
__device__ __forceinline__ void leaf_grouped_extra(const GuTile &t, const GuStage &g, const HalfGroup &G,
                                                   const ExtraBlk &E, int i, int kp, int h, float (&v)[16]) {
    const uint4 wi = G.w[i];
    const uint32_t wv[4] = {wi.x, wi.y, wi.z, wi.w};
    uint32_t opa[4], opb[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const auto r = __builtin_amdgcn_permlane32_swap(wv[d] & kNibbles, (wv[d] >> 4) & kNibbles, false, false);
        opa[d] = r[0];
        opb[d] = r[1];
    }
    const uint32_t ha = i ? G.ha.y : G.ha.x, hb = i ? G.hb.y : G.hb.x;
    const uint4 *da4 = reinterpret_cast<const uint4 *>(g.d4 + kp * 16 + 8 * h);
    const uint4 *db4 = reinterpret_cast<const uint4 *>(g.d4 + (kp + 32) * 16 + 8 * h);
    const uint4 a0 = da4[0], a1 = da4[1], b0 = db4[0], b1 = db4[1];
    const uint32_t da[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const uint32_t db[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float d8a = cvt_half_lo(ha), c4a = -4.0f * cvt_half_hi(ha);
    const float d8b = cvt_half_lo(hb), c4b = -4.0f * cvt_half_hi(hb);
    const uint4 xa = G.xa[i], xb = G.xb[i];
    float u0[16];
    v16i keep_a0, keep_b0, keep_e0;
    {
        float za[16];
        const v16i Ia = frag_mfma2(opa[0], opa[1], xa.x, xa.y);
#pragma unroll
        for (int j = 0; j < 16; ++j) za[j] = frag_value(Ia[j], d8a, c4a, da, j);
        const v16i Ie = extra_dots<0>(E, i, t.shift);
        extra_scale(g, E, i, kp + 64, h, Ie, za);
        const v16i Ib = frag_mfma2(opb[0], opb[1], xb.x, xb.y);
#pragma unroll
        for (int j = 0; j < 16; ++j) u0[j] = za[j] + frag_value(Ib[j], d8b, c4b, db, j);
        if constexpr (Dbg) { keep_a0 = Ia; keep_b0 = Ib; keep_e0 = Ie; }
    }
    {
        float za[16];
        const v16i Ia = frag_mfma2(opa[2], opa[3], xa.z, xa.w);
#pragma unroll
        for (int j = 0; j < 16; ++j) za[j] = frag_value(Ia[j], d8a, c4a, da, j);
        const v16i Ie = extra_dots<1>(E, i, t.shift);
        extra_scale(g, E, i, kp + 64, h, Ie, za);
        const v16i Ib = frag_mfma2(opb[2], opb[3], xb.z, xb.w);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = u0[j] + (za[j] + frag_value(Ib[j], d8b, c4b, db, j));
        if constexpr (Dbg) {
            store_dots<Dbg>(t, kp, keep_a0, Ia);
            store_dots<Dbg>(t, kp + 32, keep_b0, Ib);
            store_dots<Dbg>(t, kp + 64, keep_e0, Ie);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

template<bool Dbg, bool Extra = false>
__device__ __forceinline__ void leaf_grouped(const GuTile &t, const GuStage &g, const HalfGroup &G, int i, int kp, int m,
                                             int h, float (&v)[16], const ExtraBlk *E = nullptr) {
    if constexpr (Extra) {
        if (kp < t.nb - 64) {   // uniform
            leaf_grouped_extra<Dbg>(t, g, G, *E, i, kp, h, v);
            return;
        }
    }
    const uint4 wi = G.w[i];
    const uint32_t wv[4] = {wi.x, wi.y, wi.z, wi.w};
    uint32_t opa[4], opb[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const auto r = __builtin_amdgcn_permlane32_swap(wv[d] & kNibbles, (wv[d] >> 4) & kNibbles, false, false);
        opa[d] = r[0];   // block kp: low nibbles (lanes < 32), high nibbles (lanes >= 32)
        opb[d] = r[1];   // block kp + 32
    }
    const uint32_t ha = i ? G.ha.y : G.ha.x, hb = i ? G.hb.y : G.hb.x;
    const uint4 *da4 = reinterpret_cast<const uint4 *>(g.d4 + kp * 16 + 8 * h);
    const uint4 *db4 = reinterpret_cast<const uint4 *>(g.d4 + (kp + 32) * 16 + 8 * h);
    const uint4 a0 = da4[0], a1 = da4[1], b0 = db4[0], b1 = db4[1];
    const uint32_t da[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const uint32_t db[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float d8a = cvt_half_lo(ha), c4a = -4.0f * cvt_half_hi(ha);
    const float d8b = cvt_half_lo(hb), c4b = -4.0f * cvt_half_hi(hb);
    const uint4 xa = G.xa[i], xb = G.xb[i];
    float u0[16];
    v16i keep_a0, keep_b0;
    {
        const v16i Ia = frag_mfma2(opa[0], opa[1], xa.x, xa.y), Ib = frag_mfma2(opb[0], opb[1], xb.x, xb.y);
#pragma unroll
        for (int j = 0; j < 16; ++j) u0[j] = frag_value(Ia[j], d8a, c4a, da, j) + frag_value(Ib[j], d8b, c4b, db, j);
        if constexpr (Dbg) { keep_a0 = Ia; keep_b0 = Ib; }
    }
    {
        const v16i Ia = frag_mfma2(opa[2], opa[3], xa.z, xa.w), Ib = frag_mfma2(opb[2], opb[3], xb.z, xb.w);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = u0[j] + (frag_value(Ia[j], d8a, c4a, da, j) + frag_value(Ib[j], d8b, c4b, db, j));
        if constexpr (Dbg) {
            store_dots<Dbg>(t, kp, keep_a0, Ia);
            store_dots<Dbg>(t, kp + 32, keep_b0, Ib);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Tree merge of the level-1 node p (= w) as in tree_step.
__device__ __forceinline__ void tree_merge(float (*park)[16][64], int lane, int p, float (&w)[16], float (&l1)[16],
                                           float (&l2)[16], float (&res)[16]) {
    if ((p & 1) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l1[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = l1[i] + w[i];
    if ((p & 2) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l2[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = l2[i] + w[i];
    int lvl = 0;
    for (; lvl < 2; ++lvl) {
        if (((p >> (lvl + 2)) & 1) == 0) break;
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = park[lvl][i][lane] + w[i];
    }
    if (lvl < 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) park[lvl][i][lane] = w[i];
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) res[i] = w[i];
    }
}

template<bool Dbg, bool Extra = false>
__device__ __forceinline__ void fold_tree_grouped(const GuTile &t, const GuStage &g, uint32_t w_off, float (*park)[16][64],
                                                  int lane, uint4 (&wn)[2], float (&res)[16]) {
    // wn: node 0's weight half, already in flight.
    const int m = lane & 31, h = lane >> 5;
    float l1[16], l2[16];
#pragma unroll 1
    for (int p = 0; p < 16; ++p) {
        HalfGroup G;
        G.w[0] = wn[0];
        G.w[1] = wn[1];
        half_load_x(t, p, G);
        ExtraBlk E;
        if constexpr (Extra) {
            if (2 * p < t.nb - 64) extra_load(t, p, E);   // uniform
        }
        half_load_w(t, w_off, p < 15 ? p + 1 : p, wn);   // node p + 1's weights in flight during node p
        float w[16], x[16];
        leaf_grouped<Dbg, Extra>(t, g, G, 0, 2 * p, m, h, w, &E);
        leaf_grouped<Dbg, Extra>(t, g, G, 1, 2 * p + 1, m, h, x, &E);
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = w[i] + x[i];
        tree_merge(park, lane, p, w, l1, l2, res);
    }
}

// ---- H > 2048 (reference lanes holding several blocks): per-block loads.
// One block of a reference lane's chain: both fragment dots scaled into the
// lane's accumulators, acc = fma(d4, fma(float(I_f), d8, c4), acc).
template<bool Dbg>
__device__ __forceinline__ void chain_block(const GuTile &t, const BlockLoads &l, int b, float (&c0)[16],
                                            float (&c1)[16]) {
    const uint32_t d4[8] = {l.d0.x, l.d0.y, l.d0.z, l.d0.w, l.d1.x, l.d1.y, l.d1.z, l.d1.w};
    const v16i I0 = fragment_dots<0>(t, l), I1 = fragment_dots<1>(t, l);
    const float d8 = cvt_half_lo(l.hd), c4 = -4.0f * cvt_half_hi(l.hd);
    fragment_scale(c0, I0, d8, c4, d4);
    fragment_scale(c1, I1, d8, c4, d4);
    store_dots<Dbg>(t, b, I0, I1);
}

// Leaf kp for rows of more than 64 blocks: reference lanes kp and kp + 32,
// each the chain over its blocks j, j + 64, ... in increasing order (the
// reference lane array's acc[2j + f]), walked as one sequence -- kp's chain,
// then kp + 32's -- with
// each block's loads issued before the previous block is scaled.
template<bool Dbg, bool Canon = false>
__device__ __forceinline__ void fold_leaf_multi(const GuTile &t, int kp, float (&v)[16]) {
    float a0[16], a1[16], b0[16], b1[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) { a0[i] = 0.0f; a1[i] = 0.0f; b0[i] = 0.0f; b1[i] = 0.0f; }
    // nb > 64 here, so kp + 32 < nb and both chains hold a block.
    const int na = (t.nb - kp + 63) / 64, nc = (t.nb - kp - 32 + 63) / 64;
    BlockLoads cur = block_loads<Canon>(t, kp);
#pragma unroll 1
    for (int s = 0; s < na; ++s) {   // uniform
        const BlockLoads nxt = block_loads<Canon>(t, s + 1 < na ? kp + 64 * (s + 1) : kp + 32);
        chain_block<Dbg>(t, cur, kp + 64 * s, a0, a1);
        cur = nxt;
    }
#pragma unroll 1
    for (int s = 0; s < nc; ++s) {   // uniform
        BlockLoads nxt = cur;
        if (s + 1 < nc) nxt = block_loads<Canon>(t, kp + 32 + 64 * (s + 1));
        chain_block<Dbg>(t, cur, kp + 32 + 64 * s, b0, b1);
        cur = nxt;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (a0[i] + b0[i]) + (a1[i] + b1[i]);
    __builtin_amdgcn_sched_barrier(0);
}

template<bool Dbg>
__device__ __forceinline__ void fold_tree_multi(const GuTile &t, float (*park)[16][64], int lane, float (&res)[16]) {
    float l1[16], l2[16];
#pragma unroll 1
    for (int p = 0; p < 16; ++p) {
        float w[16], x[16];
        fold_leaf_multi<Dbg>(t, 2 * p, w);
        fold_leaf_multi<Dbg>(t, 2 * p + 1, x);
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = w[i] + x[i];
        if ((p & 1) == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) l1[i] = w[i];
            continue;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = l1[i] + w[i];
        if ((p & 2) == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) l2[i] = w[i];
            continue;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = l2[i] + w[i];
        int lvl = 0;
        for (; lvl < 2; ++lvl) {
            if (((p >> (lvl + 2)) & 1) == 0) break;
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i] = park[lvl][i][lane] + w[i];
        }
        if (lvl < 2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) park[lvl][i][lane] = w[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) res[i] = w[i];
        }
    }
}

// Workgroup = 2 waves: wave 0 gate rows R0..R0+31, wave 1 the same up rows,
// both for token tile `sub` (32 pairs) of an MFMA item.  A-row m of the MFMA
// is physical row 16*((m>>2)&1) + 4*(m>>3) + (m&3), so accumulator register v
// of lane half h is row 16h + v: the lane's 16 scales per block are two
// 16-byte groups of the [rows/8][blocks][8] plane, and its 16 middle values
// are elements 16h..16h+15 of one Q8_1 block.  Units are ordered
// (item, slice, sub) so the 4 tiles of an item that read the same weight rows
// are adjacent on one XCD.
// Fold: kFoldStaged (H < 2048), kFoldGrouped (H = 2048), kFoldGrouped96
// (2048 < H <= 3072: the grouped leaves plus block kp + 64 in chain A;
// 2560/640 4K Zipf layer 3.40 -> 2.83 ms with Q4_0 downs, 3.54 -> 2.98 ms
// with Q4_1, against kFoldMulti), kFoldMulti (H > 3072); one instantiation
// per shape keeps only that path's registers.
enum { kFoldStaged = 0, kFoldGrouped = 1, kFoldMulti = 2, kFoldGrouped96 = 3 };
constexpr int kGu96MaxBlocks = 96;

template<int Fold, bool Dbg>
__global__ __launch_bounds__(128, 2) void k_gate_up_mfma(FfnArgs a) {
    // Pending tree levels 3-4 per wave; after the tree the up wave's area
    // carries its result to the gate wave.
    __shared__ float park[2][2][16][64];
    __shared__ uint4 d4_lds[2][Fold == kFoldGrouped96 ? kGu96MaxBlocks : kGuMaxBlocks][4];   // [mat][block][32 halfs]
    float (*xch)[64] = park[1][0];
    const int mat = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shape.H, I = a.shape.I, nb = H / 32, nbi = I / 32;
    const int slices = nbi * kSubs;
    const Unit un = row_chunk_unit(a.routes.item_counts[1], slices);
    if (!un.ok) return;   // uniform per workgroup
    const Item *itp = a.routes.mfma_items + un.item;
    const int expert = itp->expert, first = itp->first, ncols = itp->ncols;
    const int sub = un.slice % kSubs;
    const int R0 = (un.slice / kSubs) * 32;
    if (kSub * sub >= ncols) return;   // uniform per workgroup: no tokens in this tile
    const int lane = threadIdx.x & 63;
    const int m = lane & 31, h = lane >> 5;
    const int prow = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const int j = kSub * sub + m;
    const int pair = first + std::min(j, ncols - 1);

    const size_t rbase = static_cast<size_t>(expert) * I + R0;
    const uint32_t row_bytes = static_cast<uint32_t>(nb) * 16u;
    GuTile t;
    t.wr = buffer_rsrc((mat ? a.bank.up_codes : a.bank.gate_codes) + rbase * row_bytes, 32u * row_bytes);
    t.sr = buffer_rsrc((mat ? a.bank.up_scales : a.bank.gate_scales) + rbase * nb, 32u * static_cast<uint32_t>(nb) * 2u);
    t.xr = buffer_rsrc(a.xq.codes, static_cast<uint32_t>(a.tokens) * static_cast<uint32_t>(nb) * 32u);
    t.hr = buffer_rsrc(a.xq.heads, static_cast<uint32_t>(a.tokens) * static_cast<uint32_t>(nb) * 4u);
    t.w_off = static_cast<uint32_t>(prow) * row_bytes;
    t.s_off0 = static_cast<uint32_t>(2 * h * nb) * 16u;
    t.s_off1 = t.s_off0 + static_cast<uint32_t>(nb) * 16u;
    const uint32_t tok = static_cast<uint32_t>(a.routes.pair_token[pair]);
    t.x_off = tok * static_cast<uint32_t>(nb) * 32u + 16u * h;
    t.h_off = tok * static_cast<uint32_t>(nb) * 4u;
    t.nb = nb;
    t.shift = 4 * h;
    t.dots = Dbg ? (mat ? a.up_dots : a.gate_dots) : nullptr;
    t.dot_base = (static_cast<size_t>(pair) * I + R0 + 16 * h) * nb;
    t.dot_ok = Dbg && t.dots && j < ncols;

    float res[16];
    // Node 0's weight half is issued before the scale staging, so the two
    // round trips overlap.
    const uint32_t w_off = static_cast<uint32_t>(prow) * row_bytes + 32u * 16u * h;
    uint4 wn[2] = {};
    if constexpr (Fold == kFoldGrouped || Fold == kFoldGrouped96) half_load_w(t, w_off, 0, wn);
    if constexpr (Fold != kFoldMulti) {
        // Stage the tile's scales (both matrices) and its tokens' Q8 heads.
        // Scale group g (rows 8g..8g+7) of block b is one 16-byte chunk of the
        // [rows/8][blocks][8] plane and lands at halfs 8g..8g+7 of [mat][b].
        for (int c = threadIdx.x; c < 8 * nb; c += blockDim.x) {
            const int mm = c / (4 * nb), rem = c % (4 * nb), gi = rem / nb, b = rem % nb;
            const uint16_t *plane = mm ? a.bank.up_scales : a.bank.gate_scales;
            d4_lds[mm][b][gi] = *reinterpret_cast<const uint4 *>(plane + (rbase + 8 * gi) * nb + b * 8);
        }
        __syncthreads();
        const GuStage g{reinterpret_cast<const uint32_t *>(&d4_lds[mat][0][0]), nullptr};
        if constexpr (Fold == kFoldGrouped || Fold == kFoldGrouped96)
            fold_tree_grouped<Dbg, Fold == kFoldGrouped96>(t, g, w_off, park[mat], lane, wn, res);
        else fold_tree_staged<false, Dbg>(t, g, park[mat], lane, res);
    } else {
        fold_tree_multi<Dbg>(t, park[mat], lane, res);
    }
    if (mat == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) xch[v][lane] = res[v];
    }
    __syncthreads();   // (the up wave's tree is done with park[1]; the gate wave's with park[0])
    if (mat != 0) return;
    int flags = 0;
    float mid[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) mid[v] = silu_mul(res[v], xch[v][lane], flags);
    float keep[16];
    if constexpr (Dbg) {
#pragma unroll
        for (int v = 0; v < 16; ++v) keep[v] = mid[v];
    }
    const Q8Part<2> q8 = quantize_part<2>(mid);
    if (j < ncols) {
        const size_t mb = static_cast<size_t>(pair) * nbi + R0 / 32;
        *reinterpret_cast<uint4 *>(a.mq.codes + mb * 32 + 16 * h) =
            make_uint4(q8.codes[0], q8.codes[1], q8.codes[2], q8.codes[3]);
        if (h == 0) a.mq.heads[mb] = q8.head;
        if constexpr (Dbg) {
            if (a.middle_f32)
#pragma unroll
                for (int v = 0; v < 16; ++v) a.middle_f32[static_cast<size_t>(pair) * I + R0 + 16 * h + v] = keep[v];
        }
        const int f = flags | (h == 0 ? q8.flags : 0);
        if (f) atomicOr(a.error, f);
    }
}

// ------------------------------------------------------------------ down ---
// Workgroup = 4 waves x 32 output rows = 128 rows of H.  A-row m maps to
// physical row rho = 4*(v&7) + 2*hh + (v>>3) with v = 4*(m>>3) + (m&3) and
// hh = (m>>2)&1, so accumulator register v of lane half h is row
// 4*(v&7) + 2h + (v>>3), whose scale sits at slot 16h + v of the
// [rows/32][blocks][32] plane (slot (r%4)*8 + (r%32)/4): one 32-byte read per
// lane and block.  Before the stores, lanes l and l^32 trade 8 values so each
// lane holds 16 consecutive rows (4 float4 stores per tile).
//
// I <= 512 (16 blocks): the four waves read the same middle rows, so the
// item's middle codes and heads are staged once in LDS, and each wave stages
// its 32-row scale tile there.  Weight blocks stream through a window of
// kDnWin registers: block b's register is reloaded with block b + kDnWin as
// soon as block b's A operand is formed.  With Q4_0 rows and 8 or 16 blocks
// a workgroup runs kDnSlicesPerGroup slices of 128 rows against the
// one staging: the window runs on into the next slice's blocks, and the next
// slice's scale tile goes to the other half of a double buffer.
constexpr int kDnMaxBlocks = 16;
constexpr int kDnWin = 8;
constexpr int kDnSlicesPerGroup = 4;

template<int NB, int W = 4>
struct DownStageT {
    static constexpr bool kMins = false;
    uint4 x[kDnMaxBlocks][kMfmaTile][2];     // middle codes [block][pair][32 bytes]
    uint32_t hd[kDnMaxBlocks][kMfmaTile];    // middle heads [block][pair]
    uint4 d4[NB][W][kDnMaxBlocks][4];        // [buffer][wave]: scales [block][32 slots]
};
using DownStage = DownStageT<2>;             // Q4_0 rows: 80 KiB, two workgroups per CU
// Q4_1 rows also stage their mins (80 KiB: two workgroups per CU) and take
// one slice per workgroup (a second scale buffer would not fit twice).
template<int W = 4>
struct DownStageQ41T : DownStageT<1, W> {
    static constexpr bool kMins = true;
    uint4 m4[W][kDnMaxBlocks][4];            // per wave: mins [block][32 slots]
};
using DownStageQ41 = DownStageQ41T<4>;
// Rows of 17..32 Q4_0 blocks: a workgroup of 8 waves takes two 128-row
// slices against one staging of each round (80 KiB).
using DownStage2 = DownStageT<1, 8>;

// Slices of 128 rows per work unit of the down kernel.  Running on into the
// next slice keeps block j of every slice in window register j % kDnWin only
// when the block count is a multiple of kDnWin.
__host__ __device__ constexpr int down_span(int nbi, bool q41) {
    return nbi % kDnWin == 0 && nbi <= kDnMaxBlocks && !q41 ? kDnSlicesPerGroup : 1;
}
// Work units per item.
__host__ __device__ constexpr int down_groups(int H, int nbi, bool q41) {
    const int slices = (H + 127) / 128, span = down_span(nbi, q41);
    return (slices + span - 1) / span;
}

// d4s: the wave's staged scale tile ([block][4] chunks); m4s: its staged
// Q4_1 mins (same layout), or nullptr for Q4_0 rows.  wa: the weight window
// (block b in register b % kDnWin); block b + kDnWin is read through wr
// (this slice's 32 rows, and the next slice's 32 rows at next_off when there
// is a next slice: past its end the descriptor reads zeros), at lane offset
// w_off.
template<int NS, bool Dbg, bool Q41, class Stage>
__device__ __forceinline__ void down_staged(const FfnArgs &a, const Stage &st, const uint4 (*d4s)[4], const uint4 (*m4s)[4],
                                            uint4 (&wa)[kDnWin], __amdgpu_buffer_rsrc_t wr, uint32_t next_off,
                                            uint32_t w_off, int nbi, int first, int ncols, int R0, int pslot, int lane,
                                            float (&acc)[kSubs][16]) {
    const int m = lane & 31, h = lane >> 5, shift = 4 * h;
    const uint16_t *d4h = reinterpret_cast<const uint16_t *>(&d4s[0][0]);
    if constexpr (Q41) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[s][v] = 0.0f;
    } else {
    // Seed: -8 * sum_b d4 s8, 16 blocks in one f16 MFMA.
    uint32_t dw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int k0 = 8 * h + 2 * e, k1 = k0 + 1;
        const uint32_t lo = k0 < nbi ? d4h[k0 * 32 + pslot] : 0u;
        const uint32_t hi = k1 < nbi ? d4h[k1 * 32 + pslot] : 0u;
        dw[e] = lo | (hi << 16);
    }
    const v8h da = pack8(dw);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        uint32_t sw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k0 = 8 * h + 2 * e, k1 = k0 + 1;
            const uint32_t lo = k0 < nbi ? st.hd[k0][kSub * s + m] >> 16 : 0u;
            const uint32_t hi = k1 < nbi ? st.hd[k1][kSub * s + m] & 0xffff0000u : 0u;
            sw[e] = lo | hi;
        }
        const v16f corr = __builtin_amdgcn_mfma_f32_32x32x16_f16(da, pack8(sw), v16f{}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[s][v] = -8.0f * corr[v];
    }
    }
    v16i magic;
#pragma unroll
    for (int v = 0; v < 16; ++v) magic[v] = kMagic;
    // Each step's B operand and head are read from LDS one step ahead (block
    // b + 1's first at block b's last step; past nbi they are never used).
    uint4 xb = st.x[0][m][h];
    uint32_t hx = st.hd[0][m];
#pragma unroll
    for (int b = 0; b < kDnMaxBlocks; ++b) {
        if (b < nbi) {   // uniform; a guard rather than a break keeps the loop unrolled
        const uint4 w = wa[b % kDnWin];
        const uint4 d0 = d4s[b][2 * h], d1 = d4s[b][2 * h + 1];
        const uint32_t d4[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
        uint32_t m4[8] = {};
        float d4f[16];
        if constexpr (Q41) {
            const uint4 n0 = m4s[b][2 * h], n1 = m4s[b][2 * h + 1];
            m4[0] = n0.x; m4[1] = n0.y; m4[2] = n0.z; m4[3] = n0.w;
            m4[4] = n1.x; m4[5] = n1.y; m4[6] = n1.z; m4[7] = n1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                d4f[2 * e] = cvt_half_lo(d4[e]);
                d4f[2 * e + 1] = cvt_half_hi(d4[e]);
            }
        }
        const v4i A = {static_cast<int>((w.x >> shift) & kNibbles), static_cast<int>((w.y >> shift) & kNibbles),
                       static_cast<int>((w.z >> shift) & kNibbles), static_cast<int>((w.w >> shift) & kNibbles)};
        {
            // The offset goes into the per-lane operand, which the range check covers.
            const int nb = b + kDnWin;
            const uint32_t o = nb < nbi ? static_cast<uint32_t>(nb) * 16u : next_off + static_cast<uint32_t>(nb - nbi) * 16u;
            wa[b % kDnWin] = buffer_load16(wr, w_off + o, 0);
        }
        // Each tile's MFMA is issued before the previous tile is scaled, so
        // the matrix unit works under the scaling and two results are live.
        v16i rp;
        uint32_t hp = 0;
        auto scale_prev = [&](int sp) {
            if constexpr (Q41) scale_block_q41(acc[sp], rp, hp, d4, m4);
            else scale_block_f32(acc[sp], rp, hp, d4f);
            if constexpr (Dbg) {
                const int j = kSub * sp + m;
                if (a.down_dots && j < ncols)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        a.down_dots[(static_cast<size_t>(first + j) * a.shape.H + R0 + 4 * (v & 7) + 2 * h + (v >> 3)) * nbi + b] =
                            rp[v] - kMagic;
            }
        };
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const v4i B = {static_cast<int>(xb.x), static_cast<int>(xb.y), static_cast<int>(xb.z), static_cast<int>(xb.w)};
            const v16i r = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, magic, 0, 0, 0);
            const uint32_t hs = hx;
            if (s + 1 < NS) {
                xb = st.x[b][kSub * (s + 1) + m][h];
                hx = st.hd[b][kSub * (s + 1) + m];
            } else if (b + 1 < kDnMaxBlocks) {
                xb = st.x[b + 1][m][h];
                hx = st.hd[b + 1][m];
            }
            if (s > 0) scale_prev(s - 1);
            __builtin_amdgcn_sched_barrier(0);
            rp = r;
            hp = hs;
        }
        scale_prev(NS - 1);
        }
    }
}

// down_staged for one of two staging rounds (down_two_rounds): blocks B0 ..
// B0 + 15 of the row sit at local indices 0..15.
template<int NS, bool Dbg, bool Q41, class Stage, int B0>
__device__ __forceinline__ void down_staged_round(const FfnArgs &a, const Stage &st, const uint4 (*d4s)[4], const uint4 (*m4s)[4],
                                            uint4 (&wa)[kDnWin], __amdgpu_buffer_rsrc_t wr, uint32_t next_off,
                                            uint32_t w_off, int nbi, int first, int ncols, int R0, int pslot, int lane,
                                            float (&acc)[kSubs][16]) {
    const int m = lane & 31, h = lane >> 5, shift = 4 * h;
    // Blocks B0 .. B0 + nloc - 1 are staged at local indices 0 .. nloc - 1
    // (the scales, mins, codes and heads); the weight window and the dots
    // use the block's own index.
    static_assert(B0 % kDnWin == 0, "block B0 + b sits in window register b % kDnWin");
    // (B0 == 0: every local index below kDnMaxBlocks is also below nbi, so
    // nbi itself bounds the first round.)
    const int nloc = B0 == 0 ? nbi : min(nbi - B0, kDnMaxBlocks);
    const uint16_t *d4h = reinterpret_cast<const uint16_t *>(&d4s[0][0]);
    if constexpr (Q41) {
        if constexpr (B0 == 0) {
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[s][v] = 0.0f;
        }
    } else {
    // Seed: -8 * sum_b d4 s8, 16 blocks in one f16 MFMA.
    uint32_t dw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int k0 = 8 * h + 2 * e, k1 = k0 + 1;
        const uint32_t lo = k0 < nloc ? d4h[k0 * 32 + pslot] : 0u;
        const uint32_t hi = k1 < nloc ? d4h[k1 * 32 + pslot] : 0u;
        dw[e] = lo | (hi << 16);
    }
    const v8h da = pack8(dw);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        uint32_t sw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k0 = 8 * h + 2 * e, k1 = k0 + 1;
            const uint32_t lo = k0 < nloc ? st.hd[k0][kSub * s + m] >> 16 : 0u;
            const uint32_t hi = k1 < nloc ? st.hd[k1][kSub * s + m] & 0xffff0000u : 0u;
            sw[e] = lo | hi;
        }
        const v16f corr = __builtin_amdgcn_mfma_f32_32x32x16_f16(da, pack8(sw), v16f{}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            if constexpr (B0 == 0) acc[s][v] = -8.0f * corr[v];
            else acc[s][v] = acc[s][v] + -8.0f * corr[v];
        }
    }
    }
    v16i magic;
#pragma unroll
    for (int v = 0; v < 16; ++v) magic[v] = kMagic;
    // Each step's B operand and head are read from LDS one step ahead (block
    // b + 1's first at block b's last step; past nbi they are never used).
    uint4 xb = st.x[0][m][h];
    uint32_t hx = st.hd[0][m];
#pragma unroll
    for (int b = 0; b < kDnMaxBlocks; ++b) {
        if (b < nloc) {   // uniform; a guard rather than a break keeps the loop unrolled
        const uint4 w = wa[b % kDnWin];
        const uint4 d0 = d4s[b][2 * h], d1 = d4s[b][2 * h + 1];
        const uint32_t d4[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
        uint32_t m4[8] = {};
        float d4f[16];
        if constexpr (Q41) {
            const uint4 n0 = m4s[b][2 * h], n1 = m4s[b][2 * h + 1];
            m4[0] = n0.x; m4[1] = n0.y; m4[2] = n0.z; m4[3] = n0.w;
            m4[4] = n1.x; m4[5] = n1.y; m4[6] = n1.z; m4[7] = n1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                d4f[2 * e] = cvt_half_lo(d4[e]);
                d4f[2 * e + 1] = cvt_half_hi(d4[e]);
            }
        }
        const v4i A = {static_cast<int>((w.x >> shift) & kNibbles), static_cast<int>((w.y >> shift) & kNibbles),
                       static_cast<int>((w.z >> shift) & kNibbles), static_cast<int>((w.w >> shift) & kNibbles)};
        {
            // The offset goes into the per-lane operand, which the range check covers.
            const int nb = B0 + b + kDnWin;
            const uint32_t o = nb < nbi ? static_cast<uint32_t>(nb) * 16u : next_off + static_cast<uint32_t>(nb - nbi) * 16u;
            wa[b % kDnWin] = buffer_load16(wr, w_off + o, 0);
        }
        // Each tile's MFMA is issued before the previous tile is scaled, so
        // the matrix unit works under the scaling and two results are live.
        v16i rp;
        uint32_t hp = 0;
        auto scale_prev = [&](int sp) {
            if constexpr (Q41) scale_block_q41(acc[sp], rp, hp, d4, m4);
            else scale_block_f32(acc[sp], rp, hp, d4f);
            if constexpr (Dbg) {
                const int j = kSub * sp + m;
                if (a.down_dots && j < ncols)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        a.down_dots[(static_cast<size_t>(first + j) * a.shape.H + R0 + 4 * (v & 7) + 2 * h + (v >> 3)) * nbi + B0 + b] =
                            rp[v] - kMagic;
            }
        };
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const v4i B = {static_cast<int>(xb.x), static_cast<int>(xb.y), static_cast<int>(xb.z), static_cast<int>(xb.w)};
            const v16i r = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, magic, 0, 0, 0);
            const uint32_t hs = hx;
            if (s + 1 < NS) {
                xb = st.x[b][kSub * (s + 1) + m][h];
                hx = st.hd[b][kSub * (s + 1) + m];
            } else if (b + 1 < kDnMaxBlocks) {
                xb = st.x[b + 1][m][h];
                hx = st.hd[b + 1][m];
            }
            if (s > 0) scale_prev(s - 1);
            __builtin_amdgcn_sched_barrier(0);
            rp = r;
            hp = hs;
        }
        scale_prev(NS - 1);
        }
    }
}

// Writes a wave's 32-row x (32 x nsub)-pair result tile to the pairs'
// contribution rows.  Lane half h holds rows 4q + 2h (v = q) and
// 4q + 2h + 1 (v = 8 + q), q = 0..7; after the trade lane half h holds rows
// 16h .. 16h + 15 (4 float4 stores per tile).
__device__ __forceinline__ void store_down_tile(const FfnArgs &a, const float (&acc)[kSubs][16], int nsub, int first,
                                                int ncols, int R0) {
    const int lane = threadIdx.x & 63, m = lane & 31, h = lane >> 5;
#pragma unroll
    for (int s = 0; s < kSubs; ++s) {
        if (s >= nsub) break;
        const int j = kSub * s + m;
        const bool valid = j < ncols;
        const int p = first + std::min(j, ncols - 1);
        const size_t orow = static_cast<size_t>(a.routes.pair_token[p]) * a.out_stride_k + a.routes.pair_rank[p];
        float *dst = a.out + orow * a.shape.H + R0 + 16 * h;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // v_permlane32_swap(a, b): lanes < 32 get (own a, a of lane + 32),
            // lanes >= 32 (b of lane - 32, own b) -- for both halves the
            // float4's x and z; the same for y and w.
            const auto xz = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[s][q]),
                                                             __float_as_uint(acc[s][4 + q]), false, false);
            const auto yw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[s][8 + q]),
                                                             __float_as_uint(acc[s][12 + q]), false, false);
            const float4 o = make_float4(__uint_as_float(xz[0]), __uint_as_float(yw[0]), __uint_as_float(xz[1]),
                                         __uint_as_float(yw[1]));
            if (valid) *reinterpret_cast<float4 *>(dst + 4 * q) = o;
        }
    }
}

// The staged path's slices s0 .. s1-1 for one wave, after the staging
// barrier.  wa holds slice s0's first kDnWin weight blocks; buffer 0 of
// st.d4 its scales.
template<int NS, bool Dbg, bool Q41, class Stage>
__device__ __forceinline__ void down_slices(const FfnArgs &a, Stage &st, int wave, uint4 (&wa)[kDnWin], int nbi,
                                            int expert, int first, int ncols, int s0, int s1, uint32_t w_off, int pslot) {
    const int lane = threadIdx.x & 63, H = a.shape.H;
    const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
    for (int sl = s0; sl < s1; ++sl) {
        const int R0 = sl * 128 + wave * 32;
        if (R0 >= H) break;                     // wave-uniform; later slices lie further down
        // Opaque zeros added to the lane index, the weight offset and the
        // block count keep the per-lane LDS and weight addresses (about 80
        // VGPRs) and the window's block offsets (16 SGPRs) from being
        // hoisted out of the loop into registers.
        int zero, szero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        asm volatile("s_mov_b32 %0, 0" : "=s"(szero));
        const int buf = Q41 ? 0 : (sl - s0) & 1;
        const int Rn = R0 + 128;
        const bool pf = sl + 1 < s1 && Rn < H;
        // Loads are unconditional: past the last slice the descriptors are
        // empty and read zeros.
        const size_t rc = static_cast<size_t>(expert) * H + R0, rn = static_cast<size_t>(expert) * H + (pf ? Rn : R0);
        // Rows R0 .. R0 + 31, and R0 + 128 .. R0 + 159 when there is a next slice.
        const auto wr = buffer_rsrc(a.bank.down_codes + rc * row_bytes, (pf ? 160u : 32u) * row_bytes);
        // The next slice's scale tile: nbi * 4 chunks of 16 bytes, one per lane.
        uint4 dn = make_uint4(0, 0, 0, 0);
        if constexpr (!Q41)
            dn = buffer_load16(buffer_rsrc(a.bank.down_scales + rn * nbi, pf ? static_cast<uint32_t>(nbi) * 64u : 0u),
                               16u * static_cast<uint32_t>(lane), 0);
        float acc[kSubs][16];
        const uint4 (*m4s)[4] = nullptr;
        if constexpr (Q41) m4s = st.m4[wave];
        down_staged<NS, Dbg, Q41>(a, st, st.d4[buf][wave], m4s, wa, wr, 128u * row_bytes, w_off + static_cast<uint32_t>(zero), nbi + szero,
                                  first, ncols, R0, pslot, lane + zero, acc);
        if constexpr (!Q41) {
            // The other buffer was last read by slice sl - 1 of this wave.
            if (lane < nbi * 4) st.d4[buf ^ 1][wave][lane >> 2][lane & 3] = dn;
            __builtin_amdgcn_wave_barrier();
        }
        store_down_tile(a, acc, NS, first, ncols, R0);
    }
}

// Stages blocks B0 .. B0 + 15 (those below nbi) of an item's middle codes
// and heads, and of each active wave's 32-row scale (and min) tile, at local
// block indices 0..15.  Thread t keeps one (block, half) of the code rows,
// local block (t % 32) / 2 and half t % 2, for pairs t / 32 + 8 i, and one
// block of the heads, t % 16, for pairs t / 16 + 16 i.  The descriptors end
// at the item's last pair: pairs past ncols read zero.  All loads are issued
// before the first LDS write.
template<int T>
struct DownStager {
    __amdgpu_buffer_rsrc_t xr, hr;
    const uint4 *scales, *mins;   // the wave's [nbi][4] chunks
    uint32_t pair_bytes;
    int cols, nbi, xb, xh, xj, hb, hj;

    __device__ static DownStager make(const FfnArgs &a, int first, int ncols, int nsub, int nbi, size_t rbase) {
        static_assert(kMfmaTile == 128 && kDnMaxBlocks == 16 && (T == 256 || T == 512),
                      "staging map: 256 or 512 threads, 128 pairs, 16 blocks");
        DownStager g;
        g.pair_bytes = static_cast<uint32_t>(nbi) * 32u;
        g.xr = buffer_rsrc(a.mq.codes + static_cast<size_t>(first) * g.pair_bytes, static_cast<uint32_t>(ncols) * g.pair_bytes);
        g.hr = buffer_rsrc(a.mq.heads + static_cast<size_t>(first) * nbi, static_cast<uint32_t>(ncols * nbi) * 4u);
        g.scales = reinterpret_cast<const uint4 *>(a.bank.down_scales + rbase * nbi);
        g.mins = a.bank.down_mins ? reinterpret_cast<const uint4 *>(a.bank.down_mins + rbase * nbi) : nullptr;
        g.cols = nsub * kSub;
        g.nbi = nbi;
        const int tid = static_cast<int>(threadIdx.x);
        g.xb = (tid & 31) >> 1;
        g.xh = tid & 1;
        g.xj = tid >> 5;
        g.hb = tid & 15;
        g.hj = tid >> 4;
        return g;
    }

    template<class Stage>
    __device__ void run(Stage &st, int B0, int wave, int lane, bool active) const {
        const int bx = B0 + xb, bh = B0 + hb;
        const uint32_t x_off = static_cast<uint32_t>(xj) * pair_bytes + static_cast<uint32_t>(32 * bx + 16 * xh);
        const uint32_t h_off = static_cast<uint32_t>(hj * nbi + bh) * 4u;
        // Thread t keeps (block, half) ((t % 32) / 2, t % 2) of pairs t / 32 + PX i
        // and the head of block t % 16 of pairs t / 16 + PH i.
        constexpr int PX = T / 32, PH = T / 16;
        uint4 xv[kMfmaTile / PX];
        uint32_t hv[kMfmaTile / PH];
#pragma unroll
        for (int i = 0; i < kMfmaTile / PX; ++i)
            if (PX * i < cols && bx < nbi) xv[i] = buffer_load16(xr, x_off, static_cast<uint32_t>(PX * i) * pair_bytes);
#pragma unroll
        for (int i = 0; i < kMfmaTile / PH; ++i)
            if (PH * i < cols && bh < nbi) hv[i] = buffer_load4(hr, h_off, static_cast<uint32_t>(PH * i * nbi) * 4u);
#pragma unroll
        for (int i = 0; i < kMfmaTile / PX; ++i)
            if (PX * i < cols && bx < nbi) st.x[xb][xj + PX * i][xh] = xv[i];
#pragma unroll
        for (int i = 0; i < kMfmaTile / PH; ++i)
            if (PH * i < cols && bh < nbi) st.hd[hb][hj + PH * i] = hv[i];
        const int nl = min(nbi - B0, kDnMaxBlocks);
        if (active)
            for (int c = lane; c < nl * 4; c += 64) st.d4[0][wave][c >> 2][c & 3] = scales[B0 * 4 + c];
        if constexpr (Stage::kMins) {
            if (active)
                for (int c = lane; c < nl * 4; c += 64) st.m4[wave][c >> 2][c & 3] = mins[B0 * 4 + c];
        }
    }
};

// Rows of 17..32 down blocks (I = 544..1024; the reference model's 640: 20):
// one 128-row slice per workgroup, its blocks staged in two rounds into the
// same LDS (0..15, then 16..nbi - 1) with the accumulators carried across.
// The weight window already holds blocks 16..23 when the second round
// starts.  Every wave reaches both barriers.
template<int NS, bool Dbg, bool Q41, class Stage, class Stager>
__device__ __forceinline__ void down_two_rounds(const FfnArgs &a, Stage &st, const Stager &sg, int wave, bool active,
                                                uint4 (&wa)[kDnWin], int nbi, int first, int ncols, int R0, size_t rbase,
                                                uint32_t w_off, int pslot) {
    const int lane = threadIdx.x & 63;
    const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
    // This slice's 32 rows; past them (no next slice) the descriptor reads zeros.
    const auto wr = buffer_rsrc(a.bank.down_codes + rbase * row_bytes, 32u * row_bytes);
    const uint4 (*m4s)[4] = nullptr;
    if constexpr (Q41) m4s = st.m4[wave];
    float acc[kSubs][16];
    if (active)
        down_staged_round<NS, Dbg, Q41, Stage, 0>(a, st, st.d4[0][wave], m4s, wa, wr, 32u * row_bytes, w_off, nbi, first, ncols,
                                            R0, pslot, lane, acc);
    __syncthreads();   // every wave is done with blocks 0..15
    sg.run(st, kDnMaxBlocks, wave, lane, active);
    __syncthreads();
    if (!active) return;
    down_staged_round<NS, Dbg, Q41, Stage, kDnMaxBlocks>(a, st, st.d4[0][wave], m4s, wa, wr, 32u * row_bytes, w_off, nbi, first,
                                                   ncols, R0, pslot, lane, acc);
    store_down_tile(a, acc, NS, first, ncols, R0);
}

// R2: rows of 17..32 blocks, staged in two rounds (down_two_rounds); a
// separate instantiation, so the other shapes' kernel keeps its registers.
template<bool Dbg, bool Q41, bool R2 = false>
__global__ __launch_bounds__(256, 2) void k_down_mfma(FfnArgs a) {
    __shared__ std::conditional_t<Q41, DownStageQ41, DownStage> st;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shape.H, nbi = a.shape.I / 32;
    const int slices = (H + 127) / 128;
    const bool staged = R2 || nbi <= kDnMaxBlocks;
    const int span = down_span(nbi, Q41);
    const Unit un = mfma_unit(a.routes.item_counts[1], down_groups(H, nbi, Q41));
    if (!un.ok) return;
    const Item *itp = a.routes.mfma_items + un.item;
    const int expert = itp->expert, first = itp->first, ncols = itp->ncols;
    const int s0 = un.slice * span, s1 = std::min(slices, s0 + span);
    const int R0 = s0 * 128 + wave * 32;
    const bool active = R0 < H;      // wave-uniform
    const int nsub = (ncols + kSub - 1) / kSub;
    const int m = lane & 31, h = lane >> 5;
    const int mv = 4 * (m >> 3) + (m & 3);
    const int prow = 4 * (mv & 7) + 2 * ((m >> 2) & 1) + (mv >> 3);
    const int pslot = (prow & 3) * 8 + (prow >> 2);

    const size_t rbase = static_cast<size_t>(expert) * H + (active ? R0 : 0);
    const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
    const uint16_t *scales = a.bank.down_scales + rbase * nbi;        // [nbi][32] halfs of this 32-row group
    if (staged) {
        // The first weight blocks first (their HBM latency overlaps the staging).
        const auto wr = buffer_rsrc(a.bank.down_codes + rbase * row_bytes, 32u * row_bytes);
        const uint32_t w_off = static_cast<uint32_t>(prow) * row_bytes;
        uint4 wa[kDnWin];
#pragma unroll
        for (int b = 0; b < kDnWin; ++b) wa[b] = buffer_load16(wr, w_off, static_cast<uint32_t>(b < nbi ? b : 0) * 16u);
        if constexpr (R2) {
            // Middle codes and heads of the item's pairs, every load issued
            // before the first LDS write (DownStager).
            const DownStager<256> sg = DownStager<256>::make(a, first, ncols, nsub, nbi, rbase);
            sg.run(st, 0, wave, lane, active);
            __syncthreads();
            switch (nsub) {   // two staging rounds; every wave takes part in their barriers
            case 1: down_two_rounds<1, Dbg, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
            case 2: down_two_rounds<2, Dbg, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
            case 3: down_two_rounds<3, Dbg, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
            default: down_two_rounds<4, Dbg, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
            }
            return;
        }
        // Middle codes and heads of the item's pairs, every load issued
        // before the first LDS write.  Thread t keeps one (block, half) of the
        // code rows, block (t % 32) / 2 and half t % 2, for pairs t / 32 + 8 i,
        // and one block of the heads, t % 16, for pairs t / 16 + 16 i.  The
        // descriptors end at the item's last pair: pairs past ncols read zero.
        static_assert(kMfmaTile == 128 && kDnMaxBlocks == 16, "staging map: 256 threads, 128 pairs, 16 blocks");
        const int cols = nsub * kSub;
        const uint32_t pair_bytes = static_cast<uint32_t>(nbi) * 32u;
        const auto xr = buffer_rsrc(a.mq.codes + static_cast<size_t>(first) * pair_bytes,
                                    static_cast<uint32_t>(ncols) * pair_bytes);
        const auto hr = buffer_rsrc(a.mq.heads + static_cast<size_t>(first) * nbi,
                                    static_cast<uint32_t>(ncols * nbi) * 4u);
        const int tid = static_cast<int>(threadIdx.x);
        const int xb = (tid & 31) >> 1, xh = tid & 1, xj = tid >> 5, hb = tid & 15, hj = tid >> 4;
        const uint32_t x_off = static_cast<uint32_t>(xj) * pair_bytes + static_cast<uint32_t>(32 * xb + 16 * xh);
        const uint32_t h_off = static_cast<uint32_t>(hj * nbi + hb) * 4u;
        uint4 xv[kMfmaTile / 8];
        uint32_t hv[kMfmaTile / 16];
#pragma unroll
        for (int i = 0; i < kMfmaTile / 8; ++i)
            if (8 * i < cols && xb < nbi) xv[i] = buffer_load16(xr, x_off, 8u * i * pair_bytes);
#pragma unroll
        for (int i = 0; i < kMfmaTile / 16; ++i)
            if (16 * i < cols && hb < nbi) hv[i] = buffer_load4(hr, h_off, 64u * i * static_cast<uint32_t>(nbi));
#pragma unroll
        for (int i = 0; i < kMfmaTile / 8; ++i)
            if (8 * i < cols && xb < nbi) st.x[xb][xj + 8 * i][xh] = xv[i];
#pragma unroll
        for (int i = 0; i < kMfmaTile / 16; ++i)
            if (16 * i < cols && hb < nbi) st.hd[hb][hj + 16 * i] = hv[i];
        if (active)
            for (int c = lane; c < nbi * 4; c += 64)
                st.d4[0][wave][c >> 2][c & 3] = reinterpret_cast<const uint4 *>(scales)[c];
        if constexpr (Q41) {
            const uint16_t *mins = a.bank.down_mins + rbase * nbi;   // same layout as the scales
            if (active)
                for (int c = lane; c < nbi * 4; c += 64)
                    st.m4[wave][c >> 2][c & 3] = reinterpret_cast<const uint4 *>(mins)[c];
        }
        __syncthreads();
        if (!active) return;
        switch (nsub) {
        case 1: down_slices<1, Dbg, Q41>(a, st, wave, wa, nbi, expert, first, ncols, s0, s1, w_off, pslot); break;
        case 2: down_slices<2, Dbg, Q41>(a, st, wave, wa, nbi, expert, first, ncols, s0, s1, w_off, pslot); break;
        case 3: down_slices<3, Dbg, Q41>(a, st, wave, wa, nbi, expert, first, ncols, s0, s1, w_off, pslot); break;
        default: down_slices<4, Dbg, Q41>(a, st, wave, wa, nbi, expert, first, ncols, s0, s1, w_off, pslot); break;
        }
        return;
    }
    if (!active) return;   // no barrier on this path
    float acc[kSubs][16];
    const uint32_t pairs = static_cast<uint32_t>(a.pairs_bound);
    TileArgs t;
    t.wr = buffer_rsrc(a.bank.down_codes + rbase * row_bytes, 32u * row_bytes);
    t.sr = buffer_rsrc(scales, static_cast<uint32_t>(nbi) * 64u);
    t.mr = buffer_rsrc(Q41 ? a.bank.down_mins + rbase * nbi : scales, static_cast<uint32_t>(nbi) * 64u);
    t.xr = buffer_rsrc(a.mq.codes, pairs * static_cast<uint32_t>(nbi) * 32u);
    t.hr = buffer_rsrc(a.mq.heads, pairs * static_cast<uint32_t>(nbi) * 4u);
    t.w_off = static_cast<uint32_t>(prow) * row_bytes;
    t.s_off0 = 32u * h;
    t.s_off1 = 32u * h + 16u;
    t.s_step = 64u;
#pragma unroll
    for (int s = 0; s < kSubs; ++s) {
        const uint32_t p = static_cast<uint32_t>(first + std::min(kSub * s + m, ncols - 1));
        t.x_off[s] = p * static_cast<uint32_t>(nbi) * 32u + 16u * h;
        t.h_off[s] = p * static_cast<uint32_t>(nbi) * 4u;
    }
    t.cscale = scales + pslot;
    t.cstride = 32;
    t.nb = nbi;
    t.shift = 4 * h;
    t.dots = Dbg ? a.down_dots : nullptr;
    t.dot_rows = static_cast<size_t>(H);
    t.dot_row0 = R0;
    t.dot_pair0 = first;
    t.ncols = ncols;
    t.m = m;
    t.h = h;
    tile_dispatch<Dbg, true, Q41>(t, nsub, acc);
    store_down_tile(a, acc, nsub, first, ncols, R0);
}

// Q4_0 rows of 17..32 down blocks without debug outputs: a workgroup of 8
// waves takes slices 2u (waves 0-3) and 2u + 1 (waves 4-7) of an item, so
// each staging round (down_two_rounds) serves 256 rows instead of 128.  The
// CU holds one such workgroup (8 waves at 236 VGPRs: two per SIMD, as two
// 4-wave workgroups would).
__global__ __launch_bounds__(512, 1) void k_down_mfma_pair(FfnArgs a) {
    constexpr bool Q41 = false;
    __shared__ DownStage2 st;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shape.H, nbi = a.shape.I / 32;
    const int slices = (H + 127) / 128;
    const Unit un = mfma_unit(a.routes.item_counts[1], (slices + 1) / 2);
    if (!un.ok) return;   // uniform per workgroup
    const Item *itp = a.routes.mfma_items + un.item;
    const int expert = itp->expert, first = itp->first, ncols = itp->ncols;
    const int R0 = (2 * un.slice + (wave >> 2)) * 128 + (wave & 3) * 32;
    const bool active = R0 < H;      // wave-uniform
    const int nsub = (ncols + kSub - 1) / kSub;
    const int m = lane & 31;
    const int mv = 4 * (m >> 3) + (m & 3);
    const int prow = 4 * (mv & 7) + 2 * ((m >> 2) & 1) + (mv >> 3);
    const int pslot = (prow & 3) * 8 + (prow >> 2);
    const size_t rbase = static_cast<size_t>(expert) * H + (active ? R0 : 0);
    const uint32_t row_bytes = static_cast<uint32_t>(nbi) * 16u;
    // The first weight blocks first (their HBM latency overlaps the staging).
    const auto wr = buffer_rsrc(a.bank.down_codes + rbase * row_bytes, 32u * row_bytes);
    const uint32_t w_off = static_cast<uint32_t>(prow) * row_bytes;
    uint4 wa[kDnWin];
#pragma unroll
    for (int b = 0; b < kDnWin; ++b) wa[b] = buffer_load16(wr, w_off, static_cast<uint32_t>(b) * 16u);
    const DownStager<512> sg = DownStager<512>::make(a, first, ncols, nsub, nbi, rbase);
    sg.run(st, 0, wave, lane, active);
    __syncthreads();
    switch (nsub) {   // two staging rounds; every wave takes part in their barriers
    case 1: down_two_rounds<1, false, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
    case 2: down_two_rounds<2, false, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
    case 3: down_two_rounds<3, false, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
    default: down_two_rounds<4, false, Q41>(a, st, sg, wave, active, wa, nbi, first, ncols, R0, rbase, w_off, pslot); break;
    }
}

// Upper bound on MFMA items: a group of n >= mfma_min pairs gives
// ceil(n / 128) items, and at most min(Ep, pairs / mfma_min) groups qualify.
size_t mfma_item_bound(const FfnArgs &a) {
    const size_t P = static_cast<size_t>(a.pairs_bound);
    const size_t G = std::min(P, static_cast<size_t>(a.shape.Ep));
    const size_t big = a.mfma_min >= 1 ? std::min(G, P / static_cast<size_t>(a.mfma_min)) : G;
    return std::max<size_t>(P / kMfmaTile + big, 1);
}

unsigned mfma_grid(const FfnArgs &a, int slices) {
    const size_t units = mfma_item_bound(a) * static_cast<size_t>(slices);
    const size_t round = 8 * static_cast<size_t>(kUnitChunk);
    return static_cast<unsigned>((units + round - 1) / round * round);
}

// row_chunk_unit's grid: the units rounded up to whole rounds of 8 chunks.
unsigned chunk_grid(const FfnArgs &a, int slices) {
    const size_t units = mfma_item_bound(a) * static_cast<size_t>(slices);
    const size_t round = 8 * static_cast<size_t>(kGuChunk);
    return static_cast<unsigned>((units + round - 1) / round * round);
}

// ---------------------------------------------------------------- linear ---
// One Q4_0 matrix against wide column batches (moe_linear), in the gate/up
// kernel's exact order without the SiLU epilogue.  The reference's pairwise
// tree over the 16 level-1 nodes (leaves 2p, 2p+1; leaf k' = blocks k' and
// k' + 32 and, past 64 blocks, their lane's later blocks) splits into four
// 4-node subtrees whose roots combine as (R0 + R1) + (R2 + R3): workgroup =
// one 32-row x 32-column tile, wave w builds subtree w, so a tile's
// sequential work is a quarter of the gate/up kernel's.  The waves share the
// rows' scales staged in LDS.  Ids are XCD-aware: the column tiles of one row
// tile run on one XCD, so its rows are fetched from HBM once.
__device__ __forceinline__ void subtree4_merge(int q, float (&w)[16], float (&l1)[16], float (&l2)[16],
                                               float (&res)[16]) {
    if ((q & 1) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l1[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = l1[i] + w[i];
    if ((q & 2) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l2[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) res[i] = l2[i] + w[i];
}

// wn: the wave's first node's weight half, already in flight (grouped folds).
// The two-node form for 8-wave workgroups: res = node 0 + node 1.
__device__ __forceinline__ void subtree2_merge(int q, float (&w)[16], float (&l1)[16], float (&res)[16]) {
    if ((q & 1) == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) l1[i] = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) res[i] = l1[i] + w[i];
}

// NPW level-1 nodes per wave (4: a 4-wave workgroup, 2: an 8-wave one).
template<int Fold, bool Canon, int NPW>
__device__ __forceinline__ void subtree(const GuTile &t, const GuStage &g, uint32_t w_off, int wave, int lane,
                                        uint4 (&wn)[2], float (&res)[16]) {
    static_assert(NPW == 4 || NPW == 2, "subtree: 2 or 4 nodes per wave");
    const int m = lane & 31, h = lane >> 5;
    float l1[16], l2[16];
    if constexpr (Fold == kFoldGrouped || Fold == kFoldGrouped96) {
        constexpr bool X = Fold == kFoldGrouped96;
        // Node q + 1's weight half is in flight while node q computes.
#pragma unroll 1
        for (int q = 0; q < NPW; ++q) {
            const int p = NPW * wave + q;
            HalfGroup G;
            G.w[0] = wn[0];
            G.w[1] = wn[1];
            half_load_x<Canon>(t, p, G);
            ExtraBlk E;
            if constexpr (X) {
                if (2 * p < t.nb - 64) extra_load<Canon>(t, p, E);   // uniform
            }
            half_load_w(t, w_off, q < NPW - 1 ? p + 1 : p, wn);
            float w[16], x[16];
            leaf_grouped<false, X>(t, g, G, 0, 2 * p, m, h, w, &E);
            leaf_grouped<false, X>(t, g, G, 1, 2 * p + 1, m, h, x, &E);
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i] = w[i] + x[i];
            if constexpr (NPW == 4) subtree4_merge(q, w, l1, l2, res);
            else subtree2_merge(q, w, l1, res);
        }
    } else {
#pragma unroll 1
        for (int q = 0; q < NPW; ++q) {
            const int p = NPW * wave + q;
            float w[16], x[16];
            if constexpr (Fold == kFoldStaged) {
                leaf_staged<false, false, Canon>(t, g, 2 * p, m, h, w);
                leaf_staged<false, false, Canon>(t, g, 2 * p + 1, m, h, x);
            } else {
                fold_leaf_multi<false, Canon>(t, 2 * p, w);
                fold_leaf_multi<false, Canon>(t, 2 * p + 1, x);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i] = w[i] + x[i];
            if constexpr (NPW == 4) subtree4_merge(q, w, l1, l2, res);
            else subtree2_merge(q, w, l1, res);
        }
    }
}

// Canon: the columns are canonical Q8_1 blocks, read in place (codes at
// byte 4 of each 36-byte block, the head at byte 0); else the split planes.
// W = 8: eight waves of two level-1 nodes each, the roots combined
// ((R0 + R1) + (R2 + R3)) + ((R4 + R5) + (R6 + R7)) -- the same tree levels
// as the 4-wave form's (R0 + R1) + (R2 + R3) over 4-node subtrees -- for
// launches whose 4-wave grid leaves SIMDs with one wave.
template<int Fold, bool Canon, int W = 4>
__global__ __launch_bounds__(64 * W, W == 8 ? 1 : 2) void k_linear_mfma(LinearMfmaArgs a) {
    constexpr int NPW = 16 / W, VPW = 16 / W;   // level-1 nodes and finished values per wave
    __shared__ float roots[W][16][64];          // subtree roots [wave][value][lane]
    __shared__ uint4 d4_lds[Fold == kFoldGrouped96 ? kGu96MaxBlocks : kGuMaxBlocks][4];   // [block][32 halfs]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int id = static_cast<int>(blockIdx.x), local = id >> 3;
    const int rt = (id & 7) + 8 * (local / a.col_tiles), ct = local % a.col_tiles;
    if (rt >= a.row_tiles) return;   // uniform per workgroup (grid padded to 8 row tiles)
    const int nb = a.nb, R0 = rt * 32, c0 = ct * kSub;
    const int lane = threadIdx.x & 63;
    const int m = lane & 31, h = lane >> 5;
    const int prow = 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
    const uint32_t col = static_cast<uint32_t>(std::min(c0 + m, a.N - 1));
    const uint32_t row_bytes = static_cast<uint32_t>(nb) * 16u;
    GuTile t;
    t.wr = buffer_rsrc(a.codes + static_cast<size_t>(R0) * row_bytes, 32u * row_bytes);
    t.sr = buffer_rsrc(a.scales + static_cast<size_t>(R0) * nb, 32u * static_cast<uint32_t>(nb) * 2u);
    if constexpr (Canon) {
        t.xr = buffer_rsrc(a.q8, static_cast<uint32_t>(a.N) * static_cast<uint32_t>(nb) * 36u);
        t.hr = t.xr;
        t.x_off = col * static_cast<uint32_t>(nb) * 36u + 4u + 16u * h;
        t.h_off = col * static_cast<uint32_t>(nb) * 36u;
    } else {
        t.xr = buffer_rsrc(a.xq.codes, static_cast<uint32_t>(a.N) * static_cast<uint32_t>(nb) * 32u);
        t.hr = buffer_rsrc(a.xq.heads, static_cast<uint32_t>(a.N) * static_cast<uint32_t>(nb) * 4u);
        t.x_off = col * static_cast<uint32_t>(nb) * 32u + 16u * h;
        t.h_off = col * static_cast<uint32_t>(nb) * 4u;
    }
    t.w_off = static_cast<uint32_t>(prow) * row_bytes;
    t.s_off0 = static_cast<uint32_t>(2 * h * nb) * 16u;
    t.s_off1 = t.s_off0 + static_cast<uint32_t>(nb) * 16u;
    t.nb = nb;
    t.shift = 4 * h;
    t.dots = nullptr;
    t.dot_base = 0;
    t.dot_ok = false;
    // The first node's weight half is issued before the scale staging, so the
    // two round trips overlap.
    const uint32_t w_off = static_cast<uint32_t>(prow) * row_bytes + 32u * 16u * h;
    uint4 wn[2] = {};
    if constexpr (Fold == kFoldGrouped || Fold == kFoldGrouped96) half_load_w(t, w_off, NPW * wave, wn);
    if constexpr (Fold != kFoldMulti) {
        // Scale group g (rows 8g..8g+7) of block b lands at halfs 8g..8g+7 of d4_lds[b].
        for (int c = threadIdx.x; c < 4 * nb; c += blockDim.x) {
            const int gi = c / nb, b = c % nb;
            d4_lds[b][gi] = *reinterpret_cast<const uint4 *>(a.scales + static_cast<size_t>(R0 + 8 * gi) * nb + b * 8);
        }
        __syncthreads();
    }
    const GuStage g{reinterpret_cast<const uint32_t *>(&d4_lds[0][0]), nullptr};
    float res[16];
    subtree<Fold, Canon, NPW>(t, g, w_off, wave, lane, wn, res);
#pragma unroll
    for (int v = 0; v < 16; ++v) roots[wave][v][lane] = res[v];
    __syncthreads();
    // Wave w finishes values VPW w .. VPW w + VPW - 1: rows R0 + 16h + VPW w + i
    // of column c0 + m.
    const int c = c0 + m;
    const int row = R0 + 16 * h + VPW * wave;
    if (c >= a.N || row >= a.M) return;
    float out[VPW];
#pragma unroll
    for (int i = 0; i < VPW; ++i) {
        const int v = VPW * wave + i;
        const float q0 = (roots[0][v][lane] + roots[1][v][lane]) + (roots[2][v][lane] + roots[3][v][lane]);
        if constexpr (W == 4) out[i] = q0;
        else out[i] = q0 + ((roots[4][v][lane] + roots[5][v][lane]) + (roots[6][v][lane] + roots[7][v][lane]));
    }
    float *yr = a.y + static_cast<size_t>(c) * a.M + row;
    if constexpr (W == 4) {
        if (row + 4 <= a.M && (a.M & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) {
            *reinterpret_cast<float4 *>(yr) = make_float4(out[0], out[1], out[2], out[3]);
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < VPW; ++i)
        if (row + i < a.M) yr[i] = out[i];
}

}  // namespace

namespace {
template<bool Canon, int W>
void launch_linear_mfma_t(const LinearMfmaArgs &a, unsigned grid, hipStream_t s) {
    constexpr unsigned T = 64 * W;
    // Only 64-block rows take the 8-wave form: for the other folds the
    // compiler's register allocator (with the iterative-ILP scheduler this
    // file is built with) fails on it.
    if (a.nb == kGuMaxBlocks) k_linear_mfma<kFoldGrouped, Canon, W><<<grid, T, 0, s>>>(a);
    else if (a.nb > kGuMaxBlocks && a.nb <= kGu96MaxBlocks) k_linear_mfma<kFoldGrouped96, Canon><<<grid, 256, 0, s>>>(a);
    else if (a.nb < kGuMaxBlocks) k_linear_mfma<kFoldStaged, Canon><<<grid, 256, 0, s>>>(a);
    else k_linear_mfma<kFoldMulti, Canon><<<grid, 256, 0, s>>>(a);
}
}  // namespace

hipError_t launch_linear_mfma(const LinearMfmaArgs &a, hipStream_t s) {
    const unsigned grid = static_cast<unsigned>((a.row_tiles + 7) / 8 * 8) * static_cast<unsigned>(a.col_tiles);
    const bool w8 = a.waves == 8;
    if (a.q8) {
        if (w8) launch_linear_mfma_t<true, 8>(a, grid, s);
        else launch_linear_mfma_t<true, 4>(a, grid, s);
    } else {
        if (w8) launch_linear_mfma_t<false, 8>(a, grid, s);
        else launch_linear_mfma_t<false, 4>(a, grid, s);
    }
    return hipGetLastError();
}

hipError_t launch_gate_up_mfma(const FfnArgs &a, hipStream_t s) {
    const bool dbg = a.middle_f32 || a.gate_dots || a.up_dots;
    const unsigned grid = chunk_grid(a, a.shape.I / 32 * kSubs);
    const int nb = a.shape.H / 32;
    if (nb == kGuMaxBlocks) {
        if (dbg) k_gate_up_mfma<kFoldGrouped, true><<<grid, 128, 0, s>>>(a);
        else k_gate_up_mfma<kFoldGrouped, false><<<grid, 128, 0, s>>>(a);
    } else if (nb > kGuMaxBlocks && nb <= kGu96MaxBlocks) {
        if (dbg) k_gate_up_mfma<kFoldGrouped96, true><<<grid, 128, 0, s>>>(a);
        else k_gate_up_mfma<kFoldGrouped96, false><<<grid, 128, 0, s>>>(a);
    } else if (nb < kGuMaxBlocks) {
        if (dbg) k_gate_up_mfma<kFoldStaged, true><<<grid, 128, 0, s>>>(a);
        else k_gate_up_mfma<kFoldStaged, false><<<grid, 128, 0, s>>>(a);
    } else {
        if (dbg) k_gate_up_mfma<kFoldMulti, true><<<grid, 128, 0, s>>>(a);
        else k_gate_up_mfma<kFoldMulti, false><<<grid, 128, 0, s>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_down_mfma(const FfnArgs &a, hipStream_t s) {
    const bool q41 = a.bank.down_mins != nullptr;
    const unsigned grid = mfma_grid(a, down_groups(a.shape.H, a.shape.I / 32, q41));
    // Rows of 17..32 blocks take two staging rounds; the debug build (per-block
    // dots) keeps them on the tile path, whose register use it can afford.
    const int nbi = a.shape.I / 32;
    const bool r2 = nbi > kDnMaxBlocks && nbi <= 2 * kDnMaxBlocks;
    if (a.down_dots) {
        if (q41) k_down_mfma<true, true><<<grid, 256, 0, s>>>(a);
        else k_down_mfma<true, false><<<grid, 256, 0, s>>>(a);
    } else if (r2 && !q41) {
        // Two slices per 8-wave workgroup (2560/640 4K Zipf(1.1) layer with
        // Q4_0 downs 2.70-2.71 -> 2.46 ms); with Q4_1 rows (254 VGPRs, 88 KB
        // of LDS) it ran 2.71 -> 2.75 ms, so those keep one slice per workgroup.
        const unsigned pgrid = mfma_grid(a, ((a.shape.H + 127) / 128 + 1) / 2);   // k_down_mfma_pair's units per item
        k_down_mfma_pair<<<pgrid, 512, 0, s>>>(a);
    } else if (r2) {
        k_down_mfma<false, true, true><<<grid, 256, 0, s>>>(a);
    } else if (q41) k_down_mfma<false, true><<<grid, 256, 0, s>>>(a);
    else k_down_mfma<false, false><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace moe
