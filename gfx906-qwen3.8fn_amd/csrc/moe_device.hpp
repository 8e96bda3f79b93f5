// Device primitives shared by the kernel translation units (moe_kernels.hip,
// moe_mfma.hip): fp16 conversions, the Q4_0 x Q8 block dot, the Q8_1
// quantizers with the reference's XOR-butterfly raw sum, SiLU(g)*u with the
// reference's sanitisation, and raw buffer loads.  gfx950 (CDNA4), wave64.
#pragma once

#include "moe_expf.h"
#include "moe_internal.hpp"

#include <hip/hip_fp16.h>

#if defined(__FAST_MATH__)
#error "moe kernels require strict IEEE fp32 (correctly rounded division for Q8 scales)"
#endif
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "moe kernels are written for gfx950 (CDNA4)"
#endif

#pragma clang fp contract(off)

namespace moe {
namespace {

// ------------------------------------------------------------ primitives ---
__device__ __forceinline__ float h2f(uint32_t bits) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits & 0xffffu)));
}
__device__ __forceinline__ uint32_t f2h(float v) {
    return __half_as_ushort(__float2half_rn(v));
}

// a . b (signed bytes) from a zero accumulator in one instruction: the VOP3P
// v_dot4_i32_i8 takes the 0 inline, where the builtin becomes a v_mov of 0
// into the destination plus the accumulating v_dot4c.
__device__ __forceinline__ int sdot4_first(int a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Integer block dot over one Q4_0 code chunk (16 bytes: byte j holds element j
// in its low nibble and element j+16 in its high nibble) and 32 Q8 codes
// (x0 = codes 0..15, x1 = codes 16..31).  Nibbles are 0..15, so v_dot4_i32_i8
// on the masked bytes is the exact unsigned-nibble x signed-code sum.
__device__ __forceinline__ int dot_block(uint4 w, uint4 x0, uint4 x1) {
    constexpr uint32_t m = 0x0f0f0f0fu;
    int s = sdot4_first(static_cast<int>(w.x & m), static_cast<int>(x0.x));
    s = __builtin_amdgcn_sdot4(static_cast<int>(w.y & m), static_cast<int>(x0.y), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(w.z & m), static_cast<int>(x0.z), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(w.w & m), static_cast<int>(x0.w), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((w.x >> 4) & m), static_cast<int>(x1.x), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((w.y >> 4) & m), static_cast<int>(x1.y), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((w.z >> 4) & m), static_cast<int>(x1.z), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((w.w >> 4) & m), static_cast<int>(x1.w), s, false);
    return s;
}

// The value of lane l ^ D (D = 1, 2, 4, 8, 16, 32) without the LDS round trip
// of a shuffle: DPP quad permutes for 1 and 2, a half-row mirror then a quad
// reversal for 4 (7 - i, then i ^ 3 within the quad, is i ^ 4), a rotation by
// 8 of the 16-lane row for 8, one bit-mask swizzle for 16 and
// v_permlane32_swap for 32 (the swap of a register with itself leaves the
// partner half's value in the second result for lanes < 32 and in the first
// for lanes >= 32).  D <= 16 stays within each 32-lane half, so the same
// partner serves a butterfly of width 32.  The exact XOR partner keeps the
// butterfly sums in the reference's order.
template<int D>
__device__ __forceinline__ int lane_xor(int v) {
    if constexpr (D == 1) return __builtin_amdgcn_update_dpp(v, v, 0xb1, 0xf, 0xf, false);        // quad_perm 1,0,3,2
    else if constexpr (D == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4e, 0xf, 0xf, false);   // quad_perm 2,3,0,1
    else if constexpr (D == 4) {
        const int m = __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false);                  // row_half_mirror
        return __builtin_amdgcn_update_dpp(m, m, 0x1b, 0xf, 0xf, false);                          // quad_perm 3,2,1,0
    } else if constexpr (D == 8) return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false); // row_ror:8
    else if constexpr (D == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401f);   // bit-mask mode: and 31, xor 16
    else {
        static_assert(D == 32, "lane_xor: D in 1, 2, 4, 8, 16, 32");
        const auto r = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false,
                                                        false);
        return static_cast<int>((threadIdx.x & 32) ? r[0] : r[1]);
    }
}
template<int D>
__device__ __forceinline__ float lane_xor(float v) {
    return __int_as_float(lane_xor<D>(__float_as_int(v)));
}
// A butterfly over the 32 lanes of each half: op(v, partner) for D = 1 .. 16.
template<class T, class Op>
__device__ __forceinline__ T half_butterfly(T v, Op op) {
    v = op(v, lane_xor<1>(v));
    v = op(v, lane_xor<2>(v));
    v = op(v, lane_xor<4>(v));
    v = op(v, lane_xor<8>(v));
    return op(v, lane_xor<16>(v));
}
template<int D>
__device__ __forceinline__ float xor_sum(float v) { return v + lane_xor<D>(v); }
// v + partner for D = M, M / 2, .. 1 (a butterfly sum from the widest stage).
template<int M>
__device__ __forceinline__ float xor_sum_from(float v) {
    if constexpr (M >= 1) return xor_sum_from<M / 2>(xor_sum<M>(v));
    else return v;
}

// The two fragment dots of one block in the reference CPU/MMVQ order
// (src/cpu_expert.cpp:156-213): fragment f covers code bytes 8f..8f+7, i.e.
// elements 8f..8f+7 (low nibbles, codes x0) and 16+8f..16+8f+7 (high
// nibbles, codes x1).  dot_block(w, x0, x1) is their sum.
__device__ __forceinline__ void fragment_dots(uint4 w, uint4 x0, uint4 x1, int &f0, int &f1) {
    constexpr uint32_t m = 0x0f0f0f0fu;
    f0 = sdot4_first(static_cast<int>(w.x & m), static_cast<int>(x0.x));
    f0 = __builtin_amdgcn_sdot4(static_cast<int>(w.y & m), static_cast<int>(x0.y), f0, false);
    f0 = __builtin_amdgcn_sdot4(static_cast<int>((w.x >> 4) & m), static_cast<int>(x1.x), f0, false);
    f0 = __builtin_amdgcn_sdot4(static_cast<int>((w.y >> 4) & m), static_cast<int>(x1.y), f0, false);
    f1 = sdot4_first(static_cast<int>(w.z & m), static_cast<int>(x0.z));
    f1 = __builtin_amdgcn_sdot4(static_cast<int>(w.w & m), static_cast<int>(x0.w), f1, false);
    f1 = __builtin_amdgcn_sdot4(static_cast<int>((w.z >> 4) & m), static_cast<int>(x1.z), f1, false);
    f1 = __builtin_amdgcn_sdot4(static_cast<int>((w.w >> 4) & m), static_cast<int>(x1.w), f1, false);
}

// fma(d4, t, +0) with d4 given as the lo / hi fp16 half of a word.
__device__ __forceinline__ float mul_half_lo(uint32_t h2, float t) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(t));
    return r;
}
__device__ __forceinline__ float mul_half_hi(uint32_t h2, float t) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(t));
    return r;
}

// Down projection form (K = I/32 <= 16 blocks): 16 lanes per row group, lane
// kl = block kl, eight rows per lane (row index l of w[l], scale half l of
// d4p).  The reference's order for K <= 16 blocks (src/cpu_expert.cpp:156-213)
// is: z = fma(d4, fma(float(I_f), d8, -4 s8), +0) per block and fragment;
// the 128-lane fold first adds +0 (lanes k + 32 are empty), then the two
// fragments, then the blocks pairwise in index order (XOR 1, 2, 4, 8), and
// finally +0 again (the empty upper half).  (z0 + 0) + (z1 + 0) equals
// (z0 + z1) + 0 for every pair of floats, so each +0 is done once.  Rows are
// traded during the first three stages: lane l ends with the total of row
// 4*(l & 1) + 2*(l>>1 & 1) + (l>>2 & 1); lanes l and l ^ 8 agree.
//
// Q41: Q4_1 rows (m4p holds the rows' m as d4p holds d).  Per block
// dd = half(d4*d8), ms = half(m4*s8) (RNE) and per fragment
// z = +0 + fma(float(I_f), dd, ms*0.5) (src/cpu_expert.cpp:167-194); the
// fold is the same.
template<bool Q41>
__device__ __forceinline__ float rows8_down_exact(const uint4 (&w)[8], uint4 d4p, uint4 m4p, uint4 x0, uint4 x1,
                                                  uint32_t head, bool has, int lane) {
    const float d8 = h2f(head), s8 = h2f(head >> 16), c4 = -4.0f * s8;
    const bool c0 = lane & 1, c1 = lane & 2, c2 = lane & 4;
    float v4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float z[2];   // rows i, i + 4
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int q = i + 4 * h;
            int f0, f1;
            fragment_dots(w[q], x0, x1, f0, f1);
            const uint32_t d4w = (&d4p.x)[q >> 1];
            float z0, z1;
            if constexpr (Q41) {
                const uint32_t m4w = (&m4p.x)[q >> 1];
                const float d4 = (q & 1) ? h2f(d4w >> 16) : h2f(d4w), m4 = (q & 1) ? h2f(m4w >> 16) : h2f(m4w);
                const float dd = h2f(f2h(d4 * d8)), hm = h2f(f2h(m4 * s8)) * 0.5f;
                z0 = fmaf(static_cast<float>(f0), dd, hm);
                z1 = fmaf(static_cast<float>(f1), dd, hm);
            } else {
                const float t0 = fmaf(static_cast<float>(f0), d8, c4), t1 = fmaf(static_cast<float>(f1), d8, c4);
                z0 = (q & 1) ? mul_half_hi(d4w, t0) : mul_half_lo(d4w, t0);
                z1 = (q & 1) ? mul_half_hi(d4w, t1) : mul_half_lo(d4w, t1);
            }
            z[h] = has ? (z0 + z1) + 0.0f : 0.0f;
        }
        const float send = c0 ? z[0] : z[1];
        const float keep = c0 ? z[1] : z[0];
        v4[i] = keep + lane_xor<1>(send);
        __builtin_amdgcn_sched_barrier(0);   // one row pair at a time (register pressure)
    }
    float v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float send = c1 ? v4[i] : v4[i + 2];
        const float keep = c1 ? v4[i + 2] : v4[i];
        v2[i] = keep + lane_xor<2>(send);
    }
    float v = (c2 ? v2[1] : v2[0]) + lane_xor<4>(c2 ? v2[0] : v2[1]);
    v = xor_sum<8>(v);
    return v + 0.0f;
}

// One down (row, block) chunk as rows8_down_exact forms it before its block
// tree: both fragments scaled, then (z0 + z1) + 0, or +0 for a block past the
// row end.  d4h / m4h hold the row's fp16 scale / min in their low halves.
template<bool Q41>
__device__ __forceinline__ float down_chunk(uint4 w, uint32_t d4h, uint32_t m4h, uint4 x0, uint4 x1, uint32_t head,
                                            bool has) {
    const float d8 = h2f(head), s8 = h2f(head >> 16), c4 = -4.0f * s8;
    int f0, f1;
    fragment_dots(w, x0, x1, f0, f1);
    float z0, z1;
    if constexpr (Q41) {
        const float d4 = h2f(d4h), m4 = h2f(m4h);
        const float dd = h2f(f2h(d4 * d8)), hm = h2f(f2h(m4 * s8)) * 0.5f;
        z0 = fmaf(static_cast<float>(f0), dd, hm);
        z1 = fmaf(static_cast<float>(f1), dd, hm);
    } else {
        const float t0 = fmaf(static_cast<float>(f0), d8, c4), t1 = fmaf(static_cast<float>(f1), d8, c4);
        z0 = mul_half_lo(d4h, t0);
        z1 = mul_half_lo(d4h, t1);
    }
    return has ? (z0 + z1) + 0.0f : 0.0f;
}

// Eight weight rows (w[q], scales d4p: row q at half q) against one token's
// Q8 block per lane (lane = block, H/32 <= 64), summed in the reference's
// exact fp32 order (src/cpu_expert.cpp:156-213, the gfx906 MMVQ reduction):
// per block and fragment z = fma(d4, fma(float(I_f), d8, -4 s8), +0); the
// reference's 128-lane fold adds lane k' and k'+32 per fragment, then the two
// fragments, then the blocks pairwise in index order (XOR 1, 2, 4, 8, 16).
// Rows are traded between lanes during the first stages so every lane ends
// with one row's total: lane l holds row 4*(l>>5 & 1) + 2*(l & 1) + (l>>1 & 1).
// The first stage is one v_permlane32_swap of rows i and i + 4: lanes < 32
// then hold (row i own, row i of lane + 32), lanes >= 32 (row i + 4 of lane
// - 32, own), and one add finishes both (fp32 addition commutes, so each
// pair gives the reference's bits).  Lanes with `has` false (blocks past H)
// contribute +0, as the reference's unused lanes do; Full (H/32 == 64) drops
// that select.
template<bool Full = false>
__device__ __forceinline__ float rows8_exact(const uint4 (&w)[8], uint4 d4p, uint4 x0, uint4 x1, uint32_t head,
                                             bool has, int lane) {
    const float d8 = h2f(head), c4 = -4.0f * h2f(head >> 16);
    const bool b0 = lane & 1, b1 = lane & 2;
    float v4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float z[2][2];   // [row i / i + 4][fragment]
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int q = i + 4 * h;
            int f0, f1;
            fragment_dots(w[q], x0, x1, f0, f1);
            const uint32_t d4w = (&d4p.x)[q >> 1];
            const float t0 = fmaf(static_cast<float>(f0), d8, c4), t1 = fmaf(static_cast<float>(f1), d8, c4);
            const float z0 = (q & 1) ? mul_half_hi(d4w, t0) : mul_half_lo(d4w, t0);
            const float z1 = (q & 1) ? mul_half_hi(d4w, t1) : mul_half_lo(d4w, t1);
            z[h][0] = Full || has ? z0 : 0.0f;
            z[h][1] = Full || has ? z1 : 0.0f;
        }
        float u[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(z[0][f]), __float_as_uint(z[1][f]),
                                                            false, false);
            u[f] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        v4[i] = u[0] + u[1];
        __builtin_amdgcn_sched_barrier(0);   // one row pair at a time (register pressure)
    }
    float v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float send = b0 ? v4[i] : v4[i + 2];
        const float keep = b0 ? v4[i + 2] : v4[i];
        v2[i] = keep + lane_xor<1>(send);
    }
    float v = (b1 ? v2[1] : v2[0]) + lane_xor<2>(b1 ? v2[0] : v2[1]);
    v = xor_sum<4>(v);
    v = xor_sum<8>(v);
    return xor_sum<16>(v);
}

// The same reduction for lane partials already summed over several blocks
// (lane j holds both fragments' accumulators of blocks j, j + 64, ... for 8
// rows): z[row][f] -> lane j + lane j ^ 32 per fragment (one
// v_permlane32_swap per row pair, as in rows8_exact), then the two
// fragments, then XOR 1, 2, 4, 8, 16.  Lane l ends with row
// 4*(l>>5 & 1) + 2*(l & 1) + (l>>1 & 1).
__device__ __forceinline__ float fold_rows8(const float (&z)[8][2], int lane) {
    const bool b0 = lane & 1, b1 = lane & 2;
    float v4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float u[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(z[i][f]), __float_as_uint(z[i + 4][f]),
                                                            false, false);
            u[f] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        v4[i] = u[0] + u[1];
    }
    float v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float send = b0 ? v4[i] : v4[i + 2];
        const float keep = b0 ? v4[i + 2] : v4[i];
        v2[i] = keep + lane_xor<1>(send);
    }
    float v = (b1 ? v2[1] : v2[0]) + lane_xor<2>(b1 ? v2[0] : v2[1]);
    v = xor_sum<4>(v);
    v = xor_sum<8>(v);
    return xor_sum<16>(v);
}

// fold_rows8 for 4 rows: z[row][f] -> lane j + lane j ^ 32 per fragment (row
// pairs i, i + 2), the two fragments, then XOR 1, 2, 4, 8, 16 -- per row the
// same additions in the same order.  Lane l ends with row 2*(l>>5 & 1) +
// (l & 1).
__device__ __forceinline__ float fold_rows4(const float (&z)[4][2], int lane) {
    const bool b0 = lane & 1;
    float v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float u[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(z[i][f]), __float_as_uint(z[i + 2][f]),
                                                            false, false);
            u[f] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        v2[i] = u[0] + u[1];
    }
    float v = (b0 ? v2[1] : v2[0]) + lane_xor<1>(b0 ? v2[0] : v2[1]);
    v = xor_sum<2>(v);
    v = xor_sum<4>(v);
    v = xor_sum<8>(v);
    return xor_sum<16>(v);
}

// rows8_exact for rows of 65..128 blocks: lane j holds blocks j (w, d4p, x0,
// x1, head) and j + 64 (w2, ..., present when has2).  The reference's lane
// 2j + f accumulates its blocks in ascending order,
// acc = fma(d4, fma(float(I_f), d8, -4 s8), acc) from +0 (src/cpu_expert.cpp:
// 156-213), and the accumulators are then folded as by rows8_exact.
__device__ __forceinline__ float rows8_exact2(const uint4 (&w)[8], uint4 d4p, uint4 x0, uint4 x1, uint32_t head,
                                              const uint4 (&w2)[8], uint4 d4p2, uint4 y0, uint4 y1, uint32_t head2,
                                              bool has2, int lane) {
    const float d8 = h2f(head), c4 = -4.0f * h2f(head >> 16);
    const float e8 = h2f(head2), e4 = -4.0f * h2f(head2 >> 16);
    float acc[8][2];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        int f0, f1, g0, g1;
        fragment_dots(w[q], x0, x1, f0, f1);
        fragment_dots(w2[q], y0, y1, g0, g1);
        const uint32_t da = (&d4p.x)[q >> 1] >> (16 * (q & 1)), db = (&d4p2.x)[q >> 1] >> (16 * (q & 1));
        const float a4 = h2f(da), b4 = h2f(db);
        const float a0 = fmaf(a4, fmaf(static_cast<float>(f0), d8, c4), 0.0f);
        const float a1 = fmaf(a4, fmaf(static_cast<float>(f1), d8, c4), 0.0f);
        const float s0 = fmaf(b4, fmaf(static_cast<float>(g0), e8, e4), a0);
        const float s1 = fmaf(b4, fmaf(static_cast<float>(g1), e8, e4), a1);
        acc[q][0] = has2 ? s0 : a0;
        acc[q][1] = has2 ? s1 : a1;
    }
    return fold_rows8(acc, lane);
}

// rows8_exact2 with the second block's t values already formed: lane j (has2)
// holds t2[q][f] = fma(float(I_f), d8', -4 s8') of row q and block j + 64 and
// that block's scales d4p2; the arithmetic and fold are rows8_exact2's.
__device__ __forceinline__ float rows8_exact2t(const uint4 (&w)[8], uint4 d4p, uint4 x0, uint4 x1, uint32_t head,
                                               uint4 d4p2, const float (&t2)[8][2], bool has2, int lane) {
    const float d8 = h2f(head), c4 = -4.0f * h2f(head >> 16);
    float acc[8][2];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        int f0, f1;
        fragment_dots(w[q], x0, x1, f0, f1);
        const uint32_t da = (&d4p.x)[q >> 1] >> (16 * (q & 1)), db = (&d4p2.x)[q >> 1] >> (16 * (q & 1));
        const float a4 = h2f(da), b4 = h2f(db);
        const float a0 = fmaf(a4, fmaf(static_cast<float>(f0), d8, c4), 0.0f);
        const float a1 = fmaf(a4, fmaf(static_cast<float>(f1), d8, c4), 0.0f);
        const float s0 = fmaf(b4, t2[q][0], a0);
        const float s1 = fmaf(b4, t2[q][1], a1);
        acc[q][0] = has2 ? s0 : a0;
        acc[q][1] = has2 ? s1 : a1;
    }
    return fold_rows8(acc, lane);
}

// One Q8_1 block from 32 lanes (lane32 = element index).  Semantics of the
// reference GPU quantizer (src/hip/linear.hip:121-149): a nonfinite element
// poisons its block (bit 1), an unrepresentable scale/sum/code sets bit 2,
// and a failing block is written as all zero.  The raw sum is the ascending
// XOR butterfly 1,2,4,8,16 of the (sanitised) inputs -- each stage adds the
// partner's value, so both partners hold the same sum as in the reference.
struct Q8Lane {
    int8_t code;
    uint32_t head;   // half d | half s << 16 (valid in every lane)
    int flags;       // per-block flags (valid in every lane)
};

__device__ __forceinline__ Q8Lane quantize32(float x) {
    int bad = !isfinite(x);
    if (bad) x = 0.0f;
    float amax = fabsf(x);
    amax = half_butterfly(amax, [](float a, float b) { return fmaxf(a, b); });
    bad = half_butterfly(bad, [](int a, int b) { return a | b; });
    const float sum = half_butterfly(x, [](float a, float b) { return a + b; });
    const float d = amax / 127.0f;
    const uint32_t hd = f2h(d), hs = f2h(sum);
    const bool representable = isfinite(sum) && (hs & 0x7c00u) != 0x7c00u &&
                               (hd & 0x7c00u) != 0x7c00u && (amax == 0.0f || d > 0.0f);
    const float code = (!bad && representable && amax != 0.0f) ? roundf(x / d) : 0.0f;
    int bad_code = !isfinite(code) || code < -127.0f || code > 127.0f;
    bad_code = half_butterfly(bad_code, [](int a, int b) { return a | b; });
    const bool valid = !bad && representable && !bad_code;
    Q8Lane q;
    q.code = valid ? static_cast<int8_t>(code) : int8_t{0};
    q.head = (valid && amax != 0.0f) ? (hd | (hs << 16)) : 0u;
    q.flags = (bad ? 1 : 0) | ((representable && !bad_code) ? 0 : 2);
    return q;
}

// One Q8_1 block from P lanes (P = 2 or 4): lane l holds elements
// (32/P) * part .. +32/P-1 of its block, part = l / (64/P); the partners are
// lanes l ^ 32 (and l ^ 16 for P = 4).  Same bits as quantize32: max is
// order-free, and each part's pairwise sum is an aligned subtree of the XOR
// butterfly 1..16, whose last stages combine the parts in the same order.
// codes[] gets the lane's 32/P codes (4 per word, element order); head and
// flags are valid in every lane of the block.
template<int P>
struct Q8Part {
    uint32_t codes[8 / P];
    uint32_t head;
    int flags;
};

template<int P>
__device__ __forceinline__ Q8Part<P> quantize_part(float (&v)[32 / P]) {
    constexpr int n = 32 / P;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < n; ++i)
        if (!isfinite(v[i])) { bad = 1; v[i] = 0.0f; }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(v[i]));
    float t[n];
#pragma unroll
    for (int i = 0; i < n; ++i) t[i] = v[i];
#pragma unroll
    for (int w = n / 2; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) t[i] = t[2 * i] + t[2 * i + 1];
    float sum = t[0];
    if constexpr (P == 4) {
        amax = fmaxf(amax, lane_xor<16>(amax));
        bad |= lane_xor<16>(bad);
        sum = sum + lane_xor<16>(sum);
    }
    amax = fmaxf(amax, lane_xor<32>(amax));
    bad |= lane_xor<32>(bad);
    sum = sum + lane_xor<32>(sum);   // commutative: every lane of the block agrees
    const float d = amax / 127.0f;
    const uint32_t hd = f2h(d), hs = f2h(sum);
    const bool representable = isfinite(sum) && (hs & 0x7c00u) != 0x7c00u &&
                               (hd & 0x7c00u) != 0x7c00u && (amax == 0.0f || d > 0.0f);
    const bool quant = !bad && representable && amax != 0.0f;
    int bad_code = 0;
    Q8Part<P> q;
#pragma unroll
    for (int w = 0; w < n / 4; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float c = quant ? roundf(v[4 * w + b] / d) : 0.0f;
            bad_code |= !isfinite(c) || c < -127.0f || c > 127.0f;
            word |= (static_cast<uint32_t>(static_cast<int>(c)) & 0xffu) << (8 * b);
        }
        q.codes[w] = word;
    }
    if constexpr (P == 4) bad_code |= lane_xor<16>(bad_code);
    bad_code |= lane_xor<32>(bad_code);
    const bool valid = !bad && representable && !bad_code;
#pragma unroll
    for (int w = 0; w < n / 4; ++w) q.codes[w] = valid ? q.codes[w] : 0u;
    q.head = (valid && amax != 0.0f) ? (hd | (hs << 16)) : 0u;
    q.flags = (bad ? 1 : 0) | ((representable && !bad_code) ? 0 : 2);
    return q;
}

// moe_expf's 32 64-bit table entries as 64 dwords, one per lane (lane l
// holds dword l): loaded once at kernel start, read in an epilogue with two
// lane shuffles instead of a memory access on the epilogue's critical path.
// Every lane of the wave must take part in the shuffles.
__device__ __forceinline__ uint32_t expf_table_word(int lane) {
    return reinterpret_cast<const uint32_t *>(moe_expf_table_device)[lane & 63];
}

struct LaneExpfTable {
    uint32_t word;
    __device__ __forceinline__ uint64_t operator()(int i) const {
        const uint32_t lo = static_cast<uint32_t>(__shfl(static_cast<int>(word), 2 * i, 64));
        const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(word), 2 * i + 1, 64));
        return (static_cast<uint64_t>(hi) << 32) | lo;
    }
};

// SiLU(g)*u with the reference's sanitisation (src/hip/linear.hip:106-120),
// expf's table read through `table` (MoeExpfTable: memory; LaneExpfTable:
// registers, the whole wave calling).
template<typename Table>
__device__ __forceinline__ float silu_mul(float g, float u, int &flags, const Table &table) {
    if (!isfinite(g)) { flags |= 1; g = 0.0f; }
    if (!isfinite(u)) { flags |= 1; u = 0.0f; }
    float a = g / (1.0f + moe_expf_with(-g, table));
    if (!isfinite(a)) { flags |= 2; a = 0.0f; }
    float v = a * u;
    if (!isfinite(v)) { flags |= 2; v = 0.0f; }
    return flags ? 0.0f : v;
}

__device__ __forceinline__ float silu_mul(float g, float u, int &flags) {
    return silu_mul(g, u, flags, MoeExpfTable{});
}

// -------------------------------------------------------- buffer loads ---
// Raw buffer loads: a uniform base in a buffer resource (SGPRs), a 32-bit
// per-lane offset and a uniform SGPR offset.  A wave's row loads then share
// one offset VGPR and are all issued before the first is waited for.  The
// resource covers `bytes` from `base` (dword 3 = 32-bit data format, the gfx9
// raw-buffer setting).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, off, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// The same with the nontemporal cache policy (nt): for weight streams that a
// launch reads once (cold B8 decode 34.1-34.6 -> 33.4-33.7 us per layer).
__device__ __forceinline__ uint4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, off, 2);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, lane_off, off, 0);
}

}  // namespace
}  // namespace moe
