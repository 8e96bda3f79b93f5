/*
 * moe_expf.h -- single-precision exp with the bits of the host C library.
 *
 * The reference's CPU expert computes SiLU with the host's expf
 * (src/cpu_expert.cpp:251, std::exp on a float) and its GPU kernels with the
 * device expf (src/hip/linear.hip:113); it records device/host expf parity as
 * unqualified (src/cpu_expert.hpp:73-74).  A 1-ulp difference there can move a
 * middle value across a Q8 rounding boundary, and one changed middle code of
 * the shared expert moves its token's output by ~1e-2 rms.  So the device
 * evaluates expf exactly as the host library on the target image does
 * (glibc 2.35, x86-64 FMA build), restated from the published method.
 * Source of the method: Szabolcs Nagy's expf in ARM's optimized-routines
 * (math/expf.c, MIT OR Apache-2.0 WITH LLVM-exception), which glibc adopted
 * as sysdeps/ieee754/flt-32/e_expf.c (LGPL-2.1-or-later); no code of either
 * is copied here, only the algorithm and its published polynomial and shift
 * constants, which fix the result bits:
 *
 *   k = round(x * 32/ln2), r = x * 32/ln2 - k          (double, via 1.5*2^52 shift)
 *   2^(k/32) = table[k % 32] with k/32 added to the exponent field
 *   2^(r/32) ~ C2' r + 1 + (C0' r + C1') r^2           (cubic, Horner with FMAs)
 *   result = (float)(2^(k/32) * 2^(r/32))
 *
 * where table[i] = bits(2^(i/32)) - (i << 47), computed here from the
 * mathematics, and the FMA build fuses x * 32/ln2 into both the shift and the
 * reduction.  The host build of this function (moe_expf_host) was compared
 * with the host expf over all 2^32 inputs (0 mismatches) and is compared on a
 * dense sample by the CPU tests; the device build performs the same IEEE
 * double operations and is compared on the GPU (moe_expf_device).
 */
#ifndef MOE_EXPF_H
#define MOE_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define MOE_EXPF_FN __host__ __device__ __forceinline__
#define MOE_EXPF_MEMBER __host__ __device__ __forceinline__
#else
#define MOE_EXPF_FN static inline
#define MOE_EXPF_MEMBER inline
#endif

MOE_EXPF_FN double moe_expf_asdouble(uint64_t u) {
    double d;
    __builtin_memcpy(&d, &u, sizeof d);
    return d;
}
MOE_EXPF_FN uint64_t moe_expf_asuint64(double d) {
    uint64_t u;
    __builtin_memcpy(&u, &d, sizeof u);
    return u;
}
MOE_EXPF_FN uint32_t moe_expf_asuint(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, sizeof u);
    return u;
}

/* bits(2^(i/32)) - (i << 47): adding k << 47 to entry k % 32 scales by 2^(k/32).
 * A memory table rather than a switch: with a lane-dependent index a switch
 * becomes a select chain whose 32 64-bit constants occupy registers. */
#define MOE_EXPF_TABLE_VALUES \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t moe_expf_table_device[32] = {MOE_EXPF_TABLE_VALUES};
#endif
static const uint64_t moe_expf_table_host[32] = {MOE_EXPF_TABLE_VALUES};

MOE_EXPF_FN uint64_t moe_expf_table(int i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return moe_expf_table_device[i & 31];
#else
    return moe_expf_table_host[i & 31];
#endif
}

struct MoeExpfTable {
    MOE_EXPF_MEMBER uint64_t operator()(int i) const { return moe_expf_table(i); }
};

/* The function in three steps, so that callers evaluating several values can
 * issue all table reads together: the argument reduction (k, as the shifted
 * double kd and its bits ki), the table index, and the rest given the entry. */
struct MoeExpfReduced {
    double xd, kd;
    uint64_t ki;
};

MOE_EXPF_FN MoeExpfReduced moe_expf_reduce(float x) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    MoeExpfReduced r;
    r.xd = (double)x;
    r.kd = __builtin_fma(inv_ln2_n, r.xd, shift);
    r.ki = moe_expf_asuint64(r.kd);
    return r;
}

MOE_EXPF_FN int moe_expf_index(const MoeExpfReduced &r) { return (int)(r.ki & 31u); }

MOE_EXPF_FN float moe_expf_finish(float x, const MoeExpfReduced &red, uint64_t entry) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t abstop = (moe_expf_asuint(x) >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                                   /* |x| >= 88 (top bits of 88.0f) */
        if (moe_expf_asuint(x) == 0xff800000u) return 0.0f;   /* -inf */
        if (abstop >= 0x7f8u) return x + x;                   /* +inf, nan */
        if (x > 0x1.62e42ep6f) return __builtin_inff();       /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                  /* underflow */
    }
    const double kd = red.kd - shift;
    const double r = __builtin_fma(inv_ln2_n, red.xd, -kd);
    const double s = moe_expf_asdouble(entry + (red.ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* The function with the table lookup as a parameter (the kernels' epilogues
 * pass a lookup that reads the table from registers).  The table is read
 * before any special-case return, by every lane: a lookup through lane
 * shuffles needs all lanes of the wave present. */
template<typename Table>
MOE_EXPF_FN float moe_expf_with(float x, const Table &table) {
    const MoeExpfReduced r = moe_expf_reduce(x);
    const uint64_t entry = table(moe_expf_index(r));
    return moe_expf_finish(x, r, entry);
}

MOE_EXPF_FN float moe_expf(float x) { return moe_expf_with(x, MoeExpfTable{}); }

#endif /* MOE_EXPF_H */
