/*
 * CPU oracle for the routed-MoE Q4_0 x Q8_1 expert FFN -- TEST INFRASTRUCTURE.
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, always as the checker or the CPU baseline, never as the product path.
 * Citations are to the reference at 0FL01/gfx906-qwen3.8fn (src/...).
 * Build: oracle/Makefile (gcc, -O2 -ffp-contract=off, no fast-math).
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define MO_X86 1
#define MO_AVX2 __attribute__((target("avx2,fma,f16c")))
#else
#define MO_X86 0
#endif

#if defined(__FAST_MATH__)
#error "the oracle requires strict IEEE floating point"
#endif
#pragma GCC optimize("fp-contract=off")

_Static_assert(sizeof(mo_q4_0) == 18, "Q4_0 block is 18 bytes");
_Static_assert(sizeof(mo_q8_1) == 36, "Q8_1 block is 36 bytes");

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t ld16(const uint8_t *p) { uint16_t h; memcpy(&h, p, 2); return h; }

/* ---------------------------------------------------------------- half ---- */
/* IEEE binary16 -> binary32 is exact.  quant.cpp:211-232: subnormals are
 * normalised, infinities keep their sign, NaNs keep sign/payload and are
 * quieted (F16C semantics). */
float mo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        /* m * 2^-24 is exactly representable as a normal float. */
        const float mag = (float)m * 0x1p-24f;
        return u2f(sign | f2u(mag));
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0u));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* binary32 -> binary16, round to nearest even (quant.cpp:234-260 semantics:
 * overflow to infinity, gradual underflow, NaN payload top bits + quiet bit). */
uint16_t mo_float_to_half(float value) {
    const uint32_t u = f2u(value);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? (0x200u | (m >> 13)) : 0u));
    /* Work on the 24-bit significand (implicit bit included for normals). */
    int exp = (int)e - 127;                     /* unbiased */
    uint32_t sig = e ? (m | 0x800000u) : m;     /* value = sig * 2^(exp-23), e>0 */
    if (e == 0) return sign;                    /* float subnormals are < 2^-126: half zero */
    if (exp > 15) return (uint16_t)(sign | 0x7c00u);
    /* Target: half normal needs exp >= -14, else subnormal with unit 2^-24. */
    int shift;                                  /* bits of sig dropped */
    uint32_t base;                              /* exponent field contribution */
    if (exp >= -14) { shift = 13; base = (uint32_t)(exp + 15) << 10; sig &= 0x7fffffu; }
    else { shift = -exp - 14 + 13; base = 0; }
    if (shift > 24) return sign;                /* below half of the smallest subnormal */
    const uint32_t kept = sig >> shift;
    const uint32_t rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
    uint32_t r = base + kept;                   /* carries propagate into the exponent */
    if (rem > half || (rem == half && (kept & 1u))) r += 1u;
    return (uint16_t)(sign | r);                /* r == 0x7c00 is the correct overflow */
}

/* ------------------------------------------------------------ quantize ---- */
/* quant.cpp:275-325: D = amax/127 (FP32, correctly rounded); codes are
 * roundf(x/D) with the FP32 D; d = half(D); s = half(raw sum) where the raw
 * sum is the ascending XOR butterfly (masks 1,2,4,8,16) of the 32 inputs. */
int mo_quantize_q8(const float *x, size_t n, mo_q8_1 *out) {
    if (n % 32) return MO_INVALID_ARGUMENT;
    for (size_t b = 0; b < n / 32; ++b) {
        const float *v = x + b * 32;
        float t[32], amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            if (!isfinite(v[i])) return MO_NUMERIC_ERROR;
            t[i] = v[i];
            const float a = fabsf(v[i]);
            if (a > amax) amax = a;
        }
        mo_q8_1 q;
        memset(&q, 0, sizeof q);
        if (amax == 0.0f) { out[b] = q; continue; }
        const float D = amax / 127.0f;
        if (D == 0.0f) return MO_NUMERIC_ERROR;
        q.d = mo_float_to_half(D);
        if ((q.d & 0x7c00u) == 0x7c00u) return MO_NUMERIC_ERROR;
        for (int mask = 1; mask < 32; mask <<= 1) {
            float next[32];
            for (int l = 0; l < 32; ++l) next[l] = t[l] + t[l ^ mask];
            memcpy(t, next, sizeof t);
        }
        q.s = mo_float_to_half(t[0]);
        if (!isfinite(t[0]) || (q.s & 0x7c00u) == 0x7c00u) return MO_NUMERIC_ERROR;
        for (int i = 0; i < 32; ++i) {
            const float c = roundf(v[i] / D);
            if (!isfinite(c) || c < -127.0f || c > 127.0f) return MO_NUMERIC_ERROR;
            q.qs[i] = (int8_t)c;
        }
        out[b] = q;
    }
    return MO_OK;
}

/* ----------------------------------------------------------------- dots ---- */
int32_t mo_block_dot(const uint8_t *qs, const int8_t *c) {
    int32_t s = 0;
    for (int i = 0; i < 16; ++i) {
        s += (int32_t)(qs[i] & 15u) * (int32_t)c[i];
        s += (int32_t)(qs[i] >> 4) * (int32_t)c[i + 16];
    }
    return s;
}

float mo_scaled_dot_q4_0(int32_t I, uint16_t d4, const mo_q8_1 *x) {
    const float dw = mo_half_to_float(d4), dx = mo_half_to_float(x->d), sx = mo_half_to_float(x->s);
    const float p = (float)I * dx;
    const float corr = 8.0f * sx;
    return dw * (p - corr);
}

void mo_block_dots(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, int32_t *dots) {
    const int nb = K / 32;
    for (int c = 0; c < cols; ++c)
        for (int r = 0; r < M; ++r)
            for (int k = 0; k < nb; ++k) {
                const uint8_t *blk = w + ((size_t)r * nb + k) * 18;
                dots[((size_t)c * M + r) * nb + k] = mo_block_dot(blk + 2, x[(size_t)c * nb + k].qs);
            }
}

/* Ascending serial K sum of full-block scaled dots (quant.cpp:148-165). */
void mo_matmul_full(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out) {
    const int nb = K / 32;
    for (int c = 0; c < cols; ++c)
        for (int r = 0; r < M; ++r) {
            float acc = 0.0f;
            for (int k = 0; k < nb; ++k) {
                const uint8_t *blk = w + ((size_t)r * nb + k) * 18;
                const mo_q8_1 *a = &x[(size_t)c * nb + k];
                acc += mo_scaled_dot_q4_0(mo_block_dot(blk + 2, a->qs), ld16(blk), a);
            }
            out[(size_t)c * M + r] = acc;
        }
}

/* ------------------------------------------------------ cpu_expert order --- */
/* cpu_expert.cpp:156-213.  Each block contributes two 16-code fragments:
 * f=0 covers bytes 0..7 (elements 0..7 and 16..23), f=1 bytes 8..15.  They
 * accumulate into lane 2*(k%64)+f of 128 lanes with
 *     acc = fma(d4, fma(float(I_f), d8, -4*s8), acc),
 * then lane[i] += lane[i+64] (i<64), then an ascending XOR butterfly over 64
 * lanes (masks 1..32); the row result is lane 0. */
static void fold128(float *lane, float *result) {
    for (int i = 0; i < 64; ++i) lane[i] = lane[i] + lane[i + 64];
    for (int mask = 1; mask < 64; mask <<= 1) {
        float next[64];
        for (int i = 0; i < 64; ++i) next[i] = lane[i] + lane[i ^ mask];
        memcpy(lane, next, sizeof next);
    }
    *result = lane[0];
}

static inline int32_t fragment_dot(const uint8_t *qs, const int8_t *c, int f) {
    int32_t s = 0;
    for (int j = 8 * f; j < 8 * f + 8; ++j) {
        s += (int32_t)(qs[j] & 15u) * (int32_t)c[j];
        s += (int32_t)(qs[j] >> 4) * (int32_t)c[j + 16];
    }
    return s;
}

void mo_matrix_gpu_order(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out) {
    const int nb = K / 32;
    for (int c = 0; c < cols; ++c)
        for (int r = 0; r < M; ++r) {
            float lane[128];
            for (int i = 0; i < 128; ++i) lane[i] = 0.0f;
            for (int k = 0; k < nb; ++k) {
                const uint8_t *blk = w + ((size_t)r * nb + k) * 18;
                const mo_q8_1 *a = &x[(size_t)c * nb + k];
                const float d4 = mo_half_to_float(ld16(blk));
                const float d8 = mo_half_to_float(a->d), s8 = mo_half_to_float(a->s);
                const float corr = -4.0f * s8;
                for (int f = 0; f < 2; ++f) {
                    float *acc = &lane[2 * (k % 64) + f];
                    *acc = fmaf(d4, fmaf((float)fragment_dot(blk + 2, a->qs, f), d8, corr), *acc);
                }
            }
            fold128(lane, &out[(size_t)c * M + r]);
        }
}

/* Q4_1 rows (20-byte blocks {half d; half m; u8 qs[16]}, value q*d + m) in
 * the same lane order (cpu_expert.cpp:167-194): per block dd = half(d4*d8)
 * and ms = half(m4*s8), both rounded to half (RNE), and per fragment
 *     acc = acc + fma(float(I_f), dd, ms * 0.5)
 * (a separate add, not a fused one), then the same fold. */
void mo_matrix_gpu_order_q41(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out) {
    const int nb = K / 32;
    for (int c = 0; c < cols; ++c)
        for (int r = 0; r < M; ++r) {
            float lane[128];
            for (int i = 0; i < 128; ++i) lane[i] = 0.0f;
            for (int k = 0; k < nb; ++k) {
                const uint8_t *blk = w + ((size_t)r * nb + k) * 20;
                const mo_q8_1 *a = &x[(size_t)c * nb + k];
                const float d4 = mo_half_to_float(ld16(blk)), m4 = mo_half_to_float(ld16(blk + 2));
                const float d8 = mo_half_to_float(a->d), s8 = mo_half_to_float(a->s);
                const float dd = mo_half_to_float(mo_float_to_half(d4 * d8));
                const float ms = mo_half_to_float(mo_float_to_half(m4 * s8));
                for (int f = 0; f < 2; ++f) {
                    float *acc = &lane[2 * (k % 64) + f];
                    *acc = *acc + fmaf((float)fragment_dot(blk + 4, a->qs, f), dd, ms * 0.5f);
                }
            }
            fold128(lane, &out[(size_t)c * M + r]);
        }
}

int mo_cpu_has_avx2(void) {
#if MO_X86
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c");
#else
    return 0;
#endif
}

#if MO_X86
/* Vectorized integer fragments: maddubs(unsigned nibble, signed code) pairs
 * cannot saturate (|2*15*128| < 32767), madd(.,1) widens to int32.  The low
 * 128-bit lane holds byte-pairs for nibbles x codes[0..15], the high lane the
 * high nibbles x codes[16..31]; fragment f sums dwords {2f,2f+1} of both
 * lanes -- exactly bytes 8f..8f+7 of the block, as fragment_dot does. */
MO_AVX2 static void matrix_avx2_impl(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols,
                                     float *out) {
    const int nb = K / 32;
    const __m128i low4 = _mm_set1_epi8(15);
    const __m256i ones = _mm256_set1_epi16(1);
    float lane[3][128] __attribute__((aligned(32)));
    for (int c0 = 0; c0 < cols; c0 += 3) {
        const int n = cols - c0 < 3 ? cols - c0 : 3;
        for (int r = 0; r < M; ++r) {
            for (int c = 0; c < n; ++c)
                for (int i = 0; i < 128; ++i) lane[c][i] = 0.0f;
            for (int k = 0; k < nb; ++k) {
                const uint8_t *blk = w + ((size_t)r * nb + k) * 18;
                const float d4 = _cvtsh_ss(ld16(blk));
                const __m128i packed = _mm_loadu_si128((const __m128i *)(blk + 2));
                const __m256i nib = _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(packed, 4), low4),
                                                     _mm_and_si128(packed, low4));
                for (int c = 0; c < n; ++c) {
                    const mo_q8_1 *a = &x[(size_t)(c0 + c) * nb + k];
                    const __m256i q = _mm256_loadu_si256((const __m256i *)a->qs);
                    const __m256i d32 = _mm256_madd_epi16(_mm256_maddubs_epi16(nib, q), ones);
                    const __m128i s = _mm_add_epi32(_mm256_castsi256_si128(d32),
                                                    _mm256_extracti128_si256(d32, 1));
                    const int32_t I0 = _mm_extract_epi32(s, 0) + _mm_extract_epi32(s, 1);
                    const int32_t I1 = _mm_extract_epi32(s, 2) + _mm_extract_epi32(s, 3);
                    const float d8 = _cvtsh_ss(a->d), s8 = _cvtsh_ss(a->s);
                    const float corr = -4.0f * s8;
                    float *acc = &lane[c][2 * (k % 64)];
                    acc[0] = fmaf(d4, fmaf((float)I0, d8, corr), acc[0]);
                    acc[1] = fmaf(d4, fmaf((float)I1, d8, corr), acc[1]);
                }
            }
            for (int c = 0; c < n; ++c) fold128(lane[c], &out[(size_t)(c0 + c) * M + r]);
        }
    }
}
#endif

int mo_matrix_gpu_order_avx2(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out) {
#if MO_X86
    if (!mo_cpu_has_avx2()) return MO_UNSUPPORTED_CPU;
    matrix_avx2_impl(w, K, M, x, cols, out);
    return MO_OK;
#else
    (void)w; (void)K; (void)M; (void)x; (void)cols; (void)out;
    return MO_UNSUPPORTED_CPU;
#endif
}

/* ------------------------------------------------------------- expert ----- */
typedef struct {
    float *gate, *up, *middle;   /* [cols][I] */
    mo_q8_1 *mq8;                /* [cols][I/32] */
} expert_scratch;

/* cpu_expert.cpp:233-267 (whole stage). */
static int expert_run(const uint8_t *gw, const uint8_t *uw, const uint8_t *dw, int H, int I,
                      const mo_q8_1 *x, int cols, float *y, expert_scratch *s, int use_avx2, int down_q41) {
    if (use_avx2) {
        if (mo_matrix_gpu_order_avx2(gw, H, I, x, cols, s->gate) != MO_OK) return MO_UNSUPPORTED_CPU;
        mo_matrix_gpu_order_avx2(uw, H, I, x, cols, s->up);
    } else {
        mo_matrix_gpu_order(gw, H, I, x, cols, s->gate);
        mo_matrix_gpu_order(uw, H, I, x, cols, s->up);
    }
    const size_t mid = (size_t)cols * I;
    for (size_t i = 0; i < mid; ++i) {
        const float g = s->gate[i], u = s->up[i];
        if (!isfinite(g) || !isfinite(u)) return MO_NUMERIC_ERROR;
        const float activated = g / (1.0f + expf(-g));
        const float m = activated * u;
        if (!isfinite(activated) || !isfinite(m)) return MO_NUMERIC_ERROR;
        s->middle[i] = m;
    }
    if (mo_quantize_q8(s->middle, mid, s->mq8) != MO_OK) return MO_NUMERIC_ERROR;
    if (down_q41) mo_matrix_gpu_order_q41(dw, I, H, s->mq8, cols, y);
    else if (use_avx2) mo_matrix_gpu_order_avx2(dw, I, H, s->mq8, cols, y);
    else mo_matrix_gpu_order(dw, I, H, s->mq8, cols, y);
    for (size_t i = 0; i < (size_t)cols * H; ++i)
        if (!isfinite(y[i])) return MO_NUMERIC_ERROR;
    return MO_OK;
}

static int expert_forward_impl(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int H, int I,
                               const mo_q8_1 *x, int cols, float *y, float *gate_out, float *up_out,
                               float *middle_out, mo_q8_1 *middle_q8_out, int use_avx2, int down_q41) {
    if (H <= 0 || I <= 0 || H % 32 || I % 32 || cols <= 0) return MO_INVALID_ARGUMENT;
    expert_scratch s;
    const size_t mid = (size_t)cols * I;
    s.gate = malloc(mid * sizeof(float));
    s.up = malloc(mid * sizeof(float));
    s.middle = malloc(mid * sizeof(float));
    s.mq8 = malloc(mid / 32 * sizeof(mo_q8_1));
    int rc = MO_INVALID_ARGUMENT;
    if (s.gate && s.up && s.middle && s.mq8) {
        rc = expert_run(gate, up, down, H, I, x, cols, y, &s, use_avx2, down_q41);
        if (gate_out) memcpy(gate_out, s.gate, mid * sizeof(float));
        if (up_out) memcpy(up_out, s.up, mid * sizeof(float));
        if (middle_out) memcpy(middle_out, s.middle, mid * sizeof(float));
        if (middle_q8_out) memcpy(middle_q8_out, s.mq8, mid / 32 * sizeof(mo_q8_1));
    }
    free(s.gate); free(s.up); free(s.middle); free(s.mq8);
    return rc;
}

int mo_expert_forward(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int H, int I,
                      const mo_q8_1 *x, int cols, float *y, float *gate_out, float *up_out,
                      float *middle_out, mo_q8_1 *middle_q8_out, int use_avx2) {
    return expert_forward_impl(gate, up, down, H, I, x, cols, y, gate_out, up_out, middle_out, middle_q8_out,
                               use_avx2, 0);
}

int mo_expert_forward_q41(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int H, int I,
                          const mo_q8_1 *x, int cols, float *y, float *gate_out, float *up_out,
                          float *middle_out, mo_q8_1 *middle_q8_out) {
    return expert_forward_impl(gate, up, down, H, I, x, cols, y, gate_out, up_out, middle_out, middle_q8_out,
                               0, 1);
}

/* ------------------------------------------------------------- routes ----- */
/* routes.cpp:59-115: validate the whole input first (ids in range, unique
 * per token, weights finite and >= 0), then histogram, exclusive scan and a
 * stable scatter in (token, rank) order; raw weight bits are preserved. */
int mo_route_groups(const int32_t *ids, const float *weights, int tokens, int top_k, int experts,
                    int32_t *at, int32_t *ar, int32_t *ae, float *aw, int32_t *counts,
                    int32_t *offsets) {
    if (tokens < 1 || top_k < 1 || experts < 1) return MO_INVALID_ARGUMENT;
    for (int t = 0; t < tokens; ++t)
        for (int r = 0; r < top_k; ++r) {
            const size_t i = (size_t)t * top_k + r;
            if (ids[i] < 0 || ids[i] >= experts) return MO_INVALID_ARGUMENT;
            if (!isfinite(weights[i]) || weights[i] < 0.0f) return MO_INVALID_ARGUMENT;
            for (int q = 0; q < r; ++q)
                if (ids[(size_t)t * top_k + q] == ids[i]) return MO_INVALID_ARGUMENT;
        }
    for (int e = 0; e < experts; ++e) counts[e] = 0;
    for (size_t i = 0; i < (size_t)tokens * top_k; ++i) ++counts[ids[i]];
    offsets[0] = 0;
    for (int e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *cursor = malloc(sizeof(int32_t) * (size_t)experts);
    if (!cursor) return MO_INVALID_ARGUMENT;
    for (int e = 0; e < experts; ++e) cursor[e] = offsets[e];
    for (int t = 0; t < tokens; ++t)
        for (int r = 0; r < top_k; ++r) {
            const size_t i = (size_t)t * top_k + r;
            const int32_t p = cursor[ids[i]]++;
            at[p] = t; ar[p] = r; ae[p] = ids[i];
            memcpy(&aw[p], &weights[i], sizeof(float));
        }
    free(cursor);
    return MO_OK;
}

/* session_ops.hip:307-324: y = +0, then for rank 0..k-1: y = y + (w * c). */
void mo_routed_fold(const float *contrib, const float *weights, int tokens, int top_k, int H, float *y) {
    for (int t = 0; t < tokens; ++t)
        for (int i = 0; i < H; ++i) {
            float v = 0.0f;
            for (int r = 0; r < top_k; ++r) {
                const float p = weights[(size_t)t * top_k + r] * contrib[((size_t)t * top_k + r) * H + i];
                v = v + p;
            }
            y[(size_t)t * H + i] = v;
        }
}

/* session_ops.hip:375-391: scale = 1/(1+expf(-g)); y = y + scale*s.  With no
 * gate the shared expert is an always-routed expert of weight 1.0. */
static void shared_add(const float *s, const float *gate, int t, int H, float *y) {
    float scale = 1.0f;
    if (gate) scale = 1.0f / (1.0f + expf(-gate[t]));
    for (int i = 0; i < H; ++i) {
        const float p = scale * s[i];
        y[(size_t)t * H + i] = y[(size_t)t * H + i] + p;
    }
}

/* The reference's fold with its error semantics: routed_fold
 * (session_ops.hip:307-324) then shared_sigmoid_add (:375-391), as two passes.
 * operand(): a nonfinite input sets bit 1 and reads as 0 (:161-164);
 * arithmetic(): a nonfinite result sets bit 2 and becomes 0 (:166-169).  The
 * routed pass writes 0 where it raised any flag; the shared pass reads that
 * value as its accumulator and writes 0 where it raised a flag of its own.
 * shared may be NULL (no shared add); shared_gate NULL means scale 1.0.
 * Returns the OR of all flags; y [tokens][H]. */
static float mo_operand(float x, int *flags) {
    if (!isfinite(x)) { *flags |= 1; return 0.0f; }
    return x;
}
static float mo_arith(float x, int *flags) {
    if (!isfinite(x)) { *flags |= 2; return 0.0f; }
    return x;
}
int mo_combine_flags(const float *contrib, const float *weights, const float *shared, const float *shared_gate,
                     int tokens, int top_k, int H, float *y) {
    int all = 0;
    for (int t = 0; t < tokens; ++t)
        for (int i = 0; i < H; ++i) {
            int f = 0;
            float v = 0.0f;
            for (int r = 0; r < top_k; ++r) {
                const float x = mo_operand(contrib[((size_t)t * top_k + r) * H + i], &f);
                const float w = mo_operand(weights[(size_t)t * top_k + r], &f);
                const float c = mo_arith(w * x, &f);
                v = mo_arith(v + c, &f);
            }
            v = f ? 0.0f : v;
            all |= f;
            if (shared) {
                int g = 0;
                const float x = mo_operand(shared[(size_t)t * H + i], &g);
                const float acc = mo_operand(v, &g);
                float scale = 1.0f;
                if (shared_gate) {
                    const float gate = mo_operand(shared_gate[t], &g);
                    scale = mo_arith(1.0f / (1.0f + expf(-gate)), &g);
                }
                const float c = mo_arith(scale * x, &g);
                const float sum = mo_arith(acc + c, &g);
                v = g ? 0.0f : sum;
                all |= g;
            }
            y[(size_t)t * H + i] = v;
        }
    return all;
}

/* One expert's canonical bytes: gate and up Q4_0, down Q4_0 (18-byte
 * blocks) or Q4_1 (20-byte blocks). */
static size_t expert_bytes(int H, int I, int down_q41) {
    return (size_t)H / 32 * I * (36 + (down_q41 ? 20 : 18));
}

static int moe_layer_impl(const float *x, int tokens, int H, int I, int E, int top_k,
                          const uint8_t *experts_q4, const uint8_t *shared_q4, const int32_t *ids,
                          const float *weights, const float *shared_gate, float *y, float *contrib_out,
                          mo_q8_1 *x_q8_out, const uint8_t *mask, int use_avx2, int down_q41) {
    if (tokens < 1 || H % 32 || I % 32 || E < 1 || top_k < 1) return MO_INVALID_ARGUMENT;
    const size_t nbx = (size_t)H / 32, eb = expert_bytes(H, I, down_q41), mat = (size_t)H / 32 * I * 18;
    const size_t assignments = (size_t)tokens * top_k;
    mo_q8_1 *xq = malloc(sizeof(mo_q8_1) * nbx * tokens);
    int32_t *at = malloc(4 * assignments), *ar = malloc(4 * assignments), *ae = malloc(4 * assignments);
    float *aw = malloc(4 * assignments);
    int32_t *counts = malloc(4 * (size_t)E), *offsets = malloc(4 * ((size_t)E + 1));
    float *contrib = malloc(sizeof(float) * assignments * H);
    float *row = malloc(sizeof(float) * H);
    expert_scratch s;
    s.gate = malloc(sizeof(float) * I); s.up = malloc(sizeof(float) * I);
    s.middle = malloc(sizeof(float) * I); s.mq8 = malloc(sizeof(mo_q8_1) * I / 32);
    int rc = MO_INVALID_ARGUMENT;
    if (!xq || !at || !ar || !ae || !aw || !counts || !offsets || !contrib || !row ||
        !s.gate || !s.up || !s.middle || !s.mq8) goto done;
    for (int t = 0; t < tokens; ++t) {
        if (mask && !mask[t]) { memset(xq + t * nbx, 0, sizeof(mo_q8_1) * nbx); continue; }
        rc = mo_quantize_q8(x + (size_t)t * H, (size_t)H, xq + t * nbx);
        if (rc != MO_OK) goto done;
    }
    rc = mo_route_groups(ids, weights, tokens, top_k, E, at, ar, ae, aw, counts, offsets);
    if (rc != MO_OK) goto done;
    /* Expert groups in ascending expert order; each column is independent of
     * the others in its group (cpu_expert_test "group vs individual output"). */
    for (size_t p = 0; p < assignments; ++p) {
        const int t = at[p], r = ar[p], e = ae[p];
        if (mask && !mask[t]) continue;
        const uint8_t *base = experts_q4 + (size_t)e * eb;
        rc = expert_run(base, base + mat, base + 2 * mat, H, I, xq + (size_t)t * nbx, 1,
                        contrib + ((size_t)t * top_k + r) * H, &s, use_avx2, down_q41);
        if (rc != MO_OK) goto done;
    }
    for (int t = 0; t < tokens; ++t) {
        if (mask && !mask[t]) continue;
        mo_routed_fold(contrib + (size_t)t * top_k * H, weights + (size_t)t * top_k, 1, top_k, H,
                       y + (size_t)t * H);
        if (shared_q4) {
            rc = expert_run(shared_q4, shared_q4 + mat, shared_q4 + 2 * mat, H, I, xq + (size_t)t * nbx, 1,
                            row, &s, use_avx2, down_q41);
            if (rc != MO_OK) goto done;
            shared_add(row, shared_gate, t, H, y);
        }
    }
    if (contrib_out) memcpy(contrib_out, contrib, sizeof(float) * assignments * H);
    if (x_q8_out) memcpy(x_q8_out, xq, sizeof(mo_q8_1) * nbx * tokens);
    rc = MO_OK;
done:
    free(xq); free(at); free(ar); free(ae); free(aw); free(counts); free(offsets); free(contrib);
    free(row); free(s.gate); free(s.up); free(s.middle); free(s.mq8);
    return rc;
}

int mo_moe_layer(const float *x, int tokens, int H, int I, int E, int top_k,
                 const uint8_t *experts_q4, const uint8_t *shared_q4, const int32_t *ids,
                 const float *weights, const float *shared_gate, float *y, float *contrib_out,
                 mo_q8_1 *x_q8_out, const uint8_t *mask, int use_avx2) {
    return moe_layer_impl(x, tokens, H, I, E, top_k, experts_q4, shared_q4, ids, weights, shared_gate, y,
                          contrib_out, x_q8_out, mask, use_avx2, 0);
}

int mo_moe_layer_q41(const float *x, int tokens, int H, int I, int E, int top_k,
                     const uint8_t *experts_q4, const uint8_t *shared_q4, const int32_t *ids,
                     const float *weights, const float *shared_gate, float *y, float *contrib_out,
                     mo_q8_1 *x_q8_out, const uint8_t *mask) {
    return moe_layer_impl(x, tokens, H, I, E, top_k, experts_q4, shared_q4, ids, weights, shared_gate, y,
                          contrib_out, x_q8_out, mask, 0, 1);
}

/* ----------------------------------------------------------- topology ----- */
static int read_topology(int cpu, const char *name, int *value) {
    char path[160], buf[64];
    snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/%s", cpu, name);
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return 0;
    const ssize_t n = read(fd, buf, sizeof buf - 1);
    close(fd);
    if (n <= 0) return 0;
    buf[n] = 0;
    char *end = NULL;
    errno = 0;
    const long v = strtol(buf, &end, 10);
    if (errno || end == buf) return 0;
    *value = (int)v;
    return 1;
}

/* cpu_expert.cpp:334-362: first allowed logical CPU of each (package, core). */
int mo_allowed_physical_cpus(int *cpus, int capacity, int *count) {
    cpu_set_t allowed;
    CPU_ZERO(&allowed);
    if (sched_getaffinity(0, sizeof allowed, &allowed)) return MO_INVALID_ARGUMENT;
    int pk[CPU_SETSIZE], co[CPU_SETSIZE], n = 0;
    for (int id = 0; id < CPU_SETSIZE; ++id) {
        if (!CPU_ISSET(id, &allowed)) continue;
        int p = -1, c = -1;
        if (!read_topology(id, "physical_package_id", &p) || !read_topology(id, "core_id", &c)) {
            p = -1; c = id;   /* no sysfs topology: each logical CPU is its own core */
        }
        int seen = 0;
        for (int i = 0; i < n; ++i) if (pk[i] == p && co[i] == c) { seen = 1; break; }
        if (seen) continue;
        if (n < capacity) cpus[n] = id;
        pk[n] = p; co[n] = c; ++n;
    }
    *count = n < capacity ? n : capacity;
    return n ? MO_OK : MO_INVALID_ARGUMENT;
}

/* ------------------------------------------------------------ baseline ---- */
typedef struct {
    int expert, first, columns;   /* a <=3-column tile of one expert group */
} tile_job;

typedef struct {
    /* inputs */
    const float *x; int tokens, H, I, E, top_k;
    const uint8_t *experts_q4, *shared_q4;
    const int32_t *ids; const float *weights, *shared_gate;
    float *y;
    /* state */
    mo_q8_1 *xq; int32_t *at, *ar, *ae, *counts, *offsets; float *aw, *contrib, *shared_out;
    tile_job *jobs; int njobs;
    atomic_int next_quant, next_job, next_shared, next_fold, failure;
    pthread_barrier_t barrier;
    int workers, pin, rounds;
    const int *cpus;
} pool_state;

typedef struct { pool_state *st; int id; } worker_arg;

static void run_phases(pool_state *st, expert_scratch *s, mo_q8_1 *gx, float *out) {
    const size_t nbx = (size_t)st->H / 32, eb = expert_bytes(st->H, st->I, 0);
    const size_t mat = (size_t)st->H / 32 * st->I * 18;
    const int H = st->H, I = st->I, k = st->top_k;
    /* Phase 1: quantize tokens. */
    for (;;) {
        const int t = atomic_fetch_add(&st->next_quant, 1);
        if (t >= st->tokens) break;
        if (mo_quantize_q8(st->x + (size_t)t * H, (size_t)H, st->xq + t * nbx) != MO_OK)
            atomic_store(&st->failure, MO_NUMERIC_ERROR);
    }
    pthread_barrier_wait(&st->barrier);
    /* Phase 2: expert tiles (groups are built once before timing, see below). */
    for (;;) {
        const int j = atomic_fetch_add(&st->next_job, 1);
        if (j >= st->njobs) break;
        const tile_job *job = &st->jobs[j];
        for (int c = 0; c < job->columns; ++c)
            memcpy(gx + c * nbx, st->xq + (size_t)st->at[job->first + c] * nbx, sizeof(mo_q8_1) * nbx);
        const uint8_t *base = st->experts_q4 + (size_t)job->expert * eb;
        if (expert_run(base, base + mat, base + 2 * mat, H, I, gx, job->columns, out, s, 1, 0) != MO_OK)
            atomic_store(&st->failure, MO_NUMERIC_ERROR);
        for (int c = 0; c < job->columns; ++c) {
            const int p = job->first + c;
            memcpy(st->contrib + ((size_t)st->at[p] * k + st->ar[p]) * H, out + (size_t)c * H,
                   sizeof(float) * H);
        }
    }
    /* Shared expert in 3-column tiles of consecutive tokens. */
    if (st->shared_q4) {
        for (;;) {
            const int t0 = atomic_fetch_add(&st->next_shared, 3);
            if (t0 >= st->tokens) break;
            const int n = st->tokens - t0 < 3 ? st->tokens - t0 : 3;
            const uint8_t *base = st->shared_q4;
            if (expert_run(base, base + mat, base + 2 * mat, H, I, st->xq + (size_t)t0 * nbx, n,
                           st->shared_out + (size_t)t0 * H, s, 1, 0) != MO_OK)
                atomic_store(&st->failure, MO_NUMERIC_ERROR);
        }
    }
    pthread_barrier_wait(&st->barrier);
    /* Phase 3: rank-order fold (+ shared add) per token. */
    for (;;) {
        const int t = atomic_fetch_add(&st->next_fold, 1);
        if (t >= st->tokens) break;
        mo_routed_fold(st->contrib + (size_t)t * k * H, st->weights + (size_t)t * k, 1, k, H,
                       st->y + (size_t)t * H);
        if (st->shared_q4) shared_add(st->shared_out + (size_t)t * H, st->shared_gate, t, H, st->y);
    }
}

static void *worker_main(void *p) {
    worker_arg *a = p;
    pool_state *st = a->st;
    if (st->pin && st->cpus) {
        cpu_set_t m;
        CPU_ZERO(&m);
        CPU_SET(st->cpus[a->id], &m);
        pthread_setaffinity_np(pthread_self(), sizeof m, &m);
    }
    expert_scratch s;
    s.gate = malloc(sizeof(float) * 3 * st->I); s.up = malloc(sizeof(float) * 3 * st->I);
    s.middle = malloc(sizeof(float) * 3 * st->I); s.mq8 = malloc(sizeof(mo_q8_1) * 3 * st->I / 32);
    mo_q8_1 *gx = malloc(sizeof(mo_q8_1) * 3 * st->H / 32);
    float *out = malloc(sizeof(float) * 3 * st->H);
    if (!s.gate || !s.up || !s.middle || !s.mq8 || !gx || !out) atomic_store(&st->failure, MO_INVALID_ARGUMENT);
    for (int round = 0; round < st->rounds; ++round) {
        pthread_barrier_wait(&st->barrier);   /* start of a timed layer */
        if (atomic_load(&st->failure) == MO_OK) run_phases(st, &s, gx, out);
        else { pthread_barrier_wait(&st->barrier); pthread_barrier_wait(&st->barrier); }
        pthread_barrier_wait(&st->barrier);   /* end of layer */
    }
    free(s.gate); free(s.up); free(s.middle); free(s.mq8); free(gx); free(out);
    return NULL;
}

static double now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int mo_baseline_layer(const float *x, int tokens, int H, int I, int E, int top_k,
                      const uint8_t *experts_q4, const uint8_t *shared_q4, const int32_t *ids,
                      const float *weights, const float *shared_gate, float *y, int workers, int pin,
                      int repeats, double *seconds, int *workers_used) {
    if (tokens < 1 || H % 32 || I % 32 || E < 1 || top_k < 1 || repeats < 1) return MO_INVALID_ARGUMENT;
    if (!mo_cpu_has_avx2()) return MO_UNSUPPORTED_CPU;
    int cpus[CPU_SETSIZE], ncpu = 0;
    if (mo_allowed_physical_cpus(cpus, CPU_SETSIZE, &ncpu) != MO_OK) ncpu = 1, pin = 0;
    if (workers <= 0 || workers > ncpu) workers = ncpu;
    pool_state st;
    memset(&st, 0, sizeof st);
    st.x = x; st.tokens = tokens; st.H = H; st.I = I; st.E = E; st.top_k = top_k;
    st.experts_q4 = experts_q4; st.shared_q4 = shared_q4; st.ids = ids; st.weights = weights;
    st.shared_gate = shared_gate; st.y = y; st.workers = workers; st.pin = pin; st.cpus = cpus;
    st.rounds = repeats + 1;
    const size_t A = (size_t)tokens * top_k;
    st.xq = malloc(sizeof(mo_q8_1) * (size_t)tokens * H / 32);
    st.at = malloc(4 * A); st.ar = malloc(4 * A); st.ae = malloc(4 * A); st.aw = malloc(4 * A);
    st.counts = malloc(4 * (size_t)E); st.offsets = malloc(4 * ((size_t)E + 1));
    st.contrib = malloc(sizeof(float) * A * H);
    st.shared_out = malloc(sizeof(float) * (size_t)tokens * H);
    st.jobs = malloc(sizeof(tile_job) * (A / 3 + (size_t)E + 1));
    int rc = MO_INVALID_ARGUMENT;
    if (!st.xq || !st.at || !st.ar || !st.ae || !st.aw || !st.counts || !st.offsets || !st.contrib ||
        !st.shared_out || !st.jobs) goto done;
    /* Validate once up front so a bad route fails before any thread starts;
     * the timed rounds below group again, as the reference does per layer. */
    rc = mo_route_groups(ids, weights, tokens, top_k, E, st.at, st.ar, st.ae, st.aw, st.counts, st.offsets);
    if (rc != MO_OK) goto done;
    atomic_init(&st.failure, MO_OK);
    pthread_barrier_init(&st.barrier, NULL, (unsigned)workers + 1);
    pthread_t threads[CPU_SETSIZE];
    worker_arg args[CPU_SETSIZE];
    for (int i = 0; i < workers; ++i) {
        args[i].st = &st; args[i].id = i;
        pthread_create(&threads[i], NULL, worker_main, &args[i]);
    }
    double total = 0.0;
    for (int round = 0; round < st.rounds; ++round) {
        atomic_store(&st.next_quant, 0); atomic_store(&st.next_job, 0);
        atomic_store(&st.next_shared, 0); atomic_store(&st.next_fold, 0);
        const double t0 = now_seconds();
        mo_route_groups(ids, weights, tokens, top_k, E, st.at, st.ar, st.ae, st.aw, st.counts, st.offsets);
        st.njobs = 0;
        for (int e = 0; e < E; ++e)
            for (int f = st.offsets[e]; f < st.offsets[e + 1]; f += 3) {
                tile_job *j = &st.jobs[st.njobs++];
                j->expert = e; j->first = f;
                j->columns = st.offsets[e + 1] - f < 3 ? st.offsets[e + 1] - f : 3;
            }
        pthread_barrier_wait(&st.barrier);   /* start */
        pthread_barrier_wait(&st.barrier);   /* quantize done */
        pthread_barrier_wait(&st.barrier);   /* experts done */
        pthread_barrier_wait(&st.barrier);   /* fold done */
        const double t1 = now_seconds();
        if (round > 0) total += t1 - t0;     /* round 0 is the warm-up */
    }
    for (int i = 0; i < workers; ++i) pthread_join(threads[i], NULL);
    pthread_barrier_destroy(&st.barrier);
    rc = atomic_load(&st.failure);
    *seconds = total / repeats;
    *workers_used = workers;
done:
    free(st.xq); free(st.at); free(st.ar); free(st.ae); free(st.aw); free(st.counts);
    free(st.offsets); free(st.contrib); free(st.shared_out); free(st.jobs);
    return rc;
}

/* The C library's expf over an array (the function the reference's CPU SiLU
 * calls, src/cpu_expert.cpp:251): the checker for the kernels' expf. */
void mo_expf_libm(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

/* ---- router -------------------------------------------------------------
 * mo_router_softmax restates router_softmax (src/hip/session_ops.hip:401-434):
 * 32 lanes, lane l holds logits l + 32k; nonfinite inputs count as 0 and set
 * bit 1; the row maximum; per lane a left-to-right sum of expf(x - max) from
 * +0; a width-32 XOR butterfly (1, 2, 4, 8, 16; dpp.cuh:32-36) for the total;
 * one reciprocal and a multiply per value; any flag zeroes the whole row.
 * expf is the C library's (the reference's CPU expert uses it; its GPU
 * router uses the device's, whose bits the reference does not pin:
 * src/cpu_expert.hpp:73-74).
 * mo_select_routes restates select_routes (src/session.hip:666-687): the
 * top_k largest values, ties to the lower id; 32 buckets (id % 32) summed in
 * rank order, then the XOR butterfly; denominator max(bucket 0, 1/16384);
 * weight = value * (1 / denominator).  An invalid denominator (the reference
 * throws) sets bit 2 and gives zero weights.  Both return their flags. */
static inline float mo_finite_or(float x, int *flags, int bit) {
    if (!isfinite(x)) { *flags |= bit; return 0.0f; }
    return x;
}

int mo_router_softmax(const float *logits, int tokens, int experts, float *prob) {
    int all = 0;
    const int per = experts / 32;
    for (int t = 0; t < tokens; ++t) {
        const float *row = logits + (size_t)t * experts;
        float *out = prob + (size_t)t * experts;
        int flags = 0;
        float lane_max[32], lane_sum[32];
        for (int l = 0; l < 32; ++l) {
            float m = -INFINITY;
            for (int k = 0; k < per; ++k) m = fmaxf(m, mo_finite_or(row[l + 32 * k], &flags, 1));
            lane_max[l] = m;
        }
        float maximum = -INFINITY;
        for (int l = 0; l < 32; ++l) maximum = fmaxf(maximum, lane_max[l]);
        for (int l = 0; l < 32; ++l) {
            float total = 0.0f;
            for (int k = 0; k < per; ++k) {
                const float x = mo_finite_or(row[l + 32 * k], &flags, 0);
                const float shifted = mo_finite_or(x - maximum, &flags, 2);
                const float w = mo_finite_or(expf(shifted), &flags, 2);
                out[l + 32 * k] = w;
                total = mo_finite_or(total + w, &flags, 2);
            }
            lane_sum[l] = total;
        }
        for (int d = 1; d < 32; d <<= 1) {
            float next[32];
            for (int l = 0; l < 32; ++l) next[l] = lane_sum[l] + lane_sum[l ^ d];
            memcpy(lane_sum, next, sizeof next);
        }
        const float total = mo_finite_or(lane_sum[0], &flags, 2);
        if (!(total > 0.0f)) flags |= 2;
        const float inverse = total > 0.0f ? mo_finite_or(1.0f / total, &flags, 2) : 0.0f;
        for (int e = 0; e < experts; ++e) out[e] = mo_finite_or(out[e] * inverse, &flags, 2);
        if (flags)
            for (int e = 0; e < experts; ++e) out[e] = 0.0f;
        all |= flags;
    }
    return all;
}

int mo_select_routes(const float *prob, int tokens, int experts, int top_k, int32_t *ids, float *weights) {
    int all = 0;
    for (int t = 0; t < tokens; ++t) {
        const float *row = prob + (size_t)t * experts;
        int32_t *id = ids + (size_t)t * top_k;
        float *wt = weights + (size_t)t * top_k;
        for (int i = 0; i < top_k; ++i) {   /* selection: largest value, then lowest id */
            int best = -1;
            for (int e = 0; e < experts; ++e) {
                int taken = 0;
                for (int q = 0; q < i; ++q) taken |= id[q] == e;
                if (taken) continue;
                if (best < 0 || row[e] > row[best]) best = e;   /* ascending e: ties keep the lower id */
            }
            id[i] = best;
        }
        float buckets[32] = {0};
        for (int i = 0; i < top_k; ++i) buckets[id[i] % 32] += row[id[i]];
        for (int d = 1; d < 32; d <<= 1) {
            float next[32];
            for (int l = 0; l < 32; ++l) next[l] = buckets[l] + buckets[l ^ d];
            memcpy(buckets, next, sizeof next);
        }
        const float floor_ = 1.0f / 16384.0f;
        const float denominator = buckets[0] < floor_ ? floor_ : buckets[0];
        int flags = 0;
        if (!(denominator > 0) || !isfinite(denominator)) flags = 2;
        const float inverse = flags ? 0.0f : 1.0f / denominator;
        for (int i = 0; i < top_k; ++i) wt[i] = row[id[i]] * inverse;
        all |= flags;
    }
    return all;
}
