/*
 * CPU oracle for the routed-MoE Q4_0 x Q8_1 expert FFN.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
 * path is compared against, and the CPU baseline that bench.py times beside it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library never links, loads or falls back to it.
 *
 * It restates, in plain C, the arithmetic of the reference's CPU path
 * (0FL01/gfx906-qwen3.8fn, read-only at /root/reference):
 *   - Q4_0 / Q8_1 block formats                      src/quant.hpp:8-18
 *   - half <-> float, RNE, subnormals, NaN quieting  src/quant.cpp:211-260
 *   - quantize_q8 (FP32 amax/127 codes, raw XOR sum)  src/quant.cpp:275-325
 *   - integer block dot over unsigned nibbles        src/quant.cpp:48-55
 *   - Q4_0 full-block scaled dot                     src/quant.cpp:88-93
 *   - ascending full-block matmul (3-column tiles)   src/quant.cpp:141-167,
 *                                                    src/linear_reference.cpp:148-199
 *   - cpu_expert two-fragment / FMA / 128-lane XOR order
 *                                                    src/cpu_expert.cpp:156-213
 *   - cpu_expert whole-expert execute                src/cpu_expert.cpp:216-272
 *   - RouteGroups::prepare counting sort             src/routes.cpp:59-115
 *   - routed_fold rank-order left fold               src/hip/session_ops.hip:307-324
 *   - shared_sigmoid_add                             src/hip/session_ops.hip:375-391
 *   - allowed physical CPU discovery                 src/cpu_expert.cpp:334-362
 *
 * Every function is pinned by the tests under tests/ (golden vectors written
 * by the compiled reference in oracle/_ref, literal known answers from the
 * reference's own tests, closed forms and brute force on tiny inputs).
 *
 * Shapes are generic: hidden H and intermediate I must be multiples of 32.
 * Weights use the canonical 18-byte Q4_0 layout [row][block], rows contiguous.
 * Activations/outputs are token-major: x[t*H + i], y[t*H + i].
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct { uint16_t d; uint8_t qs[16]; } mo_q4_0;            /* 18 bytes */
typedef struct { uint16_t d, s; int8_t qs[32]; } mo_q8_1;          /* 36 bytes */

enum {
    MO_OK = 0,
    MO_INVALID_ARGUMENT = 1,
    MO_NUMERIC_ERROR = 2,
    MO_UNSUPPORTED_CPU = 3,
};

float mo_half_to_float(uint16_t bits);
uint16_t mo_float_to_half(float value);

/* src/quant.cpp:275-325.  n must be a multiple of 32.  Returns MO_OK or
 * MO_NUMERIC_ERROR (nonfinite input, FP32 scale underflow for a nonzero block,
 * half overflow of scale or raw sum, rounded code outside [-127,127]).  On
 * error, output blocks before the failing block are written, later ones not. */
int mo_quantize_q8(const float *x, size_t n, mo_q8_1 *out);

/* src/quant.cpp:48-55: sum_{i<16} (qs[i]&15)*c[i] + (qs[i]>>4)*c[i+16]. */
int32_t mo_block_dot(const uint8_t *qs, const int8_t *codes);

/* src/quant.cpp:88-93: d4 * (float(I)*d8 - 8*s8), separately rounded. */
float mo_scaled_dot_q4_0(int32_t integer_dot, uint16_t d4, const mo_q8_1 *x);

/* Per-block int32 dots, dots[(c*M + r)*(K/32) + k].  x is [cols][K/32]. */
void mo_block_dots(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, int32_t *dots);

/* Ascending full-block fp32 matmul (quant.cpp:141-167 / linear_reference.cpp
 * projection()).  out[c*M + r].  x is [cols][K/32]. */
void mo_matmul_full(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out);

/* cpu_expert.cpp:156-213 (matrix_gpu_order<Q4_0>), scalar restatement with
 * explicit fmaf.  out[c*M + r]. */
void mo_matrix_gpu_order(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out);

/* Same arithmetic, AVX2/FMA/F16C vectorized integer dots (bit-identical).
 * Returns MO_UNSUPPORTED_CPU when the host lacks AVX2/FMA/F16C. */
int mo_matrix_gpu_order_avx2(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out);
int mo_cpu_has_avx2(void);

/* cpu_expert.cpp:216-272 whole stage for one expert and `cols` gathered Q8
 * columns (x is [cols][H/32]): gate/up in gpu order, host expf SiLU, middle
 * quantize_q8, down in gpu order.  Optional outputs (may be NULL): gate/up/
 * middle [cols][I] fp32, middle_q8 [cols][I/32].  y is [cols][H] unweighted.
 * use_avx2 selects the vectorized projection (bit-identical results). */
int mo_expert_forward(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                      int H, int I, const mo_q8_1 *x, int cols, float *y,
                      float *gate_out, float *up_out, float *middle_out,
                      mo_q8_1 *middle_q8_out, int use_avx2);

/* routes.cpp:59-115.  ids/weights [tokens][top_k].  Outputs:
 * assign_token/rank/expert/weight [tokens*top_k] grouped by ascending expert,
 * within a group by token then rank; counts [experts]; offsets [experts+1]. */
int mo_route_groups(const int32_t *ids, const float *weights, int tokens, int top_k, int experts,
                    int32_t *assign_token, int32_t *assign_rank, int32_t *assign_expert,
                    float *assign_weight, int32_t *counts, int32_t *offsets);

/* session_ops.hip:307-324.  contributions [tokens][top_k][H] unweighted,
 * weights [tokens][top_k].  y = +0; for r: y = y + (w*c), separately rounded. */
void mo_routed_fold(const float *contributions, const float *weights, int tokens, int top_k,
                    int H, float *y);

/* session_ops.hip:307-324 then :375-391 with their flag semantics: a
 * nonfinite operand sets bit 1 and reads as 0, a nonfinite result sets bit 2
 * and becomes 0; the routed fold writes 0 where it raised a flag, the shared
 * sigmoid add (skipped when shared is NULL; scale 1 when shared_gate is NULL)
 * starts from that value and writes 0 where it raised one.  Returns the OR of
 * the flags. */
int mo_combine_flags(const float *contributions, const float *weights, const float *shared,
                     const float *shared_gate, int tokens, int top_k, int H, float *y);

/* Whole MoE layer, reference order:
 *   Q8 of x -> groups -> per (token,rank) expert forward (cpu_expert order)
 *   -> contributions -> rank-order fold -> optional shared expert add.
 * experts_q4 holds E experts, each [gate I*H/32 | up I*H/32 | down H*I/32]
 * 18-byte blocks.  shared_q4 may be NULL (no shared expert).  shared_gate
 * [tokens] may be NULL (scale 1.0) or raw logits (scale = 1/(1+expf(-g))).
 * contributions_out [tokens][top_k][H] and x_q8_out [tokens][H/32] may be
 * NULL.  token_mask (may be NULL) restricts the work to tokens whose mask
 * byte is nonzero (others' outputs are left untouched). */
int mo_moe_layer(const float *x, int tokens, int H, int I, int E, int top_k,
                 const uint8_t *experts_q4, const uint8_t *shared_q4,
                 const int32_t *ids, const float *weights, const float *shared_gate,
                 float *y, float *contributions_out, mo_q8_1 *x_q8_out,
                 const uint8_t *token_mask, int use_avx2);

/* CPU baseline: the same layer with a pool of pinned worker threads, one per
 * allowed physical core (cpu_expert.cpp:334-362), jobs = expert groups split
 * into <=3-column tiles (cpu_expert.hpp:10).  Times quantize -> all groups ->
 * rank-order fold (+shared) with CLOCK_MONOTONIC, after one warm-up, over
 * `repeats` runs; returns the mean seconds per layer in *seconds.
 * workers <= 0 selects every allowed physical core; *workers_used reports it. */
int mo_baseline_layer(const float *x, int tokens, int H, int I, int E, int top_k,
                      const uint8_t *experts_q4, const uint8_t *shared_q4,
                      const int32_t *ids, const float *weights, const float *shared_gate,
                      float *y, int workers, int pin, int repeats,
                      double *seconds, int *workers_used);

/* Physical-core representatives (first allowed sibling per (package,core)). */
int mo_allowed_physical_cpus(int *cpus, int capacity, int *count);

/* The C library's expf over an array (checker for the kernels' expf). */
void mo_expf_libm(const float *x, float *y, size_t n);

/* Q4_1 down rows (20-byte blocks {half d; half m; qs[16]}) in the cpu_expert
 * order with the half-rounded d4*d8 and m4*s8 products (cpu_expert.cpp:167-194),
 * and the whole expert / layer with Q4_1 down matrices (gate/up stay Q4_0;
 * an expert's canonical bytes are [gate 18-B blocks | up | down 20-B blocks]). */
void mo_matrix_gpu_order_q41(const uint8_t *w, int K, int M, const mo_q8_1 *x, int cols, float *out);
int mo_expert_forward_q41(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int H, int I,
                          const mo_q8_1 *x, int cols, float *y, float *gate_out, float *up_out,
                          float *middle_out, mo_q8_1 *middle_q8_out);
int mo_moe_layer_q41(const float *x, int tokens, int H, int I, int E, int top_k,
                     const uint8_t *experts_q4, const uint8_t *shared_q4, const int32_t *ids,
                     const float *weights, const float *shared_gate, float *y, float *contrib_out,
                     mo_q8_1 *x_q8_out, const uint8_t *mask);

/* Router: softmax over each row of `experts` logits (experts % 32 == 0) as
 * router_softmax (src/hip/session_ops.hip:401-434), and top_k selection with
 * the XOR-bucket denominator as select_routes (src/session.hip:666-687).
 * Both return the OR of their flags (1 invalid input, 2 arithmetic). */
int mo_router_softmax(const float *logits, int tokens, int experts, float *prob);
int mo_select_routes(const float *prob, int tokens, int experts, int top_k, int32_t *ids, float *weights);

#ifdef __cplusplus
}
#endif
#endif
