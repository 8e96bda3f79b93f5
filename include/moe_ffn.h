/*
 * moe_ffn.h -- C ABI of the MI355X (gfx950) routed-MoE Q4_0 x Q8_1 expert FFN.
 *
 * Drop-in boundary for the routed expert path of 0FL01/gfx906-qwen3.8fn.  It
 * replaces everything between "token activations + host/device route ids and
 * weights" and "routed (+shared) FFN aggregate [N][H] fp32" in the reference's
 * Layer::ffn (src/session.hip:1446-1541, 1384-1410), i.e. the work of
 *   RouteGroups::prepare / upload_routes     src/routes.cpp:59-115, src/session.hip:393-410
 *   launch_quantize_q8_1                     src/hip/linear.cuh:107-108
 *   launch_moe_gather_q8 / launch_moe_scatter src/hip/session_ops.cuh:175-199
 *   launch_quantized_linear{,_short,_tiled}  src/hip/linear.cuh:70-87
 *   launch_silu_up_q8_1                      src/hip/linear.cuh:15-17
 *   launch_routed_fold / launch_scaled_add   src/hip/session_ops.cuh:104-114
 *   launch_shared_sigmoid_add_rows           src/hip/session_ops.cuh:213-214
 *   Experts::project/run/run_group/run_chunk src/session.hip:976-1078
 *
 * Conventions (kept from src/hip/linear.cuh:35-45, src/hip/session_ops.cuh:22-45):
 *   - every entry point returns a status (0 = success; otherwise a hipError_t
 *     value: 1 = invalid value, 2 = out of memory, 801 = not supported);
 *   - shape / null / alignment checks happen BEFORE any HIP call;
 *   - launchers only enqueue on the explicit stream (NULL = default stream);
 *     success means "enqueued", not "completed";
 *   - no hidden synchronisation, no allocation outside moe_ffn_create;
 *   - `error` is a caller-owned device int, zeroed by the caller in stream
 *     order; kernels atomically OR bit 1 (nonfinite / invalid input: bad
 *     expert id, duplicate id within a token, negative or nonfinite route
 *     weight) and bit 2 (arithmetic: Q8 not representable, nonfinite result).
 *     Kernels never clear it; a failing Q8 block is written as all zero.
 *   - one owner per layer handle; calls on one handle must not overlap.
 *
 * Formats (src/quant.hpp:8-18): Q4_0 = 18-byte block {half d; u8 qs[16]},
 * element j<16 = qs[j]&15, j>=16 = qs[j-16]>>4, value (q-8)*d.  Q8_1 =
 * 36-byte block {half d; half s; i8 qs[32]} with codes chosen by the FP32
 * scale amax/127 and s = half of the raw-input XOR-butterfly sum.
 */
#ifndef MOE_FFN_H
#define MOE_FFN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Down-projection block format (gate and up are always Q4_0).  Q4_1 =
 * 20-byte block {half d; half m; u8 qs[16]}, value q*d + m, as the
 * checkpoint's layers 0-5 store ffn_down_exps (src/expert_main.cpp:83-84);
 * its dot uses half-rounded d4*d8 and m4*s8 products (src/quant.cpp:95-100,
 * src/cpu_expert.cpp:167-194). */
enum { MOE_DOWN_Q4_0 = 0, MOE_DOWN_Q4_1 = 1 };

typedef struct moe_ffn_config {
    int hidden;        /* H: multiple of 32, 32..16384 */
    int intermediate;  /* I: multiple of 32, 32..16384 */
    int experts;       /* E: routed experts, 1..4096 */
    int top_k;         /* routes per token, 1..32, <= experts */
    int has_shared;    /* 1: one shared expert, always routed (src/session.hip:1384-1410) */
    int max_tokens;    /* capacity of forward(), 1..65536 */
    int down_type;     /* MOE_DOWN_Q4_0 (0) or MOE_DOWN_Q4_1 (1): format of the down matrices */
} moe_ffn_config;

typedef struct moe_ffn_layer moe_ffn_layer;

/* Expert weight bank in the reference's canonical layout: for each expert,
 * gate [I rows][H/32 blocks], then up [I][H/32], then down [H][I/32], 18-byte
 * Q4_0 blocks (down: 20-byte Q4_1 blocks when down_type is Q4_1), rows contiguous (src/session.hip:700-716 expert slots,
 * src/model.hpp:109-111).  `shared_q4` has the same per-expert layout.
 *
 * moe_ffn_create: uploads from HOST memory, repacking on the device into the
 * MI355X layout (code planes + scale planes); this is the only call that
 * allocates or synchronises.  Replaces the Experts/GpuExpert constructors
 * (src/session.hip:689-745, src/gpu_expert.hpp:9, src/hip/expert.hip:205-228). */
int moe_ffn_create(const moe_ffn_config *config, const void *experts_q4, const void *shared_q4,
                   int device, moe_ffn_layer **layer);

/* Same, from canonical bytes already resident in device memory (e.g. a
 * checkpoint loaded straight into HBM). */
int moe_ffn_create_from_device(const moe_ffn_config *config, const void *experts_q4_device,
                               const void *shared_q4_device, int device, moe_ffn_layer **layer);

/* Same, from the routed-expert tensors as the reference holds them: three
 * host tensors gate_exps [E][I][H/32], up_exps [E][I][H/32], down_exps
 * [E][H][I/32] of 18-byte Q4_0 blocks (down: Q4_1 20-byte blocks when
 * down_type says so) (GGUF ffn_{gate,up,down}_exps, rank 3
 * [input, output, expert]; Experts::ram, src/session.hip:700-716,
 * src/model.hpp:109-111), plus the shared expert's three matrices (NULL when
 * the layer has none).  Lets Experts' loaded tensors be handed over as is. */
int moe_ffn_create_tensors(const moe_ffn_config *config, const void *gate_exps, const void *up_exps,
                           const void *down_exps, const void *shared_gate, const void *shared_up,
                           const void *shared_down, int device, moe_ffn_layer **layer);

/* Synthetic weight bank generated on the device (for benchmarks of banks too
 * large to stage through the host): per block d = half(|N(0,0.02)|) and
 * uniform codes, from a counter-based hash of (seed, block index).  The bytes
 * are reproducible by moe_ffn_export_expert. */
int moe_ffn_create_synthetic(const moe_ffn_config *config, uint64_t seed, int device,
                             moe_ffn_layer **layer);

int moe_ffn_destroy(moe_ffn_layer *layer);

/* Device bytes held by a layer (weights + workspace for max_tokens). */
int moe_ffn_memory_bytes(const moe_ffn_config *config, size_t *weight_bytes, size_t *workspace_bytes);

/* Copy expert `expert` (0..E-1, or E for the shared expert) back to HOST in
 * the canonical layout above (synchronous; test/diagnostic use). */
int moe_ffn_export_expert(moe_ffn_layer *layer, int expert, void *host_q4);

/* The routed expert FFN of one MoE layer (replaces src/session.hip:1446-1541
 * plus shared_project/shared_add :1384-1410).  All pointers are DEVICE memory:
 *   x        [tokens][H] fp32 FFN input
 *   ids      [tokens][top_k] int32 expert ids (0..E-1, distinct per token)
 *   weights  [tokens][top_k] fp32 normalised route weights (finite, >= 0)
 *   shared_gate [tokens] fp32 raw shared-expert gate logits, or NULL for a
 *            gate of 1.0 (ignored when the layer has no shared expert)
 *   y        [tokens][H] fp32 output: y = +0; y = y + w_r*expert_r(x) for
 *            r = 0..top_k-1 in rank order; y = y + sigmoid(g)*shared(x)
 * tokens in 1..max_tokens.  Enqueue only, no host round trip for routing. */
int moe_ffn_forward(moe_ffn_layer *layer, const float *x, const int32_t *ids, const float *weights,
                    int tokens, const float *shared_gate, float *y, int *error, void *stream);

/* forward() from an already quantized input: x_q8 = canonical Q8_1 blocks
 * [tokens][H/32] (36 bytes each, 4-byte aligned), as the reference's FFN
 * receives its original Q8 rows f(21) (src/session.hip:1446-1460).  Same
 * outputs as forward() on the x those blocks quantize. */
int moe_ffn_forward_q8(moe_ffn_layer *layer, const void *x_q8, const int32_t *ids, const float *weights,
                       int tokens, const float *shared_gate, float *y, int *error, void *stream);

/* ------------------------------------------------------------------------
 * Stage entry points (parity tests and component timing).
 * ---------------------------------------------------------------------- */

/* fp32 [columns][width] -> canonical Q8_1 [columns][width/32] (36-byte
 * blocks).  Replaces launch_quantize_q8_1 (src/hip/linear.cuh:107-108,
 * kernel src/hip/linear.hip:99-150); width multiple of 32, 32..16384,
 * columns 1..65536.  Bit-exact with the reference quantize_q8. */
int moe_quantize_q8_1(const float *x, void *q8, int width, int columns, int *error, void *stream);

/* Route grouping on the device (replaces RouteGroups::prepare,
 * src/routes.cpp:59-115, and upload_routes src/session.hip:393-410).
 * Outputs (device): counts [E], offsets [E+1], route_token / route_rank
 * [tokens*top_k] grouped by ascending expert, then token, then rank. */
int moe_ffn_group_routes(moe_ffn_layer *layer, const int32_t *ids, const float *weights, int tokens,
                         int32_t *counts, int32_t *offsets, int32_t *route_token,
                         int32_t *route_rank, int *error, void *stream);

/* Kernel path selection for the single-expert stages below: MFMA = the
 * int8-MFMA kernels of the grouped forward (AUTO selects them); STREAM = the
 * per-token streaming-dot kernels. */
enum { MOE_PATH_AUTO = 0, MOE_PATH_STREAM = 1, MOE_PATH_MFMA = 2 };

/* One expert's gate/up projections fused with SiLU(gate)*up and Q8_1
 * quantization of the middle (replaces Experts::project's gate/up MMVQ +
 * launch_silu_up_q8_1, src/session.hip:976-991, src/hip/linear.hip:509-525).
 *   x_q8      [columns][H/32] canonical Q8_1 (device)
 *   middle    [columns][I] fp32 SiLU(g)*u (device, may be NULL)
 *   middle_q8 [columns][I/32] canonical Q8_1 (device)
 *   gate_dots, up_dots [columns][I][H/32] int32 per-block dots (device, may be NULL)
 * expert in 0..E (E = shared).  columns 1..max_tokens. */
int moe_ffn_expert_gate_up(moe_ffn_layer *layer, int expert, const void *x_q8, int columns,
                           float *middle, void *middle_q8, int32_t *gate_dots, int32_t *up_dots,
                           int path, int *error, void *stream);

/* One expert's down projection of a canonical Q8_1 middle
 * [columns][I/32] -> y [columns][H] fp32 unweighted (src/session.hip:992-998).
 * down_dots [columns][H][I/32] int32 (may be NULL). */
int moe_ffn_expert_down(moe_ffn_layer *layer, int expert, const void *middle_q8, int columns,
                        float *y, int32_t *down_dots, int path, int *error, void *stream);

/* Timing of one resident expert (ExpertTiming, src/gpu_expert.hpp:6).
 *   upload_ms          create: weight allocation, copy and repack until complete
 *   resident_ms        device time per forward (events around the repeats)
 *   completed_wall_ms  host wall time per forward, from before the first timed
 *                      forward until the output is back in host memory */
typedef struct moe_expert_timing {
    double upload_ms;
    double resident_ms;
    double completed_wall_ms;
} moe_expert_timing;

/* GpuExpert::run (src/gpu_expert.hpp:16, src/hip/expert.hip:228-241): one
 * expert's whole forward, fp32 x -> Q8_1 -> gate/up -> SiLU*up -> Q8_1 ->
 * down, on HOST buffers x [columns][H] and y [columns][H].  Uploads x once,
 * runs one untimed forward and checks its error word, then times `repeats`
 * forwards between events on `stream` and reads y back; synchronous.
 * columns 1..max_tokens, repeats 1..10000.  path: MOE_PATH_STREAM or
 * MOE_PATH_MFMA, or MOE_PATH_AUTO for the kernels forward() would give a
 * group of `columns` pairs.  *flags receives the error word (bit 1:
 * nonfinite x, bit 2: x not representable in Q8_1; the reference's
 * check_error throws on either); when the warm-up raises it, the call
 * returns 0 without timing (timing and y untouched).
 * Uses the layer's workspace: calls on one layer must not overlap. */
int moe_ffn_expert_run(moe_ffn_layer *layer, int expert, const float *x, int columns, float *y, int repeats,
                       int path, int *flags, moe_expert_timing *timing, void *stream);

/* Rank-order weighted combine (replaces launch_routed_fold +
 * launch_shared_sigmoid_add_rows, src/hip/session_ops.hip:307-324, 375-391):
 *   contributions [tokens][top_k][H] unweighted expert outputs
 *   weights [tokens][top_k], shared [tokens][H] or NULL, shared_gate [tokens] or NULL
 *   y [tokens][H] = +0 (+ w_r*c_r for r in rank order) (+ sigmoid(g)*shared). */
int moe_combine(const float *contributions, const float *weights, const float *shared,
                const float *shared_gate, int tokens, int top_k, int hidden, float *y, int *error,
                void *stream);

/* Debug view of the last forward() on this layer (device copies, any may be
 * NULL): x_q8 [tokens][H/32] canonical Q8_1 of the input, middle_q8
 * [tokens*top_k (+tokens)][I/32] canonical Q8_1 in grouped pair order,
 * route_token/route_rank [tokens*top_k] grouped order.  Enqueue only, on
 * `stream`.  When the last forward took the ungrouped decode path, this call
 * groups its routes again, so that forward's ids and weights must still be
 * valid; any flag that raises goes to a word inside the layer, never to the
 * forward's `error`. */
int moe_ffn_debug_last(moe_ffn_layer *layer, void *x_q8, void *middle_q8, int32_t *route_token,
                       int32_t *route_rank, void *stream);

/* Profiling hook: re-enqueue one stage of the last forward() on `stream`
 * with the same inputs (which must still be valid): 0 = quantize + group,
 * 1 = gate/up + SiLU + Q8, 2 = down, 3 = rank-order fold.  Lets a benchmark
 * time the kernels of one stage alone between events on that stream. */
enum { MOE_STAGE_PREPARE = 0, MOE_STAGE_GATE_UP = 1, MOE_STAGE_DOWN = 2, MOE_STAGE_FOLD = 3 };
int moe_ffn_replay_stage(moe_ffn_layer *layer, int stage, void *stream);

/* Stage profiler.  moe_ffn_profile(layer, n) creates timing events for the
 * next n forward() calls (n = 0 releases them; this call allocates host-side
 * event objects and may synchronise).  Each profiled forward records an event
 * before its first stage and after every stage on its own stream.
 * moe_ffn_profile_read waits for the last recorded forward and returns the
 * summed milliseconds per stage (MOE_STAGE_* order, 4 values) over the
 * forwards recorded since the last read, and their count; it then rearms the
 * same events for the next n forwards. */
int moe_ffn_profile(moe_ffn_layer *layer, int forwards);
int moe_ffn_profile_read(moe_ffn_layer *layer, double *stage_ms, int *forwards);

/* Last-forward statistics (host, synchronous: waits for the last forward's
 * stream, which must still exist, and for nothing else): work items per path
 * and the number of experts (incl. shared) that received tokens.  After a
 * decode-path forward it groups that forward's routes again on that stream
 * (its ids and weights must still be valid), flagging into a word inside the
 * layer, never into the forward's `error`.  Like every call here that needs
 * the layer's device current (create, destroy, export, expert_run), it
 * leaves the caller's current device as it found it. */
int moe_ffn_last_stats(moe_ffn_layer *layer, int32_t *stream_items, int32_t *mfma_items,
                       int32_t *active_experts);

/* SiLU exponential checks.  The kernels evaluate expf(-g) of SiLU and of the
 * shared-expert sigmoid gate with the bits of the host C library's expf (the
 * function src/cpu_expert.cpp:251 calls), so the middle matches the CPU
 * reference bit for bit; the reference's device expf (src/hip/linear.hip:113)
 * does not.  moe_expf_device enqueues y[i] = expf(x[i]) on the GPU with the
 * kernels' function; moe_expf_host runs the same code on the CPU.  No
 * counterpart in the reference: they exist for parity tests. */
int moe_expf_device(const float *x, float *y, int n, void *stream);
int moe_expf_host(const float *x, float *y, size_t n);

/* Router: replaces launch_router_softmax (src/hip/session_ops.hip:519-527,
 * kernel :401-434) followed by the host's select_routes
 * (src/session.hip:666-687) and the probability download / route upload
 * around them (src/session.hip:1422-1433, 393-410).  For each token row of
 * `experts` fp32 logits (device): the softmax in router_softmax's order (32
 * lanes, lane l holding logits l + 32k, XOR-butterfly total, reciprocal
 * multiply; nonfinite input zeroes the row and sets bit 1), then the top_k
 * largest probabilities (ties to the lower id) with weights normalised by the
 * 32-bucket XOR sum floored at 1/16384.  Writes ids / weights [tokens][top_k]
 * on the device, ready for moe_ffn_forward, and the probabilities
 * [tokens][experts] when `probabilities` is not NULL.  expf has the host C
 * library's bits.  experts % 32 == 0, 32 <= experts <= 1024, top_k <= 32. */
int moe_router_select(const float *logits, int tokens, int experts, int top_k, float *probabilities,
                      int32_t *ids, float *weights, int *error, void *stream);

/* Measurement hook: enqueue a plain streaming read of `bytes` (a multiple of
 * 16, buffer 16-byte aligned) from device memory; `sink` is a device word the
 * kernel never writes in practice.  Timing it at a kernel's byte count gives
 * the practical HBM read ceiling for a launch of that size.  No counterpart
 * in the reference. */
int moe_read_probe(const void *buffer, size_t bytes, void *sink, void *stream);

/* ------------------------------------------------------------------------
 * Quantized linear projections (the non-expert Q4 matrices around the FFN).
 * ---------------------------------------------------------------------- */

/* Weight types, numbered as the reference's TensorType (src/model.hpp:17-20). */
enum { MOE_TYPE_Q4_0 = 2, MOE_TYPE_Q4_1 = 3 };

typedef struct moe_linear moe_linear;

/* One resident matrix, the counterpart of the reference's Matrix
 * (src/session.hip:559-591) for its Q4_0 / Q4_1 tensors and of the
 * QuantizedDeviceMatrix it hands to launch_quantized_linear*
 * (src/hip/linear.cuh:27-32).  `weights` = canonical GGUF blocks
 * [output][input/32] (18-byte Q4_0 or 20-byte Q4_1, 2-byte aligned), on the
 * host or (weights_on_device = 1) on `device`; they are copied into the
 * handle's own planes, so the caller may free them afterwards.  input:
 * multiple of 32, 32..16384; output 1..16384.  max_columns (0..65536) sizes
 * the Q8_1 workspace of moe_linear_apply.  Allocates; synchronises the
 * device once. */
int moe_linear_create(int type, int input, int output, int max_columns, const void *weights, int weights_on_device,
                      int device, moe_linear **out);
int moe_linear_destroy(moe_linear *linear);
/* Canonical weight bytes the handle was created from. */
int moe_linear_bytes(const moe_linear *linear, size_t *weight_bytes);

/* y [columns][output] fp32 = W x for canonical Q8_1 columns x_q8
 * [columns][input/32] (36-byte blocks, 4-byte aligned).  Replaces
 * launch_quantized_linear / _short / _tiled (src/hip/linear.cuh:70-87,
 * src/hip/linear.hip:444-490) for Q4_0 / Q4_1, with the same fp32 order
 * (bit-identical outputs), columns 1..65536 in one launch.  x_q8 is read in
 * place (no workspace), so calls on one handle may overlap.  Enqueue only. */
int moe_linear_forward_q8(moe_linear *linear, const void *x_q8, int columns, float *y, void *stream);

/* Matrix::apply for Q4 types (src/session.hip:561-591): fp32 x
 * [columns][input] is quantized to Q8_1 into the handle's workspace
 * (launch_quantize_q8_1 semantics; flags OR-ed into `error`), then
 * forward_q8.  columns 1..max_columns.  Calls on one handle must not
 * overlap (they share the workspace). */
int moe_linear_apply(moe_linear *linear, const float *x, int columns, float *y, int *error, void *stream);

/* moe_linear_apply without the handle's workspace: the Q8_1 staging of x
 * lives in a static device array of the library, 4 MiB per GPU (held until
 * the process ends), so this call allocates nothing and works on handles
 * created with max_columns = 0.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Limit: columns * (input/32) * 36
 * <= 4 MiB (e.g. 1820 columns at input 2048), else 1 (invalid value) before
 * any HIP call; the handle's device must be current (moe_linear_create set
 * the array up for it), else 1.  Same outputs and flags as moe_linear_apply.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (on any handle or stream) race.  Issue them on one stream, or order
 * the streams.  A host thread that enters this call while another thread is
 * inside it for the same GPU gets 216 (hipErrorContextAlreadyInUse) and
 * nothing is enqueued. */
int moe_linear_apply_noalloc(moe_linear *linear, const float *x, int columns, float *y, int *error,
                             void *stream);

#ifdef __cplusplus
}
#endif
#endif
