// Internal types shared by the kernels (moe_kernels.hip) and the layer /
// C-ABI code (moe_layer.hip).  gfx950 (CDNA4) only, wave64.
//
// HBM layout of one layer (all experts resident; the reference streams them
// over PCIe into an LRU of GPU slots instead, src/session.hip:689-745):
//   code planes   gate/up [E'][I][H/32][16 B], down [E'][H][I/32][16 B]
//   scale planes  gate/up [E'][I][H/32] fp16,  down [E'][H][I/32] fp16
// where E' = E + shared.  Canonical 18-byte Q4_0 blocks (src/quant.hpp:8) are
// split into a 16-byte-aligned code plane (one dwordx4 per block, coalesced
// across a wave) and a scale plane.  Activations use the same split:
//   Q8 code plane [rows][blocks][32 B] and a header plane [rows][blocks] of
//   u32 = half d | half s << 16 (the two header fields of the 36-byte Q8_1).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace moe {

// Makes `device` current for one host call of the C ABI and restores the
// caller's current device on every return path (the calls that allocate,
// copy or synchronise need their handle's device current; the caller's
// choice of device must survive them).
class DeviceScope {
public:
    explicit DeviceScope(int device) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        ok_ = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceScope() {
        if (prev_ >= 0) (void)hipSetDevice(prev_);
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;
    bool ok() const { return ok_; }

private:
    int prev_ = -1;
    bool ok_ = false;
};

// Routing and tiling constants.
inline constexpr int kStreamTokens = 4;     // tokens per streaming (decode) work item
inline constexpr int kMfmaTile = 128;       // tokens per MFMA work item (4 waves x 32)
inline constexpr int kSmallGroupTokens = 256;  // single-workgroup grouping limit

// Scale-plane order.  Scales are grouped so that one 16-byte load gives a
// lane the 8 scales the streaming kernels need for its block:
//   gate/up (kScaleGroupGateUp):  [rows/8][blocks][8]    row r at slot r % 8
//   down    (kScaleGroupDown):    [rows/32][blocks][32]  row r at slot (r % 4) * 8 + (r % 32) / 4
// `row` counts rows across experts (expert * rows_per_expert + r); rows per
// expert are multiples of 32, so groups never straddle experts.
inline constexpr int kScaleGroupGateUp = 8;
inline constexpr int kScaleGroupDown = 32;
__host__ __device__ inline size_t scale_index(size_t row, int kb, int blocks_per_row, int group) {
    if (group == kScaleGroupGateUp)
        return ((row / 8) * blocks_per_row + kb) * 8 + row % 8;
    return ((row / 32) * blocks_per_row + kb) * 32 + (row % 4) * 8 + (row % 32) / 4;
}

struct Bank {
    const uint8_t *gate_codes, *up_codes, *down_codes;
    const uint16_t *gate_scales, *up_scales, *down_scales;
    const uint16_t *down_mins;   // Q4_1 down matrices: fp16 m per block (scale order); nullptr for Q4_0
};

// A work item: one expert group slice of <= kStreamTokens (stream path) or
// <= kMfmaTile (MFMA path) consecutive grouped pairs.  Streaming items carry
// their pairs' tokens and ranks inline so a kernel can issue activation loads
// straight after the (scalar) item load.
struct Item {
    int expert, first, ncols, pad;
    int token[kStreamTokens];
    int rank[kStreamTokens];
};

struct Shape {
    int H, I, E, Ep, k;   // Ep = E + has_shared
};

struct RouteOut {
    int32_t *counts;       // [Ep]
    int32_t *offsets;      // [Ep+1]
    int32_t *pair_token;   // [P']
    int32_t *pair_rank;    // [P']  (rank k = shared expert)
    int32_t *pos_of;       // [N*k] grouped position of (t, r) or -1
    Item *stream_items;    // [<= P'/kStreamTokens + Ep]
    Item *mfma_items;      // [<= P'/kMfmaTile + Ep]
    int32_t *item_counts;  // [0] stream items, [1] mfma items, [2] active groups, [3] grouped pairs
    uint32_t *bitmap;      // large path: [W][Ep] token bitmaps
    uint32_t *wprefix;     // large path: [W][Ep] per-word exclusive popcount prefix
};

struct Act {               // split-plane Q8 rows
    uint8_t *codes;        // [rows][blocks][32]
    uint32_t *heads;       // [rows][blocks]
};

// ----------------------------------------------------------------------------
// Kernel launchers (moe_kernels.hip).  All return hipGetLastError() after the
// enqueue; argument validation is done by the callers in moe_layer.hip.
hipError_t launch_quantize_canonical(const float *x, void *q8, int width, int columns, int *error,
                                     hipStream_t s);
hipError_t launch_quantize_planes(const float *x, Act out, int width, int columns, int *error,
                                  hipStream_t s);
hipError_t launch_canonical_to_planes(const void *q8, Act out, int blocks, hipStream_t s);
hipError_t launch_planes_to_canonical(Act in, void *q8, int blocks, hipStream_t s);

// Weight planes of one matrix kind (codes / scales = plane bases).  The call
// covers plane blocks [block0, block0 + blocks); rows hold `blocks_per_row`
// blocks and scales use scale group `group`.
// mins == nullptr: 18-byte Q4_0 canonical blocks; else 20-byte Q4_1 blocks
// whose m goes to / comes from the mins plane.
hipError_t launch_repack_weights(const uint8_t *canonical, uint8_t *codes, uint16_t *scales, uint16_t *mins,
                                 size_t blocks, size_t block0, int blocks_per_row, int group, hipStream_t s);
hipError_t launch_unpack_weights(const uint8_t *codes, const uint16_t *scales, const uint16_t *mins,
                                 uint8_t *canonical, size_t blocks, size_t block0, int blocks_per_row, int group,
                                 hipStream_t s);
// Synthetic blocks: hashed from (seed, hash0 + plane block index).
hipError_t launch_synthetic_weights(uint8_t *codes, uint16_t *scales, uint16_t *mins, size_t blocks, size_t hash0,
                                    int blocks_per_row, int group, uint64_t seed, hipStream_t s);

// Quantize x into `xq` and group routes (tokens <= kSmallGroupTokens path or
// the multi-kernel path).  mfma_min = smallest group that goes to MFMA (0 = never).
hipError_t launch_prepare(const float *x, const int32_t *ids, const float *weights, int tokens,
                          Shape shape, Act xq, RouteOut routes, int mfma_min, int *error,
                          hipStream_t s);

// Single-expert stage setup: pairs 0..columns-1 = tokens 0..columns-1 of
// expert `expert`; all columns go to one path (use_mfma).
hipError_t launch_single_expert_items(Shape shape, RouteOut routes, int expert, int columns,
                                      int use_mfma, hipStream_t s);

struct FfnArgs {
    Shape shape;
    Bank bank;
    Act xq;            // activations [tokens]
    Act mq;            // middle [pairs]
    RouteOut routes;
    float *out;        // contributions: row = token*out_stride_k + rank
    int out_stride_k;  // rows per token in `out` (k+1 for forward, 1 for stages)
    int tokens;
    int pairs_bound;   // upper bound on grouped pairs (for grid sizing)
    int mfma_min;      // groups of >= mfma_min pairs are MFMA items (0: none; 1: all)
    float *middle_f32; // optional [pairs][I]
    int32_t *gate_dots, *up_dots, *down_dots;  // optional per-block dots [pair][rows][blocks]
    int *error;
    int cu_count;      // compute units of the device (persistent grids)
};

// Ungrouped decode path (few tokens, mostly one token per expert): work is
// indexed by (token, rank) directly, so no grouping runs.  The middle Q8 row
// of pair (t, r) is t * (k + has_shared) + r.
struct DecodeArgs {
    FfnArgs f;
    const float *x;            // [tokens][H]
    const int32_t *ids;        // [tokens][k]
    const float *weights;      // [tokens][k]
    const float *shared_gate;  // [tokens] or nullptr
    float *y;                  // [tokens][H]
    const void *x_q8;          // canonical Q8_1 [tokens][H/32] used instead of x, or nullptr
};
inline constexpr int kDecodeMaxBlocksH = 128;  // H/32 <= 128: one or two blocks per lane
inline constexpr int kDecodeMaxBlocksI = 32;   // I/32 <= 32: 16 lanes per down row, one or two blocks each
inline constexpr int kDecodeMaxPairs = 16;     // k + has_shared <= 16: one wave per rank in the fold
// gate/up + SiLU + Q8 (quantizes each token's x on the fly; rank 0 / slice 0
// also writes the token's x Q8 planes for debugging).
hipError_t launch_decode_gate_up(const DecodeArgs &d, hipStream_t s);
// down + rank-order fold + shared add into y.
hipError_t launch_decode_down_fold(const DecodeArgs &d, hipStream_t s);
// Debug view: the decode-layout middle Q8 rows in grouped pair order, as
// canonical 36-byte blocks (routes must hold the grouping of the same batch).
hipError_t launch_decode_middle_grouped(Act mq, RouteOut routes, Shape shape, int tokens, void *q8,
                                        hipStream_t s);

hipError_t launch_gate_up(const FfnArgs &a, bool mfma, hipStream_t s);
hipError_t launch_down(const FfnArgs &a, bool mfma, hipStream_t s);
// Int8-MFMA kernels over the MFMA items (moe_mfma.hip).
hipError_t launch_gate_up_mfma(const FfnArgs &a, hipStream_t s);
hipError_t launch_down_mfma(const FfnArgs &a, hipStream_t s);

// One Q4_0 matrix (planes, rows padded to a multiple of 32) against N
// columns in split Q8 planes, in the reference MMVQ fp32 order, on int8 MFMA
// (moe_mfma.hip); used by moe_linear for wide column counts.
struct LinearMfmaArgs {
    const uint8_t *codes;     // [Mp][nb][16 B]
    const uint16_t *scales;   // [Mp/8][nb][8]
    Act xq;                   // [N][nb] planes, read when q8 is null
    const uint8_t *q8;        // canonical Q8_1 columns [N][nb][36 B] {d, s, qs[32]}, or null
    float *y;                 // [N][M]
    int nb, M, N;
    int row_tiles;            // Mp / 32
    int col_tiles;            // ceil(N / 32)
    int waves;                // waves per workgroup: 4, or 8 (two tree nodes a wave)
};
hipError_t launch_linear_mfma(const LinearMfmaArgs &a, hipStream_t s);

hipError_t launch_fold(const float *contributions, size_t token_stride, const float *weights, int k,
                       const int32_t *pos_of, const float *shared, size_t shared_stride,
                       const float *shared_gate, int tokens, int H, float *y, int *error,
                       hipStream_t s);

hipError_t launch_fill_u32(uint32_t *p, uint32_t value, size_t count, hipStream_t s);
// Router softmax + top-k selection, one token per 64-thread block
// (experts % 32 == 0, experts <= 1024, top_k <= 32); prob may be null.
hipError_t launch_router(const float *logits, int tokens, int experts, int top_k, float *prob, int32_t *ids,
                         float *weights, int *error, hipStream_t s);
hipError_t launch_read_probe(const void *p, size_t bytes, uint32_t *sink, hipStream_t s);
hipError_t launch_expf(const float *x, float *y, int n, hipStream_t s);

}  // namespace moe
