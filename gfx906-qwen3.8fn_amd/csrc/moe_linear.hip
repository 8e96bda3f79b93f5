// Quantized linear projections (Q4_0 / Q4_1 weights x Q8_1 activations) for
// the non-expert matrices around the MoE FFN: the MI355X counterpart of the
// reference's launch_quantized_linear{,_short,_tiled}
// (src/hip/linear.hip:444-490, contract src/hip/linear.cuh:24-87) and of
// Matrix::apply for its Q4 types (src/session.hip:559-591).
//
// fp32 order.  The reference's MMVQ kernel (src/hip/linear.hip:214-262) runs
// 128 threads per row set: thread t takes fragment t % 2 of blocks
// t / 2, t / 2 + 64, ... in ascending order, accumulating
//   Q4_0: acc = fma(d4, fma(float(I_f), d8, -4 s8), acc)
//   Q4_1: acc = acc + fma(float(I_f), half(d4 d8), half(m4 s8) / 2)
// (accumulate32, src/hip/linear.hip:195-222); wave 1's accumulator is added
// to wave 0's lane-wise and the 64 lanes are summed by an ascending XOR
// butterfly.  This is the order src/cpu_expert.cpp:156-213 restates on the
// CPU (lane 2 (k % 64) + f, fold lane i + 64, XOR 1..32).  Here one wave64
// covers all 128 reference lanes: lane j holds both fragments of blocks
// j, j + 64, ...; the fold is "lane j + lane j ^ 32 per fragment", then the
// two fragments, then XOR 1..16 -- the same additions on the same values, so
// every output is bit-identical to the reference's.
//
// Layout.  At creation the canonical [output][input/32] blocks are split into
// a code plane [rows][blocks][16 B] and fp16 scale (and Q4_1 min) planes
// [rows/8][blocks][8], rows padded to a multiple of 32 with zero blocks, so a
// lane's 8 row codes are eight 16-byte loads and its 8 scales one more.
//
// Wide batches (Q4_0, at least 32 columns and kMfmaMinOutputs outputs) go to
// int8 MFMA instead (k_linear_mfma in moe_mfma.hip): the same fp32 order, with
// the per-fragment integer dots from v_mfma_i32_32x32x16_i8.  forward_q8's
// MFMA launch reads the caller's canonical blocks in place (any column
// count); apply quantizes into split planes in the handle's workspace.
//
// Work: one wave per (8 rows, column tile).  The wave loads its 8 rows'
// blocks once per 4 columns (2 when a row has more than 64 blocks) and keeps
// them in registers while it reads the columns' Q8_1 blocks straight from the
// caller's canonical 36-byte array.
// Workgroup ids are XCD-aware (id % 8 = XCD): the column tiles of one row
// slice run on one XCD, so that slice's rows are fetched from HBM once.
#include "moe_device.hpp"
#include "moe_ffn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <new>

namespace moe {
namespace {

constexpr int kLinearCols = 4;          // column-tile granularity of the Q4_1 two-slot form (G = 2)
constexpr int kLinearWaveTarget = 2048; // waves a launch aims for (8 XCDs x 32 CUs x 8)

struct LinearArgs {
    const uint8_t *codes;    // [Mp][nb][16 B]
    const uint16_t *scales;  // [Mp/8][nb][8]
    const uint16_t *mins;    // Q4_1: same order as scales; Q4_0: nullptr
    const uint8_t *x;        // canonical Q8_1 [N][nb][36 B]
    float *y;                // [N][M]
    int nb, M, N;
    int slices;              // Mp / ROWS
    int tiles, tile_cols;    // column tiles per slice; columns per tile (multiple of kLinearCols)
};

// HOLD = block slots (64 blocks each) whose weights are loaded together;
// G = columns accumulated per pass over the weights; ROWS = rows per wave
// (8, or 4: half an 8-row scale group, a.slices = Mp / 4).
template<bool Q41, int HOLD, int G, int ROWS = 8>
__global__ __launch_bounds__(64, ROWS == 4 ? (G == 4 ? 3 : 4) : 2) void k_linear(LinearArgs a) {
    const int lane = threadIdx.x;
    const int id = static_cast<int>(blockIdx.x), local = id >> 3;
    const int slice = (id & 7) + 8 * (local / a.tiles), tile = local % a.tiles;
    if (slice >= a.slices) return;   // uniform per workgroup (grid padded to 8 slices)
    const int c0 = tile * a.tile_cols, c1 = min(c0 + a.tile_cols, a.N);
    if (c0 >= c1) return;
    const int nb = a.nb, row0 = slice * ROWS, slots = (nb + 63) / 64;
    const uint32_t row_bytes = static_cast<uint32_t>(nb) * 16u;
    const auto wr = buffer_rsrc(a.codes + static_cast<size_t>(row0) * row_bytes, ROWS * row_bytes);
    // The slice's scale group (8 rows) and, for 4 rows, its half of each
    // block's 8 scales.
    const size_t g0 = static_cast<size_t>(row0 & ~7);
    const uint32_t shalf = static_cast<uint32_t>(row0 & 4) * 2u;
    const auto sr = buffer_rsrc(a.scales + g0 * nb, row_bytes);
    const auto mr = buffer_rsrc(Q41 ? a.mins + g0 * nb : a.scales, row_bytes);
    const auto xr = buffer_rsrc(a.x, static_cast<uint32_t>(static_cast<size_t>(a.N) * nb * 36));
    const int rho = ROWS == 8 ? 4 * ((lane >> 5) & 1) + 2 * (lane & 1) + ((lane >> 1) & 1)
                              : 2 * ((lane >> 5) & 1) + (lane & 1);
    for (int c = c0; c < c1; c += G) {   // uniform
        float acc[G][ROWS][2];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[g][r][0] = acc[g][r][1] = 0.0f;
        for (int i0 = 0; i0 < slots; i0 += HOLD) {   // uniform
            uint4 w[HOLD][ROWS];
            float d4[HOLD][ROWS], m4[HOLD][ROWS];
            bool has[HOLD];
            uint32_t kk[HOLD];
#pragma unroll
            for (int h = 0; h < HOLD; ++h) {
                const int k = lane + 64 * (i0 + h);
                // Lanes past the row end (or past the last slot) load block 0
                // and keep their accumulators: every load is unconditional.
                has[h] = i0 + h < slots && k < nb;
                kk[h] = has[h] ? static_cast<uint32_t>(k) : 0u;
#pragma unroll
                for (int r = 0; r < ROWS; ++r) w[h][r] = buffer_load16(wr, kk[h] * 16u, r * row_bytes);
                uint32_t dw[4], mw[4];
                if constexpr (ROWS == 8) {
                    const uint4 dp = buffer_load16(sr, kk[h] * 16u, 0);
                    dw[0] = dp.x; dw[1] = dp.y; dw[2] = dp.z; dw[3] = dp.w;
                } else {
                    const auto dp = __builtin_amdgcn_raw_buffer_load_b64(sr, kk[h] * 16u + shalf, 0, 0);
                    dw[0] = dp[0]; dw[1] = dp[1]; dw[2] = dw[3] = 0u;
                }
#pragma unroll
                for (int r = 0; r < ROWS; ++r) d4[h][r] = h2f(dw[r >> 1] >> (16 * (r & 1)));
                if constexpr (Q41) {
                    if constexpr (ROWS == 8) {
                        const uint4 mp = buffer_load16(mr, kk[h] * 16u, 0);
                        mw[0] = mp.x; mw[1] = mp.y; mw[2] = mp.z; mw[3] = mp.w;
                    } else {
                        const auto mp = __builtin_amdgcn_raw_buffer_load_b64(mr, kk[h] * 16u + shalf, 0, 0);
                        mw[0] = mp[0]; mw[1] = mp[1]; mw[2] = mw[3] = 0u;
                    }
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) m4[h][r] = h2f(mw[r >> 1] >> (16 * (r & 1)));
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                if (c + g >= c1) break;   // uniform
                const uint32_t xs = static_cast<uint32_t>(static_cast<size_t>(c + g) * nb * 36);
#pragma unroll
                for (int h = 0; h < HOLD; ++h) {
                    const uint32_t xo = kk[h] * 36u;
                    const uint32_t head = buffer_load4(xr, xo, xs);
                    const uint4 x0 = buffer_load16(xr, xo + 4u, xs);
                    const uint4 x1 = buffer_load16(xr, xo + 20u, xs);
                    const float d8 = h2f(head), s8 = h2f(head >> 16), c4 = -4.0f * s8;
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) {
                        int f[2];
                        fragment_dots(w[h][r], x0, x1, f[0], f[1]);
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            float v;
                            if constexpr (Q41) {
                                const float dd = h2f(f2h(d4[h][r] * d8)), hm = h2f(f2h(m4[h][r] * s8)) * 0.5f;
                                v = acc[g][r][q] + fmaf(static_cast<float>(f[q]), dd, hm);
                            } else {
                                v = fmaf(d4[h][r], fmaf(static_cast<float>(f[q]), d8, c4), acc[g][r][q]);
                            }
                            acc[g][r][q] = has[h] ? v : acc[g][r][q];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (c + g >= c1) break;   // uniform
            float v;
            if constexpr (ROWS == 8) v = fold_rows8(acc[g], lane);
            else v = fold_rows4(acc[g], lane);
            const int row = row0 + rho;
            if ((lane & (ROWS == 8 ? 28 : 30)) == 0 && row < a.M) a.y[static_cast<size_t>(c + g) * a.M + row] = v;
        }
    }
}

}  // namespace
}  // namespace moe

// Activation staging of moe_linear_apply_noalloc: a file-scope device array,
// one copy per GPU the library runs on, held until the process ends.  Its
// name is a host-side stand-in, never a device address: host code uses only
// the per-device address that hipGetSymbolAddress returns (noalloc_scratch).
constexpr size_t kNoallocScratchBytes = size_t{4} << 20;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
uint8_t *scratch_ptr[kMaxDevices] = {};
// Set while a host thread is inside moe_linear_apply_noalloc for that GPU: a
// second thread that enters meanwhile is refused instead of enqueueing work
// on the same array.  (Calls enqueued one after another on different streams
// can still overlap on the GPU; that is the caller's to order.)
std::atomic<int> scratch_busy[kMaxDevices] = {};

// Looks up (once per device, with that device current) the device address of
// `scratch`.  Called by moe_linear_create, the library's set-up call, so that
// the no-allocation entry point itself only reads the table.
hipError_t init_noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_ptr[device]) return hipSuccess;
    void *p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess) return r;
    if (!p) return hipErrorInvalidSymbol;
    scratch_ptr[device] = static_cast<uint8_t *>(p);
    return hipSuccess;
}

uint8_t *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    return scratch_ptr[device];
}
}  // namespace

// ------------------------------------------------------------------ C ABI ---
struct moe_linear {
    int type = 0, input = 0, output = 0, max_columns = 0, device = 0;
    int mfma_mode = -1;          // MOE_LINEAR_MFMA at creation: 0 never, 1 whenever eligible, -1 by size
    int vector_g = 0;            // MOE_LINEAR_G at creation: columns per pass of k_linear (1, 2, 4), 0 by size
    int vector_rows = 0;         // MOE_LINEAR_ROWS at creation: rows per wave of k_linear (4, 8), 0 by size
    int nb = 0, Mp = 0;
    uint8_t *planes = nullptr;   // codes | scales | mins (one allocation)
    uint8_t *codes = nullptr;
    uint16_t *scales = nullptr, *mins = nullptr;
    // apply's activation workspace, max_columns x nb x 36 B: canonical Q8_1
    // blocks (narrow batches) or split planes (wide batches on MFMA).
    void *q8 = nullptr;
};

namespace {

constexpr int kInvalid = hipErrorInvalidValue;
constexpr int kMfmaMinColumns = 32;        // one MFMA column tile
// Outputs (rows x columns) from which the MFMA kernel beats the vector one
// (MI355X, cold weights, vector / MFMA us with the per-launch vector plans
// and the 8-wave MFMA form: 2048 x 2048 at 32 / 48 / 64 columns 6.6 / 9.9 /
// 10.6 against 8.65 / 8.87 / 9.0; 512 rows at 128 / 192 / 256 columns 6.35 /
// 9.8 / 10.6 against 8.3 / 8.6 / 8.9; 2560 x 2560 at 48 columns 19.0 against
// 13.3; 8192 rows at 32 columns 56.8 against 48.2).
constexpr long kMfmaMinOutputs = 96 * 1024;

bool aligned(const void *p, size_t a) { return p && reinterpret_cast<uintptr_t>(p) % a == 0; }
size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

void release(moe_linear *L) {
    if (!L) return;
    if (L->planes) (void)hipFree(L->planes);
    if (L->q8) (void)hipFree(L->q8);
    delete L;
}

int block_bytes(int type) { return type == MOE_TYPE_Q4_1 ? 20 : 18; }

}  // namespace

extern "C" {

int moe_linear_create(int type, int input, int output, int max_columns, const void *weights, int weights_on_device,
                      int device, moe_linear **out) {
    if (!out) return kInvalid;
    *out = nullptr;
    if ((type != MOE_TYPE_Q4_0 && type != MOE_TYPE_Q4_1) || input < 32 || input > 16384 || input % 32 ||
        output < 1 || output > 16384 || max_columns < 0 || max_columns > 65536 || !aligned(weights, 2))
        return kInvalid;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return kInvalid;
    moe::DeviceScope scope(device);   // the caller's current device is restored on return
    if (!scope.ok()) return kInvalid;
    auto *L = new (std::nothrow) moe_linear;
    if (!L) return hipErrorOutOfMemory;
    L->type = type;
    L->input = input;
    L->output = output;
    L->max_columns = max_columns;
    L->device = device;
    L->nb = input / 32;
    if (const char *env = std::getenv("MOE_LINEAR_MFMA")) L->mfma_mode = std::atoi(env) ? 1 : 0;
    if (const char *env = std::getenv("MOE_LINEAR_G")) {
        const int g = std::atoi(env);
        L->vector_g = g == 1 || g == 2 || g == 4 ? g : 0;
    }
    if (const char *env = std::getenv("MOE_LINEAR_ROWS")) {
        const int r = std::atoi(env);
        L->vector_rows = r == 4 || r == 8 ? r : 0;
    }
    L->Mp = static_cast<int>(round_up(static_cast<size_t>(output), 32));
    const size_t pblocks = static_cast<size_t>(L->Mp) * L->nb;
    const size_t code_bytes = round_up(pblocks * 16, 256), scale_bytes = round_up(pblocks * 2, 256);
    const size_t total = code_bytes + scale_bytes * (type == MOE_TYPE_Q4_1 ? 2 : 1);
    hipError_t r = hipMalloc(&L->planes, total);
    if (r != hipSuccess) { release(L); return r; }
    L->codes = L->planes;
    L->scales = reinterpret_cast<uint16_t *>(L->planes + code_bytes);
    L->mins = type == MOE_TYPE_Q4_1 ? reinterpret_cast<uint16_t *>(L->planes + code_bytes + scale_bytes) : nullptr;
    if (max_columns > 0 && (r = hipMalloc(&L->q8, static_cast<size_t>(max_columns) * L->nb * 36)) != hipSuccess) {
        release(L);
        return r;
    }
    // Padding rows stay zero blocks (d = 0): their sums are computed and dropped.
    if ((r = hipMemset(L->planes, 0, total)) != hipSuccess) { release(L); return r; }
    const size_t blocks = static_cast<size_t>(output) * L->nb, bytes = blocks * block_bytes(type);
    const uint8_t *canonical = static_cast<const uint8_t *>(weights);
    void *staging = nullptr;
    if (!weights_on_device) {
        if ((r = hipMalloc(&staging, bytes)) != hipSuccess) { release(L); return r; }
        if ((r = hipMemcpy(staging, weights, bytes, hipMemcpyHostToDevice)) != hipSuccess) {
            (void)hipFree(staging);
            release(L);
            return r;
        }
        canonical = static_cast<const uint8_t *>(staging);
    }
    r = moe::launch_repack_weights(canonical, L->codes, L->scales, L->mins, blocks, 0, L->nb, moe::kScaleGroupGateUp,
                                   nullptr);
    if (r == hipSuccess) r = hipDeviceSynchronize();
    if (r == hipSuccess) r = init_noalloc_scratch(device);
    if (staging) (void)hipFree(staging);
    if (r != hipSuccess) { release(L); return r; }
    *out = L;
    return 0;
}

int moe_linear_destroy(moe_linear *L) {
    if (!L) return kInvalid;
    moe::DeviceScope scope(L->device);
    release(L);
    return 0;
}

int moe_linear_bytes(const moe_linear *L, size_t *weight_bytes) {
    if (!L || !weight_bytes) return kInvalid;
    *weight_bytes = static_cast<size_t>(L->output) * L->nb * block_bytes(L->type);
    return 0;
}

namespace {

// MFMA for wide Q4_0 batches that fit the staging area (`capacity` columns).
bool use_mfma_within(const moe_linear *L, int columns, int capacity) {
    if (L->type != MOE_TYPE_Q4_0 || columns < kMfmaMinColumns || columns > capacity || L->mfma_mode == 0)
        return false;
    return L->mfma_mode == 1 || static_cast<long>(L->output) * columns >= kMfmaMinOutputs;
}
bool use_mfma(const moe_linear *L, int columns) { return use_mfma_within(L, columns, L->max_columns); }

// Split Q8 planes for `columns` columns at `base` (codes, then heads).
moe::Act staging_planes(const moe_linear *L, void *base_ptr, int columns) {
    auto *base = static_cast<uint8_t *>(base_ptr);
    return moe::Act{base, reinterpret_cast<uint32_t *>(base + static_cast<size_t>(columns) * L->nb * 32)};
}
moe::Act workspace_planes(const moe_linear *L, int columns) { return staging_planes(L, L->q8, columns); }

// x_q8: canonical Q8_1 columns read in place, else the split planes xq.
int launch_mfma(const moe_linear *L, moe::Act xq, const void *x_q8, int columns, float *y, hipStream_t s) {
    moe::LinearMfmaArgs a{};
    a.codes = L->codes;
    a.scales = L->scales;
    a.xq = xq;
    a.q8 = static_cast<const uint8_t *>(x_q8);
    a.y = y;
    a.nb = L->nb;
    a.M = L->output;
    a.N = columns;
    a.row_tiles = L->Mp / 32;
    a.col_tiles = (columns + 31) / 32;
    // 8-wave workgroups (two tree nodes a wave) for 64-block rows where the
    // 4-wave grid gives at most one workgroup per CU (us, 4 -> 8 waves,
    // forward_q8 cold: 2048 x 2048 at N = 80 / 128 10.5 / 11.1 -> 9.45 /
    // 10.5, 2048 x 512 at N = 320 / 512 10.2 / 10.9 -> 9.25 / 10.45, 2048 x
    // 1024 at N = 160 / 256 10.3 / 10.9 -> 9.35 / 10.5; larger grids lose:
    // 2048 x 2048 at N = 192 / 1032 16.0 / 54.5 -> 17.2 / 67.5).
    a.waves = L->nb == 64 && static_cast<long>(a.row_tiles) * a.col_tiles <= 256 ? 8 : 4;
    return moe::launch_linear_mfma(a, s);
}

// Column tiling of one vector launch over `slices` row slices: G columns per
// pass over the held weights and `tile_cols` columns per wave.
struct VectorPlan {
    int G, tile_cols, tiles;
};

// G = 4 shares each weight load among the most columns but needs 219 VGPRs
// (2 waves per SIMD at 8 rows); G = 2 (141 VGPRs, 3 waves) and G = 1 (68, 7
// waves) read the weights again from L2 per pass and give matrices with few
// slices enough waves.  The largest G whose launch still has about 2048 waves
// wins (MI355X, cold weights, 8 rows, us at G = 4 / 2 / 1: 8192 x 8192 at N = 8
// 20.1 / 21.8 / 25.1, N = 4 15.8 / 13.6 / 15.5, N = 2 11.9 / 11.9 / 10.3;
// 2560 x 640 at N = 8 5.96 / 4.43 / 3.96; 2048 x 512 at N = 16 4.21 / 3.33 /
// 3.08).  One column: G = 4 (9.6 against 11.1 us at G = 1).  hold2: the
// two-slot form, G = 2 at a granularity of 4 columns.
VectorPlan vector_plan(int slices, int columns, int forced_g, bool hold2) {
    int G = hold2 ? 2 : forced_g;
    if (G == 0) {
        const long s = slices;
        G = columns == 1 || s * ((columns + 3) / 4) >= moe::kLinearWaveTarget ? 4
            : s * ((columns + 1) / 2) >= moe::kLinearWaveTarget               ? 2
                                                                              : 1;
    }
    const int gran = hold2 ? moe::kLinearCols : G;
    const int target = G == 4 || hold2 ? moe::kLinearWaveTarget
                       : G == 2        ? 2 * moe::kLinearWaveTarget
                                       : 4 * moe::kLinearWaveTarget;
    // Column tiles: enough waves to cover the chip, each tile a whole number
    // of passes.
    const int groups = (columns + gran - 1) / gran;
    const int tiles = std::max(1, std::min(groups, (target + slices - 1) / slices));
    const int per = (groups + tiles - 1) / tiles;
    const int tile_cols = per * gran;
    return VectorPlan{G, tile_cols, (columns + tile_cols - 1) / tile_cols};
}

// The vector kernel on canonical Q8_1 columns x_q8.
int launch_vector(const moe_linear *L, const void *x_q8, int columns, float *y, hipStream_t s) {
    moe::LinearArgs a{};
    a.codes = L->codes;
    a.scales = L->scales;
    a.mins = L->mins;
    a.x = static_cast<const uint8_t *>(x_q8);
    a.y = y;
    a.nb = L->nb;
    a.M = L->output;
    a.N = columns;
    const bool q41 = L->type == MOE_TYPE_Q4_1;
    const int slices8 = (L->output + 7) / 8;
    // A single column on rows of more than 64 blocks takes two slots per load
    // round when that covers the row (65..128 blocks) or the matrix has
    // fewer than 1024 slices (us, one slot -> two: Q4_0 2560 x 640 3.43 ->
    // 3.16, 4096 x 1024 3.67 -> 3.34, 2560 x 8192 5.43 -> 5.11, 8192 x 2048
    // 6.44 -> 5.97, but 8192 x 8192 9.77 -> 10.96; Q4_1 2560 x 640 3.46 ->
    // 3.17).  Every other batch takes one slot (Q4_1 2560 x 640 at N = 8
    // 6.25 -> 3.89 us, 8192 x 8192 at N = 4 / 8 20.2 / 22.8 -> 14.7 / 20.8 us
    // against two slots).
    const bool hold2 = L->nb > 64 && columns == 1 && (L->nb <= 128 || slices8 < 1024);
    VectorPlan p = vector_plan(slices8, columns, L->vector_g, hold2);
    // Rows per wave: 4 (130 / 81 / 56 VGPRs at G = 4 / 2 / 1: 3, 6 and 8
    // waves per SIMD) where the 8-row launch leaves the chip short of waves
    // or runs one column per pass on rows of at most 128 blocks; it reads
    // each column's blocks twice as often.  us, 8 rows -> 4: 8192 x 8192 at
    // N = 1 9.8 -> 8.8, 2048 x 2048 at N = 2 / 8 3.12 / 3.84 -> 2.83 / 3.66,
    // 2560 x 640 at N = 8 / 31 3.96 / 5.71 -> 3.34 / 5.28, 2048 x 512 at
    // N = 16 3.09 -> 2.85, Q4_1 640 x 2560 at N = 1 2.93 -> 2.69; but 8192 x
    // 8192 at N = 2 / 8 10.3 / 19.2 -> 11.0 / 24.3 and 1024 x 8192 at N = 8
    // 6.6 -> 7.5.
    int rows = L->vector_rows;
    if (rows == 0)
        rows = !hold2 && (static_cast<long>(slices8) * p.tiles < moe::kLinearWaveTarget || (p.G == 1 && L->nb <= 128))
                   ? 4
                   : 8;
    if (hold2) rows = 8;
    a.slices = rows == 4 ? (L->output + 3) / 4 : slices8;
    if (rows == 4) p = vector_plan(a.slices, columns, L->vector_g, false);
    a.tile_cols = p.tile_cols;
    a.tiles = p.tiles;
    const size_t grid = round_up(static_cast<size_t>(a.slices), 8) * a.tiles;
    if (grid > 0x7fffffffu) return kInvalid;
    const dim3 g(static_cast<unsigned>(grid)), b(64);
    const int G = p.G;
    if (q41) {
        if (hold2) moe::k_linear<true, 2, 2><<<g, b, 0, s>>>(a);
        else if (rows == 4 && G == 4) moe::k_linear<true, 1, 4, 4><<<g, b, 0, s>>>(a);
        else if (rows == 4 && G == 2) moe::k_linear<true, 1, 2, 4><<<g, b, 0, s>>>(a);
        else if (rows == 4) moe::k_linear<true, 1, 1, 4><<<g, b, 0, s>>>(a);
        else if (G == 4) moe::k_linear<true, 1, 4><<<g, b, 0, s>>>(a);
        else if (G == 2) moe::k_linear<true, 1, 2><<<g, b, 0, s>>>(a);
        else moe::k_linear<true, 1, 1><<<g, b, 0, s>>>(a);
    } else {
        // Past one column Q4_0 takes one block slot per load round: 8192 x
        // 8192 at N = 8 / 16, 22.9 / 39.1 us with two slots and 2 columns per
        // round against 19.8 / 33.6 us at one slot and 4 columns (MI355X,
        // cold weights).
        if (hold2) moe::k_linear<false, 2, 2><<<g, b, 0, s>>>(a);
        else if (rows == 4 && G == 4) moe::k_linear<false, 1, 4, 4><<<g, b, 0, s>>>(a);
        else if (rows == 4 && G == 2) moe::k_linear<false, 1, 2, 4><<<g, b, 0, s>>>(a);
        else if (rows == 4) moe::k_linear<false, 1, 1, 4><<<g, b, 0, s>>>(a);
        else if (G == 4) moe::k_linear<false, 1, 4><<<g, b, 0, s>>>(a);
        else if (G == 2) moe::k_linear<false, 1, 2><<<g, b, 0, s>>>(a);
        else moe::k_linear<false, 1, 1><<<g, b, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace

int moe_linear_forward_q8(moe_linear *L, const void *x_q8, int columns, float *y, void *stream) {
    if (!L || !aligned(x_q8, 4) || !aligned(y, 4) || columns < 1 || columns > 65536) return kInvalid;
    const auto s = static_cast<hipStream_t>(stream);
    // The MFMA kernel reads the canonical blocks in place: no staging, so
    // any column count qualifies.
    if (use_mfma_within(L, columns, 65536)) return launch_mfma(L, moe::Act{}, x_q8, columns, y, s);
    return launch_vector(L, x_q8, columns, y, s);
}

int moe_linear_apply(moe_linear *L, const float *x, int columns, float *y, int *error, void *stream) {
    if (!L || !aligned(x, 4) || !aligned(y, 4) || !aligned(error, 4) || columns < 1 || columns > L->max_columns)
        return kInvalid;
    const auto s = static_cast<hipStream_t>(stream);
    if (use_mfma(L, columns)) {
        const moe::Act xq = workspace_planes(L, columns);
        const hipError_t r = moe::launch_quantize_planes(x, xq, L->input, columns, error, s);
        if (r != hipSuccess) return r;
        return launch_mfma(L, xq, nullptr, columns, y, s);
    }
    const hipError_t r = moe::launch_quantize_canonical(x, L->q8, L->input, columns, error, s);
    if (r != hipSuccess) return r;
    return moe_linear_forward_q8(L, L->q8, columns, y, stream);
}

int moe_linear_apply_noalloc(moe_linear *L, const float *x, int columns, float *y, int *error, void *stream) {
    if (!L || !aligned(x, 4) || !aligned(y, 4) || !aligned(error, 4) || columns < 1) return kInvalid;
    // The staging (canonical Q8_1 blocks, or the MFMA kernel's split planes:
    // 36 bytes per block either way) must fit the static array.
    if (static_cast<size_t>(columns) * L->nb * 36 > kNoallocScratchBytes) return kInvalid;
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device != L->device) return kInvalid;
    uint8_t *ws = noalloc_scratch(device);
    if (!ws) return hipErrorNotInitialized;
    if (scratch_busy[device].exchange(1, std::memory_order_acquire)) return hipErrorContextAlreadyInUse;
    struct Release {
        std::atomic<int> &flag;
        ~Release() { flag.store(0, std::memory_order_release); }
    } release_busy{scratch_busy[device]};
    const auto s = static_cast<hipStream_t>(stream);
    const int capacity = static_cast<int>(kNoallocScratchBytes / (static_cast<size_t>(L->nb) * 36));
    if (use_mfma_within(L, columns, capacity)) {
        const moe::Act xq = staging_planes(L, ws, columns);
        const hipError_t r = moe::launch_quantize_planes(x, xq, L->input, columns, error, s);
        if (r != hipSuccess) return r;
        return launch_mfma(L, xq, nullptr, columns, y, s);
    }
    const hipError_t r = moe::launch_quantize_canonical(x, ws, L->input, columns, error, s);
    if (r != hipSuccess) return r;
    return launch_vector(L, ws, columns, y, s);
}

}  // extern "C"
