// A compiled C++ caller of the C ABI, written the way the reference's session
// would bind it (src/session.hip:700-716 for the tensors, :1422-1433 and
// :1446-1541 for the router and the FFN call): it includes moe_ffn.h, hands
// over three routed-expert tensors [E][rows][blocks] plus the shared expert's
// matrices with moe_ffn_create_tensors, and on its own hipStream_t runs
// moe_router_select on router logits and moe_ffn_forward on the device routes.
//
// Weights, x and logits come from an integer hash (below), so the expected
// outputs can be written by the CPU oracle without shipping the weights:
// tests/golden/make_abi_case.py writes tests/golden/abi_caller_case.bin with
// the oracle's ids, weights and y for three batches (2 tokens: the decode
// path, no shared gate; 24 tokens: grouped streaming, gated; 3 tokens: the
// decode path, gated).  Every path follows the reference's fp32 order, so
// every value must match bit for bit.
//
// Gated batches follow the reference's shared_project: the shared expert's
// scalar gate logit per token is the dense H -> 1 projection of the FFN input
// (launch_dense_linear into f(16), src/session.hip:1399-1402), which stays
// with the caller; moe_ffn_forward then takes those logits as `shared_gate`
// and applies sigmoid(g) to the shared expert's row (shared_add,
// src/session.hip:1404-1410).  Here the projection is a plain fp32 dot product
// on the host in element order, which the case generator repeats.
//
// Usage: abi_caller <case.bin>   (exit 0 = pass)
#include "moe_ffn.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

constexpr int kH = 2048, kI = 512, kE = 32, kK = 4;

uint64_t mix(uint64_t z) {   // splitmix64 finaliser
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Q4_0 block `g` of matrix kind m (0 gate, 1 up, 2 down) of expert e (kE =
// the shared expert): d = half with bits 0x1C00 | (h & 0x3FF), i.e. in
// [2^-7, 2^-6), and 16 hashed code bytes.
void block(int m, int e, size_t g, uint8_t out[18]) {
    const uint64_t h = mix((static_cast<uint64_t>(m) << 56) ^ (static_cast<uint64_t>(e) << 40) ^ g);
    const uint16_t d = static_cast<uint16_t>(0x1C00u | (h & 0x3FFu));
    std::memcpy(out, &d, 2);
    const uint64_t c0 = mix(h), c1 = mix(h + 1);
    std::memcpy(out + 2, &c0, 8);
    std::memcpy(out + 10, &c1, 8);
}

std::vector<uint8_t> matrix(int m, int e, int rows, int blocks_per_row) {
    std::vector<uint8_t> v(static_cast<size_t>(rows) * blocks_per_row * 18);
    for (size_t g = 0; g < static_cast<size_t>(rows) * blocks_per_row; ++g) block(m, e, g, v.data() + g * 18);
    return v;
}

float hashed(uint64_t tag, size_t i, float scale) {
    return static_cast<float>(static_cast<int>(mix(tag + i) & 0xFFFFu) - 32768) * scale;
}

// The shared gate's dense H -> 1 projection of each token row: g[t] = sum of
// x[t][i] * gate_w[i], products rounded to fp32 and added left to right.
#pragma clang fp contract(off)
std::vector<float> gate_logits(const std::vector<float> &x, const std::vector<float> &gate_w, int n) {
    std::vector<float> g(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) {
        float acc = 0.0f;
        for (int i = 0; i < kH; ++i) {
            const float p = x[static_cast<size_t>(t) * kH + i] * gate_w[static_cast<size_t>(i)];
            acc = acc + p;
        }
        g[static_cast<size_t>(t)] = acc;
    }
    return g;
}

#define CHECK(call)                                                                       \
    do {                                                                                  \
        const int st_ = static_cast<int>(call);                                           \
        if (st_ != 0) {                                                                   \
            std::fprintf(stderr, "%s failed with status %d (line %d)\n", #call, st_, __LINE__); \
            return 1;                                                                     \
        }                                                                                 \
    } while (0)

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) { std::fprintf(stderr, "usage: %s <case.bin>\n", argv[0]); return 2; }
    FILE *f = std::fopen(argv[1], "rb");
    if (!f) { std::fprintf(stderr, "cannot open %s\n", argv[1]); return 2; }
    int32_t head[8];
    if (std::fread(head, 4, 8, f) != 8 || head[0] != 0x4D4F4532 || head[1] != kH || head[2] != kI || head[3] != kE ||
        head[4] != kK) {
        std::fprintf(stderr, "bad case file header\n");
        return 2;
    }
    const int ncases = head[5];
    if (ncases < 1 || ncases > 8) return 2;
    std::vector<int> tokens(ncases), gated(ncases);
    if (std::fread(tokens.data(), 4, ncases, f) != static_cast<size_t>(ncases) ||
        std::fread(gated.data(), 4, ncases, f) != static_cast<size_t>(ncases))
        return 2;
    // The shared gate's projection weights (ffn_gate_inp_shexp, H floats).
    std::vector<float> gate_w(kH);
    for (int i = 0; i < kH; ++i) gate_w[static_cast<size_t>(i)] = hashed(0x6A7E000000ull, static_cast<size_t>(i), 1.0f / 1048576);

    // The routed-expert tensors as Experts::ram holds them: [E][rows][blocks].
    std::vector<uint8_t> gate, up, down;
    for (int e = 0; e < kE; ++e) {
        auto g = matrix(0, e, kI, kH / 32), u = matrix(1, e, kI, kH / 32), d = matrix(2, e, kH, kI / 32);
        gate.insert(gate.end(), g.begin(), g.end());
        up.insert(up.end(), u.begin(), u.end());
        down.insert(down.end(), d.begin(), d.end());
    }
    const auto sg = matrix(0, kE, kI, kH / 32), su = matrix(1, kE, kI, kH / 32), sd = matrix(2, kE, kH, kI / 32);

    int max_tokens = 0;
    for (int n : tokens) max_tokens = n > max_tokens ? n : max_tokens;
    moe_ffn_config cfg{};
    cfg.hidden = kH;
    cfg.intermediate = kI;
    cfg.experts = kE;
    cfg.top_k = kK;
    cfg.has_shared = 1;
    cfg.max_tokens = max_tokens;
    cfg.down_type = MOE_DOWN_Q4_0;
    moe_ffn_layer *layer = nullptr;
    CHECK(moe_ffn_create_tensors(&cfg, gate.data(), up.data(), down.data(), sg.data(), su.data(), sd.data(), 0,
                                 &layer));
    hipStream_t stream = nullptr;
    CHECK(hipStreamCreate(&stream));

    int failures = 0;
    for (int c = 0; c < ncases; ++c) {
        const int n = tokens[c];
        std::vector<float> x(static_cast<size_t>(n) * kH), logits(static_cast<size_t>(n) * kE);
        for (size_t i = 0; i < x.size(); ++i) x[i] = hashed(0xA5C0000000ull + 0x1000000ull * c, i, 1.0f / 16384);
        for (size_t i = 0; i < logits.size(); ++i) logits[i] = hashed(0xD3F0000000ull + 0x1000000ull * c, i, 1.0f / 8192);
        std::vector<int32_t> want_ids(static_cast<size_t>(n) * kK);
        std::vector<float> want_w(static_cast<size_t>(n) * kK), want_y(static_cast<size_t>(n) * kH);
        if (std::fread(want_ids.data(), 4, want_ids.size(), f) != want_ids.size() ||
            std::fread(want_w.data(), 4, want_w.size(), f) != want_w.size() ||
            std::fread(want_y.data(), 4, want_y.size(), f) != want_y.size()) {
            std::fprintf(stderr, "case file truncated\n");
            return 2;
        }
        float *dx = nullptr, *dlogits = nullptr, *dw = nullptr, *dy = nullptr, *dgate = nullptr;
        int32_t *dids = nullptr;
        int *derr = nullptr;
        if (gated[c]) {   // f(16): the scalar gate logits, before the FFN call
            const std::vector<float> g = gate_logits(x, gate_w, n);
            CHECK(hipMalloc(&dgate, g.size() * 4));
            CHECK(hipMemcpy(dgate, g.data(), g.size() * 4, hipMemcpyHostToDevice));
        }
        CHECK(hipMalloc(&dx, x.size() * 4));
        CHECK(hipMalloc(&dlogits, logits.size() * 4));
        CHECK(hipMalloc(&dids, want_ids.size() * 4));
        CHECK(hipMalloc(&dw, want_w.size() * 4));
        CHECK(hipMalloc(&dy, want_y.size() * 4));
        CHECK(hipMalloc(&derr, 4));
        CHECK(hipMemcpyAsync(dx, x.data(), x.size() * 4, hipMemcpyHostToDevice, stream));
        CHECK(hipMemcpyAsync(dlogits, logits.data(), logits.size() * 4, hipMemcpyHostToDevice, stream));
        CHECK(hipMemsetAsync(derr, 0, 4, stream));
        // Router on the device, then the routed FFN on its routes: no host
        // round trip between them (the reference downloads probabilities and
        // uploads routes here, src/session.hip:1422-1433, 393-410).
        CHECK(moe_router_select(dlogits, n, kE, kK, nullptr, dids, dw, derr, stream));
        CHECK(moe_ffn_forward(layer, dx, dids, dw, n, dgate, dy, derr, stream));
        std::vector<int32_t> ids(want_ids.size());
        std::vector<float> w(want_w.size()), y(want_y.size());
        int err = -1;
        CHECK(hipMemcpyAsync(ids.data(), dids, ids.size() * 4, hipMemcpyDeviceToHost, stream));
        CHECK(hipMemcpyAsync(w.data(), dw, w.size() * 4, hipMemcpyDeviceToHost, stream));
        CHECK(hipMemcpyAsync(y.data(), dy, y.size() * 4, hipMemcpyDeviceToHost, stream));
        CHECK(hipMemcpyAsync(&err, derr, 4, hipMemcpyDeviceToHost, stream));
        CHECK(hipStreamSynchronize(stream));
        const bool ids_ok = std::memcmp(ids.data(), want_ids.data(), ids.size() * 4) == 0;
        const bool w_ok = std::memcmp(w.data(), want_w.data(), w.size() * 4) == 0;
        size_t ydiff = 0;
        for (size_t i = 0; i < y.size(); ++i) ydiff += std::memcmp(&y[i], &want_y[i], 4) != 0;
        const bool ok = err == 0 && ids_ok && w_ok && ydiff == 0;
        std::printf("case %d: %d tokens, %s, error word %d, ids %s, weights %s, y %zu of %zu values differ: %s\n", c,
                    n, gated[c] ? "shared gate" : "no shared gate", err, ids_ok ? "equal" : "DIFFER",
                    w_ok ? "bit-equal" : "DIFFER", ydiff, y.size(), ok ? "ok" : "FAIL");
        failures += !ok;
        CHECK(hipFree(dx));
        CHECK(hipFree(dlogits));
        CHECK(hipFree(dids));
        CHECK(hipFree(dw));
        CHECK(hipFree(dy));
        CHECK(hipFree(derr));
        if (dgate) CHECK(hipFree(dgate));
    }
    std::fclose(f);
    CHECK(hipStreamDestroy(stream));
    CHECK(moe_ffn_destroy(layer));
    std::printf("%s\n", failures ? "FAIL" : "PASS");
    return failures ? 1 : 0;
}
