// extern "C" wrapper around the reference's own CPU path, compiled in this
// container from the reference sources where they lie (/root/reference/src:
// quant.cpp, cpu_expert.cpp, routes.cpp, linear_reference.cpp) by
// oracle/Makefile into oracle/_ref/libref.so.  TEST INFRASTRUCTURE ONLY: it is
// used to pin the C restatement in oracle/moe_oracle.c and to write the golden
// fixtures under tests/golden/.  No reference source is copied; this file only
// calls the reference's public C++ API:
//   quant.hpp:20-42, linear_reference.hpp:15-16, cpu_expert.hpp:24-78,
//   routes.hpp:28-65.
#include "cpu_expert.hpp"
#include "linear_reference.hpp"
#include "quant.hpp"
#include "routes.hpp"

#include <cstring>
#include <exception>
#include <span>

using namespace qwen;

namespace {
template<class F> int guarded(F f) {
    try { f(); return 0; }
    catch (const std::invalid_argument&) { return 1; }
    catch (...) { return 2; }
}
QMatrix q4(const void* w, int input, int output) {
    const auto bytes = static_cast<std::size_t>(input / 32) * static_cast<std::size_t>(output) * sizeof(Q4_0);
    return {TensorType::Q4_0, input, output, {static_cast<const std::byte*>(w), bytes}};
}
}  // namespace

extern "C" {

float ref_half_to_float(std::uint16_t h) { return half_to_float(h); }
std::uint16_t ref_float_to_half(float f) { return float_to_half(f); }
int ref_cpu_has_avx2() { return cpu_has_avx2() ? 1 : 0; }

int ref_quantize_q8(const float* x, std::size_t n, void* out) {
    return guarded([&] {
        quantize_q8({x, n}, {static_cast<Q8_1*>(out), n / 32});
    });
}

float ref_dot_q4_0(const void* block, const void* q8) {
    return dot_q4_scalar(block, TensorType::Q4_0, *static_cast<const Q8_1*>(q8));
}

// variant 0 = matmul_scalar, 1 = matmul_avx2, 2 = matmul_q8_reference (N<=3).
int ref_matmul(int variant, const void* w, int input, int output, const void* x, int columns, float* out) {
    return guarded([&] {
        const auto m = q4(w, input, output);
        const std::span<const Q8_1> in{static_cast<const Q8_1*>(x), static_cast<std::size_t>(input / 32 * columns)};
        const std::span<float> o{out, static_cast<std::size_t>(output) * static_cast<std::size_t>(columns)};
        if (variant == 0) matmul_scalar(m, in, columns, o);
        else if (variant == 1) matmul_avx2(m, in, columns, o);
        else matmul_q8_reference(m, in, columns, o);
    });
}

// Whole CPU expert at the reference's fixed shape (gate/up 2560->640,
// Q4_0 down 640->2560), columns 1..3.  x is [columns][80] Q8_1.  Optional
// outputs copy the published scratch prefixes (gate/up/middle [columns][640],
// middle_q8 [columns][20]).  Returns the CpuExpertStatus value.
int ref_cpu_expert(const void* gate, const void* up, const void* down, const void* x, int columns,
                   float* out, float* gate_out, float* up_out, float* middle_out, void* middle_q8_out) {
    int status = -1;
    const int rc = guarded([&] {
        static CpuExpertScratch scratch;
        const CpuExpert expert(q4(gate, 2560, 640), q4(up, 2560, 640), q4(down, 640, 2560));
        CpuExpertJob job;
        job.expert = &expert;
        job.columns = columns;
        job.output = {out, static_cast<std::size_t>(columns) * 2560};
        for (int c = 0; c < columns; ++c)
            job.input[static_cast<std::size_t>(c)] = {static_cast<const Q8_1*>(x) + c * 80, 80};
        status = static_cast<int>(run_cpu_expert(job, scratch));
        const auto mid = static_cast<std::size_t>(columns) * 640;
        if (gate_out) std::memcpy(gate_out, scratch.gate.data(), mid * sizeof(float));
        if (up_out) std::memcpy(up_out, scratch.up.data(), mid * sizeof(float));
        if (middle_out) std::memcpy(middle_out, scratch.middle.data(), mid * sizeof(float));
        if (middle_q8_out) std::memcpy(middle_q8_out, scratch.middle_q8.data(), mid / 32 * sizeof(Q8_1));
    });
    return rc ? 100 + rc : status;
}

// The same expert with a Q4_1 down matrix (640 -> 2560, 20-byte blocks), as
// the checkpoint's layers 0-5 hold it.  Outputs y, middle and middle_q8.
int ref_cpu_expert_q41(const void* gate, const void* up, const void* down, const void* x, int columns,
                       float* out, float* middle_out, void* middle_q8_out) {
    int status = -1;
    const int rc = guarded([&] {
        static CpuExpertScratch scratch;
        const auto down_bytes = static_cast<std::size_t>(640 / 32) * 2560 * sizeof(Q4_1);
        const QMatrix d{TensorType::Q4_1, 640, 2560, {static_cast<const std::byte*>(down), down_bytes}};
        const CpuExpert expert(q4(gate, 2560, 640), q4(up, 2560, 640), d);
        CpuExpertJob job;
        job.expert = &expert;
        job.columns = columns;
        job.output = {out, static_cast<std::size_t>(columns) * 2560};
        for (int c = 0; c < columns; ++c)
            job.input[static_cast<std::size_t>(c)] = {static_cast<const Q8_1*>(x) + c * 80, 80};
        status = static_cast<int>(run_cpu_expert(job, scratch));
        const auto mid = static_cast<std::size_t>(columns) * 640;
        if (middle_out) std::memcpy(middle_out, scratch.middle.data(), mid * sizeof(float));
        if (middle_q8_out) std::memcpy(middle_q8_out, scratch.middle_q8.data(), mid / 32 * sizeof(Q8_1));
    });
    return rc ? 100 + rc : status;
}

// RouteGroups::prepare (512 experts, top-10).  Outputs the grouped
// assignments as four parallel arrays plus counts[512].
int ref_route_groups(const std::int32_t* ids, const float* weights, int tokens, std::int32_t* token,
                     std::int32_t* rank, std::int32_t* expert, float* weight, std::int32_t* counts) {
    return guarded([&] {
        RouteGroups groups(tokens, tokens <= 1024 ? RouteGroups::Bound::chunk1024
                                                  : RouteGroups::Bound::layerwise16384);
        const auto n = static_cast<std::size_t>(tokens) * 10;
        groups.prepare({ids, n}, {weights, n}, tokens);
        const auto a = groups.assignments();
        for (std::size_t i = 0; i < a.size(); ++i) {
            token[i] = a[i].token; rank[i] = a[i].rank; expert[i] = a[i].expert;
            std::memcpy(&weight[i], &a[i].weight, sizeof(float));
        }
        const auto c = groups.counts();
        for (std::size_t e = 0; e < c.size(); ++e) counts[e] = c[e];
    });
}

}  // extern "C"
