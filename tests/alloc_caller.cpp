// Host-allocation check of the C ABI's launch paths, in the spirit of the
// reference's heap monitor (tests/cpu_expert_test.cpp:20-55, which counts
// operator new on every thread while CPU jobs run).
//
// This program replaces the global operator new / delete and malloc / calloc /
// realloc / free for the whole process (the HIP runtime's calls included) and
// attributes each allocation to its call site: the return address lies inside
// libmoe_ffn.so's executable segments or it does not.  After one warm-up call
// of each entry point it repeats the calls a forward pass makes (quantize,
// router, decode / grouped-streaming / grouped-MFMA forwards, combine, the
// quantized linear with and without its workspace) and requires that none of
// them allocated from inside the library.  Allocations made by the HIP runtime
// on the library's behalf (its per-launch bookkeeping) are counted and printed
// but are not the library's to avoid.
//
// Usage: alloc_caller   (exit 0 = no allocation from the library)
#include "moe_ffn.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>
#include <link.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

extern "C" void *__libc_malloc(size_t);
extern "C" void *__libc_calloc(size_t, size_t);
extern "C" void *__libc_realloc(void *, size_t);
extern "C" void __libc_free(void *);

namespace heap {
std::atomic<bool> enabled{false};
std::atomic<unsigned long> total{0}, library{0};
uintptr_t text_lo[8], text_hi[8];
int ntext = 0;

void count(const void *ret) noexcept {
    if (!enabled.load(std::memory_order_relaxed)) return;
    total.fetch_add(1, std::memory_order_relaxed);
    const auto a = reinterpret_cast<uintptr_t>(ret);
    for (int i = 0; i < ntext; ++i)
        if (a >= text_lo[i] && a < text_hi[i]) library.fetch_add(1, std::memory_order_relaxed);
}

// The executable segments of the loaded object whose path ends in `name`
// (a function pointer taken in the executable may point at its own PLT
// entry, so the library is found by name).
int find_text(const char *name) {
    dl_iterate_phdr(
        [](dl_phdr_info *p, size_t, void *data) -> int {
            const char *want = static_cast<const char *>(data);
            const size_t n = std::strlen(p->dlpi_name), m = std::strlen(want);
            if (n < m || std::strcmp(p->dlpi_name + n - m, want) != 0) return 0;
            for (int i = 0; i < p->dlpi_phnum && ntext < 8; ++i) {
                const auto &ph = p->dlpi_phdr[i];
                if (ph.p_type == PT_LOAD && (ph.p_flags & PF_X)) {
                    text_lo[ntext] = p->dlpi_addr + ph.p_vaddr;
                    text_hi[ntext] = text_lo[ntext] + ph.p_memsz;
                    ++ntext;
                }
            }
            return 1;
        },
        const_cast<char *>(name));
    return ntext;
}
}  // namespace heap

extern "C" void *malloc(size_t n) {
    heap::count(__builtin_return_address(0));
    return __libc_malloc(n);
}
extern "C" void *calloc(size_t n, size_t s) {
    heap::count(__builtin_return_address(0));
    return __libc_calloc(n, s);
}
extern "C" void *realloc(void *p, size_t n) {
    heap::count(__builtin_return_address(0));
    return __libc_realloc(p, n);
}
extern "C" void free(void *p) { __libc_free(p); }

namespace {
void *cpp_alloc(size_t n, const void *ret) {
    heap::count(ret);
    if (void *p = __libc_malloc(n ? n : 1)) return p;
    throw std::bad_alloc();
}
void *cpp_aligned(size_t n, size_t a, const void *ret) {
    heap::count(ret);
    void *p = nullptr;
    if (posix_memalign(&p, a < sizeof(void *) ? sizeof(void *) : a, n ? n : 1) == 0) return p;
    throw std::bad_alloc();
}
}  // namespace

void *operator new(size_t n) { return cpp_alloc(n, __builtin_return_address(0)); }
void *operator new[](size_t n) { return cpp_alloc(n, __builtin_return_address(0)); }
void *operator new(size_t n, const std::nothrow_t &) noexcept {
    heap::count(__builtin_return_address(0));
    return __libc_malloc(n ? n : 1);
}
void *operator new[](size_t n, const std::nothrow_t &) noexcept {
    heap::count(__builtin_return_address(0));
    return __libc_malloc(n ? n : 1);
}
void *operator new(size_t n, std::align_val_t a) { return cpp_aligned(n, size_t(a), __builtin_return_address(0)); }
void *operator new[](size_t n, std::align_val_t a) { return cpp_aligned(n, size_t(a), __builtin_return_address(0)); }
void operator delete(void *p) noexcept { __libc_free(p); }
void operator delete[](void *p) noexcept { __libc_free(p); }
void operator delete(void *p, size_t) noexcept { __libc_free(p); }
void operator delete[](void *p, size_t) noexcept { __libc_free(p); }
void operator delete(void *p, std::align_val_t) noexcept { __libc_free(p); }
void operator delete[](void *p, std::align_val_t) noexcept { __libc_free(p); }
void operator delete(void *p, size_t, std::align_val_t) noexcept { __libc_free(p); }
void operator delete[](void *p, size_t, std::align_val_t) noexcept { __libc_free(p); }

namespace {

constexpr int kH = 2048, kI = 512, kE = 32, kK = 4;

#define CHECK(call)                                                                            \
    do {                                                                                       \
        const int st_ = static_cast<int>(call);                                                \
        if (st_ != 0) {                                                                        \
            std::fprintf(stderr, "%s failed with status %d (line %d)\n", #call, st_, __LINE__); \
            std::exit(1);                                                                      \
        }                                                                                      \
    } while (0)

struct Case {
    const char *what;
    unsigned long total, library;
};

}  // namespace

int main() {
    if (!heap::find_text("/libmoe_ffn.so")) {
        std::fprintf(stderr, "cannot locate libmoe_ffn.so's text segment\n");
        return 2;
    }
    // A 32-expert layer (synthetic weights, made on the device) and a Q4_0
    // linear 2048 -> 2048.
    moe_ffn_config cfg{kH, kI, kE, kK, 1, 512, MOE_DOWN_Q4_0};
    moe_ffn_layer *layer = nullptr;
    CHECK(moe_ffn_create_synthetic(&cfg, 11, 0, &layer));
    std::vector<uint8_t> w(static_cast<size_t>(kH) * (kH / 32) * 18);
    for (size_t i = 0; i < w.size(); ++i) w[i] = static_cast<uint8_t>((i * 2654435761u) >> 24);
    for (size_t b = 0; b < w.size(); b += 18) { w[b] = 0x00; w[b + 1] = 0x20; }   // d = half 0x2000
    moe_linear *lin = nullptr;
    CHECK(moe_linear_create(MOE_TYPE_Q4_0, kH, kH, 512, w.data(), 0, 0, &lin));

    const int N = 300;
    float *x = nullptr, *y = nullptr, *logits = nullptr, *wts = nullptr, *contrib = nullptr, *ly = nullptr;
    int32_t *ids = nullptr;
    int *err = nullptr;
    void *q8 = nullptr;
    CHECK(hipMalloc(&x, sizeof(float) * N * kH));
    CHECK(hipMalloc(&y, sizeof(float) * N * kH));
    CHECK(hipMalloc(&ly, sizeof(float) * N * kH));
    CHECK(hipMalloc(&logits, sizeof(float) * N * kE));
    CHECK(hipMalloc(&ids, sizeof(int32_t) * N * kK));
    CHECK(hipMalloc(&wts, sizeof(float) * N * kK));
    CHECK(hipMalloc(&contrib, sizeof(float) * N * kK * kH));
    CHECK(hipMalloc(&q8, static_cast<size_t>(N) * (kH / 32) * 36));
    CHECK(hipMalloc(&err, sizeof(int)));
    std::vector<float> hx(static_cast<size_t>(N) * kH), hl(static_cast<size_t>(N) * kE);
    for (size_t i = 0; i < hx.size(); ++i) hx[i] = static_cast<float>(static_cast<int>((i * 40503u) % 2001u) - 1000) / 700.0f;
    for (size_t i = 0; i < hl.size(); ++i) hl[i] = static_cast<float>(static_cast<int>((i * 7919u) % 997u) - 498) / 150.0f;
    CHECK(hipMemcpy(x, hx.data(), sizeof(float) * hx.size(), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(logits, hl.data(), sizeof(float) * hl.size(), hipMemcpyHostToDevice));
    CHECK(hipMemset(contrib, 0, sizeof(float) * N * kK * kH));
    CHECK(hipMemset(err, 0, sizeof(int)));
    hipStream_t s = nullptr;
    CHECK(hipStreamCreate(&s));

    // The calls of one pass; `tokens` picks the forward's path (2: decode,
    // 24: grouped streaming, 300: grouped with MFMA items).
    auto pass = [&](int tokens) {
        CHECK(moe_quantize_q8_1(x, q8, kH, tokens, err, s));
        CHECK(moe_router_select(logits, tokens, kE, kK, nullptr, ids, wts, err, s));
        CHECK(moe_ffn_forward(layer, x, ids, wts, tokens, nullptr, y, err, s));
        CHECK(moe_ffn_forward_q8(layer, q8, ids, wts, tokens, nullptr, y, err, s));
        CHECK(moe_combine(contrib, wts, nullptr, nullptr, tokens, kK, kH, y, err, s));
        CHECK(moe_linear_apply(lin, x, tokens, ly, err, s));
        CHECK(moe_linear_forward_q8(lin, q8, tokens, ly, s));
        CHECK(moe_linear_apply_noalloc(lin, x, tokens, ly, err, s));
    };
    std::vector<Case> cases;
    for (int tokens : {2, 24, 300}) {
        pass(tokens);   // warm-up: first launches load code objects
        CHECK(hipStreamSynchronize(s));
        heap::total = 0;
        heap::library = 0;
        heap::enabled = true;
        for (int r = 0; r < 20; ++r) pass(tokens);
        heap::enabled = false;
        CHECK(hipStreamSynchronize(s));
        const char *what = tokens == 2 ? "2 tokens (decode path)" : tokens == 24 ? "24 tokens (grouped, streaming)"
                                                                                : "300 tokens (grouped, MFMA)";
        cases.push_back(Case{what, heap::total.load(), heap::library.load()});
    }
    int flag = -1;
    CHECK(hipMemcpy(&flag, err, sizeof(int), hipMemcpyDeviceToHost));
    int failures = flag != 0;
    for (const Case &c : cases) {
        std::printf("%s: 20 passes of 8 entry points, %lu allocations from the library, %lu in the process "
                    "(HIP runtime)\n", c.what, c.library, c.total);
        failures += c.library != 0;
    }
    std::printf("error word %d\n", flag);
    CHECK(hipStreamDestroy(s));
    for (void *p : {static_cast<void *>(x), static_cast<void *>(y), static_cast<void *>(ly),
                    static_cast<void *>(logits), static_cast<void *>(ids), static_cast<void *>(wts),
                    static_cast<void *>(contrib), q8, static_cast<void *>(err)})
        CHECK(hipFree(p));
    CHECK(moe_linear_destroy(lin));
    CHECK(moe_ffn_destroy(layer));
    std::printf("%s\n", failures ? "FAIL" : "PASS");
    return failures ? 1 : 0;
}
