// libm_check.cpp -- test infrastructure: compares the library's restatement
// of tanhf / expf (freetoken-rs_amd/csrc/ft_libm.hpp, the source the kernels
// compile) with this host's libm over ranges of f32 bit patterns. Called by
// tests/test_libm.py through ctypes; never linked into the product.
//
// Built with -ffp-contract=off (see oracle/Makefile), the same contraction
// rule the HIP library is compiled with.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <atomic>

#include "../freetoken-rs_amd/csrc/ft_libm.hpp"

namespace {

inline uint32_t fbits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    return u;
}

// Equal results, NaN equal to NaN (the sign and payload of a NaN result are
// not compared: both sides only ever return x + x or 1/x +- 1 for NaN input).
inline bool same(float a, float b) { return (a != a && b != b) || fbits(a) == fbits(b); }

template <typename F, typename G>
int64_t sweep(uint64_t lo, uint64_t hi, int threads, uint32_t* first_bad, F mine, G ref) {
    if (threads < 1) threads = 1;
    std::atomic<int64_t> bad{0};
    std::atomic<uint64_t> first{~0ull};
    std::vector<std::thread> pool;
    const uint64_t n = hi - lo;
    for (int t = 0; t < threads; ++t) {
        pool.emplace_back([&, t]() {
            const uint64_t a = lo + n * t / threads, b = lo + n * (t + 1) / threads;
            int64_t local = 0;
            uint64_t f = ~0ull;
            for (uint64_t u = a; u < b; ++u) {
                float x;
                const uint32_t w = (uint32_t)u;
                std::memcpy(&x, &w, 4);
                if (!same(mine(x), ref(x))) {
                    ++local;
                    if (u < f) f = u;
                }
            }
            bad += local;
            uint64_t cur = first.load();
            while (f < cur && !first.compare_exchange_weak(cur, f)) {}
        });
    }
    for (auto& th : pool) th.join();
    if (first_bad) *first_bad = (uint32_t)first.load();
    return bad.load();
}

}  // namespace

extern "C" {

// Number of f32 bit patterns u in [lo, hi) whose tanh differs from libm's
// tanhf; *first_bad = the lowest such pattern (0xFFFFFFFF if none).
int64_t lc_sweep_tanhf(uint64_t lo, uint64_t hi, int threads, uint32_t* first_bad) {
    return sweep(lo, hi, threads, first_bad, [](float x) { return ft::libm::tanhf_glibc(x); },
                 [](float x) { return tanhf(x); });
}

int64_t lc_sweep_expf(uint64_t lo, uint64_t hi, int threads, uint32_t* first_bad) {
    return sweep(lo, hi, threads, first_bad, [](float x) { return ft::libm::expf_glibc(x); },
                 [](float x) { return expf(x); });
}


float lc_tanhf(float x) { return ft::libm::tanhf_glibc(x); }
float lc_expf(float x) { return ft::libm::expf_glibc(x); }
}
