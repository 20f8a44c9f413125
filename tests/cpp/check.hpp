// Test support for the C++ host tests: a named-case runner, seeded N(0,1)
// inputs (SplitMix64 + Box-Muller), 16-bit / fp8 codecs through the oracle, and
// the parity metrics of the Python tests (normwise ||gpu - ref||_inf /
// ||ref||_inf; bit-exact comparisons).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace check {

struct Case {
    const char *name;
    std::function<void()> body;
};

inline std::vector<Case> &cases() {
    static std::vector<Case> all;
    return all;
}

struct Register {
    Register(const char *name, std::function<void()> body) { cases().push_back({name, std::move(body)}); }
};

struct Failure {
    std::string what;
};

#define CASE(name)                                   \
    static void name();                              \
    static check::Register reg_##name(#name, name);  \
    static void name()

#define EXPECT(cond, ...)                                                      \
    do {                                                                       \
        if (!(cond)) {                                                         \
            char buf_[512];                                                    \
            std::snprintf(buf_, sizeof buf_, __VA_ARGS__);                     \
            throw check::Failure{std::string(#cond) + ": " + buf_};            \
        }                                                                      \
    } while (0)

// Run every case (or those whose name contains `filter`), printing one line per
// case before and after it, flushed, so a failure names its case.
inline int run_all(int argc, char **argv) {
    const char *filter = argc > 1 ? argv[1] : nullptr;
    int failed = 0, ran = 0;
    for (const Case &c : cases()) {
        if (filter && !std::strstr(c.name, filter)) continue;
        std::printf("case %s ...\n", c.name);
        std::fflush(stdout);
        ++ran;
        try {
            c.body();
            std::printf("case %s ok\n", c.name);
        } catch (const Failure &f) {
            ++failed;
            std::printf("case %s FAILED: %s\n", c.name, f.what.c_str());
        } catch (const std::exception &e) {
            ++failed;
            std::printf("case %s FAILED (exception): %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d cases, %d failed\n", ran, failed);
    return failed ? 1 : 0;
}

// SplitMix64 -> uniform -> Box-Muller N(mean, std), in f32
inline std::vector<float> normal(uint64_t seed, size_t n, float mean = 0.0f, float sd = 1.0f) {
    uint64_t s = seed;
    auto next = [&s] {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    std::vector<float> out(n);
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = ((next() >> 11) + 1.0) * 0x1.0p-53, u2 = (next() >> 11) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 6.283185307179586476925 * u2;
        out[i] = (float)(mean + sd * r * std::cos(a));
        if (i + 1 < n) out[i + 1] = (float)(mean + sd * r * std::sin(a));
    }
    return out;
}

inline double normwise(const std::vector<float> &got, const std::vector<float> &ref) {
    double scale = 0.0, diff = 0.0;
    for (size_t i = 0; i < ref.size(); ++i) {
        scale = std::fmax(scale, std::fabs((double)ref[i]));
        diff = std::fmax(diff, std::fabs((double)got[i] - (double)ref[i]));
    }
    return scale > 0 ? diff / scale : diff;
}

}  // namespace check
