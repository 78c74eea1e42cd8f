// test_utils.hpp -- assertion macros and runner with the same names and output
// shape as the reference's tests/test_utils.h (ASSERT, ASSERT_NEAR, TestCase,
// run_tests), written with printf because this toolchain has no <print>.
#pragma once

#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

struct TestCase {
    std::string name;
    std::function<bool()> fn;
};

#define ASSERT(cond, msg)                                                                  \
    do {                                                                                   \
        if (!(cond)) {                                                                     \
            std::printf("    x at %s:%d -- %s: %s\n", __FILE__, __LINE__, msg, #cond);      \
            return false;                                                                  \
        }                                                                                  \
    } while (0)

#define ASSERT_NEAR(a, b, eps, msg)                                                                   \
    do {                                                                                              \
        const double _a = static_cast<double>(a), _b = static_cast<double>(b);                        \
        if (std::abs(_a - _b) > static_cast<double>(eps)) {                                          \
            std::printf("    x at %s:%d -- %s: %g ~ %g (eps=%g)\n", __FILE__, __LINE__, msg, _a, _b,  \
                        static_cast<double>(eps));                                                    \
            return false;                                                                             \
        }                                                                                             \
    } while (0)

inline int run_tests(const std::vector<TestCase>& tests) {
    int passed = 0, failed = 0;
    for (const auto& t : tests) {
        std::printf("  ....  %s\n", t.name.c_str());
        std::fflush(stdout);
        bool ok = false;
        try {
            ok = t.fn();
        } catch (const std::exception& e) {
            std::printf("    x uncaught exception: %s\n", e.what());
        }
        std::printf("  %s  %s\n", ok ? "PASS" : "FAIL", t.name.c_str());
        std::fflush(stdout);
        (ok ? passed : failed) += 1;
    }
    std::printf("\n%d/%d passed\n", passed, passed + failed);
    return failed > 0 ? 1 : 0;
}
