// check.hpp -- the check harness of the C++ operator tests.
//
// A case is a function void(check::Context&).  Its checks go through the
// CHECK_* macros: each counts itself, and the first one that fails records
// file, line, the condition and (for CHECK_CLOSE) both values, then leaves the
// case.  check::main runs a table of cases in order -- all of them, or those
// whose name contains one of the command-line arguments -- prints one line
// per case and a tally, and returns the number of failed cases (at most 99).
#pragma once

#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace check {

class Context {
public:
    int checks = 0;
    bool failed = false;
    std::string where, detail;

    bool ok() const { return !failed; }
    void fail(const char* file, int line, std::string text) {
        if (failed) return;  // keep the first failure
        failed = true;
        const char* base = std::strrchr(file, '/');
        where = std::string(base ? base + 1 : file) + ":" + std::to_string(line);
        detail = std::move(text);
    }
};

using Body = void (*)(Context&);
struct Case {
    const char* name;
    Body body;
};

inline bool selected(const char* name, int argc, char** argv) {
    if (argc < 2) return true;
    for (int i = 1; i < argc; ++i)
        if (std::strstr(name, argv[i])) return true;
    return false;
}

inline int main(const std::vector<Case>& cases, int argc, char** argv) {
    int run = 0, bad = 0, total_checks = 0;
    for (const Case& k : cases) {
        if (!selected(k.name, argc, argv)) continue;
        ++run;
        std::printf("[run ] %s\n", k.name);
        std::fflush(stdout);
        Context c;
        try {
            k.body(c);
        } catch (const std::exception& e) {
            c.fail("(exception)", 0, e.what());
        }
        total_checks += c.checks;
        if (c.ok()) {
            std::printf("[ ok ] %s (%d checks)\n", k.name, c.checks);
        } else {
            ++bad;
            std::printf("[FAIL] %s at %s: %s\n", k.name, c.where.c_str(), c.detail.c_str());
        }
        std::fflush(stdout);
    }
    std::printf("%d case(s), %d check(s): %d failed\n", run, total_checks, bad);
    return bad > 99 ? 99 : bad;
}

}  // namespace check

#define CHECK_TRUE(ctx, cond, what)                                                   \
    do {                                                                              \
        ++(ctx).checks;                                                               \
        if (!(cond)) {                                                                \
            (ctx).fail(__FILE__, __LINE__, std::string(what) + " -- false: " #cond);  \
            return;                                                                   \
        }                                                                             \
    } while (0)

#define CHECK_CLOSE(ctx, got, want, tol, what)                                                              \
    do {                                                                                                    \
        ++(ctx).checks;                                                                                     \
        const double g_ = static_cast<double>(got), w_ = static_cast<double>(want);                         \
        const double t_ = static_cast<double>(tol);                                                         \
        if (!(std::fabs(g_ - w_) <= t_)) {                                                                  \
            char b_[160];                                                                                   \
            std::snprintf(b_, sizeof b_, " -- got %.9g, want %.9g, |diff| %.3g > %.3g", g_, w_,             \
                          std::fabs(g_ - w_), t_);                                                          \
            (ctx).fail(__FILE__, __LINE__, std::string(what) + b_);                                         \
            return;                                                                                         \
        }                                                                                                   \
    } while (0)
