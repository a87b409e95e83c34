// Minimal test registry shared by the C++ test binaries: TEST(name, "cpu" |
// "gpu"), CHECK, CHECK_THROWS, and a main that runs one suite:
//   <binary> cpu|gpu   -> exit status 0 when every test of that suite passes.
// Include it in exactly one translation unit per binary.
#pragma once

#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "gpu.hpp"

namespace harness {

struct Case {
    const char* name;
    const char* kind;
    void (*fn)();
};
inline std::vector<Case>& registry() {
    static std::vector<Case> cases;
    return cases;
}
struct Registrar {
    Registrar(const char* name, const char* kind, void (*fn)()) { registry().push_back({name, kind, fn}); }
};
struct Failure {
    std::string what;
};

#define TEST(name, kind)                                            \
    static void name();                                             \
    static harness::Registrar registrar_##name(#name, kind, name); \
    static void name()
#define CHECK(cond)                                                                                     \
    do {                                                                                                \
        if (!(cond)) throw harness::Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond}; \
    } while (0)
#define CHECK_THROWS(expr)                                                                                  \
    do {                                                                                                    \
        bool thrown_ = false;                                                                               \
        try {                                                                                               \
            expr;                                                                                           \
        } catch (const nvr::Error&) {                                                                       \
            thrown_ = true;                                                                                 \
        }                                                                                                   \
        if (!thrown_) throw harness::Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": no throw: " #expr}; \
    } while (0)

// Throws unless `expr` throws nvr::Error of the given Fault kind.
#define CHECK_FAULT(expr, kind)                                                                             \
    do {                                                                                                    \
        bool thrown_ = false;                                                                               \
        try {                                                                                               \
            expr;                                                                                           \
        } catch (const nvr::Error& e_) {                                                                    \
            if (e_.fault() != (kind))                                                                       \
                throw harness::Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": fault " +   \
                                       nvr::fault_name(e_.fault()) + " (" + e_.what() + "), expected " +   \
                                       nvr::fault_name(kind)};                                              \
            thrown_ = true;                                                                                 \
        }                                                                                                   \
        if (!thrown_) throw harness::Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": no throw: " #expr}; \
    } while (0)

}  // namespace harness

int main(int argc, char** argv) {
    if (argc < 2 || (std::strcmp(argv[1], "cpu") != 0 && std::strcmp(argv[1], "gpu") != 0)) {
        std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
        return 2;
    }
    int failed = 0, ran = 0;
    for (const harness::Case& c : harness::registry()) {
        if (std::strcmp(c.kind, argv[1]) != 0) continue;
        ++ran;
        std::printf("%s ... ", c.name);
        std::fflush(stdout);
        try {
            c.fn();
            std::printf("ok\n");
        } catch (const harness::Failure& f) {
            ++failed;
            std::printf("FAILED: %s\n", f.what.c_str());
        } catch (const std::exception& e) {
            ++failed;
            std::printf("FAILED: exception: %s\n", e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d of %d passed\n", ran - failed, ran);
    return failed == 0 && ran > 0 ? 0 : 1;
}
