// Minimal checks for the C++ test mains (never compiled out, unlike
// assert() under -DNDEBUG).
#pragma once
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>

#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond))                                                                  \
            throw std::runtime_error(std::string(__FILE__) + ":" +                    \
                                     std::to_string(__LINE__) + ": CHECK(" #cond ")"); \
    } while (0)

#define CHECK_THROWS(expr, Type)                                                      \
    do {                                                                              \
        bool thrown_ = false;                                                         \
        try {                                                                         \
            expr;                                                                     \
        } catch (const Type&) {                                                       \
            thrown_ = true;                                                           \
        }                                                                             \
        if (!thrown_)                                                                 \
            throw std::runtime_error(std::string(__FILE__) + ":" +                    \
                                     std::to_string(__LINE__) + ": no " #Type);       \
    } while (0)

inline int run_test(const char* name, void (*fn)()) {
    try {
        fn();
        std::printf("  PASS %s\n", name);
        return 0;
    } catch (const std::exception& e) {
        std::printf("  FAIL %s: %s\n", name, e.what());
        return 1;
    }
}
