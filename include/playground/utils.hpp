// playground/utils.hpp -- check macro.
// Reference: results/naive_cycle4/include/playground/utils.hpp:6-14 (prints
// the failed condition with file:line and exits with EXIT_FAILURE).
#pragma once

#include <cstdio>
#include <cstdlib>

#define PLAYGROUND_CHECK(condition)                                                  \
    do {                                                                             \
        if (!(condition)) {                                                          \
            std::fprintf(stderr, "[Playground] Check failed at %s:%d for \"%s\"\n",  \
                         __FILE__, __LINE__, #condition);                            \
            std::exit(EXIT_FAILURE);                                                 \
        }                                                                            \
    } while (0)

#define PLAYGROUND_HIP_CHECK(expr)                                                   \
    do {                                                                             \
        hipError_t e_ = (expr);                                                      \
        if (e_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "[Playground] HIP error %s at %s:%d for \"%s\"\n",  \
                         hipGetErrorString(e_), __FILE__, __LINE__, #expr);          \
            std::exit(EXIT_FAILURE);                                                 \
        }                                                                            \
    } while (0)
