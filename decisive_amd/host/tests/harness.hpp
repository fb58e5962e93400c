// harness.hpp -- a minimal test runner for the host-layer tests.
#pragma once

#include <cstdio>
#include <functional>
#include <string>
#include <vector>

namespace harness {

struct Case {
    const char *name;
    std::function<void()> fn;
};

inline std::vector<Case> &cases() {
    static std::vector<Case> c;
    return c;
}
inline int &failures() {
    static int f = 0;
    return f;
}

struct Register {
    Register(const char *name, std::function<void()> fn) { cases().push_back({name, std::move(fn)}); }
};

inline int run_all(int argc, char **argv) {
    int ran = 0;
    for (const Case &c : cases()) {
        if (argc > 1 && std::string(argv[1]) != c.name) continue;
        int before = failures();
        printf("[ RUN  ] %s\n", c.name);
        fflush(stdout);
        c.fn();
        printf("[ %s ] %s\n", failures() == before ? " OK " : "FAIL", c.name);
        fflush(stdout);
        ran++;
    }
    printf("%d test(s), %d failed check(s)\n", ran, failures());
    return failures() == 0 && ran > 0 ? 0 : 1;
}

}  // namespace harness

#define TEST(name)                                            \
    static void name();                                       \
    static harness::Register reg_##name(#name, name);         \
    static void name()

#define CHECK(cond)                                                                       \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond);      \
            harness::failures()++;                                                        \
        }                                                                                 \
    } while (0)

#define CHECK_EQ(a, b)                                                                    \
    do {                                                                                  \
        auto va_ = (a);                                                                   \
        auto vb_ = (b);                                                                   \
        if (!(va_ == vb_)) {                                                              \
            fprintf(stderr, "%s:%d: CHECK_EQ failed: %s == %s\n", __FILE__, __LINE__, #a, #b); \
            harness::failures()++;                                                        \
        }                                                                                 \
    } while (0)
