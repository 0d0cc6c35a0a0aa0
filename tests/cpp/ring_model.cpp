// A model of the greedy ring (x0ne-core/oracle/tests/cpu_oracle.rs:566-614, restated): the
// engine's own rules (x0ne-engine_amd/csrc/ring.h, included, not copied) drive a ring of RING
// words over every `ahead` the engine accepts (1 .. 15) and every request of 1 .. 70 tokens. A
// ring word is never rewritten before the caller took it, no step is launched past the tokens
// asked, at most `ahead` steps are in flight, and every token asked is launched. The same for
// greedy_timed's loop (RING - 1 steps ahead, tokens collected in order). Exit status 0: all hold.
#include <cstdio>
#include <cstdlib>

#include "ring.h"

using namespace x0ne;

#define CHECK(c, ...)                                  \
    do {                                               \
        if (!(c)) {                                    \
            std::fprintf(stderr, __VA_ARGS__);         \
            std::fprintf(stderr, " (line %d)\n", __LINE__); \
            std::exit(1);                              \
        }                                              \
    } while (0)

int main() {
    constexpr long NONE = -1;
    long checks = 0;
    for (size_t ahead = 1; ahead <= RING - 1; ++ahead) {
        for (size_t max_tokens = 1; max_tokens <= 70; ++max_tokens) {
            long ring[RING];
            for (auto& w : ring) w = NONE;  // ring word -> the step whose token it holds, not taken
            size_t taken = 0, launched = 0;
            auto fill = [&]() {
                while (greedy_may_launch(launched, taken, max_tokens, ahead)) {
                    const size_t j = launched + 1;
                    CHECK(ring[ring_word(j)] == NONE, "ahead %zu: step %zu overwrites step %ld", ahead, j,
                          ring[ring_word(j)]);
                    ring[ring_word(j)] = (long)j;
                    launched = j;
                    ++checks;
                }
            };
            fill();
            while (taken < max_tokens) {
                if (taken > 0) {
                    CHECK(ring[ring_word(taken)] == (long)taken, "ahead %zu: token %zu is not in its word", ahead,
                          taken);
                    ring[ring_word(taken)] = NONE;
                }
                taken += 1;
                fill();
                CHECK(launched < max_tokens, "a step past the tokens asked");
                CHECK(launched + 1 - taken <= ahead, "ahead %zu: %zu steps in flight", ahead, launched + 1 - taken);
            }
            CHECK(launched == max_tokens - 1, "every token asked was launched");
            for (long w : ring) CHECK(w == NONE, "a token left in the ring");
        }
    }
    // greedy_timed: step i's token into word i, collected in order once RING - 1 are outstanding.
    for (size_t n = 1; n <= 70; ++n) {
        long ring[RING];
        for (auto& w : ring) w = NONE;
        size_t next = 1, collected = 0;
        auto collect = [&](size_t j) {
            CHECK(ring[ring_word(j)] == (long)j, "timed: token %zu is not in its word", j);
            ring[ring_word(j)] = NONE;
            ++collected;
        };
        for (size_t i = 1; i < n; ++i) {
            CHECK(ring[ring_word(i)] == NONE, "timed: step %zu overwrites step %ld", i, ring[ring_word(i)]);
            ring[ring_word(i)] = (long)i;
            if (timed_must_collect(i, next)) collect(next++);
            CHECK(i + 1 - next <= RING - 1, "timed: %zu steps outstanding", i + 1 - next);
            ++checks;
        }
        while (next < n) collect(next++);
        CHECK(collected + 1 == n, "timed: %zu of %zu tokens collected", collected + 1, n);
    }
    std::printf("ring model: %ld launches checked\n", checks);
    return 0;
}
