// The host's ring of device greedy tokens (engine.rs:67-79, :1267-1343): RING pinned words, each
// with its event; step j's token is copied into word j % RING. Plain C++ (no device code), so the
// rules below are the ones the engine runs and the ones the CPU model test drives.
#pragma once
#include <stddef.h>

namespace x0ne {

constexpr size_t RING = 16;  // engine.rs:70: GREEDY_AHEAD_MAX + 1

inline size_t ring_word(size_t step) { return step % RING; }

// A greedy session (Greedy::fill, engine.rs:1322-1343): `taken` tokens handed to the caller,
// steps 1 .. `launched` launched (token 0 is the prompt's own). Step launched + 1 is launched
// while it is a token the request still wants (below max_tokens) and fewer than `ahead` steps
// lie beyond the last token taken. With ahead < RING no word is rewritten before it is taken.
inline bool greedy_may_launch(size_t launched, size_t taken, size_t max_tokens, size_t ahead) {
    const size_t taken_m1 = taken ? taken - 1 : 0;
    return launched + 1 < max_tokens && launched - taken_m1 < ahead;
}

// Engine::greedy_timed's loop (engine.rs:1065-1135): after launching step i, with `next` the
// first token not yet collected, the host collects `next` once RING - 1 steps are outstanding,
// so the word step i + 1 will use is free again.
inline bool timed_must_collect(size_t i, size_t next) { return i + 1 - next >= RING - 1; }

}  // namespace x0ne
