"""The arena on host memory, against a byte model, without a GPU: the counterpart of
x0ne-core/oracle/tests/cpu_arena.rs. Plans are aligned, disjoint and inside the one allocation;
writes land exactly on their bytes and a refused write changes nothing; a scrub zeroes the
ClientData regions and nothing else; slices of another arena, and plans at the edge of u64,
are refused (arena.rs:163-303)."""
import ctypes as C

import numpy as np
import pytest

from common import O

POISON = 0xA5
ALIGN = 256


def new_arena():
    from x0ne_core.arena import Arena
    return Arena()


def random_plan(rng: O.Rng, n: int, max_len=5000):
    """A random plan and the model of where each region must be: the end of the plan rounded up
    to 256 (arena.rs:174-198); an empty region is refused and moves nothing."""
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    a = new_arena()
    model = []
    end = 0
    for i in range(n):
        if rng.chance(8):
            before = a.planned_bytes()
            with pytest.raises(ArenaError):
                a.alloc("empty", 0, Class.CLIENT_DATA)
            assert a.planned_bytes() == before and len(a.regions()) == len(model)
        length = rng.range(1, max_len)
        cls = Class.CLIENT_DATA if rng.chance(2) else Class.WEIGHTS
        s = a.alloc(f"r{i}", length, cls)
        offset = (end + ALIGN - 1) // ALIGN * ALIGN
        end = offset + length
        assert (s.offset, s.len) == (offset, length), f"region {i}"
        assert a.planned_bytes() == end, "the plan ends where its last region ends"
        model.append((s, length, cls))
    return a, model


def test_random_plans_are_aligned_disjoint_and_inside_the_allocation():
    for seed in range(200):
        rng = O.Rng(seed)
        a, model = random_plan(rng, rng.range(1, 40))
        regions = a.regions()
        assert len(regions) == len(model)
        end = 0
        for i, ((label, cls, off, ln), (s, length, mcls)) in enumerate(zip(regions, model)):
            assert label == f"r{i}" and cls == mcls and ln == length == s.len and off == s.offset
            assert off % ALIGN == 0, f"seed {seed} region {i}"
            assert off >= end, f"seed {seed}: regions overlap or are out of order"
            end = off + ln
            assert end <= a.planned_bytes()
        a.freeze(None)
        assert a.frozen()
        assert len(a.regions()) == len(model)


def test_random_writes_reads_and_scrubs_match_a_byte_model():
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    for seed in range(60):
        rng = O.Rng(1000 + seed)
        a, model = random_plan(rng, rng.range(1, 24), 3000)
        total = a.planned_bytes()
        a.freeze(None)
        bytes_ = np.full(total, POISON, np.uint8)
        for op in range(200):
            s, length, cls = model[rng.below(len(model))]
            at = rng.range(0, length + 8)
            n = rng.range(0, 300)
            kind = rng.below(3)
            if kind == 0:
                data = np.array([rng.below(256) for _ in range(n)], np.uint8)
                if at + n <= length:
                    a.write(s, at, data)
                    bytes_[s.offset + at:s.offset + at + n] = data
                else:
                    with pytest.raises(ArenaError):
                        a.write(s, at, data)
            elif kind == 1:
                if at + n <= length:
                    got = np.frombuffer(a.read(s, at, n), np.uint8)
                    assert (got == bytes_[s.offset + at:s.offset + at + n]).all(), f"seed {seed} op {op}"
                else:
                    with pytest.raises(ArenaError):
                        a.read(s, at, n)
            else:
                zeroed = a.scrub_client_data()
                want = 0
                for s2, l2, c2 in model:
                    if c2 == Class.CLIENT_DATA:
                        bytes_[s2.offset:s2.offset + l2] = 0
                        want += l2
                assert zeroed == want
        # The whole backing, padding included, is what the model says.
        host = (C.c_uint8 * max(total, 1)).from_address(a.addr(model[0][0], 0) - model[0][0].offset) if total else []
        assert total == 0 or (np.frombuffer(host, np.uint8)[:total] == bytes_).all(), f"seed {seed}"


def test_addresses_and_spans_stay_inside_their_slice():
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    a = new_arena()
    s = a.alloc("x", 1000, Class.CLIENT_DATA)
    t = a.alloc("y", 10, Class.WEIGHTS)
    a.freeze(None)
    base = a.addr(s, 0)
    assert a.addr(s, 999) == base + 999
    for at in (1000, 1001, 2 ** 64 - 1):  # an address names a byte of the slice (arena.rs:278-287)
        with pytest.raises(ArenaError):
            a.addr(s, at)
    assert a.span(s, 10, 990) == base + 10
    for at, n in [(10, 991), (0, 0), (1001, 1), (2 ** 64 - 1, 2), (1, 2 ** 64 - 1)]:  # nor an empty span
        with pytest.raises(ArenaError):
            a.span(s, at, n)
    assert a.addr(t, 0) % ALIGN == 0


def test_a_slice_of_another_arena_is_refused_on_every_entry_point():
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    a, b = new_arena(), new_arena()
    sa = a.alloc("x", 64, Class.CLIENT_DATA)
    b.alloc("x", 64, Class.CLIENT_DATA)
    a.freeze(None)
    b.freeze(None)
    for call in (lambda: b.write(sa, 0, b"\x01"), lambda: b.read(sa, 0, 1), lambda: b.addr(sa, 0),
                 lambda: b.span(sa, 0, 1)):
        with pytest.raises(ArenaError):
            call()


def test_plans_at_the_edge_of_u64_are_refused_not_wrapped():
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    a = new_arena()
    a.alloc("x", 100, Class.WEIGHTS)
    for n in [2 ** 64 - 1, 2 ** 64 - 100, 2 ** 64 - 256]:
        with pytest.raises(ArenaError):
            a.alloc("big", n, Class.WEIGHTS)
    assert a.planned_bytes() == 100  # a refused plan changes nothing


def test_an_arena_is_planned_then_frozen_once():
    from x0ne_core import ArenaError
    from x0ne_core.arena import Class
    a = new_arena()
    s = a.alloc("x", 16, Class.CLIENT_DATA)
    with pytest.raises(ArenaError):
        a.write(s, 0, b"\x00")  # not frozen yet
    a.freeze(None)
    with pytest.raises(ArenaError):
        a.alloc("late", 16, Class.WEIGHTS)
    with pytest.raises(ArenaError):
        a.freeze(None)
    assert np.frombuffer(a.read(s, 0, 16), np.uint8).tolist() == [POISON] * 16
