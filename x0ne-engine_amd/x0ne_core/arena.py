"""The arena (x0ne-core/runtime/src/arena.rs) over the C ABI: plan regions while Building, one
allocation at freeze, checked addressing once Frozen; ClientData is what a scrub zeroes."""
from __future__ import annotations

import ctypes as C
from enum import IntEnum

import numpy as np

from ._lib import Slice, check, lib

ALIGN = 256  # arena.rs:37


class Class(IntEnum):
    WEIGHTS = 0
    CLIENT_DATA = 1


class Arena:
    def __init__(self, handle=None, owned=True):
        if handle is None:
            h = C.c_void_p()
            check(lib().x0ne_arena_new(C.byref(h)))
            handle = h
        self.h = handle
        self.owned = owned

    def close(self):
        if getattr(self, "h", None) and self.owned:
            lib().x0ne_arena_free(self.h)
        self.h = None

    def __del__(self):
        self.close()

    def alloc(self, label: str, length: int, cls: Class) -> Slice:
        s = Slice()
        check(lib().x0ne_arena_alloc(self.h, label.encode(), int(length), int(cls), C.byref(s)), "alloc")
        return s

    def planned_bytes(self) -> int:
        return lib().x0ne_arena_planned_bytes(self.h)

    def freeze(self, gpu=None):
        """freeze(allocate): device memory of `gpu`, or host memory poisoned with 0xA5."""
        check(lib().x0ne_arena_freeze(self.h, gpu.h if gpu is not None else None), "freeze")
        self._gpu = gpu  # keeps the device alive as long as its memory
        return self

    def frozen(self) -> bool:
        return bool(lib().x0ne_arena_is_frozen(self.h))

    def write(self, s: Slice, at: int, data) -> None:
        b = np.ascontiguousarray(data).view(np.uint8).ravel() if not isinstance(data, (bytes, bytearray)) \
            else np.frombuffer(bytes(data), np.uint8)
        check(lib().x0ne_arena_write(self.h, s, int(at), b.ctypes.data, b.size), "write")

    def read(self, s: Slice, at: int, n: int) -> bytes:
        out = np.empty(int(n), np.uint8)
        check(lib().x0ne_arena_read(self.h, s, int(at), out.ctypes.data, out.size), "read")
        return out.tobytes()

    def read_array(self, s: Slice, at: int, count: int, dtype) -> np.ndarray:
        dt = np.dtype(dtype)
        return np.frombuffer(self.read(s, at, count * dt.itemsize), dt).copy()

    def addr(self, s: Slice, at: int = 0) -> int:
        out = C.c_uint64()
        check(lib().x0ne_arena_addr(self.h, s, int(at), C.byref(out)), "addr")
        return out.value

    def ptr(self, s: Slice) -> int:
        return self.addr(s, 0)

    def span(self, s: Slice, at: int, length: int) -> int:
        out = C.c_uint64()
        check(lib().x0ne_arena_span(self.h, s, int(at), int(length), C.byref(out)), "span")
        return out.value

    def scrub_client_data(self) -> int:
        out = C.c_uint64()
        check(lib().x0ne_arena_scrub(self.h, C.byref(out)), "scrub")
        return out.value

    def slices(self):
        """(label, class, Slice) of every region, in plan order."""
        out = []
        for i, (label, cls, _, _) in enumerate(self.regions()):
            s = Slice()
            check(lib().x0ne_arena_region_slice(self.h, i, C.byref(s)))
            out.append((label, cls, s))
        return out

    def regions(self):
        out = []
        buf = C.create_string_buffer(256)
        cls, off, ln = C.c_uint32(), C.c_uint64(), C.c_uint64()
        for i in range(lib().x0ne_arena_region_count(self.h)):
            check(lib().x0ne_arena_region(self.h, i, buf, 256, C.byref(cls), C.byref(off), C.byref(ln)))
            out.append((buf.value.decode(), Class(cls.value), off.value, ln.value))
        return out
