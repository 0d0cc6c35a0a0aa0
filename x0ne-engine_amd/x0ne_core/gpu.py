"""The device and the kernel-launch API (x0ne-core/runtime/src/gpu.rs) over the C ABI."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

from ._lib import ArgC, Counts, GemvFusedC, SplitPlanC, check, lib


class Param(IntEnum):
    """Kinds of kernel parameters (kernels/src/lib.rs:127-132)."""
    PTR = 0
    U32 = 1
    F32 = 2

    def size(self) -> int:
        return 8 if self is Param.PTR else 4


@dataclass(frozen=True)
class Arg:
    """A launch argument (gpu.rs:281-314): Arg.ptr(addr), Arg.u32(v), Arg.f32(v)."""
    kind: Param
    value: object

    @staticmethod
    def ptr(v: int) -> "Arg":
        return Arg(Param.PTR, int(v))

    @staticmethod
    def u32(v: int) -> "Arg":
        return Arg(Param.U32, int(v))

    @staticmethod
    def f32(v: float) -> "Arg":
        return Arg(Param.F32, float(v))

    @staticmethod
    def of(v) -> "Arg":
        """From a Python value the way Arg::from does: float -> F32, int -> U32 if it fits a
        pointer-free u32 argument is wanted, use Arg.u32/Arg.ptr explicitly otherwise."""
        if isinstance(v, Arg):
            return v
        if isinstance(v, float):
            return Arg.f32(v)
        raise TypeError("use Arg.ptr / Arg.u32 / Arg.f32")

    def c(self) -> ArgC:
        a = ArgC()
        a.kind = int(self.kind)
        if self.kind is Param.PTR:
            a.ptr = self.value
        elif self.kind is Param.U32:
            a.u32 = self.value & 0xFFFFFFFF
        else:
            a.f32 = self.value
        return a


def _args(args):
    arr = (ArgC * max(1, len(args)))()
    for i, a in enumerate(args):
        arr[i] = a.c()
    return arr


def kernel_names() -> list[str]:
    L = lib()
    return [L.x0ne_kernel_name(i).decode() for i in range(L.x0ne_kernel_count())]


def params_of(name: str):
    """The parameter kinds of a kernel (lib.rs:146-151); None for an unknown name."""
    buf = (C.c_uint32 * 32)()
    n = lib().x0ne_kernel_params(name.encode(), buf, 32)
    if n == C.c_size_t(-1).value:
        return None
    return [Param(buf[i]) for i in range(n)]


def check_args(name: str, args) -> None:
    """check_args (gpu.rs:317-333): raises GpuError naming the first wrong argument."""
    check(lib().x0ne_check_args(name.encode(), _args(args), len(args)))


def kernel_set() -> str:
    buf = C.create_string_buffer(512)
    lib().x0ne_kernel_set(buf, 512)
    return buf.value.decode()


@dataclass
class SplitPlan:
    """gpu.rs SplitPlan: P, the grid, the group size, whether a grouped kernel serves it."""
    splits: int
    grid_x: int
    group: int
    grouped: bool
    per_cu: int

    def c(self) -> SplitPlanC:
        return SplitPlanC(self.splits, self.grid_x, self.group, int(self.grouped), self.per_cu)


class Graph:
    def __init__(self, gpu: "Gpu", handle):
        self.gpu, self.h = gpu, handle

    def nodes(self) -> int:
        return lib().x0ne_graph_nodes(self.h)

    def close(self):
        if self.h:
            lib().x0ne_graph_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Gpu:
    """Gpu::new (gpu.rs:799-928): device 0, one stream."""

    def __init__(self):
        h = C.c_void_p()
        check(lib().x0ne_gpu_new(C.byref(h)), "Gpu::new")
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().x0ne_gpu_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def sync(self):
        check(lib().x0ne_gpu_sync(self.h), "sync")

    def describe(self) -> str:
        buf = C.create_string_buffer(512)
        check(lib().x0ne_gpu_describe(self.h, buf, 512))
        return buf.value.decode()

    def compute_units(self) -> int:
        return lib().x0ne_gpu_compute_units(self.h)

    def mem_info(self):
        f, t = C.c_uint64(), C.c_uint64()
        check(lib().x0ne_gpu_mem_info(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def counts(self) -> dict:
        c = Counts()
        check(lib().x0ne_gpu_counts(self.h, C.byref(c)))
        return c.as_dict()

    def launch(self, name: str, grid, block: int, args):
        """Gpu::launch (gpu.rs:1031-1086): checked against the kernel table, not synchronised."""
        if isinstance(grid, int):
            grid = (grid, 1)
        if len(grid) == 3:
            check(lib().x0ne_gpu_launch_3d(self.h, name.encode(), *grid, block, _args(args), len(args)), name)
            return
        gx, gy = grid
        check(lib().x0ne_gpu_launch(self.h, name.encode(), gx, gy, block, _args(args), len(args)), name)

    def gemv(self, w: int, rows: int, cols: int, x: int, n: int, y: int, out_f32: bool):
        """Gpu::gemm (gpu.rs:1098-1149): Y[n][rows] = X[n][cols] W^T on device addresses."""
        check(lib().x0ne_gpu_gemv(self.h, w, rows, cols, x, n, y, int(out_f32)), "gemv")

    def gemm_tiled(self, tile: int, w: int, rows: int, cols: int, x: int, n: int, y: int, out_f32: bool,
                   layout: int = 0):
        """The tiled matrix-core GEMM with block tile `tile` (x0ne_gpu_gemm_tiled; 0 picks one),
        layout bit 0 W in 16-row panels, bit 1 X in panels."""
        check(lib().x0ne_gpu_gemm_tiled(self.h, tile, layout, w, rows, cols, x, n, y, int(out_f32)), "gemm_tiled")

    def gemv_fused(self, **fields) -> None:
        """One fused decode GEMV instance (x0ne_gpu_gemv_fused) on device addresses."""
        d = GemvFusedC(**fields)
        check(lib().x0ne_gpu_gemv_fused(self.h, C.byref(d)), "gemv_fused")

    def gemv_fused_blocks(self, **fields) -> int:
        d = GemvFusedC(**fields)
        return int(lib().x0ne_gpu_gemv_fused_blocks(self.h, C.byref(d)))

    def split_plan(self, q_heads: int, kv_heads: int) -> SplitPlan:
        p = SplitPlanC()
        check(lib().x0ne_gpu_split_plan(self.h, q_heads, kv_heads, C.byref(p)), "split_plan")
        return SplitPlan(p.splits, p.grid_x, p.group, bool(p.grouped), p.per_cu)

    def attention_split(self, plan: SplitPlan, last_block: bool, q, k, v, pages, state, counter, out, pos,
                        q_heads, kv_heads, max_ctx, scale):
        pc = plan.c()
        check(lib().x0ne_gpu_attention_split(self.h, C.byref(pc), int(last_block), q, k, v, pages, state, counter,
                                              out, pos, q_heads, kv_heads, max_ctx, scale), "split-K attention")

    def attention_split_scratch(self, plan: SplitPlan, last_block: bool, q, k, v, pages, out, pos, q_heads, kv_heads,
                                max_ctx, scale):
        """attention_split with the states and counters in the library's static scratch array
        (x0ne_gpu_attention_split_scratch: no workspace argument, no allocation)."""
        pc = plan.c()
        check(lib().x0ne_gpu_attention_split_scratch(self.h, C.byref(pc), int(last_block), q, k, v, pages, out, pos,
                                                      q_heads, kv_heads, max_ctx, scale), "split-K attention (scratch)")

    def time_attention(self, q_heads: int, kv_heads: int, ctx: int, splits: int, iters: int, seed: int = 0):
        """the isolated split-K decode attention over more than 512 MiB of
        rotating K/V planes; (mean kernel µs per launch, planes rotated)."""
        us, planes = C.c_double(), C.c_uint32()
        check(lib().x0ne_gpu_time_attention(self.h, q_heads, kv_heads, ctx, splits, iters, seed, C.byref(us),
                                            C.byref(planes)), "time_attention")
        return us.value, planes.value

    def capture(self, launches) -> Graph:
        """Gpu::capture (gpu.rs:1170-1217): records the launches `launches()` makes."""
        check(lib().x0ne_gpu_capture_begin(self.h), "capture")
        err = None
        try:
            launches()
        except Exception as e:  # the capture must still be closed
            err = e
        h = C.c_void_p()
        st = lib().x0ne_gpu_capture_end(self.h, C.byref(h))
        if err is not None:
            if h:
                lib().x0ne_graph_free(h)
            raise err
        check(st, "capture")
        return Graph(self, h)

    def launch_graph(self, g: Graph):
        check(lib().x0ne_gpu_launch_graph(self.h, g.h), "launch_graph")


def split_state_bytes(q_heads: int, splits: int) -> int:
    return lib().x0ne_split_state_bytes(q_heads, splits)
