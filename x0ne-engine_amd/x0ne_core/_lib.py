"""Loads libx0ne_core.so (built in-tree by x0ne-engine_amd/build.py) and declares its C ABI
(include/x0ne_core.h). There is no fallback: without the library every call raises."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# X0NE_CORE_LIB: another build of this library (build.py --asan: the host code under
# AddressSanitizer, for the CPU suite).
LIB_PATH = os.environ.get("X0NE_CORE_LIB") or os.path.join(HERE, "libx0ne_core.so")

OK, ERR_IO, ERR_FORMAT, ERR_ARENA, ERR_NOT_IMPLEMENTED, ERR_GPU = range(6)


class Error(Exception):
    """The reference's Error (x0ne-core/runtime/src/error.rs:4-15)."""


class IoError(Error):
    """Error::Io"""


class FormatError(Error):
    """Error::Format: refused before any device work."""


class ArenaError(Error):
    """Error::Arena"""


class NotImplementedFeature(Error):
    """Error::NotImplemented"""


class GpuError(Error):
    """Error::Gpu"""


_ERRORS = {ERR_IO: IoError, ERR_FORMAT: FormatError, ERR_ARENA: ArenaError,
           ERR_NOT_IMPLEMENTED: NotImplementedFeature, ERR_GPU: GpuError}


class Slice(C.Structure):
    """A planned region of an arena (arena.rs:49-53)."""
    _fields_ = [("arena", C.c_uint64), ("offset", C.c_uint64), ("len", C.c_uint64)]

    def __repr__(self):
        return f"Slice(arena={self.arena}, offset={self.offset}, len={self.len})"


class Counts(C.Structure):
    """Driver-call tallies (gpu.rs:93-103)."""
    _fields_ = [(n, C.c_uint64) for n in
                ("launches", "graph_launches", "gemms", "htod", "dtoh", "memsets", "syncs")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class ArgC(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("u32", C.c_uint32), ("f32", C.c_float),
                ("pad", C.c_uint32), ("ptr", C.c_uint64)]


class SplitPlanC(C.Structure):
    _fields_ = [("splits", C.c_uint32), ("grid_x", C.c_uint32), ("group", C.c_uint32),
                ("grouped", C.c_uint32), ("per_cu", C.c_uint32)]


class PosStatsC(C.Structure):
    """x0ne_pos_stats: PosStats (engine.rs:60-64)."""
    _fields_ = [("argmax", C.c_uint32), ("logsumexp", C.c_float), ("next_logprob", C.c_float)]


class GemvFusedC(C.Structure):
    """x0ne_gemv_fused: one fused decode GEMV instance on caller buffers."""
    _fields_ = [(n, C.c_uint64) for n in ("w", "x", "res_in", "res_out", "delta", "norm_w", "embed", "tokens",
                                          "y", "partial", "counter", "token_out", "pos")] + \
               [(n, C.c_uint32) for n in ("rows", "cols", "vocab", "advance")] + [("eps", C.c_float)] + \
               [(n, C.c_uint32) for n in ("prologue", "epilogue", "f64_sums")]


class EngineOptionsC(C.Structure):
    _fields_ = [("max_ctx", C.c_uint64), ("page_seed", C.c_uint64), ("sums", C.c_uint32),
                ("prefill_chunk", C.c_uint32), ("max_batch", C.c_uint32), ("reserved", C.c_uint32)]


_lib = None

# Every function include/x0ne_core.h declares: name -> (argtypes, restype).
P = C.c_void_p
U32, U64, SZ, I32, F32, F64 = C.c_uint32, C.c_uint64, C.c_size_t, C.c_int, C.c_float, C.c_double
ST = C.c_int
SIGNATURES = {
    "x0ne_last_error": ([C.c_char_p, SZ], SZ),
    "x0ne_kernel_set": ([C.c_char_p, SZ], SZ),
    "x0ne_gpu_new": ([C.POINTER(P)], ST),
    "x0ne_gpu_free": ([P], None),
    "x0ne_gpu_sync": ([P], ST),
    "x0ne_gpu_describe": ([P, C.c_char_p, SZ], ST),
    "x0ne_gpu_compute_units": ([P], U32),
    "x0ne_gpu_mem_info": ([P, C.POINTER(U64), C.POINTER(U64)], ST),
    "x0ne_gpu_counts": ([P, C.POINTER(Counts)], ST),
    "x0ne_kernel_count": ([], SZ),
    "x0ne_kernel_name": ([SZ], C.c_char_p),
    "x0ne_kernel_params": ([C.c_char_p, C.POINTER(U32), SZ], SZ),
    "x0ne_check_args": ([C.c_char_p, C.POINTER(ArgC), SZ], ST),
    "x0ne_gpu_launch": ([P, C.c_char_p, U32, U32, U32, C.POINTER(ArgC), SZ], ST),
    "x0ne_gpu_launch_3d": ([P, C.c_char_p, U32, U32, U32, U32, C.POINTER(ArgC), SZ], ST),
    "x0ne_gpu_gemv": ([P, U64, U64, U64, U64, U64, U64, I32], ST),
    "x0ne_gpu_gemm_tiled": ([P, U32, U32, U64, U64, U64, U64, U64, U64, I32], ST),
    "x0ne_gpu_gemv_fused_blocks": ([P, C.POINTER(GemvFusedC)], U32),
    "x0ne_gpu_gemv_fused": ([P, C.POINTER(GemvFusedC)], ST),
    "x0ne_gpu_split_plan": ([P, U32, U32, C.POINTER(SplitPlanC)], ST),
    "x0ne_gpu_attention_split": ([P, C.POINTER(SplitPlanC), I32, U64, U64, U64, U64, U64, U64, U64, U64,
                                  U32, U32, U32, F32], ST),
    "x0ne_gpu_attention_split_scratch": ([P, C.POINTER(SplitPlanC), I32, U64, U64, U64, U64, U64, U64,
                                          U32, U32, U32, F32], ST),
    "x0ne_split_state_bytes": ([U32, U32], U64),
    "x0ne_gpu_time_attention": ([P, U32, U32, U32, U32, U32, U64, C.POINTER(F64), C.POINTER(U32)], ST),
    "x0ne_gpu_capture_begin": ([P], ST),
    "x0ne_gpu_capture_end": ([P, C.POINTER(P)], ST),
    "x0ne_gpu_launch_graph": ([P, P], ST),
    "x0ne_graph_nodes": ([P], SZ),
    "x0ne_graph_free": ([P], None),
    "x0ne_arena_new": ([C.POINTER(P)], ST),
    "x0ne_arena_free": ([P], None),
    "x0ne_arena_alloc": ([P, C.c_char_p, U64, U32, C.POINTER(Slice)], ST),
    "x0ne_arena_planned_bytes": ([P], U64),
    "x0ne_arena_freeze": ([P, P], ST),
    "x0ne_arena_write": ([P, Slice, U64, P, U64], ST),
    "x0ne_arena_read": ([P, Slice, U64, P, U64], ST),
    "x0ne_arena_addr": ([P, Slice, U64, C.POINTER(U64)], ST),
    "x0ne_arena_span": ([P, Slice, U64, U64, C.POINTER(U64)], ST),
    "x0ne_arena_scrub": ([P, C.POINTER(U64)], ST),
    "x0ne_arena_region_count": ([P], SZ),
    "x0ne_arena_region": ([P, SZ, C.c_char_p, SZ, C.POINTER(U32), C.POINTER(U64), C.POINTER(U64)], ST),
    "x0ne_arena_region_slice": ([P, SZ, C.POINTER(Slice)], ST),
    "x0ne_arena_is_frozen": ([P], I32),
    "x0ne_engine_load_from": ([C.c_char_p, SZ, C.POINTER(C.c_char_p), C.POINTER(P), C.POINTER(U64),
                               C.c_char_p, C.POINTER(EngineOptionsC), C.POINTER(P)], ST),
    "x0ne_engine_load_synthetic": ([C.c_char_p, U64, F64, C.POINTER(EngineOptionsC), C.POINTER(P)], ST),
    "x0ne_engine_load": ([C.c_char_p, C.POINTER(EngineOptionsC), C.POINTER(P)], ST),
    "x0ne_engine_free": ([P], None),
    "x0ne_engine_session": ([P, C.POINTER(U32), SZ, C.POINTER(P)], ST),
    "x0ne_session_logits": ([P, C.POINTER(C.POINTER(F32)), C.POINTER(SZ)], ST),
    "x0ne_session_position": ([P], SZ),
    "x0ne_session_step": ([P, U32], ST),
    "x0ne_session_finish": ([P], ST),
    "x0ne_session_drop": ([P], None),
    "x0ne_session_into_greedy": ([P, SZ, SZ, C.POINTER(P)], ST),
    "x0ne_greedy_next": ([P, C.POINTER(U32)], ST),
    "x0ne_greedy_taken": ([P], SZ),
    "x0ne_greedy_position": ([P], SZ),
    "x0ne_greedy_finish": ([P], ST),
    "x0ne_greedy_drop": ([P], None),
    "x0ne_engine_greedy_timed": ([P, C.POINTER(U32), SZ, SZ, C.POINTER(U32), C.POINTER(F64)], ST),
    "x0ne_engine_greedy_with_last_logits": ([P, C.POINTER(U32), SZ, SZ, C.POINTER(U32), C.POINTER(F32)], ST),
    "x0ne_engine_decode_timed": ([P, C.POINTER(U32), SZ, SZ, SZ, C.POINTER(U32), C.POINTER(F64)], ST),
    "x0ne_engine_greedy_batch": ([P, C.POINTER(U32), SZ, SZ, SZ, C.POINTER(U32), C.POINTER(F64), C.POINTER(F32)], ST),
    "x0ne_engine_decode_batch_timed": ([P, C.POINTER(U32), SZ, SZ, SZ, SZ, C.POINTER(U32), C.POINTER(F64)], ST),
    "x0ne_engine_set_decode_mode": ([P, U32], ST),
    "x0ne_engine_decode_mode": ([P], U32),
    "x0ne_engine_set_decode_attention": ([P, U32], ST),
    "x0ne_engine_decode_attention": ([P], U32),
    "x0ne_engine_set_split_merge": ([P, U32], ST),
    "x0ne_engine_split_merge": ([P], U32),
    "x0ne_engine_logits_at": ([P, C.POINTER(U32), SZ, C.POINTER(SZ), SZ, U32, C.POINTER(F32)], ST),
    "x0ne_engine_moe_routing": ([P, C.POINTER(U32), SZ, C.POINTER(U32), SZ, C.POINTER(SZ)], ST),
    "x0ne_engine_run": ([P, C.POINTER(U32), SZ, U32, C.POINTER(SZ), SZ, C.POINTER(PosStatsC), C.POINTER(F32)], ST),
    "x0ne_engine_describe": ([P, C.c_char_p, SZ], ST),
    "x0ne_engine_graph_nodes": ([P], SZ),
    "x0ne_engine_splits": ([P], U32),
    "x0ne_engine_counts": ([P, C.POINTER(Counts)], ST),
    "x0ne_engine_client_data_is_zero": ([P, C.POINTER(I32)], ST),
    "x0ne_engine_host_buffers_are_zero": ([P], I32),
    "x0ne_engine_max_ctx": ([P], U64),
    "x0ne_engine_sums": ([P], U32),
    "x0ne_engine_arena": ([P], P),
    "x0ne_engine_page": ([P, U64, C.POINTER(U32)], ST),
    "x0ne_engine_time_kernel": ([P, U32, U32, C.POINTER(F64), C.POINTER(F64), C.POINTER(U64)], ST),
    "x0ne_engine_time_batch_kernel": ([P, U32, U32, U32, C.POINTER(F64), C.POINTER(F64), C.POINTER(U64)], ST),
}


def lib():
    """The loaded library; raises (never falls back) when it is missing or incomplete."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with x0ne-engine_amd/build.py "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)  # AttributeError names a symbol the header declares but the library lacks
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(4096)
    lib().x0ne_last_error(buf, 4096)
    return buf.value.decode(errors="replace")


def check(status: int, what: str = ""):
    """Raises the Error variant of a non-zero status, with the library's message."""
    if status == OK:
        return
    cls = _ERRORS.get(status, Error)
    raise cls(f"{what}: {last_error()}" if what else last_error())
