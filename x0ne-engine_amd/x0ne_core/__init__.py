"""x0ne Core for MI355X: the Qwen3 dense bf16 decode engine on hand-written gfx950 kernels.

The Python face of include/x0ne_core.h, mirroring the reference's Rust runtime crate
(x0ne-core/runtime/src): Engine / Session / Greedy (engine.rs), Gpu and the kernel-launch API
(gpu.rs), Arena (arena.rs), Kernels (ops.rs). Every call goes to libx0ne_core.so; there is no
CPU fallback."""
from ._lib import (ArenaError, Error, FormatError, GpuError, IoError, NotImplementedFeature, Slice, last_error,
                   lib)
from .arena import ALIGN, Arena, Class
from .engine import (GREEDY_AHEAD, GREEDY_AHEAD_MAX, DecodeAttention, DecodeMode, Engine, EngineOptions, Greedy,
                     Route, Session, SplitMerge)
from .gpu import Arg, Gpu, Graph, Param, SplitPlan, check_args, kernel_names, kernel_set, params_of, split_state_bytes

__all__ = [
    "ALIGN", "Arena", "ArenaError", "Arg", "Class", "DecodeAttention", "DecodeMode", "Engine", "EngineOptions", "Error",
    "FormatError", "GREEDY_AHEAD", "GREEDY_AHEAD_MAX", "Gpu", "GpuError", "Graph", "Greedy", "IoError",
    "NotImplementedFeature", "Param", "Route", "Session", "Slice", "SplitMerge", "SplitPlan", "check_args", "kernel_names",
    "kernel_set", "last_error", "lib", "params_of", "split_state_bytes",
]
