"""The C-ABI library without a GPU: it loads, it exports every function include/x0ne_core.h
declares (and the Python mirror binds each with the header's arity), the kernel table matches the
kernel declarations of kernels.h parameter for parameter, and every call that needs a device says
so with X0NE_ERR_GPU instead of failing another way (the drop-in boundary, a line each of
x0ne-core/runtime/src/{gpu.rs, arena.rs, engine.rs} re-exported in C)."""
import ctypes as C
import os
import re

import pytest

from common import ROOT

HEADER = os.path.join(ROOT, "include", "x0ne_core.h")
KERNELS_H = os.path.join(ROOT, "x0ne-engine_amd", "csrc", "kernels.h")


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^[A-Za-z_][A-Za-z_0-9 \*]*?\b(x0ne_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, re.M | re.S):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else args.count(",") + 1
        decls[m.group(1)] = n
    return decls


def test_the_header_declares_the_boundary_the_reference_binds():
    decls = header_functions()
    # The entry points a Rust wrapper of x0ne-core/runtime needs (engine.rs, gpu.rs, arena.rs).
    for name in ["x0ne_engine_load_from", "x0ne_engine_load", "x0ne_engine_run", "x0ne_engine_moe_routing", "x0ne_engine_session", "x0ne_session_logits", "x0ne_session_step",
                 "x0ne_session_finish", "x0ne_session_into_greedy", "x0ne_greedy_next", "x0ne_greedy_finish",
                 "x0ne_engine_greedy_timed", "x0ne_engine_describe", "x0ne_engine_free", "x0ne_arena_new",
                 "x0ne_arena_alloc", "x0ne_arena_freeze", "x0ne_arena_write", "x0ne_arena_read", "x0ne_arena_addr",
                 "x0ne_arena_scrub", "x0ne_gpu_launch", "x0ne_gpu_gemv", "x0ne_gpu_capture_begin",
                 "x0ne_gpu_capture_end", "x0ne_gpu_launch_graph", "x0ne_gpu_split_plan", "x0ne_last_error"]:
        assert name in decls, name
    assert len(decls) >= 60


def test_the_library_exports_every_declared_function():
    from x0ne_core._lib import lib
    L = lib()
    missing = [n for n in header_functions() if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_the_python_mirror_binds_every_function_with_the_headers_arity():
    from x0ne_core._lib import SIGNATURES
    decls = header_functions()
    for name, n in decls.items():
        assert name in SIGNATURES, f"{name} has no binding"
        assert len(SIGNATURES[name][0]) == n, f"{name}: {len(SIGNATURES[name][0])} arguments bound, header has {n}"


RUST_SYS = os.path.join(ROOT, "x0ne-engine_amd", "rust", "x0ne-core-runtime-mi355x", "src", "sys.rs")


def test_the_rust_crates_bindings_are_the_headers():
    """The Rust crate (x0ne-engine_amd/rust/x0ne-core-runtime-mi355x, x0ne-core/runtime's drop-in)
    cannot be compiled here (no cargo); its raw bindings are held to the header instead: every
    extern function it declares is declared in include/x0ne_core.h with the same number of
    parameters and exported by the library, and its options, statistics and counts structs have
    the header's fields in order."""
    from x0ne_core._lib import lib
    decls = header_functions()
    text = open(RUST_SYS).read()
    block = text[text.index('extern "C" {'):]
    fns = re.findall(r"pub fn (x0ne_[a-z0-9_]+)\s*\(([^)]*)\)", block, re.S)
    assert len(fns) >= 35
    L = lib()
    for name, args in fns:
        n = 0 if not args.strip() else args.strip().rstrip(",").count(",") + 1
        assert name in decls, f"{name}: not in the header"
        assert decls[name] == n, f"{name}: {n} parameters in Rust, {decls[name]} in the header"
        assert hasattr(L, name), f"{name}: not exported"
    header = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    c_to_rust = {"uint64_t": "u64", "uint32_t": "u32", "float": "f32", "double": "f64"}
    for name in ["x0ne_engine_options", "x0ne_pos_stats", "x0ne_counts", "x0ne_arg", "x0ne_split_plan",
                 "x0ne_gemv_fused", "x0ne_slice"]:
        # repr(C) with the header's fields, in order and of the same types: the same layout.
        m = re.search(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct %s \{(.*?)\}" % name, text, re.S)
        assert m, f"{name}: no repr(C) struct in sys.rs"
        rf = re.findall(r"pub (\w+): (\w+)", m.group(1))
        body = re.search(r"typedef struct \{([^}]*)\}\s*%s;" % name, header, re.S).group(1)
        cf = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            ctype, names = decl.split(None, 1)
            cf += [(n.strip(), c_to_rust[ctype]) for n in names.split(",")]
        assert rf == cf, f"{name}: Rust fields {rf}, header fields {cf}"
    for const, value in re.findall(r"#define (X0NE_\w+) (\d+)u?\b", header):
        if re.search(r"pub const %s\b" % const, text):
            assert re.search(r"pub const %s: \w+ = %s;" % (const, value), text), const


RUST_SRC = os.path.join(ROOT, "x0ne-engine_amd", "rust", "x0ne-core-runtime-mi355x", "src")


def test_the_rust_crate_has_the_references_kernel_launch_and_arena_api():
    """gpu.rs and arena.rs of the drop-in crate carry the public items of x0ne-core/runtime's
    (gpu.rs:262-314, 317-333, 958-985, 988-1008, 1031-1238, 1343-1364, 1383-1387; arena.rs:37-303)
    with the reference's signatures, and every sys:: function they, engine.rs and lib.rs call is
    one sys.rs declares (held to the header by the test above). The crate is not compiled here
    (no cargo); this is the check that holds its surface to the reference's."""
    sys_text = open(os.path.join(RUST_SRC, "sys.rs")).read()
    declared = set(re.findall(r"pub fn (x0ne_[a-z0-9_]+)", sys_text))
    squash = lambda t: re.sub(r"\s+", " ", t)
    gpu = squash(open(os.path.join(RUST_SRC, "gpu.rs")).read())
    arena = squash(open(os.path.join(RUST_SRC, "arena.rs")).read())
    lib = open(os.path.join(RUST_SRC, "lib.rs")).read()
    for m in ["pub mod gpu;", "pub mod arena;", "pub mod engine;", "pub mod st;"]:
        assert m in lib, m
    for sig in ["pub enum Arg { Ptr(u64), U32(u32), F32(f32), }",
                "pub fn param(&self) -> Param",
                "pub fn check_args(name: &str, params: &[Param], args: &[Arg]) -> Result<()>",
                "pub struct SplitPlan", "pub kernel: Kernel", "pub grid_x: u32", "pub group: u32",
                "pub grouped: bool", "pub per_sm: u32", "pub splits: u32",
                "pub fn new() -> Result<Gpu>",
                "pub fn split_plan(&self, q_heads: usize, kv_heads: usize) -> Result<SplitPlan>",
                "pub fn allocate(&self, len: u64) -> Result<DeviceBacking>",
                "pub unsafe fn launch(&self, k: Kernel, grid: (u32, u32), block: u32, args: &[Arg]) -> Result<()>",
                "pub unsafe fn gemm(&self, w: u64, rows: usize, cols: usize, x: u64, n: usize, y: u64, out: Out) -> Result<()>",
                "pub fn capture(&self, f: impl FnOnce() -> Result<()>) -> Result<Graph>",
                "pub unsafe fn launch_graph(&self, g: &Graph) -> Result<()>",
                "pub fn sync(&self) -> Result<()>", "pub fn counts(&self) -> Counts",
                "pub fn mem_info(&self) -> Result<(u64, u64)>", "pub fn nodes(&self) -> usize",
                "pub enum Out { Bf16, F32, }", "pub kernel_launches: u64",
                "macro_rules! launch { ($gpu:expr, $k:expr, $grid:expr, $block:expr; $($arg:expr),* $(,)?)"]:
        assert sig in gpu, f"gpu.rs: {sig}"
    for sig in ["pub const ALIGN: u64", "pub enum Class { Weights, ClientData, }",
                "pub fn offset(&self) -> u64", "pub fn len(&self) -> u64",
                "pub struct Region { pub label: String, pub class: Class, pub offset: u64, pub len: u64, }",
                "pub fn new() -> Self",
                "pub fn alloc(&mut self, label: &str, len: u64, class: Class) -> Result<Slice>",
                "pub fn planned_bytes(&self) -> u64",
                "pub fn freeze<B: Backing>(self, allocate: impl FnOnce(u64) -> Result<B>) -> Result<Arena<Frozen<B>>>",
                "pub fn write(&mut self, s: Slice, at: u64, data: &[u8]) -> Result<()>",
                "pub fn read(&self, s: Slice, at: u64, out: &mut [u8]) -> Result<()>",
                "pub fn scrub_client_data(&mut self) -> Result<u64>",
                "pub fn addr(&self, s: Slice, at: u64) -> Result<u64>",
                "pub fn ptr(&self, s: Slice) -> Result<u64>",
                "pub fn span(&self, s: Slice, at: u64, len: u64) -> Result<u64>",
                "pub fn allocate(len: u64) -> Result<Self>"]:
        assert sig in arena, f"arena.rs: {sig}"
    assert "ALIGN: u64 = sys::X0NE_ARENA_ALIGN" in arena
    assert re.search(r"pub const X0NE_ARENA_ALIGN: u64 = 256;", sys_text)
    for f in ["gpu.rs", "arena.rs", "engine.rs", "lib.rs", "error.rs", "st.rs"]:
        used = set(re.findall(r"sys::(x0ne_[a-z0-9_]+)\s*\(", open(os.path.join(RUST_SRC, f)).read()))
        assert used <= declared, f"{f} calls {sorted(used - declared)}, not declared in sys.rs"
    # Every unsafe block carries its reason, as the reference's code does.
    for f in ["gpu.rs", "arena.rs"]:
        lines = open(os.path.join(RUST_SRC, f)).read().splitlines()
        for i, line in enumerate(lines):
            if re.search(r"unsafe \{", line) and "unsafe impl" not in line:
                window = "\n".join(lines[max(0, i - 4):i + 1])
                assert "SAFETY" in window, f"{f}:{i + 1}: an unsafe block without a SAFETY comment"


def kernel_declarations():
    """Parameter kinds of each kernel in kernels.h, with the declaration macros expanded."""
    text = open(KERNELS_H).read()
    kinds = {}

    def kind(p):
        p = p.strip()
        if "*" in p:
            return "p"
        if p.startswith("float"):
            return "f"
        if p.startswith("uint32_t"):
            return "u"
        raise AssertionError(f"parameter {p!r}")

    # Each #define X0NE_DECLARE_NAME(params) with a continued body, expanded at its uses.
    plain, expanded = text, []
    for m in re.finditer(r"#define (X0NE_DECLARE_\w+)\(([^)]*)\)((?:.*\\\n)+.*\n)", text):
        name, params = m.group(1), [q.strip() for q in m.group(2).split(",")]
        body = m.group(3).replace("\\\n", "\n")
        plain = plain.replace(m.group(0), "")
        for use in re.finditer(r"^" + name + r"\(([^)]*)\)", text, re.M):
            b = body
            for q, v in zip(params, [x.strip() for x in use.group(1).split(",")]):
                b = b.replace("##" + q + "##", v).replace("##" + q, v)
            expanded.append(b)
        assert re.search(r"^" + name + r"\(", text, re.M), f"{name} is never used"
    for src in [plain] + expanded:
        for m in re.finditer(r"__global__ void (x0ne_\w+)\s*\(([^)]*)\)", src, re.S):
            kinds[m.group(1)] = "".join(kind(p) for p in m.group(2).split(","))
    return kinds


def test_the_kernel_table_is_the_kernel_declarations():
    from x0ne_core import gpu
    decl = kernel_declarations()
    names = gpu.kernel_names()
    assert sorted(names) == sorted(decl), "the table lists exactly the declared kernels"
    for n in names:
        got = "".join({0: "p", 1: "u", 2: "f"}[int(p)] for p in gpu.params_of(n))
        assert got == decl[n], f"{n}: table {got}, declaration {decl[n]}"


def test_a_launch_is_checked_against_the_table_before_any_device():
    from x0ne_core import gpu
    from x0ne_core.gpu import Arg
    with pytest.raises(Exception):
        gpu.check_args("x0ne_advance_u32", [Arg.u32(1)])  # a pointer is expected
    with pytest.raises(Exception):
        gpu.check_args("x0ne_advance_u32", [])
    with pytest.raises(Exception):
        gpu.check_args("no_such_kernel", [])
    gpu.check_args("x0ne_advance_u32", [Arg.ptr(0)])


def test_without_a_gpu_device_calls_fail_with_the_gpu_error():
    from x0ne_core import Engine, EngineOptions, GpuError
    from x0ne_core.gpu import Gpu
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(GpuError):
        Gpu()
    cfg = {"model_type": "qwen3", "dtype": "bfloat16", "hidden_act": "silu", "attention_bias": False,
           "hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 1, "num_attention_heads": 2,
           "num_key_value_heads": 1, "head_dim": 128, "vocab_size": 100, "max_position_embeddings": 256,
           "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": True}
    with pytest.raises(GpuError):
        Engine.load_synthetic(cfg, 0, 0.02, EngineOptions(max_ctx=64))


def test_the_error_codes_are_the_references_variants():
    from x0ne_core import _lib
    L = _lib.lib()
    # x0ne_status values are fixed by the header: OK 0, IO 1, FORMAT 2, ARENA 3, NOT_IMPLEMENTED 4, GPU 5.
    text = open(HEADER).read()
    for name, v in [("X0NE_OK", 0), ("X0NE_ERR_IO", 1), ("X0NE_ERR_FORMAT", 2), ("X0NE_ERR_ARENA", 3),
                    ("X0NE_ERR_NOT_IMPLEMENTED", 4), ("X0NE_ERR_GPU", 5)]:
        assert re.search(rf"\b{name}\s*=\s*{v}\b", text), name
    buf = C.create_string_buffer(256)
    L.x0ne_last_error(buf, 256)  # callable without a device
