//! The C ABI of libx0ne_core.so (include/x0ne_core.h), the entry points this crate wraps.
#![allow(non_camel_case_types)]
use std::ffi::{c_char, c_int, c_void};

#[repr(C)]
pub struct x0ne_engine {
    _p: [u8; 0],
}
#[repr(C)]
pub struct x0ne_session {
    _p: [u8; 0],
}
#[repr(C)]
pub struct x0ne_greedy {
    _p: [u8; 0],
}
#[repr(C)]
pub struct x0ne_gpu {
    _p: [u8; 0],
}
#[repr(C)]
pub struct x0ne_graph {
    _p: [u8; 0],
}
#[repr(C)]
pub struct x0ne_arena {
    _p: [u8; 0],
}

/// x0ne_engine_options.sums
pub const X0NE_SUMS_DEFAULT: u32 = 0;
pub const X0NE_SUMS_F64: u32 = 1;
pub const X0NE_SUMS_F32: u32 = 2;

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct x0ne_engine_options {
    pub max_ctx: u64,
    pub page_seed: u64,
    pub sums: u32,
    pub prefill_chunk: u32,
    pub max_batch: u32,
    pub reserved: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct x0ne_pos_stats {
    pub argmax: u32,
    pub logsumexp: f32,
    pub next_logprob: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug, PartialEq, Eq)]
pub struct x0ne_counts {
    pub launches: u64,
    pub graph_launches: u64,
    pub gemms: u64,
    pub htod: u64,
    pub dtoh: u64,
    pub memsets: u64,
    pub syncs: u64,
}

/// x0ne_param
pub const X0NE_PARAM_PTR: u32 = 0;
pub const X0NE_PARAM_U32: u32 = 1;
pub const X0NE_PARAM_F32: u32 = 2;

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct x0ne_arg {
    pub kind: u32,
    pub u32: u32,
    pub f32: f32,
    pub pad: u32,
    pub ptr: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct x0ne_split_plan {
    pub splits: u32,
    pub grid_x: u32,
    pub group: u32,
    pub grouped: u32,
    pub per_cu: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct x0ne_gemv_fused {
    pub w: u64,
    pub x: u64,
    pub res_in: u64,
    pub res_out: u64,
    pub delta: u64,
    pub norm_w: u64,
    pub embed: u64,
    pub tokens: u64,
    pub y: u64,
    pub partial: u64,
    pub counter: u64,
    pub token_out: u64,
    pub pos: u64,
    pub rows: u32,
    pub cols: u32,
    pub vocab: u32,
    pub advance: u32,
    pub eps: f32,
    pub prologue: u32,
    pub epilogue: u32,
    pub f64_sums: u32,
}

/// x0ne_class (arena.rs:42-45)
pub const X0NE_CLASS_WEIGHTS: u32 = 0;
pub const X0NE_CLASS_CLIENT_DATA: u32 = 1;
pub const X0NE_ARENA_ALIGN: u64 = 256;

#[repr(C)]
#[derive(Clone, Copy, Default, Debug, PartialEq, Eq)]
pub struct x0ne_slice {
    pub arena: u64,
    pub offset: u64,
    pub len: u64,
}

pub const X0NE_OK: c_int = 0;
pub const X0NE_ERR_IO: c_int = 1;
pub const X0NE_ERR_FORMAT: c_int = 2;
pub const X0NE_ERR_ARENA: c_int = 3;
pub const X0NE_ERR_NOT_IMPLEMENTED: c_int = 4;
pub const X0NE_ERR_GPU: c_int = 5;

extern "C" {
    pub fn x0ne_last_error(buf: *mut c_char, len: usize) -> usize;
    pub fn x0ne_kernel_set(buf: *mut c_char, len: usize) -> usize;

    // The device (gpu.rs).
    pub fn x0ne_gpu_new(out: *mut *mut x0ne_gpu) -> c_int;
    pub fn x0ne_gpu_free(g: *mut x0ne_gpu);
    pub fn x0ne_gpu_sync(g: *mut x0ne_gpu) -> c_int;
    pub fn x0ne_gpu_describe(g: *const x0ne_gpu, buf: *mut c_char, len: usize) -> c_int;
    pub fn x0ne_gpu_compute_units(g: *const x0ne_gpu) -> u32;
    pub fn x0ne_gpu_mem_info(g: *const x0ne_gpu, free_bytes: *mut u64, total_bytes: *mut u64) -> c_int;
    pub fn x0ne_gpu_counts(g: *const x0ne_gpu, out: *mut x0ne_counts) -> c_int;
    pub fn x0ne_kernel_count() -> usize;
    pub fn x0ne_kernel_name(i: usize) -> *const c_char;
    pub fn x0ne_kernel_params(name: *const c_char, out: *mut u32, cap: usize) -> usize;
    pub fn x0ne_check_args(name: *const c_char, args: *const x0ne_arg, n: usize) -> c_int;
    pub fn x0ne_gpu_launch(g: *mut x0ne_gpu, name: *const c_char, gx: u32, gy: u32, block: u32, args: *const x0ne_arg,
                           n: usize) -> c_int;
    pub fn x0ne_gpu_gemv(g: *mut x0ne_gpu, w: u64, rows: u64, cols: u64, x: u64, n: u64, y: u64, out_f32: c_int)
                         -> c_int;
    pub fn x0ne_gpu_split_plan(g: *const x0ne_gpu, q_heads: u32, kv_heads: u32, out: *mut x0ne_split_plan) -> c_int;
    pub fn x0ne_gpu_capture_begin(g: *mut x0ne_gpu) -> c_int;
    pub fn x0ne_gpu_capture_end(g: *mut x0ne_gpu, out: *mut *mut x0ne_graph) -> c_int;
    pub fn x0ne_gpu_launch_graph(g: *mut x0ne_gpu, graph: *const x0ne_graph) -> c_int;
    pub fn x0ne_graph_nodes(graph: *const x0ne_graph) -> usize;
    pub fn x0ne_graph_free(graph: *mut x0ne_graph);

    // The arena (arena.rs).
    pub fn x0ne_arena_new(out: *mut *mut x0ne_arena) -> c_int;
    pub fn x0ne_arena_free(a: *mut x0ne_arena);
    pub fn x0ne_arena_alloc(a: *mut x0ne_arena, label: *const c_char, len: u64, cls: u32, out: *mut x0ne_slice)
                            -> c_int;
    pub fn x0ne_arena_planned_bytes(a: *const x0ne_arena) -> u64;
    pub fn x0ne_arena_freeze(a: *mut x0ne_arena, g: *mut x0ne_gpu) -> c_int;
    pub fn x0ne_arena_write(a: *mut x0ne_arena, s: x0ne_slice, at: u64, data: *const c_void, len: u64) -> c_int;
    pub fn x0ne_arena_read(a: *const x0ne_arena, s: x0ne_slice, at: u64, out: *mut c_void, len: u64) -> c_int;
    pub fn x0ne_arena_addr(a: *const x0ne_arena, s: x0ne_slice, at: u64, out: *mut u64) -> c_int;
    pub fn x0ne_arena_span(a: *const x0ne_arena, s: x0ne_slice, at: u64, len: u64, out: *mut u64) -> c_int;
    pub fn x0ne_arena_scrub(a: *mut x0ne_arena, zeroed: *mut u64) -> c_int;
    pub fn x0ne_arena_region_count(a: *const x0ne_arena) -> usize;
    pub fn x0ne_arena_region(a: *const x0ne_arena, i: usize, label_buf: *mut c_char, label_len: usize, cls: *mut u32,
                             offset: *mut u64, len: *mut u64) -> c_int;
    pub fn x0ne_arena_is_frozen(a: *const x0ne_arena) -> c_int;

    // The engine (engine.rs).
    pub fn x0ne_engine_load_from(config_json: *const c_char, n_files: usize, names: *const *const c_char,
                                 data: *const *const u8, lens: *const u64, index_json: *const c_char,
                                 opts: *const x0ne_engine_options, out: *mut *mut x0ne_engine) -> c_int;
    pub fn x0ne_engine_load(model_dir: *const c_char, opts: *const x0ne_engine_options,
                            out: *mut *mut x0ne_engine) -> c_int;
    pub fn x0ne_engine_free(e: *mut x0ne_engine);

    pub fn x0ne_engine_session(e: *mut x0ne_engine, prompt: *const u32, n: usize, out: *mut *mut x0ne_session)
                               -> c_int;
    pub fn x0ne_session_logits(s: *const x0ne_session, ptr: *mut *const f32, len: *mut usize) -> c_int;
    pub fn x0ne_session_position(s: *const x0ne_session) -> usize;
    pub fn x0ne_session_step(s: *mut x0ne_session, token: u32) -> c_int;
    pub fn x0ne_session_finish(s: *mut x0ne_session) -> c_int;
    pub fn x0ne_session_drop(s: *mut x0ne_session);
    pub fn x0ne_session_into_greedy(s: *mut x0ne_session, max_tokens: usize, ahead: usize,
                                    out: *mut *mut x0ne_greedy) -> c_int;
    pub fn x0ne_greedy_next(g: *mut x0ne_greedy, token: *mut u32) -> c_int;
    pub fn x0ne_greedy_taken(g: *const x0ne_greedy) -> usize;
    pub fn x0ne_greedy_position(g: *const x0ne_greedy) -> usize;
    pub fn x0ne_greedy_finish(g: *mut x0ne_greedy) -> c_int;
    pub fn x0ne_greedy_drop(g: *mut x0ne_greedy);

    pub fn x0ne_engine_greedy_timed(e: *mut x0ne_engine, prompt: *const u32, n_prompt: usize, n: usize,
                                    tokens: *mut u32, times: *mut f64) -> c_int;
    pub fn x0ne_engine_greedy_with_last_logits(e: *mut x0ne_engine, prompt: *const u32, n_prompt: usize, n: usize,
                                               tokens: *mut u32, logits: *mut f32) -> c_int;
    pub fn x0ne_engine_set_decode_mode(e: *mut x0ne_engine, mode: u32) -> c_int;
    pub fn x0ne_engine_decode_mode(e: *const x0ne_engine) -> u32;
    pub fn x0ne_engine_set_decode_attention(e: *mut x0ne_engine, attention: u32) -> c_int;
    pub fn x0ne_engine_decode_attention(e: *const x0ne_engine) -> u32;
    pub fn x0ne_engine_set_split_merge(e: *mut x0ne_engine, merge: u32) -> c_int;
    pub fn x0ne_engine_split_merge(e: *const x0ne_engine) -> u32;
    pub fn x0ne_engine_logits_at(e: *mut x0ne_engine, ids: *const u32, n: usize, positions: *const usize,
                                 n_positions: usize, route: u32, rows: *mut f32) -> c_int;
    pub fn x0ne_engine_run(e: *mut x0ne_engine, ids: *const u32, n: usize, route: u32, keep: *const usize,
                           n_keep: usize, stats: *mut x0ne_pos_stats, rows: *mut f32) -> c_int;
    pub fn x0ne_engine_moe_routing(e: *mut x0ne_engine, ids: *const u32, n: usize, out: *mut u32, cap: usize,
                                   written: *mut usize) -> c_int;
    pub fn x0ne_engine_describe(e: *const x0ne_engine, buf: *mut c_char, len: usize) -> c_int;
    pub fn x0ne_engine_graph_nodes(e: *const x0ne_engine) -> usize;
    pub fn x0ne_engine_splits(e: *const x0ne_engine) -> u32;
    pub fn x0ne_engine_counts(e: *const x0ne_engine, out: *mut x0ne_counts) -> c_int;
    pub fn x0ne_engine_client_data_is_zero(e: *const x0ne_engine, out: *mut c_int) -> c_int;
    pub fn x0ne_engine_host_buffers_are_zero(e: *const x0ne_engine) -> c_int;
    pub fn x0ne_engine_max_ctx(e: *const x0ne_engine) -> u64;
    pub fn x0ne_engine_sums(e: *const x0ne_engine) -> u32;
}
