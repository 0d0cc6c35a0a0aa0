//! The C ABI of libx0ne_core.so (include/x0ne_core.h), the entry points this crate wraps.
#![allow(non_camel_case_types)]
use std::ffi::{c_char, c_int};

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
#[derive(Clone, Copy, Default)]
pub struct x0ne_engine_options {
    pub max_ctx: u64,
    pub page_seed: u64,
    pub f64_sums: u32,
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
#[derive(Clone, Copy, Default)]
pub struct x0ne_counts {
    pub launches: u64,
    pub graph_launches: u64,
    pub gemms: u64,
    pub htod: u64,
    pub dtoh: u64,
    pub memsets: u64,
    pub syncs: u64,
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
}
