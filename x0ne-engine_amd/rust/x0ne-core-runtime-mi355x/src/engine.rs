//! Engine, Session and Greedy (x0ne-core/runtime/src/engine.rs) over libx0ne_core.so: the same
//! signatures and borrowing rules. A Session borrows its Engine mutably (one request at a time);
//! its logits are valid until its next step or finish (the borrow of &self enforces it); a
//! Session or Greedy dropped without finish zeroes the client bytes all the same.
use std::ffi::{c_int, CString};
use std::marker::PhantomData;

use crate::error::check;
use crate::st::SliceSource;
use crate::{sys, Error, Result};

/// Prompt rows per prefill pass of this engine's f32 path (the reference's is 512, engine.rs:67;
/// a 2048-row pass gives the prefill GEMM enough output tiles to fill MI355X's 256 compute units).
/// The exact mode, the default, feeds a prompt one exact step per token.
pub const PREFILL_CHUNK: usize = 2048;
/// Steps ahead of the host in a greedy session by default, and at most (engine.rs:67-79).
pub const GREEDY_AHEAD: usize = 2;
pub const GREEDY_AHEAD_MAX: usize = 15;

#[derive(Clone, Copy, Debug)]
pub struct EngineOptions {
    pub max_ctx: usize,
}

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Route {
    Prefill = 0,
    Decode = 1,
}

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum DecodeMode {
    Eager = 0,
    Graph = 1,
}

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum DecodeAttention {
    SplitK = 0,
    PerHead = 1,
}

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum SplitMerge {
    Kernel = 0,
    LastBlock = 1,
}

/// PosStats (engine.rs:57-64).
#[derive(Clone, Copy, Debug, Default)]
pub struct PosStats {
    pub argmax: u32,
    pub logsumexp: f32,
    pub next_logprob: f32,
}

pub use crate::gpu::Counts;

pub struct Engine {
    h: *mut sys::x0ne_engine,
    vocab: usize,
}

// As the reference's Gpu (gpu.rs:768): Send, not Sync; callers serialise through a Mutex.
unsafe impl Send for Engine {}

fn options(o: EngineOptions) -> sys::x0ne_engine_options {
    sys::x0ne_engine_options { max_ctx: o.max_ctx as u64, ..Default::default() }
}

fn vocab_of(config_json: &str) -> usize {
    // The library has checked the config; its vocab_size sizes the rows handed back.
    config_json
        .split("\"vocab_size\"")
        .nth(1)
        .and_then(|rest| rest.trim_start().strip_prefix(':'))
        .map(|rest| rest.trim_start().chars().take_while(|c| c.is_ascii_digit()).collect::<String>())
        .and_then(|d| d.parse().ok())
        .unwrap_or(0)
}

impl Engine {
    /// Engine::load_from (engine.rs:301-309): a Qwen3 checkpoint from safetensors in memory.
    pub fn load_from(config_json: &str, src: &SliceSource<'_>, opts: EngineOptions) -> Result<Engine> {
        let cfg = CString::new(config_json).map_err(|_| Error::Format("config.json: a NUL byte".into()))?;
        let names: Vec<*const std::ffi::c_char> = src.names.iter().map(|n| n.as_ptr()).collect();
        let data: Vec<*const u8> = src.files.iter().map(|f| f.as_ptr()).collect();
        let lens: Vec<u64> = src.files.iter().map(|f| f.len() as u64).collect();
        let index = src.index.as_ref().map_or(std::ptr::null(), |c| c.as_ptr());
        let o = options(opts);
        let mut h = std::ptr::null_mut();
        // SAFETY: every pointer is valid for the call; the library keeps none of them.
        check(unsafe {
            sys::x0ne_engine_load_from(cfg.as_ptr(), names.len(), names.as_ptr(), data.as_ptr(), lens.as_ptr(),
                                       index, &o, &mut h)
        })?;
        Ok(Engine { h, vocab: vocab_of(config_json) })
    }

    /// Engine::load (engine.rs:292-297): config.json, then model.safetensors or the shards its
    /// model.safetensors.index.json names.
    pub fn load(model_dir: &std::path::Path, opts: EngineOptions) -> Result<Engine> {
        use std::os::unix::ffi::OsStrExt;
        let dir = CString::new(model_dir.as_os_str().as_bytes())
            .map_err(|_| Error::Format("model_dir: a NUL byte".into()))?;
        let o = options(opts);
        let mut h = std::ptr::null_mut();
        // SAFETY: as above.
        check(unsafe { sys::x0ne_engine_load(dir.as_ptr(), &o, &mut h) })?;
        let config = std::fs::read_to_string(model_dir.join("config.json"))?;
        Ok(Engine { h, vocab: vocab_of(&config) })
    }

    /// Engine::session (engine.rs:389-406): prefills `prompt`, holds the last position's logits.
    pub fn session(&mut self, prompt: &[u32]) -> Result<Session<'_>> {
        let mut s = std::ptr::null_mut();
        // SAFETY: the prompt is read during the call only.
        check(unsafe { sys::x0ne_engine_session(self.h, prompt.as_ptr(), prompt.len(), &mut s) })?;
        Ok(Session { s, _e: PhantomData })
    }

    pub fn greedy(&mut self, prompt: &[u32], n: usize) -> Result<Vec<u32>> {
        Ok(self.greedy_timed(prompt, n)?.0)
    }

    /// Engine::greedy_timed (engine.rs:1026-1038): n tokens and the seconds (from the call) at
    /// which each was on the host.
    pub fn greedy_timed(&mut self, prompt: &[u32], n: usize) -> Result<(Vec<u32>, Vec<f64>)> {
        let (mut t, mut s) = (vec![0u32; n], vec![0f64; n]);
        // SAFETY: the output buffers hold n values each.
        check(unsafe {
            sys::x0ne_engine_greedy_timed(self.h, prompt.as_ptr(), prompt.len(), n, t.as_mut_ptr(), s.as_mut_ptr())
        })?;
        Ok((t, s))
    }

    /// Engine::greedy_with_last_logits (engine.rs:1042-1063).
    pub fn greedy_with_last_logits(&mut self, prompt: &[u32], n: usize) -> Result<(Vec<u32>, Vec<f32>)> {
        let (mut t, mut l) = (vec![0u32; n], vec![0f32; self.vocab]);
        // SAFETY: tokens holds n values, logits vocab_size.
        check(unsafe {
            sys::x0ne_engine_greedy_with_last_logits(self.h, prompt.as_ptr(), prompt.len(), n, t.as_mut_ptr(),
                                                     l.as_mut_ptr())
        })?;
        Ok((t, l))
    }

    /// Engine::run (engine.rs:928-1006): stats at every position, full rows at `keep`.
    pub fn run(&mut self, ids: &[u32], route: Route, keep: &[usize]) -> Result<(Vec<PosStats>, Vec<Vec<f32>>)> {
        let mut stats = vec![sys::x0ne_pos_stats::default(); ids.len().max(1)];
        let mut rows = vec![0f32; keep.len() * self.vocab];
        // SAFETY: stats holds ids.len() entries, rows keep.len() rows of vocab_size.
        check(unsafe {
            sys::x0ne_engine_run(self.h, ids.as_ptr(), ids.len(), route as u32, keep.as_ptr(), keep.len(),
                                 stats.as_mut_ptr(), rows.as_mut_ptr())
        })?;
        let stats = stats[..ids.len()]
            .iter()
            .map(|s| PosStats { argmax: s.argmax, logsumexp: s.logsumexp, next_logprob: s.next_logprob })
            .collect();
        Ok((stats, rows.chunks_exact(self.vocab.max(1)).map(|r| r.to_vec()).collect()))
    }

    pub fn stats(&mut self, ids: &[u32], route: Route) -> Result<Vec<PosStats>> {
        Ok(self.run(ids, route, &[])?.0)
    }

    /// Engine::logits_at (engine.rs:1012-1020).
    pub fn logits_at(&mut self, ids: &[u32], positions: &[usize], route: Route) -> Result<Vec<Vec<f32>>> {
        let mut rows = vec![0f32; positions.len() * self.vocab];
        // SAFETY: rows holds positions.len() rows of vocab_size.
        check(unsafe {
            sys::x0ne_engine_logits_at(self.h, ids.as_ptr(), ids.len(), positions.as_ptr(), positions.len(),
                                       route as u32, rows.as_mut_ptr())
        })?;
        Ok(rows.chunks_exact(self.vocab.max(1)).map(|r| r.to_vec()).collect())
    }

    /// Engine::moe_routing (engine.rs:612-640): [position][layer][top_k] expert ids.
    pub fn moe_routing(&mut self, ids: &[u32], layers: usize, top_k: usize) -> Result<Vec<u32>> {
        let mut out = vec![0u32; ids.len() * layers * top_k];
        let mut written = 0usize;
        // SAFETY: out holds its length.
        check(unsafe {
            sys::x0ne_engine_moe_routing(self.h, ids.as_ptr(), ids.len(), out.as_mut_ptr(), out.len(), &mut written)
        })?;
        out.truncate(written);
        Ok(out)
    }

    pub fn decode_mode(&self) -> DecodeMode {
        // SAFETY: a live engine.
        if unsafe { sys::x0ne_engine_decode_mode(self.h) } == 0 { DecodeMode::Eager } else { DecodeMode::Graph }
    }
    pub fn set_decode_mode(&mut self, mode: DecodeMode) -> Result<()> {
        check(unsafe { sys::x0ne_engine_set_decode_mode(self.h, mode as u32) })
    }
    pub fn decode_attention(&self) -> DecodeAttention {
        if unsafe { sys::x0ne_engine_decode_attention(self.h) } == 1 {
            DecodeAttention::PerHead
        } else {
            DecodeAttention::SplitK
        }
    }
    /// Engine::set_decode_attention (engine.rs:531-539): re-captures the decode graph.
    pub fn set_decode_attention(&mut self, a: DecodeAttention) -> Result<()> {
        check(unsafe { sys::x0ne_engine_set_decode_attention(self.h, a as u32) })
    }
    pub fn split_merge(&self) -> SplitMerge {
        if unsafe { sys::x0ne_engine_split_merge(self.h) } == 1 { SplitMerge::LastBlock } else { SplitMerge::Kernel }
    }
    /// Engine::set_split_merge (engine.rs:547-560).
    pub fn set_split_merge(&mut self, m: SplitMerge) -> Result<()> {
        check(unsafe { sys::x0ne_engine_set_split_merge(self.h, m as u32) })
    }

    /// Engine::describe (engine.rs:578-606).
    pub fn describe(&self) -> String {
        let mut buf = vec![0u8; 2048];
        // SAFETY: the buffer is writable for its length.
        let _ = unsafe { sys::x0ne_engine_describe(self.h, buf.as_mut_ptr().cast(), buf.len()) };
        let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
        String::from_utf8_lossy(&buf[..end]).into_owned()
    }
    pub fn graph_nodes(&self) -> usize {
        unsafe { sys::x0ne_engine_graph_nodes(self.h) }
    }
    pub fn splits(&self) -> u32 {
        unsafe { sys::x0ne_engine_splits(self.h) }
    }
    pub fn max_ctx(&self) -> usize {
        unsafe { sys::x0ne_engine_max_ctx(self.h) as usize }
    }
    pub fn counts(&self) -> Counts {
        let mut c = sys::x0ne_counts::default();
        let _ = unsafe { sys::x0ne_engine_counts(self.h, &mut c) };
        c.into()
    }
    /// The engine runs the exact mode (f64 sums, the oracle's rounding points): what
    /// EngineOptions { max_ctx } gives a dense model decoding one sequence. This build's; the
    /// reference's engine has the f32 path only.
    pub fn exact(&self) -> bool {
        unsafe { sys::x0ne_engine_sums(self.h) == sys::X0NE_SUMS_F64 }
    }
    pub fn client_data_is_zero(&self) -> Result<bool> {
        let mut z: c_int = 0;
        check(unsafe { sys::x0ne_engine_client_data_is_zero(self.h, &mut z) })?;
        Ok(z != 0)
    }
    pub fn host_buffers_are_zero(&self) -> bool {
        unsafe { sys::x0ne_engine_host_buffers_are_zero(self.h) != 0 }
    }
}

impl Drop for Engine {
    fn drop(&mut self) {
        // SAFETY: the handle came from a load; Sessions borrowing it are gone (the borrow checker).
        unsafe { sys::x0ne_engine_free(self.h) }
    }
}

/// A request on the engine (engine.rs:1137-1243).
pub struct Session<'e> {
    s: *mut sys::x0ne_session,
    _e: PhantomData<&'e mut Engine>,
}

impl<'e> Session<'e> {
    /// The f32 logits of the last position; valid until the next step or finish.
    pub fn logits(&self) -> &[f32] {
        let (mut p, mut n) = (std::ptr::null(), 0usize);
        // SAFETY: the library's pinned row outlives &self: it changes only at step or finish,
        // which take &mut self or self.
        unsafe {
            if sys::x0ne_session_logits(self.s, &mut p, &mut n) != sys::X0NE_OK || p.is_null() {
                return &[];
            }
            std::slice::from_raw_parts(p, n)
        }
    }
    pub fn position(&self) -> usize {
        unsafe { sys::x0ne_session_position(self.s) }
    }
    pub fn step(&mut self, token: u32) -> Result<()> {
        check(unsafe { sys::x0ne_session_step(self.s, token) })
    }
    /// Session::finish: zeroes the client bytes.
    pub fn finish(self) -> Result<()> {
        let s = self.s;
        std::mem::forget(self);
        check(unsafe { sys::x0ne_session_finish(s) })
    }
    /// Session::into_greedy_ahead (engine.rs:1199-1243): the session is consumed (freed by the
    /// library even on error, its client bytes zeroed).
    pub fn into_greedy_ahead(self, max_tokens: usize, ahead: usize) -> Result<Greedy<'e>> {
        let s = self.s;
        std::mem::forget(self);
        let mut g = std::ptr::null_mut();
        check(unsafe { sys::x0ne_session_into_greedy(s, max_tokens, ahead, &mut g) })?;
        Ok(Greedy { g, _e: PhantomData })
    }
    pub fn into_greedy(self, max_tokens: usize) -> Result<Greedy<'e>> {
        self.into_greedy_ahead(max_tokens, GREEDY_AHEAD)
    }
}

impl Drop for Session<'_> {
    fn drop(&mut self) {
        unsafe { sys::x0ne_session_drop(self.s) }
    }
}

/// A session deciding greedy tokens on the device (engine.rs:1245-1344).
pub struct Greedy<'e> {
    g: *mut sys::x0ne_greedy,
    _e: PhantomData<&'e mut Engine>,
}

impl Greedy<'_> {
    pub fn next_token(&mut self) -> Result<u32> {
        let mut t = 0u32;
        check(unsafe { sys::x0ne_greedy_next(self.g, &mut t) })?;
        Ok(t)
    }
    pub fn taken(&self) -> usize {
        unsafe { sys::x0ne_greedy_taken(self.g) }
    }
    pub fn position(&self) -> usize {
        unsafe { sys::x0ne_greedy_position(self.g) }
    }
    pub fn finish(self) -> Result<()> {
        let g = self.g;
        std::mem::forget(self);
        check(unsafe { sys::x0ne_greedy_finish(g) })
    }
}

impl Drop for Greedy<'_> {
    fn drop(&mut self) {
        unsafe { sys::x0ne_greedy_drop(self.g) }
    }
}
