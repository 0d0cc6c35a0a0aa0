//! x0ne Core's runtime API (x0ne-core/runtime, crate x0ne_core_runtime) on MI355X: the engine,
//! its sessions, the kernel-launch API (gpu), the KV arena (arena) and the safetensors source of
//! the reference, over libx0ne_core.so's C ABI (include/x0ne_core.h), whose hand-written gfx950
//! kernels replace the CUDA cubins and cuBLAS.
pub mod arena;
pub mod engine;
mod error;
pub mod gpu;
pub mod st;
pub mod sys;

pub use error::{Error, Result};

/// lib.rs:26-31: the kernel set's fingerprint and the compiler that built it (for MI355X: the
/// SHA-256 prefix of the HIP sources and the hipcc version, where the CUDA build reported the
/// cubins' hash and the nvcc release).
pub fn kernel_set() -> (&'static str, &'static str) {
    static SET: std::sync::OnceLock<(String, String)> = std::sync::OnceLock::new();
    let (a, b) = SET.get_or_init(|| {
        let mut buf = vec![0u8; 512];
        // SAFETY: the buffer is writable for its length.
        unsafe { sys::x0ne_kernel_set(buf.as_mut_ptr().cast(), buf.len()) };
        let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
        let s = String::from_utf8_lossy(&buf[..end]).into_owned();
        // "kernels <sha>, gfx950, <compiler>"
        let sha = s.split(',').next().unwrap_or("").trim_start_matches("kernels ").trim().to_string();
        let compiler = s.splitn(3, ',').nth(2).unwrap_or("").trim().to_string();
        (sha, compiler)
    });
    (a.as_str(), b.as_str())
}
