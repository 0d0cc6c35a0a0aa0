//! The reference's Error (x0ne-core/runtime/src/error.rs:4-40): one variant per x0ne_status.
use std::fmt;

#[derive(Debug)]
pub enum Error {
    Io(std::io::Error),
    /// A refused config, checkpoint or request: raised before any device work.
    Format(String),
    Arena(String),
    NotImplemented(&'static str),
    Gpu(String),
}

pub type Result<T> = std::result::Result<T, Error>;

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            Error::Io(e) => write!(f, "io: {e}"),
            Error::Format(m) => write!(f, "format: {m}"),
            Error::Arena(m) => write!(f, "arena: {m}"),
            Error::NotImplemented(m) => write!(f, "not implemented: {m}"),
            Error::Gpu(m) => write!(f, "gpu: {m}"),
        }
    }
}

impl std::error::Error for Error {
    fn source(&self) -> Option<&(dyn std::error::Error + 'static)> {
        match self {
            Error::Io(e) => Some(e),
            _ => None,
        }
    }
}

impl From<std::io::Error> for Error {
    fn from(e: std::io::Error) -> Self {
        Error::Io(e)
    }
}

/// The status of a call, with the calling thread's message of the library's last failure.
pub(crate) fn check(status: std::ffi::c_int) -> Result<()> {
    use crate::sys;
    if status == sys::X0NE_OK {
        return Ok(());
    }
    let mut buf = vec![0u8; 4096];
    // SAFETY: the buffer is writable for its length; the library writes at most len - 1 bytes
    // and a terminating NUL.
    unsafe { sys::x0ne_last_error(buf.as_mut_ptr().cast(), buf.len()) };
    let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
    let msg = String::from_utf8_lossy(&buf[..end]).into_owned();
    Err(match status {
        sys::X0NE_ERR_IO => Error::Io(std::io::Error::other(msg)),
        sys::X0NE_ERR_FORMAT => Error::Format(msg),
        sys::X0NE_ERR_ARENA => Error::Arena(msg),
        sys::X0NE_ERR_NOT_IMPLEMENTED => Error::NotImplemented(intern(msg)),
        _ => Error::Gpu(msg),
    })
}

/// The reference's NotImplemented carries a `&'static str`; the library's messages for it are a
/// small fixed set (one per unsupported configuration), so each distinct one is leaked once and
/// reused.
fn intern(msg: String) -> &'static str {
    use std::collections::HashSet;
    use std::sync::{Mutex, OnceLock};
    static SEEN: OnceLock<Mutex<HashSet<&'static str>>> = OnceLock::new();
    let mut seen = SEEN.get_or_init(|| Mutex::new(HashSet::new())).lock().unwrap_or_else(|e| e.into_inner());
    if let Some(s) = seen.get(msg.as_str()) {
        return s;
    }
    let s: &'static str = Box::leak(msg.into_boxed_str());
    seen.insert(s);
    s
}
