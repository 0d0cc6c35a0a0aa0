//! The KV arena of x0ne-core/runtime/src/arena.rs over libx0ne_core.so: one allocation planned
//! region by region (`Arena<Building>::alloc`), made once (`freeze`), then read, written,
//! addressed and scrubbed through checked slices (`Arena<Frozen<B>>`). The typestate is the
//! reference's: nothing is allocated after freeze, and a slice of another arena is refused. The
//! memory is the library's (`x0ne_arena_freeze`): one device allocation on a `Gpu`, or host
//! memory poisoned with 0xA5 (`HostBacking`) for tests without a device.
use std::ffi::CString;
use std::sync::Arc;

use crate::error::check;
use crate::gpu::{DeviceBacking, Handle};
use crate::{sys, Error, Result};

/// Offsets are multiples of this (arena.rs:37).
pub const ALIGN: u64 = sys::X0NE_ARENA_ALIGN;

/// What a region holds (arena.rs:39-45). `ClientData` is everything derived from a request: KV
/// cache, activations, logits, scratch. `scrub_client_data` zeroes it.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Class {
    Weights,
    ClientData,
}

impl Class {
    fn raw(self) -> u32 {
        match self {
            Class::Weights => sys::X0NE_CLASS_WEIGHTS,
            Class::ClientData => sys::X0NE_CLASS_CLIENT_DATA,
        }
    }
}

/// A planned region. Only valid for the arena that issued it (arena.rs:47-65).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub struct Slice(sys::x0ne_slice);

impl Slice {
    pub fn offset(&self) -> u64 {
        self.0.offset
    }
    pub fn len(&self) -> u64 {
        self.0.len
    }
    pub fn is_empty(&self) -> bool {
        self.0.len == 0
    }
}

#[derive(Debug, Clone)]
pub struct Region {
    pub label: String,
    pub class: Class,
    pub offset: u64,
    pub len: u64,
}

/// The memory behind a frozen arena: what `freeze`'s allocate callback returns
/// (arena.rs:76-91). Sealed: the library makes the allocation on the backing's device, or in
/// host memory.
pub trait Backing: Sized + private::Sealed {
    fn len(&self) -> u64;
    fn is_empty(&self) -> bool {
        self.len() == 0
    }
}

/// A backing whose bytes have a device address (one contiguous allocation).
pub trait DeviceAddressed: Backing {}

mod private {
    pub trait Sealed {
        /// The device handle the library allocates on, or None for host memory.
        fn device(&self) -> Option<std::sync::Arc<crate::gpu::Handle>>;
    }
}

/// Host memory, poisoned with 0xA5 so that bytes never written stand out (arena.rs:93-136).
#[derive(Debug)]
pub struct HostBacking(u64);

impl HostBacking {
    pub fn allocate(len: u64) -> Result<Self> {
        usize::try_from(len).map_err(|_| Error::Arena("size exceeds host usize".into()))?;
        Ok(HostBacking(len))
    }
}

impl private::Sealed for HostBacking {
    fn device(&self) -> Option<Arc<Handle>> {
        None
    }
}
impl Backing for HostBacking {
    fn len(&self) -> u64 {
        self.0
    }
}
// The library's host arenas have addresses too (host pointers); the engine's tests read them.
impl DeviceAddressed for HostBacking {}

impl private::Sealed for DeviceBacking {
    fn device(&self) -> Option<Arc<Handle>> {
        Some(self.gpu.clone())
    }
}
impl Backing for DeviceBacking {
    fn len(&self) -> u64 {
        self.len
    }
}
impl DeviceAddressed for DeviceBacking {}

/// The library's arena handle, freed once.
struct Raw(*mut sys::x0ne_arena);

impl Drop for Raw {
    fn drop(&mut self) {
        // SAFETY: freed once, here (the device memory with it, on the handle's stream).
        unsafe { sys::x0ne_arena_free(self.0) };
    }
}

pub struct Building {
    raw: Raw,
}

pub struct Frozen<B: Backing> {
    raw: Raw,
    regions: Vec<Region>,
    mem: B,
    /// Keeps the device handle (stream and context) alive while the arena's memory is.
    _device: Option<Arc<Handle>>,
}

pub struct Arena<S> {
    state: S,
}

// As the reference's: an arena moves between threads with its engine.
unsafe impl Send for Building {}
unsafe impl<B: Backing + Send> Send for Frozen<B> {}

impl Default for Arena<Building> {
    fn default() -> Self {
        Self::new()
    }
}

fn regions_of(a: *const sys::x0ne_arena) -> Vec<Region> {
    // SAFETY: a live arena handle.
    let n = unsafe { sys::x0ne_arena_region_count(a) };
    (0..n)
        .filter_map(|i| {
            let mut label = vec![0u8; 256];
            let (mut cls, mut offset, mut len) = (0u32, 0u64, 0u64);
            // SAFETY: the label buffer is writable for its length; the rest are live locals.
            let st = unsafe {
                sys::x0ne_arena_region(a, i, label.as_mut_ptr().cast(), label.len(), &mut cls, &mut offset, &mut len)
            };
            if st != sys::X0NE_OK {
                return None;
            }
            let end = label.iter().position(|&b| b == 0).unwrap_or(label.len());
            Some(Region {
                label: String::from_utf8_lossy(&label[..end]).into_owned(),
                class: if cls == sys::X0NE_CLASS_CLIENT_DATA { Class::ClientData } else { Class::Weights },
                offset,
                len,
            })
        })
        .collect()
}

impl Arena<Building> {
    /// A Building arena (arena.rs:163-172). Panics only if the library cannot allocate its
    /// bookkeeping (host memory).
    pub fn new() -> Self {
        let mut a = std::ptr::null_mut();
        // SAFETY: `a` is a live local; freed by `Raw::drop`.
        let st = unsafe { sys::x0ne_arena_new(&mut a) };
        assert!(st == sys::X0NE_OK && !a.is_null(), "x0ne_arena_new failed");
        Arena { state: Building { raw: Raw(a) } }
    }

    /// Plans `len` bytes at the next multiple of ALIGN (arena.rs:174-198): an empty region or a
    /// size overflow is Error::Arena.
    pub fn alloc(&mut self, label: &str, len: u64, class: Class) -> Result<Slice> {
        let c = CString::new(label).map_err(|_| Error::Arena(format!("{label:?}: label holds a NUL")))?;
        let mut s = sys::x0ne_slice::default();
        // SAFETY: a live building arena; `c` outlives the call; `s` is a live local.
        check(unsafe { sys::x0ne_arena_alloc(self.state.raw.0, c.as_ptr(), len, class.raw(), &mut s) })?;
        Ok(Slice(s))
    }

    /// Bytes the single allocation will take.
    pub fn planned_bytes(&self) -> u64 {
        // SAFETY: a live arena handle.
        unsafe { sys::x0ne_arena_planned_bytes(self.state.raw.0) }
    }

    pub fn regions(&self) -> Vec<Region> {
        regions_of(self.state.raw.0)
    }

    /// Makes the one allocation (arena.rs:210-225): `allocate(size)` names the memory (a
    /// `Gpu::allocate` backing or `HostBacking::allocate`), the library allocates it. Consumes
    /// the builder: nothing can be added afterwards.
    pub fn freeze<B: Backing>(self, allocate: impl FnOnce(u64) -> Result<B>) -> Result<Arena<Frozen<B>>> {
        let size = self.planned_bytes();
        let mem = allocate(size.max(1))?;
        if mem.len() < size {
            return Err(Error::Arena(format!("backing gave {} bytes for {size}", mem.len())));
        }
        let raw = self.state.raw;
        let device = private::Sealed::device(&mem);
        let g = device.as_ref().map_or(std::ptr::null_mut(), |h| h.0);
        // SAFETY: a live building arena; `g` is null or a live device handle that the frozen
        // arena keeps alive (`_device`) as long as its memory.
        check(unsafe { sys::x0ne_arena_freeze(raw.0, g) })?;
        let regions = regions_of(raw.0);
        Ok(Arena { state: Frozen { raw, regions, mem, _device: device } })
    }
}

impl<B: Backing> Arena<Frozen<B>> {
    /// Writes `data` at byte `at` of slice `s` (arena.rs:242-245), checked against the slice and
    /// the arena (Error::Arena); a device arena copies synchronously on its device's stream.
    pub fn write(&mut self, s: Slice, at: u64, data: &[u8]) -> Result<()> {
        // SAFETY: a live frozen arena; `data` is readable for its length.
        check(unsafe { sys::x0ne_arena_write(self.state.raw.0, s.0, at, data.as_ptr().cast(), data.len() as u64) })
    }

    pub fn read(&self, s: Slice, at: u64, out: &mut [u8]) -> Result<()> {
        // SAFETY: a live frozen arena; `out` is writable for its length.
        check(unsafe { sys::x0ne_arena_read(self.state.raw.0, s.0, at, out.as_mut_ptr().cast(), out.len() as u64) })
    }

    /// Zeroes every `ClientData` region; returns the bytes zeroed. Weights are untouched
    /// (arena.rs:253-265).
    pub fn scrub_client_data(&mut self) -> Result<u64> {
        let mut zeroed = 0u64;
        // SAFETY: a live frozen arena; `zeroed` is a live local.
        check(unsafe { sys::x0ne_arena_scrub(self.state.raw.0, &mut zeroed) })?;
        Ok(zeroed)
    }

    pub fn regions(&self) -> &[Region] {
        &self.state.regions
    }

    pub fn backing(&self) -> &B {
        &self.state.mem
    }
}

impl<B: DeviceAddressed> Arena<Frozen<B>> {
    /// Address of byte `at` of slice `s`, checked against the slice (arena.rs:276-288).
    pub fn addr(&self, s: Slice, at: u64) -> Result<u64> {
        let mut out = 0u64;
        // SAFETY: a live frozen arena; `out` is a live local.
        check(unsafe { sys::x0ne_arena_addr(self.state.raw.0, s.0, at, &mut out) })?;
        Ok(out)
    }

    /// Address of slice `s`.
    pub fn ptr(&self, s: Slice) -> Result<u64> {
        self.addr(s, 0)
    }

    /// Address of the `len` bytes at byte `at` of slice `s`, all of them inside it
    /// (arena.rs:295-303).
    pub fn span(&self, s: Slice, at: u64, len: u64) -> Result<u64> {
        let mut out = 0u64;
        // SAFETY: a live frozen arena; `out` is a live local.
        check(unsafe { sys::x0ne_arena_span(self.state.raw.0, s.0, at, len, &mut out) })?;
        Ok(out)
    }
}
