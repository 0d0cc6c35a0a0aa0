//! The kernel-launch API of x0ne-core/runtime/src/gpu.rs over libx0ne_core.so: `Gpu::{new, launch,
//! gemm, capture, launch_graph, split_plan, allocate, counts, mem_info, sync}`, `Arg`,
//! `check_args` and the `launch!` macro, with the reference's names, argument meanings and
//! errors. The kernels are this library's gfx950 code; its table (x0ne_kernel_name,
//! x0ne_kernel_params) stands for `x0ne_core_kernels::{KERNEL_NAMES, KERNEL_PARAMS}`, and every
//! launch is checked against it before the device sees it.
use std::ffi::{c_char, CStr, CString};
use std::sync::atomic::{AtomicU64, Ordering};
use std::sync::{Arc, OnceLock};

use crate::error::check;
use crate::{sys, Error, Result};

/// The C type of a kernel parameter (`x0ne_core_kernels::Param`, kernels/src/lib.rs).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Param {
    Ptr,
    U32,
    F32,
}

impl Param {
    /// Bytes of the parameter in a launch's argument buffer.
    pub fn size(&self) -> usize {
        match self {
            Param::Ptr => 8,
            Param::U32 | Param::F32 => 4,
        }
    }

    fn from_raw(v: u32) -> Option<Param> {
        match v {
            sys::X0NE_PARAM_PTR => Some(Param::Ptr),
            sys::X0NE_PARAM_U32 => Some(Param::U32),
            sys::X0NE_PARAM_F32 => Some(Param::F32),
            _ => None,
        }
    }
}

/// One kernel argument, by the C type of its parameter (gpu.rs:281-314).
#[derive(Debug, Clone, Copy, PartialEq)]
pub enum Arg {
    Ptr(u64),
    U32(u32),
    F32(f32),
}

impl Arg {
    pub fn param(&self) -> Param {
        match self {
            Arg::Ptr(_) => Param::Ptr,
            Arg::U32(_) => Param::U32,
            Arg::F32(_) => Param::F32,
        }
    }

    fn raw(&self) -> sys::x0ne_arg {
        let mut a = sys::x0ne_arg::default();
        match *self {
            Arg::Ptr(v) => {
                a.kind = sys::X0NE_PARAM_PTR;
                a.ptr = v;
            }
            Arg::U32(v) => {
                a.kind = sys::X0NE_PARAM_U32;
                a.u32 = v;
            }
            Arg::F32(v) => {
                a.kind = sys::X0NE_PARAM_F32;
                a.f32 = v;
            }
        }
        a
    }
}

/// A device address.
impl From<u64> for Arg {
    fn from(v: u64) -> Self {
        Arg::Ptr(v)
    }
}

impl From<u32> for Arg {
    fn from(v: u32) -> Self {
        Arg::U32(v)
    }
}

impl From<f32> for Arg {
    fn from(v: f32) -> Self {
        Arg::F32(v)
    }
}

/// `args` against the declared parameters of kernel `name`: as many, each of the same C type
/// (gpu.rs:317-333, the same messages).
pub fn check_args(name: &str, params: &[Param], args: &[Arg]) -> Result<()> {
    if args.len() != params.len() {
        return Err(Error::Gpu(format!("{name}: {} arguments for {} parameters", args.len(), params.len())));
    }
    match args.iter().zip(params).position(|(a, p)| a.param() != *p) {
        Some(i) => Err(Error::Gpu(format!(
            "{name}: argument {i} is {:?}, the kernel takes {:?}",
            args[i].param(),
            params[i]
        ))),
        None => Ok(()),
    }
}

/// Most parameters a launch passes (the table's kernels take 20 at most).
const MAX_ARGS: usize = 24;

struct Entry {
    c: &'static CStr,
    name: &'static str,
    params: Vec<Param>,
}

/// The library's kernel table, read once: its names are static strings of the loaded library.
fn table() -> &'static [Entry] {
    static TABLE: OnceLock<Vec<Entry>> = OnceLock::new();
    TABLE.get_or_init(|| {
        // SAFETY: the count and the names are the library's static table.
        let n = unsafe { sys::x0ne_kernel_count() };
        (0..n)
            .filter_map(|i| {
                // SAFETY: i is below the count; the pointer is a static NUL-terminated name.
                let p: *const c_char = unsafe { sys::x0ne_kernel_name(i) };
                if p.is_null() {
                    return None;
                }
                // SAFETY: a NUL-terminated string that lives as long as the library (the process).
                let c: &'static CStr = unsafe { CStr::from_ptr(p) };
                let name = c.to_str().ok()?;
                let mut raw = [0u32; MAX_ARGS];
                // SAFETY: `raw` is writable for its length.
                let k = unsafe { sys::x0ne_kernel_params(p, raw.as_mut_ptr(), raw.len()) };
                if k > raw.len() {
                    return None;
                }
                let params = raw[..k].iter().map(|&v| Param::from_raw(v)).collect::<Option<Vec<_>>>()?;
                Some(Entry { c, name, params })
            })
            .collect()
    })
}

/// The kernels of the table, by name (KERNEL_NAMES).
pub fn kernel_names() -> Vec<&'static str> {
    table().iter().map(|e| e.name).collect()
}

/// The declared parameters of kernel `name` (params_of, kernels/src/lib.rs:146-151).
pub fn params_of(name: &str) -> Option<&'static [Param]> {
    table().iter().find(|e| e.name == name).map(|e| e.params.as_slice())
}

/// A kernel of the table, with its declared parameters and the id of the `Gpu` that resolved it
/// (`Gpu::launch` refuses it on any other, gpu.rs:1038-1043).
#[derive(Clone, Copy)]
pub struct Kernel {
    entry: usize,
    gpu: u64,
}

impl Kernel {
    pub fn name(&self) -> &'static str {
        table()[self.entry].name
    }
    pub fn params(&self) -> &'static [Param] {
        table()[self.entry].params.as_slice()
    }
}

/// How the split-K decode attention is launched for one geometry (gpu.rs:258-276).
#[derive(Clone, Copy)]
pub struct SplitPlan {
    pub kernel: Kernel,
    /// Blocks along x: kv heads when a block serves a GQA group, else q heads.
    pub grid_x: u32,
    /// q heads served by one block (1 for the per-q-head kernel).
    pub group: u32,
    /// A grouped kernel: it takes a counter and an output and can merge in its last block.
    pub grouped: bool,
    /// Blocks of the kernel one compute unit holds at once (the reference's per SM).
    pub per_sm: u32,
    /// P, blocks along y: the slices of the context.
    pub splits: u32,
}

/// Driver-call tallies (gpu.rs:733-741).
#[derive(Debug, Clone, Copy, PartialEq, Eq, Default)]
pub struct Counts {
    pub kernel_launches: u64,
    pub graph_launches: u64,
    pub gemms: u64,
    pub htod: u64,
    pub dtoh: u64,
    pub memsets: u64,
    pub syncs: u64,
}

impl From<sys::x0ne_counts> for Counts {
    fn from(c: sys::x0ne_counts) -> Self {
        Counts {
            kernel_launches: c.launches,
            graph_launches: c.graph_launches,
            gemms: c.gemms,
            htod: c.htod,
            dtoh: c.dtoh,
            memsets: c.memsets,
            syncs: c.syncs,
        }
    }
}

/// Output element type of a GEMM.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Out {
    Bf16,
    F32,
}

/// The library's device handle, shared by the `Gpu`, its graphs and its arenas' backings, so it
/// is freed after the last of them (the reference's `Arc<Core>`, gpu.rs:85-160).
#[doc(hidden)]
pub struct Handle(pub(crate) *mut sys::x0ne_gpu);

// SAFETY: as the reference's Core (gpu.rs:111-114): the handle's calls bind the device first and
// the owners serialise their use.
unsafe impl Send for Handle {}
unsafe impl Sync for Handle {}

impl Drop for Handle {
    fn drop(&mut self) {
        // SAFETY: freed once, here, after every owner is gone; the library drains the stream first.
        unsafe { sys::x0ne_gpu_free(self.0) };
    }
}

/// A captured launch sequence, instantiated once, replayed with `Gpu::launch_graph`.
pub struct Graph {
    h: *mut sys::x0ne_graph,
    _gpu: Arc<Handle>,
}

// SAFETY: the graph is an immutable handle replayed under the owning Gpu, as the reference's.
unsafe impl Send for Graph {}

impl Graph {
    pub fn nodes(&self) -> usize {
        // SAFETY: a live graph of this wrapper.
        unsafe { sys::x0ne_graph_nodes(self.h) }
    }
}

impl Drop for Graph {
    fn drop(&mut self) {
        // SAFETY: destroyed once, here.
        unsafe { sys::x0ne_graph_free(self.h) };
    }
}

/// The single device allocation an arena asks for (`Gpu::allocate`); the allocation itself is
/// made by the arena's freeze on this device (x0ne_arena_freeze), which owns and frees it. It
/// keeps the device handle alive as long as the arena.
pub struct DeviceBacking {
    pub(crate) gpu: Arc<Handle>,
    pub(crate) len: u64,
}

pub struct Gpu {
    /// Unique in the process, never reused: a Kernel carries it.
    id: u64,
    h: Arc<Handle>,
    /// Architecture and compute units (the reference's `arch` and `sms`).
    pub arch: &'static str,
    pub sms: u32,
    /// The library's description: name, architecture, CUs, driver and runtime versions.
    pub name: String,
}

// As the reference's (gpu.rs:768): Send, not Sync; callers serialise through a Mutex.
unsafe impl Send for Gpu {}

static NEXT_GPU: AtomicU64 = AtomicU64::new(1);

fn name_c(name: &str) -> Result<CString> {
    CString::new(name).map_err(|_| Error::Gpu(format!("kernel name {name:?}")))
}

impl Gpu {
    /// GPU 0 with one stream at the default priority and the kernel table checked against the
    /// loaded code object (gpu.rs:799-928). Error::Gpu without a usable gfx950 device.
    pub fn new() -> Result<Gpu> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: `raw` is a live local; freed by `Handle::drop`.
        check(unsafe { sys::x0ne_gpu_new(&mut raw) })?;
        let h = Arc::new(Handle(raw));
        let mut buf = vec![0u8; 512];
        // SAFETY: the buffer is writable for its length.
        check(unsafe { sys::x0ne_gpu_describe(raw, buf.as_mut_ptr().cast(), buf.len()) })?;
        let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
        Ok(Gpu {
            id: NEXT_GPU.fetch_add(1, Ordering::Relaxed),
            // SAFETY: a live device handle.
            sms: unsafe { sys::x0ne_gpu_compute_units(raw) },
            h,
            arch: "gfx950",
            name: String::from_utf8_lossy(&buf[..end]).into_owned(),
        })
    }

    /// Kernel `name` of the table, for this Gpu's launches.
    pub fn kernel(&self, name: &str) -> Result<Kernel> {
        match table().iter().position(|e| e.name == name) {
            Some(entry) => Ok(Kernel { entry, gpu: self.id }),
            None => Err(Error::Gpu(format!("no kernel {name}"))),
        }
    }

    /// The split-K decode attention for a geometry (gpu.rs:958-985): a block serves the q heads
    /// of one kv head when the group size has a grouped kernel (1, 2, 4, 8), else one q head; P
    /// is one wave of that kernel over the device's compute units.
    pub fn split_plan(&self, q_heads: usize, kv_heads: usize) -> Result<SplitPlan> {
        let u = |v: usize| u32::try_from(v).map_err(|_| Error::Gpu("head count exceeds u32".into()));
        let mut p = sys::x0ne_split_plan::default();
        // SAFETY: a live device handle; `p` is a live local.
        check(unsafe { sys::x0ne_gpu_split_plan(self.h.0, u(q_heads)?, u(kv_heads)?, &mut p) })?;
        let kernel = if p.grouped != 0 {
            self.kernel(&format!("x0ne_attention_decode_split_g{}_bf16", p.group))?
        } else {
            self.kernel("x0ne_attention_decode_split_bf16")?
        };
        Ok(SplitPlan {
            kernel,
            grid_x: p.grid_x,
            group: p.group,
            grouped: p.grouped != 0,
            per_sm: p.per_cu,
            splits: p.splits,
        })
    }

    /// The single device allocation of an arena (`Arena::freeze`): `len` bytes on this device.
    pub fn allocate(&self, len: u64) -> Result<DeviceBacking> {
        Ok(DeviceBacking { gpu: self.h.clone(), len })
    }

    /// Launches `k` on the stream with `args`, one per parameter. Refused before the device sees
    /// them: a kernel of another `Gpu`, and arguments that differ from the kernel's declared
    /// parameters in number or C type (`check_args`; the library checks them again).
    ///
    /// # Safety
    ///
    /// Every pointer argument is a device address of this device, valid for every byte the
    /// kernel reads or writes at this grid with these sizes, until the launch is done on the
    /// stream.
    pub unsafe fn launch(&self, k: Kernel, grid: (u32, u32), block: u32, args: &[Arg]) -> Result<()> {
        if k.gpu != self.id {
            return Err(Error::Gpu(format!("{}: a kernel of Gpu {}, launched by Gpu {}", k.name(), k.gpu, self.id)));
        }
        check_args(k.name(), k.params(), args)?;
        if args.len() > MAX_ARGS {
            return Err(Error::Gpu(format!("{}: {} arguments, at most {MAX_ARGS}", k.name(), args.len())));
        }
        let raw: Vec<sys::x0ne_arg> = args.iter().map(Arg::raw).collect();
        // SAFETY: a live device handle, a static kernel name, `raw` outlives the call; the device
        // addresses are the caller's contract.
        check(unsafe {
            sys::x0ne_gpu_launch(self.h.0, table()[k.entry].c.as_ptr(), grid.0, grid.1, block, raw.as_ptr(), raw.len())
        })
    }

    /// `Y[n][rows] = X[n][cols] W^T` with `W [rows][cols]`, all row-major, bf16 in, f32
    /// accumulation (gpu.rs:1098-1149): one row is the bandwidth-bound GEMV, a few rows the
    /// few-row matrix-core GEMM, more the tiled matrix-core GEMM, all this library's kernels.
    ///
    /// # Safety
    ///
    /// `w`, `x` and `y` are device addresses of this device holding `rows * cols` bf16,
    /// `n * cols` bf16 and `n * rows` values of `out`; `y` overlaps neither `w` nor `x`; all three
    /// stay allocated until the GEMM is done on the stream.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn gemm(&self, w: u64, rows: usize, cols: usize, x: u64, n: usize, y: u64, out: Out) -> Result<()> {
        let f32_out = match out {
            Out::Bf16 => 0,
            Out::F32 => 1,
        };
        // SAFETY: a live device handle; the three matrices are the caller's contract.
        check(unsafe { sys::x0ne_gpu_gemv(self.h.0, w, rows as u64, cols as u64, x, n as u64, y, f32_out) })
    }

    /// Captures every launch `f` issues on the stream into one graph and instantiates it
    /// (gpu.rs:1170-1223). Mode GLOBAL: an allocation, a synchronization or a host copy inside
    /// `f` fails the capture. The capture is ended whether `f` succeeds or not.
    pub fn capture(&self, f: impl FnOnce() -> Result<()>) -> Result<Graph> {
        // SAFETY: a live device handle.
        check(unsafe { sys::x0ne_gpu_capture_begin(self.h.0) })?;
        let body = f();
        let mut g = std::ptr::null_mut();
        // SAFETY: ends the capture begun above; `g` is a live local.
        let ended = check(unsafe { sys::x0ne_gpu_capture_end(self.h.0, &mut g) });
        let graph = if g.is_null() { None } else { Some(Graph { h: g, _gpu: self.h.clone() }) };
        body?;
        ended?;
        graph.ok_or_else(|| Error::Gpu("the capture made no graph".into()))
    }

    /// Replays a captured graph on the stream. A graph of another `Gpu` is refused.
    ///
    /// # Safety
    ///
    /// Every device range the captured launches use is still allocated, as their contract
    /// required at capture, until the replay is done on the stream.
    pub unsafe fn launch_graph(&self, g: &Graph) -> Result<()> {
        // SAFETY: live handles; the library refuses a graph another device handle captured.
        check(unsafe { sys::x0ne_gpu_launch_graph(self.h.0, g.h) })
    }

    pub fn sync(&self) -> Result<()> {
        // SAFETY: a live device handle.
        check(unsafe { sys::x0ne_gpu_sync(self.h.0) })
    }

    /// Driver calls made through this device handle so far.
    pub fn counts(&self) -> Counts {
        let mut c = sys::x0ne_counts::default();
        // SAFETY: a live device handle; `c` is a live local.
        let _ = unsafe { sys::x0ne_gpu_counts(self.h.0, &mut c) };
        c.into()
    }

    /// (free, total) device bytes.
    pub fn mem_info(&self) -> Result<(u64, u64)> {
        let (mut free, mut total) = (0u64, 0u64);
        // SAFETY: a live device handle; two live locals.
        check(unsafe { sys::x0ne_gpu_mem_info(self.h.0, &mut free, &mut total) })?;
        Ok((free, total))
    }
}

/// `Gpu::launch` with the arguments as Rust values: u64 for a device address, u32, f32 (any
/// other type does not compile). It calls `Gpu::launch`, so it is used inside `unsafe` under the
/// same contract (gpu.rs:1383-1387).
#[macro_export]
macro_rules! launch {
    ($gpu:expr, $k:expr, $grid:expr, $block:expr; $($arg:expr),* $(,)?) => {
        $gpu.launch($k, $grid, $block, &[$($crate::gpu::Arg::from($arg)),*])
    };
}
