"""The kernel surface the parity tests call (x0ne-core/runtime/src/ops.rs, `Kernels`): each entry
point plans an arena for its inputs and outputs, freezes it (the one allocation), uploads, runs
one kernel on GPU 0 and reads the result back.

Values are numpy arrays: bf16 as uint16 bit patterns, f32 as float32, ids as uint32. K and V
are given in the reference's logical layout [position][kv_heads][128] and scattered into the
paged layout [pages][kv_heads][16][128] by `page_of` (logical page -> physical page; identity
when None); slots past ctx hold a NaN pattern, so a kernel that reads one shows it."""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from ._lib import FormatError, GpuError
from .arena import Arena, Class
from .gpu import Arg, Gpu, SplitPlan, split_state_bytes

HEAD_DIM = 128
PAGE = 16
SPLIT_STATE = HEAD_DIM + 4
PREFILL_COLS = 128  # columns (row, q head) per block of x0ne_attention_prefill_g*_bf16
PREFILL_THREADS = 256  # its block
PREFILL_EXACT_COLS = 64  # columns per block of x0ne_attention_prefill_exact_g*_bf16
PREFILL_EXACT_THREADS = 256  # its block
NAN_BF16 = 0x7FC0


@dataclass(frozen=True)
class Heads:
    q_heads: int
    kv_heads: int
    head_dim: int = HEAD_DIM

    @property
    def q_dim(self):
        return self.q_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    def check(self):
        """ops.rs:32-47: head_dim 128, q_heads a multiple of kv_heads."""
        if self.head_dim != HEAD_DIM:
            raise FormatError(f"head_dim {self.head_dim} (kernels are built for {HEAD_DIM})")
        if self.kv_heads == 0 or self.q_heads % self.kv_heads:
            raise FormatError(f"{self.q_heads} q heads for {self.kv_heads} kv heads")


@dataclass(frozen=True)
class CacheAt:
    """Where the KV write lands (ops.rs:130-136): layer `layer` of `layers`, position `pos`."""
    layers: int
    max_ctx: int
    layer: int
    pos: int


@dataclass
class QkvOut:
    q: np.ndarray
    k_row: np.ndarray
    v_row: np.ndarray
    rest_untouched: bool


def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """1 / theta^(2i / d) in f32 (ops.rs:210-214), as the host computes it for the device."""
    t = np.float32(theta)
    return np.array([np.float32(1.0) / np.float32(t ** (np.float32(2 * i) / np.float32(head_dim)))
                     for i in range(head_dim // 2)], np.float32)


def attn_scale(head_dim: int) -> float:
    """ops.rs:217-219"""
    return float(np.float32(1.0 / math.sqrt(head_dim)))


def n_pages(ctx: int) -> int:
    return (ctx + PAGE - 1) // PAGE


def to_pages(rows: np.ndarray, kv_heads: int, page_of, pool: int, fill=NAN_BF16, dim_major=False) -> np.ndarray:
    """[ctx][kv_heads * 128] bf16 -> K pages [pool][kv_heads][16][128], or V pages
    [pool][kv_heads][128][16] when dim_major; row p at page page_of[p // 16], slot p % 16."""
    ctx = rows.shape[0] if rows.ndim == 2 else rows.size // (kv_heads * HEAD_DIM)
    rows = rows.reshape(ctx, kv_heads, HEAD_DIM)
    out = np.full((pool, kv_heads, PAGE, HEAD_DIM), fill, np.uint16)
    for p in range(ctx):
        out[page_of[p // PAGE], :, p % PAGE, :] = rows[p]
    return np.ascontiguousarray(out.transpose(0, 1, 3, 2)) if dim_major else out


def to_panels(m) -> np.ndarray:
    """[n][cols] (cols a multiple of 8) -> the panel layout of the batched step (ceil(n / 16)
    panels of [cols / 8][16][8], rows past n zero), flattened."""
    m = np.asarray(m)
    n, cols = m.shape
    tiles = -(-n // 16)
    full = np.zeros((tiles * 16, cols), m.dtype)
    full[:n] = m
    return np.ascontiguousarray(full.reshape(tiles, 16, cols // 8, 8).transpose(0, 2, 1, 3)).reshape(-1)


def from_panels(flat, n: int, cols: int) -> np.ndarray:
    """The inverse of to_panels: rows 0 .. n - 1 of [n][cols]."""
    tiles = -(-n // 16)
    p = np.asarray(flat)[:tiles * 16 * cols].reshape(tiles, cols // 8, 16, 8).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(p.reshape(tiles * 16, cols)[:n])


def v_offset(page: int, kv_heads: int, kh: int, slot: int, dim: int) -> int:
    """Element index of (slot, dim) of kv head kh in V page `page` (dim-major pages)."""
    return ((page * kv_heads + kh) * HEAD_DIM + dim) * PAGE + slot


class Kernels:
    """GPU 0 with this library's kernels (ops.rs:229-238)."""

    def __init__(self, gpu: Gpu | None = None):
        self.gpu = gpu or Gpu()

    def _arena(self):
        return Arena()

    def _freeze(self, a: Arena) -> Arena:
        return a.freeze(self.gpu)

    # -- embedding (ops.rs:240-270) --
    def embedding(self, table: np.ndarray, hidden: int, token: int) -> np.ndarray:
        if hidden == 0 or hidden % 8 or table.size % hidden:
            raise FormatError(f"embedding: hidden {hidden}, table of {table.size}")
        vocab = table.size // hidden
        a = self._arena()
        t = a.alloc("table", table.size * 2, Class.WEIGHTS)
        tok = a.alloc("token", 4, Class.CLIENT_DATA)
        out = a.alloc("out", hidden * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(t, 0, table.astype(np.uint16))
        a.write(tok, 0, np.array([token & 0xFFFFFFFF], np.uint32))
        self.gpu.launch("x0ne_embedding_bf16", 1, 128,
                        [Arg.ptr(a.ptr(t)), Arg.ptr(a.ptr(tok)), Arg.ptr(a.ptr(out)), Arg.u32(hidden), Arg.u32(vocab)])
        self.gpu.sync()
        return a.read_array(out, 0, hidden, np.uint16)

    # -- add_rmsnorm (ops.rs:272-300) --
    def add_rmsnorm_panel(self, residual, x, w, eps: float):
        """The batched step's norm over rows ([n][h] residual f32 and x bf16 bits, one launch):
        (residual after, out [n][h] read back from its panels)."""
        residual = np.ascontiguousarray(residual, np.float32)
        n, h = residual.shape
        tiles = -(-n // 16)
        a = self._arena()
        r = a.alloc("residual", residual.nbytes, Class.CLIENT_DATA)
        xs = a.alloc("x", n * h * 2, Class.CLIENT_DATA)
        ws = a.alloc("w", h * 2, Class.WEIGHTS)
        out = a.alloc("out", tiles * 16 * h * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        a.write(r, 0, residual)
        a.write(xs, 0, np.asarray(x, np.uint16))
        a.write(ws, 0, np.asarray(w, np.uint16))
        self.gpu.launch("x0ne_add_rmsnorm_panel_bf16", n, 256,
                        [Arg.ptr(a.ptr(r)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(out)), Arg.u32(h),
                         Arg.f32(eps)])
        self.gpu.sync()
        return (a.read_array(r, 0, n * h, np.float32).reshape(n, h),
                from_panels(a.read_array(out, 0, tiles * 16 * h, np.uint16), n, h))

    def add_rmsnorm(self, residual, x, w, eps: float):
        residual = np.ascontiguousarray(residual, np.float32)
        h = residual.size
        if h == 0 or x.size != h or w.size != h:
            raise FormatError("add_rmsnorm: lengths differ")
        a = self._arena()
        r = a.alloc("residual", h * 4, Class.CLIENT_DATA)
        xs = a.alloc("x", h * 2, Class.CLIENT_DATA)
        ws = a.alloc("w", h * 2, Class.WEIGHTS)
        out = a.alloc("out", h * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(r, 0, residual)
        a.write(xs, 0, x.astype(np.uint16))
        a.write(ws, 0, w.astype(np.uint16))
        self.gpu.launch("x0ne_add_rmsnorm_bf16", 1, 256,
                        [Arg.ptr(a.ptr(r)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(out)), Arg.u32(h),
                         Arg.f32(eps)])
        self.gpu.sync()
        return a.read_array(r, 0, h, np.float32), a.read_array(out, 0, h, np.uint16)

    # -- qk_norm_rope_kv_write (ops.rs:302-384), paged --
    def qk_norm_rope_kv_write(self, qkv, q_norm, k_norm, heads: Heads, theta: float, eps: float, at: CacheAt,
                              page_of=None, pool=None, table: bool = False) -> QkvOut:
        """table: the prefill pass's kernel (x0ne_qk_norm_rope_kv_write_rows_bf16), reading cos and
        sin from the RoPE table (filled here for max_ctx positions) instead of computing them."""
        heads.check()
        hd, qd, kvd = heads.head_dim, heads.q_dim, heads.kv_dim
        if qkv.size != qd + 2 * kvd or q_norm.size != hd or k_norm.size != hd:
            raise FormatError("qk_norm_rope_kv_write: lengths")
        if at.layer >= at.layers or at.pos >= at.max_ctx:
            raise FormatError(f"qk_norm_rope_kv_write: {at} out of range")
        SENTINEL = 0xA5
        pages = n_pages(at.max_ctx)
        page_of = list(range(pages)) if page_of is None else list(page_of)
        pool = pool or pages
        plane = pool * heads.kv_heads * PAGE * HEAD_DIM * 2
        cache_bytes = at.layers * 2 * plane
        a = self._arena()
        x = a.alloc("qkv", qkv.size * 2, Class.CLIENT_DATA)
        qn = a.alloc("q_norm", hd * 2, Class.WEIGHTS)
        kn = a.alloc("k_norm", hd * 2, Class.WEIGHTS)
        inv = a.alloc("inv_freq", hd // 2 * 4, Class.WEIGHTS)
        pt = a.alloc("page_table", len(page_of) * 4, Class.WEIGHTS)
        q = a.alloc("q", qd * 2, Class.CLIENT_DATA)
        cache = a.alloc("cache", cache_bytes, Class.CLIENT_DATA)
        pos = a.alloc("pos", 4, Class.CLIENT_DATA)
        cs = a.alloc("rope_cs", at.max_ctx * (hd // 2) * 16, Class.CLIENT_DATA) if table else None
        self._freeze(a)
        a.write(x, 0, qkv.astype(np.uint16))
        a.write(qn, 0, q_norm.astype(np.uint16))
        a.write(kn, 0, k_norm.astype(np.uint16))
        a.write(inv, 0, inv_freq(hd, theta))
        if table:
            self._rope_table(a.ptr(inv), a.ptr(cs), at.max_ctx, hd)
        a.write(pt, 0, np.array(page_of, np.uint32))
        a.write(cache, 0, np.full(cache_bytes, SENTINEL, np.uint8))
        a.write(pos, 0, np.array([at.pos], np.uint32))
        k_off = at.layer * 2 * plane
        v_off = k_off + plane
        name, grid, block = (("x0ne_qk_norm_rope_kv_write_rows_bf16", (heads.q_heads + heads.kv_heads + 3) // 4, 256)
                             if table else ("x0ne_qk_norm_rope_kv_write_bf16", heads.q_heads + heads.kv_heads, 64))
        self.gpu.launch(name, grid, block,
                        [Arg.ptr(a.ptr(x)), Arg.ptr(a.ptr(qn)), Arg.ptr(a.ptr(kn)), Arg.ptr(a.ptr(cs if table else inv)),
                         Arg.ptr(a.ptr(q)), Arg.ptr(a.addr(cache, k_off)), Arg.ptr(a.addr(cache, v_off)),
                         Arg.ptr(a.ptr(pt)), Arg.ptr(a.ptr(pos)), Arg.u32(heads.q_heads), Arg.u32(heads.kv_heads),
                         Arg.u32(at.max_ctx), Arg.f32(eps)])
        self.gpu.sync()
        q_out = a.read_array(q, 0, qd, np.uint16)
        allb = np.frombuffer(a.read(cache, 0, cache_bytes), np.uint8)
        page = page_of[at.pos // PAGE]
        written = np.zeros(cache_bytes, bool)
        k_rows, v_rows = [], []
        for kh in range(heads.kv_heads):
            s = k_off + ((page * heads.kv_heads + kh) * PAGE + at.pos % PAGE) * HEAD_DIM * 2
            written[s:s + HEAD_DIM * 2] = True
            k_rows.append(allb[s:s + HEAD_DIM * 2].view(np.uint16))
            # V pages are dim-major: the row is 128 elements 16 apart.
            idx = np.array([v_offset(page, heads.kv_heads, kh, at.pos % PAGE, d) for d in range(HEAD_DIM)])
            for b in (0, 1):
                written[v_off + 2 * idx + b] = True
            v_rows.append(allb.view(np.uint16)[(v_off // 2) + idx].copy())
        rest = bool(np.all(allb[~written] == SENTINEL))
        return QkvOut(q_out, np.concatenate(k_rows), np.concatenate(v_rows), rest)

    # -- gemv (ops.rs:386-451, the cuBLAS call) --
    def _gemv(self, w, rows, cols, x, out_f32):
        if rows == 0 or cols == 0 or w.size != rows * cols or x.size != cols:
            raise FormatError(f"gemv: W {w.size} for {rows}x{cols}, x {x.size}")
        ob = 4 if out_f32 else 2
        a = self._arena()
        ws = a.alloc("w", w.size * 2, Class.WEIGHTS)
        xs = a.alloc("x", cols * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", rows * ob, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ws, 0, w.astype(np.uint16))
        a.write(xs, 0, x.astype(np.uint16))
        self.gpu.gemv(a.ptr(ws), rows, cols, a.ptr(xs), 1, a.ptr(ys), out_f32)
        self.gpu.sync()
        return a.read_array(ys, 0, rows, np.float32 if out_f32 else np.uint16)

    # x0ne_gpu_gemm_tiled's block tiles (features x tokens) and operand layouts
    TILE_AUTO, TILE_256x256, TILE_256x128, TILE_128x128 = 0, 1, 2, 3
    W_PANELS, X_PANELS = 1, 2

    def gemm(self, w, rows, cols, x, n, out_f32, tile=None, layout=0) -> np.ndarray:
        """Gpu::gemm over n rows of X (gpu.rs:1098-1149): Y[n][rows] = X[n][cols] W^T, the
        few-row matrix-core kernel from 2 to 64 rows, the tiled matrix-core GEMM past them;
        tile names a block tile of the tiled GEMM (x0ne_gpu_gemm_tiled) at any row count, and
        layout asks it to read W and/or X in 16-row panels (uploaded as such from the row-major
        arguments); returns Y (f32, or bf16 bits)."""
        if rows == 0 or cols == 0 or n == 0 or w.size != rows * cols or x.size != n * cols:
            raise FormatError(f"gemm: W {w.size} for {rows}x{cols}, X {x.size} for {n} rows")
        if layout and tile is None:
            raise FormatError("gemm: a panel layout needs the tiled GEMM (tile; 0 picks one)")
        ob = 4 if out_f32 else 2
        wv = np.asarray(w).astype(np.uint16)
        xv = np.asarray(x).astype(np.uint16)
        if layout & self.W_PANELS:
            wv = to_panels(wv.reshape(rows, cols))
        if layout & self.X_PANELS:
            xv = to_panels(xv.reshape(n, cols))
        a = self._arena()
        ws = a.alloc("w", wv.size * 2, Class.WEIGHTS)
        xs = a.alloc("x", xv.size * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", n * rows * ob, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ws, 0, wv)
        a.write(xs, 0, xv)
        if tile is None:
            self.gpu.gemv(a.ptr(ws), rows, cols, a.ptr(xs), n, a.ptr(ys), out_f32)
        else:
            self.gpu.gemm_tiled(tile, a.ptr(ws), rows, cols, a.ptr(xs), n, a.ptr(ys), out_f32, layout)
        self.gpu.sync()
        return a.read_array(ys, 0, n * rows, np.float32 if out_f32 else np.uint16).reshape(n, rows)

    # -- the fused decode GEMV instances (gemv.hip) --
    PRO_X, PRO_NORM, PRO_EMBED_NORM = 0, 1, 2
    EPI_BF16, EPI_F32, EPI_SWIGLU, EPI_ARGMAX = 0, 1, 2, 3

    def gemv_fused(self, w, rows: int, cols: int, prologue: int, epilogue: int, f64_sums: bool = False, x=None,
                   residual=None, delta=None, norm_w=None, embed=None, token: int = 0, vocab: int = 0,
                   eps: float = 1e-6, advance: bool = False, pos: int = 0) -> dict:
        """One launch of a decode GEMV with its fused prologue and epilogue (x0ne_gpu_gemv_fused),
        the instances the decode step runs: PRO_X takes x (bf16 bits); PRO_NORM takes the f32
        residual, delta and norm_w (bf16) and also returns the new residual; PRO_EMBED_NORM takes
        the embedding table ([vocab][cols] bf16), the token and norm_w. EPI_BF16 / EPI_F32 return
        y; EPI_SWIGLU returns the inter = rows / 2 activations; EPI_ARGMAX the f32 logits, the
        token, the position after (pos, advanced when asked) and the counter after (0)."""
        w = np.ascontiguousarray(w, np.uint16)
        if w.size != rows * cols:
            raise FormatError(f"gemv_fused: W {w.size} for {rows}x{cols}")
        out_rows = rows // 2 if epilogue == self.EPI_SWIGLU else rows
        ob = 4 if epilogue in (self.EPI_F32, self.EPI_ARGMAX) else 2
        a = self._arena()
        s = {"w": a.alloc("w", w.size * 2, Class.WEIGHTS), "y": a.alloc("y", out_rows * ob, Class.CLIENT_DATA)}
        if prologue == self.PRO_X:
            s["x"] = a.alloc("x", cols * 2, Class.CLIENT_DATA)
        if prologue in (self.PRO_NORM, self.PRO_EMBED_NORM):
            s["norm_w"] = a.alloc("norm_w", cols * 2, Class.WEIGHTS)
            s["res_out"] = a.alloc("res_out", cols * 4, Class.CLIENT_DATA)
        if prologue == self.PRO_NORM:
            s["res_in"] = a.alloc("res_in", cols * 4, Class.CLIENT_DATA)
            s["delta"] = a.alloc("delta", cols * 2, Class.CLIENT_DATA)
        if prologue == self.PRO_EMBED_NORM:
            s["embed"] = a.alloc("embed", vocab * cols * 2, Class.WEIGHTS)
            s["tokens"] = a.alloc("tokens", 4, Class.CLIENT_DATA)
        fields = dict(rows=rows, cols=cols, prologue=prologue, epilogue=epilogue, f64_sums=int(f64_sums),
                      vocab=vocab, eps=eps, advance=int(advance))
        blocks = 0
        if epilogue == self.EPI_ARGMAX:
            blocks = self.gpu.gemv_fused_blocks(w=16, y=16, x=16, res_in=16, delta=16, norm_w=16, embed=16,
                                                tokens=16, partial=16, counter=16, token_out=16, pos=16, **fields)
            if blocks == 0:
                raise FormatError("gemv_fused: instance refused")
            s["partial"] = a.alloc("partial", blocks * 12, Class.CLIENT_DATA)
            s["counter"] = a.alloc("counter", 4, Class.CLIENT_DATA)
            s["token_out"] = a.alloc("token_out", 4, Class.CLIENT_DATA)
            s["pos"] = a.alloc("pos", 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        a.write(s["w"], 0, w)
        if "x" in s:
            a.write(s["x"], 0, np.ascontiguousarray(x, np.uint16))
        if "norm_w" in s:
            a.write(s["norm_w"], 0, np.ascontiguousarray(norm_w, np.uint16))
        if "res_in" in s:
            a.write(s["res_in"], 0, np.ascontiguousarray(residual, np.float32))
            a.write(s["delta"], 0, np.ascontiguousarray(delta, np.uint16))
        if "embed" in s:
            a.write(s["embed"], 0, np.ascontiguousarray(embed, np.uint16))
            a.write(s["tokens"], 0, np.array([token], np.uint32))
        if "pos" in s:
            a.write(s["pos"], 0, np.array([pos], np.uint32))
        self.gpu.gemv_fused(**{k: a.ptr(v) for k, v in s.items()}, **fields)
        self.gpu.sync()
        out = {"y": a.read_array(s["y"], 0, out_rows, np.float32 if ob == 4 else np.uint16)}
        if "res_out" in s:
            out["residual"] = a.read_array(s["res_out"], 0, cols, np.float32)
        if epilogue == self.EPI_ARGMAX:
            out["token"] = int(a.read_array(s["token_out"], 0, 1, np.uint32)[0])
            out["pos"] = int(a.read_array(s["pos"], 0, 1, np.uint32)[0])
            out["counter"] = int(a.read_array(s["counter"], 0, 1, np.uint32)[0])
            out["blocks"] = blocks
        return out

    def gemv_f32_out(self, w, rows, cols, x) -> np.ndarray:
        return self._gemv(w, rows, cols, x, True)

    def gemv_bf16_out(self, w, rows, cols, x) -> np.ndarray:
        return self._gemv(w, rows, cols, x, False)

    # -- attention (ops.rs:453-681) --
    def probe_bf16_round(self, base: int, n: int, read: bool = False):
        """The device's bf16 rounding of the f32 values whose bits are base .. base + n - 1: how many
        differ from the rounding stated on the bits, and (read) the rounded bits."""
        if n == 0 or base + n > 1 << 32:
            raise FormatError("probe_bf16_round: range")
        a = self._arena()
        cnt = a.alloc("counter", 4, Class.CLIENT_DATA)
        out = a.alloc("out", n * 2, Class.CLIENT_DATA) if read else None
        self._freeze(a)
        a.scrub_client_data()
        self.gpu.launch("x0ne_probe_bf16_round", min((n + 255) // 256, 8192), 256,
                        [Arg.u32(base), Arg.u32(n), Arg.ptr(a.ptr(out) if read else 0), Arg.ptr(a.ptr(cnt))])
        self.gpu.sync()
        differ = int(np.frombuffer(a.read(cnt, 0, 4), np.uint32)[0])
        bits = np.frombuffer(a.read(out, 0, n * 2), np.uint16).copy() if read else None
        return differ, bits

    def _rope_table(self, inv_ptr: int, cs_ptr: int, positions: int, head_dim: int):
        self.gpu.launch("x0ne_rope_table_f64", (positions * (head_dim // 2) + 255) // 256, 256,
                        [Arg.ptr(inv_ptr), Arg.ptr(cs_ptr), Arg.u32(positions)])

    def rope_table(self, head_dim: int, theta: float, positions: int) -> np.ndarray:
        """The fused decode attention's RoPE table, [positions][head_dim / 2][cos, sin] in f64: the
        cosine and sine of (double)((float)p * inv_freq[i]) (the angle of rope.cu:7-47)."""
        if positions == 0:
            raise FormatError("rope_table: no positions")
        a = self._arena()
        inv = a.alloc("inv_freq", head_dim // 2 * 4, Class.WEIGHTS)
        cs = a.alloc("rope_cs", positions * (head_dim // 2) * 16, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(inv, 0, inv_freq(head_dim, theta))
        self._rope_table(a.ptr(inv), a.ptr(cs), positions, head_dim)
        self.gpu.sync()
        raw = a.read(cs, 0, positions * (head_dim // 2) * 16)
        return np.frombuffer(raw, np.float64).reshape(positions, head_dim // 2, 2).copy()

    def _kv_arena(self, q, k, v, ctx, h: Heads, page_of, pool, extra):
        pages = n_pages(ctx)
        page_of = list(range(pages)) if page_of is None else list(page_of)[:pages]
        pool = pool or (max(page_of) + 1)
        kp = to_pages(np.asarray(k, np.uint16)[:ctx * h.kv_dim].reshape(ctx, h.kv_dim), h.kv_heads, page_of, pool)
        vp = to_pages(np.asarray(v, np.uint16)[:ctx * h.kv_dim].reshape(ctx, h.kv_dim), h.kv_heads, page_of, pool,
                      dim_major=True)
        a = self._arena()
        sl = {
            "q": a.alloc("q", q.size * 2, Class.CLIENT_DATA),
            "k": a.alloc("k", kp.nbytes, Class.CLIENT_DATA),
            "v": a.alloc("v", vp.nbytes, Class.CLIENT_DATA),
            "pt": a.alloc("page_table", len(page_of) * 4, Class.WEIGHTS),
            "pos": a.alloc("pos", 4, Class.CLIENT_DATA),
        }
        for name, size in extra:
            sl[name] = a.alloc(name, size, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        a.write(sl["q"], 0, np.asarray(q, np.uint16))
        a.write(sl["k"], 0, kp)
        a.write(sl["v"], 0, vp)
        a.write(sl["pt"], 0, np.array(page_of, np.uint32))
        self._uploaded = (kp, vp)
        return a, sl

    def _check_attention(self, q, k, v, ctx, h: Heads, rows=1):
        h.check()
        if ctx == 0 or q.size != rows * h.q_dim or k.size < ctx * h.kv_dim or v.size < ctx * h.kv_dim:
            raise FormatError("attention: lengths")

    def attention_decode(self, q, k, v, ctx: int, h: Heads, page_of=None, pool=None) -> np.ndarray:
        """The per-head kernel (the reference's E2 witness)."""
        self._check_attention(q, k, v, ctx, h)
        a, s = self._kv_arena(q, k, v, ctx, h, page_of, pool, [("out", h.q_dim * 2)])
        a.write(s["pos"], 0, np.array([ctx - 1], np.uint32))
        self.gpu.launch("x0ne_attention_decode_bf16", h.q_heads, 256,
                        [Arg.ptr(a.ptr(s["q"])), Arg.ptr(a.ptr(s["k"])), Arg.ptr(a.ptr(s["v"])),
                         Arg.ptr(a.ptr(s["pt"])), Arg.ptr(a.ptr(s["out"])), Arg.ptr(a.ptr(s["pos"])),
                         Arg.u32(h.q_heads), Arg.u32(h.kv_heads), Arg.u32(ctx), Arg.f32(attn_scale(h.head_dim))])
        self.gpu.sync()
        return a.read_array(s["out"], 0, h.q_dim, np.uint16)

    def split_plan(self, h: Heads) -> SplitPlan:
        h.check()
        return self.gpu.split_plan(h.q_heads, h.kv_heads)

    def attention_decode_split(self, q, k, v, ctx: int, h: Heads, last_block=None, splits=None, page_of=None,
                               pool=None) -> np.ndarray:
        """Split-K (ops.rs:491-573): the plan's P unless `splits` is given; the merge kernel, or the
        grouped kernel's last block (last_block True; the default for a grouped plan)."""
        self._check_attention(q, k, v, ctx, h)
        plan = self.split_plan(h)
        if splits is not None:
            plan.splits = int(splits)
        if last_block is None:
            last_block = plan.grouped
        a, s = self._kv_arena(q, k, v, ctx, h, page_of, pool,
                              [("out", h.q_dim * 2), ("state", split_state_bytes(h.q_heads, plan.splits)),
                               ("counter", h.kv_heads * 4)])
        a.write(s["pos"], 0, np.array([ctx - 1], np.uint32))
        self.gpu.attention_split(plan, last_block, a.ptr(s["q"]), a.ptr(s["k"]), a.ptr(s["v"]), a.ptr(s["pt"]),
                                 a.ptr(s["state"]), a.ptr(s["counter"]), a.ptr(s["out"]), a.ptr(s["pos"]),
                                 h.q_heads, h.kv_heads, ctx, attn_scale(h.head_dim))
        self.gpu.sync()
        counts = a.read_array(s["counter"], 0, h.kv_heads, np.uint32)
        if counts.any():
            raise GpuError(f"split-K counters not reset: {counts.tolist()}")
        return a.read_array(s["out"], 0, h.q_dim, np.uint16)

    def attention_decode_split_scratch(self, q, k, v, ctx: int, h: Heads, last_block=None, splits=None,
                                       page_of=None, pool=None) -> np.ndarray:
        """attention_decode_split through x0ne_gpu_attention_split_scratch: the states and
        counters in the library's static scratch array, nothing allocated for them."""
        self._check_attention(q, k, v, ctx, h)
        plan = self.split_plan(h)
        if splits is not None:
            plan.splits = int(splits)
        if last_block is None:
            last_block = plan.grouped
        a, s = self._kv_arena(q, k, v, ctx, h, page_of, pool, [("out", h.q_dim * 2)])
        a.write(s["pos"], 0, np.array([ctx - 1], np.uint32))
        self.gpu.attention_split_scratch(plan, last_block, a.ptr(s["q"]), a.ptr(s["k"]), a.ptr(s["v"]),
                                         a.ptr(s["pt"]), a.ptr(s["out"]), a.ptr(s["pos"]), h.q_heads, h.kv_heads,
                                         ctx, attn_scale(h.head_dim))
        self.gpu.sync()
        return a.read_array(s["out"], 0, h.q_dim, np.uint16)

    def attention_rope_decode(self, qkv, q_norm, k_norm, eps: float, theta: float, k, v, ctx: int, h: Heads,
                              last_block=True, splits=None, page_of=None, pool=None, exact=False):
        """The engine's fused decode attention (one launch per layer): QK-norm + RoPE of the q
        heads of the packed qkv row at position ctx - 1, that position's K/V row written into its
        page, then split-K attention over keys 0..ctx-1 (k, v hold rows 0..ctx-2). last_block
        False runs the merge kernel after it. Returns (out, k_row, v_row) with the K/V row read
        back from the cache (the composition of ops.rs:138-208 and ops.rs:491-573). exact: the
        exact mode's kernel (f64 scores, softmax and sums, split-K with f64 states merged by the
        last block; it needs last_block)."""
        h.check()
        qd, kvd = h.q_dim, h.kv_dim
        if ctx == 0 or qkv.size != qd + 2 * kvd or k.size < (ctx - 1) * kvd or v.size < (ctx - 1) * kvd:
            raise FormatError("attention_rope_decode: lengths")
        # The exact kernel has no f64 merge kernel behind it: refused before any device work.
        if exact and not last_block:
            raise FormatError("attention_rope_decode: the exact kernel merges in its last block")
        plan = self.split_plan(h)
        if not plan.grouped:
            raise FormatError(f"attention_rope_decode: no grouped kernel for group {h.q_heads // h.kv_heads}")
        if splits is not None:
            plan.splits = int(splits)
        nan_row = np.full(kvd, NAN_BF16, np.uint16)
        kf = np.concatenate([np.asarray(k, np.uint16)[:(ctx - 1) * kvd], nan_row])
        vf = np.concatenate([np.asarray(v, np.uint16)[:(ctx - 1) * kvd], nan_row])
        hd = h.head_dim
        a, s = self._kv_arena(np.asarray(qkv, np.uint16), kf, vf, ctx, h, page_of, pool,
                              [("out", qd * 2), ("state", split_state_bytes(h.q_heads, plan.splits) * (2 if exact else 1)),
                               ("counter", h.kv_heads * 4), ("q_norm", hd * 2), ("k_norm", hd * 2),
                               ("inv_freq", hd // 2 * 4), ("rope_cs", ctx * (hd // 2) * 16)])
        a.write(s["pos"], 0, np.array([ctx - 1], np.uint32))
        a.write(s["q_norm"], 0, np.asarray(q_norm, np.uint16))
        a.write(s["k_norm"], 0, np.asarray(k_norm, np.uint16))
        a.write(s["inv_freq"], 0, inv_freq(hd, theta))
        self._rope_table(a.ptr(s["inv_freq"]), a.ptr(s["rope_cs"]), ctx, hd)
        counter = a.ptr(s["counter"]) if last_block else 0
        name = "exact" if exact else ""
        self.gpu.launch(f"x0ne_attention_rope_decode_{name + '_' if name else ''}g{plan.group}_bf16",
                        (h.kv_heads, plan.splits), 256,
                        [Arg.ptr(a.ptr(s["q"])), Arg.ptr(a.ptr(s["q_norm"])), Arg.ptr(a.ptr(s["k_norm"])),
                         Arg.ptr(a.ptr(s["inv_freq"])), Arg.ptr(a.ptr(s["rope_cs"])), Arg.ptr(a.ptr(s["k"])),
                         Arg.ptr(a.ptr(s["v"])),
                         Arg.ptr(a.ptr(s["pt"])), Arg.ptr(a.ptr(s["state"])), Arg.ptr(counter),
                         Arg.ptr(a.ptr(s["out"])), Arg.ptr(a.ptr(s["pos"])), Arg.u32(h.q_heads),
                         Arg.u32(h.kv_heads), Arg.u32(ctx), Arg.u32(plan.splits),
                         Arg.f32(attn_scale(hd)), Arg.f32(eps)])
        if not last_block:
            self.gpu.launch("x0ne_attention_merge_bf16", h.q_heads, 64,
                            [Arg.ptr(a.ptr(s["state"])), Arg.ptr(a.ptr(s["out"])), Arg.ptr(a.ptr(s["pos"])),
                             Arg.u32(ctx), Arg.u32(plan.splits)])
        self.gpu.sync()
        counts = a.read_array(s["counter"], 0, h.kv_heads, np.uint32)
        if counts.any():
            raise GpuError(f"split-K counters not reset: {counts.tolist()}")
        pages = n_pages(ctx)
        page_of = list(range(pages)) if page_of is None else list(page_of)
        pg, slot = page_of[(ctx - 1) // PAGE], (ctx - 1) % PAGE
        # The planes as the kernel left them: the K row and V column of position ctx - 1 in page
        # pg, and every other element as uploaded (ops.rs:322-373, the sentinel check).
        k_all = a.read_array(s["k"], 0, s["k"].len // 2, np.uint16)
        v_all = a.read_array(s["v"], 0, s["v"].len // 2, np.uint16)
        k_up, v_up = self._uploaded
        pool = k_all.size // (h.kv_heads * PAGE * HEAD_DIM)
        k4 = k_all.reshape(pool, h.kv_heads, PAGE, HEAD_DIM)
        v4 = v_all.reshape(pool, h.kv_heads, HEAD_DIM, PAGE)
        k_rows = [k4[pg, kh, slot, :].copy() for kh in range(h.kv_heads)]
        v_rows = [v4[pg, kh, :, slot].copy() for kh in range(h.kv_heads)]
        k_rest, v_rest = k4.copy(), v4.copy()
        k_rest[pg, :, slot, :] = k_up.reshape(k4.shape)[pg, :, slot, :]
        v_rest[pg, :, :, slot] = v_up.reshape(v4.shape)[pg, :, :, slot]
        self.kv_rest_untouched = bool((k_rest.ravel() == k_up.ravel()).all() and (v_rest.ravel() == v_up.ravel()).all())
        return a.read_array(s["out"], 0, qd, np.uint16), np.concatenate(k_rows), np.concatenate(v_rows)

    def attention_rope_decode_batch(self, qkv, q_norm, k_norm, eps: float, theta: float, ks, vs, ctxs, h: Heads,
                                    splits: int, max_ctx: int, page_seed: int = 0):
        """The batched step's fused decode attention for B independent sequences in one launch
        (grid (kv_heads, P, B)): sequence b's packed qkv row qkv[b] at position ctxs[b] - 1 over
        its keys 0..ctxs[b]-1 (ks[b], vs[b] hold its rows 0..ctxs[b]-2), each sequence in its
        own run of ceil(max_ctx / 16) entries of one shuffled page table over shared K/V planes.
        Returns out [B][q_dim] (the kernel writes it in panels) and the K/V rows written at each
        sequence's position."""
        h.check()
        qd, kvd, hd = h.q_dim, h.kv_dim, h.head_dim
        B = len(ctxs)
        qkv = np.asarray(qkv, np.uint16).reshape(B, qd + 2 * kvd)
        if B == 0 or len(ks) != B or len(vs) != B or any(c == 0 or c > max_ctx for c in ctxs):
            raise FormatError("attention_rope_decode_batch: lengths")
        plan = self.split_plan(h)
        if not plan.grouped:
            raise FormatError(f"attention_rope_decode_batch: no grouped kernel for group {h.q_heads // h.kv_heads}")
        plan.splits = int(splits)
        sp = n_pages(max_ctx)
        pool = B * sp
        order = np.arange(pool, dtype=np.uint32)
        if page_seed:
            np.random.default_rng(page_seed).shuffle(order)
        kp = np.full((pool, h.kv_heads, PAGE, HEAD_DIM), NAN_BF16, np.uint16)
        vp = np.full((pool, h.kv_heads, PAGE, HEAD_DIM), NAN_BF16, np.uint16)
        for b, c in enumerate(ctxs):
            rk = np.asarray(ks[b], np.uint16)[:(c - 1) * kvd].reshape(c - 1, h.kv_heads, HEAD_DIM)
            rv = np.asarray(vs[b], np.uint16)[:(c - 1) * kvd].reshape(c - 1, h.kv_heads, HEAD_DIM)
            for p in range(c - 1):
                kp[order[b * sp + p // PAGE], :, p % PAGE, :] = rk[p]
                vp[order[b * sp + p // PAGE], :, p % PAGE, :] = rv[p]
        vp = np.ascontiguousarray(vp.transpose(0, 1, 3, 2))
        a = self._arena()
        sl = {name: a.alloc(name, size, cls) for name, size, cls in [
            ("qkv", qkv.nbytes, Class.CLIENT_DATA), ("k", kp.nbytes, Class.CLIENT_DATA),
            ("v", vp.nbytes, Class.CLIENT_DATA), ("pt", pool * 4, Class.WEIGHTS), ("pos", B * 4, Class.CLIENT_DATA),
            ("out", -(-B // 16) * 16 * qd * 2, Class.CLIENT_DATA),
            ("state", B * split_state_bytes(h.q_heads, plan.splits), Class.CLIENT_DATA),
            ("counter", B * h.kv_heads * 4, Class.CLIENT_DATA), ("q_norm", hd * 2, Class.WEIGHTS),
            ("k_norm", hd * 2, Class.WEIGHTS), ("inv_freq", hd // 2 * 4, Class.WEIGHTS),
            ("rope_cs", max_ctx * (hd // 2) * 16, Class.WEIGHTS)]}
        self._freeze(a)
        a.scrub_client_data()
        a.write(sl["qkv"], 0, qkv)
        a.write(sl["k"], 0, kp)
        a.write(sl["v"], 0, vp)
        a.write(sl["pt"], 0, order)
        a.write(sl["pos"], 0, np.array([c - 1 for c in ctxs], np.uint32))
        a.write(sl["q_norm"], 0, np.asarray(q_norm, np.uint16))
        a.write(sl["k_norm"], 0, np.asarray(k_norm, np.uint16))
        a.write(sl["inv_freq"], 0, inv_freq(hd, theta))
        self._rope_table(a.ptr(sl["inv_freq"]), a.ptr(sl["rope_cs"]), max_ctx, hd)
        self.gpu.launch(f"x0ne_attention_rope_decode_batch_g{plan.group}_bf16", (h.kv_heads, plan.splits, B), 256,
                        [Arg.ptr(a.ptr(sl["qkv"])), Arg.ptr(a.ptr(sl["q_norm"])), Arg.ptr(a.ptr(sl["k_norm"])),
                         Arg.ptr(a.ptr(sl["inv_freq"])), Arg.ptr(a.ptr(sl["rope_cs"])), Arg.ptr(a.ptr(sl["k"])),
                         Arg.ptr(a.ptr(sl["v"])), Arg.ptr(a.ptr(sl["pt"])), Arg.ptr(a.ptr(sl["state"])),
                         Arg.ptr(a.ptr(sl["counter"])), Arg.ptr(a.ptr(sl["out"])), Arg.ptr(a.ptr(sl["pos"])),
                         Arg.u32(h.q_heads), Arg.u32(h.kv_heads), Arg.u32(max_ctx), Arg.u32(plan.splits),
                         Arg.f32(attn_scale(hd)), Arg.f32(eps), Arg.u32(sp)])
        self.gpu.sync()
        counts = a.read_array(sl["counter"], 0, B * h.kv_heads, np.uint32)
        if counts.any():
            raise GpuError(f"split-K counters not reset: {counts.tolist()}")
        out = from_panels(a.read_array(sl["out"], 0, sl["out"].len // 2, np.uint16), B, qd)
        k_all = a.read_array(sl["k"], 0, kp.size, np.uint16).reshape(kp.shape)
        v_all = a.read_array(sl["v"], 0, vp.size, np.uint16).reshape(vp.shape)
        k_rows, v_rows = [], []
        k_rest, v_rest = k_all.copy(), v_all.copy()
        for b, c in enumerate(ctxs):
            pg, slot = order[b * sp + (c - 1) // PAGE], (c - 1) % PAGE
            k_rows.append(k_all[pg, :, slot, :].reshape(-1).copy())
            v_rows.append(v_all[pg, :, :, slot].reshape(-1).copy())
            k_rest[pg, :, slot, :] = kp[pg, :, slot, :]
            v_rest[pg, :, :, slot] = vp[pg, :, :, slot]
        # Every sequence's K row and V column at its own position, nothing else (ops.rs:322-373).
        self.kv_rest_untouched = bool((k_rest == kp).all() and (v_rest == vp).all())
        return out, k_rows, v_rows

    FEW_KERNELS = {(1, 1): 8, (1, 2): 8, (1, 4): 8, (1, 8): 8, (2, 1): 8, (2, 2): 8, (4, 1): 8}
    FEW_SWIGLU = {(1, 1), (1, 2), (2, 1), (4, 1)}

    def gemm_few(self, w, rows, cols, x, n, mode: int, block: int = 256, rg: int = 1, x_panel: bool = False,
                 y_panel: bool = False, w_panel: bool = False) -> np.ndarray:
        """One few-row GEMM kernel itself (x0ne_gemm_few_t{TT}_r{RG}[_swiglu]_bf16, TT = 1, 2
        or 4 tiles of 16 rows of X by n): mode 0 bf16 Y, 1 f32 Y, 2 SwiGLU over the packed
        [gate; up] W of 2 rows rows (act [n][rows] bf16); `rg` row groups of 16 per block;
        x_panel / y_panel / w_panel: X and W handed over, Y read back, in the panel layout
        (returned row-major either way; a W panel needs rows a multiple of 16)."""
        wrows = 2 * rows if mode == 2 else rows
        tt = 1 if n <= 16 else 2 if n <= 32 else 4
        if w.size != wrows * cols or x.size != n * cols or not 1 <= n <= 64 or cols % 8 or \
                (tt, rg) not in self.FEW_KERNELS or (mode == 2 and (tt, rg) not in self.FEW_SWIGLU) or \
                block // 64 > self.FEW_KERNELS[(tt, rg)]:
            raise FormatError("gemm_few: lengths or variant")
        if y_panel and (mode == 1 or rows % 8):
            raise FormatError("gemm_few: a Y panel is bf16 with rows a multiple of 8")
        if w_panel and rows % 16:
            raise FormatError("gemm_few: a W panel needs rows a multiple of 16")
        name = f"x0ne_gemm_few_t{tt}_r{rg}{'_swiglu' if mode == 2 else ''}_bf16"
        ob = 4 if mode == 1 else 2
        xin = to_panels(np.asarray(x, np.uint16).reshape(n, cols)) if x_panel else np.asarray(x, np.uint16)
        yrows = -(-n // 16) * 16 if y_panel else n
        a = self._arena()
        ws = a.alloc("w", w.size * 2, Class.WEIGHTS)
        xs = a.alloc("x", xin.size * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", yrows * rows * ob, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        win = np.asarray(w, np.uint16)
        a.write(ws, 0, to_panels(win.reshape(wrows, cols)) if w_panel else win)
        a.write(xs, 0, xin)
        flags = (1 if mode == 1 else 0) | (2 if x_panel else 0) | (4 if y_panel else 0) | (8 if w_panel else 0)
        self.gpu.launch(name, (rows + 16 * rg - 1) // (16 * rg), block,
                        [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ys)), Arg.u32(rows), Arg.u32(cols),
                         Arg.u32(n), Arg.u32(flags)])
        self.gpu.sync()
        y = a.read_array(ys, 0, yrows * rows, np.float32 if mode == 1 else np.uint16)
        return from_panels(y, n, rows) if y_panel else y.reshape(n, rows)

    def gemm_few_bal(self, w, rows: int, cols: int, x, n: int, mode: int, block: int = 256, T: int = 0,
                     calls: int = 1):
        """x0ne_gemm_few_bal_bf16, the balanced few-row kernel (one block per run of T of the
        groups' steps, X and W handed over in panels): mode 0 bf16 Y, 1 f32 Y. T 0 takes the
        runs the runtime takes (ceil(groups steps / CUs)). `calls` launches in a row (the last
        one's Y). Returns (Y [n][rows], every count left zero)."""
        groups, steps = rows // 16, -(-cols // 32)
        if T == 0:
            T = -(-groups * steps // self.gpu.compute_units())
        if w.size != rows * cols or x.size != n * cols or not 1 <= n <= 16 or cols % 8 or rows % 16 or mode not in (0, 1) \
                or not block // 64 <= T <= 4 * steps + 1 or block // 64 > 8:
            raise FormatError("gemm_few_bal: lengths or run")
        cmax = -(-steps // T) + 1
        ob = 4 if mode == 1 else 2
        a = self._arena()
        ws = a.alloc("w", w.size * 2, Class.WEIGHTS)
        xin = to_panels(np.asarray(x, np.uint16).reshape(n, cols))
        xs = a.alloc("x", xin.size * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", n * rows * ob, Class.CLIENT_DATA)
        parts = a.alloc("parts", groups * cmax * 256 * 4, Class.CLIENT_DATA)
        counts = a.alloc("counts", groups * 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        a.write(ws, 0, to_panels(np.asarray(w, np.uint16).reshape(rows, cols)))
        a.write(xs, 0, xin)
        for _ in range(calls):
            self.gpu.launch("x0ne_gemm_few_bal_bf16", -(-groups * steps // T), block,
                            [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ys)), Arg.u32(rows), Arg.u32(cols),
                             Arg.u32(n), Arg.u32((1 if mode == 1 else 0) | 2 | 8), Arg.u32(T), Arg.ptr(a.ptr(parts)),
                             Arg.ptr(a.ptr(counts))])
        self.gpu.sync()
        y = a.read_array(ys, 0, n * rows, np.float32 if mode == 1 else np.uint16).reshape(n, rows)
        return y, bool((a.read_array(counts, 0, groups, np.uint32) == 0).all())

    def gemm_f64(self, w, rows: int, cols: int, x, n: int, out_f32: bool, tt: int = 0, ks: int = 1,
                 tq: int = 0) -> np.ndarray:
        """x0ne_gemm_f64_t{TT}_bf16, the exact mode's projection: Y [n][rows] = X [n][cols] W^T,
        every bf16 product summed in f64 on the matrix cores, Y f32 or bf16 (bits) of the f32
        of the sum. tt 1, 2 or 4: tiles of 16 tokens per wavefront; tq 1..8: the 4-token-quad
        kernel x0ne_gemm_f64_q{TQ}_bf16 (n <= 4 tq); both 0: the kernel the engine takes for n
        (quads up to 32 rows). ks > 1 cuts K into ks slices whose f64 partial sums
        x0ne_gemm_f64_reduce adds."""
        if tt == 0 and tq == 0:
            if n <= 32:
                tq = -(-n // 4)
            else:
                tt = 4
        if w.size != rows * cols or x.size != n * cols or cols % 8 or n == 0 or rows == 0 or ks < 1 or \
                (tq == 0 and tt not in (1, 2, 4)) or (tq and (tt or not 1 <= tq <= 8 or n > 4 * tq)):
            raise FormatError("gemm_f64: lengths")
        ob = 4 if out_f32 else 2
        a = self._arena()
        ws = a.alloc("w", w.size * 2, Class.WEIGHTS)
        xs = a.alloc("x", x.size * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", n * rows * ob, Class.CLIENT_DATA)
        parts = a.alloc("parts", max(ks, 2) * n * rows * 8, Class.CLIENT_DATA)
        self._freeze(a)
        a.scrub_client_data()
        a.write(ws, 0, np.asarray(w, np.uint16))
        a.write(xs, 0, np.asarray(x, np.uint16))
        tiles = -(-rows // 64) * (1 if tq else -(-n // (16 * tt)))
        self.gpu.launch(f"x0ne_gemm_f64_q{tq}_bf16" if tq else f"x0ne_gemm_f64_t{tt}_bf16", -(-tiles * ks // 4), 256,
                        [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ys)), Arg.u32(rows), Arg.u32(cols),
                         Arg.u32(n), Arg.u32(1 if out_f32 else 0), Arg.u32(ks), Arg.ptr(a.ptr(parts))])
        if ks > 1:
            self.gpu.launch("x0ne_gemm_f64_reduce", -(-n * rows // 256), 256,
                            [Arg.ptr(a.ptr(parts)), Arg.ptr(a.ptr(ys)), Arg.u32(rows), Arg.u32(n), Arg.u32(ks),
                             Arg.u32(1 if out_f32 else 0)])
        self.gpu.sync()
        return a.read_array(ys, 0, n * rows, np.float32 if out_f32 else np.uint16).reshape(n, rows)

    def panel(self, m, rows: int, cols: int) -> np.ndarray:
        """x0ne_panel_bf16: the [rows][cols] bf16 matrix m copied into 16-row panels on the device
        (flat, rows x cols values; left as the destination held it, 0xFFFF here, when rows is not a
        multiple of 16 or cols of 8)."""
        m = np.asarray(m, np.uint16).reshape(-1)
        if m.size != rows * cols or rows == 0 or cols == 0:
            raise FormatError("panel: lengths")
        a = self._arena()
        src = a.alloc("src", m.size * 2, Class.WEIGHTS)
        dst = a.alloc("dst", m.size * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(src, 0, m)
        a.write(dst, 0, np.full(m.size, 0xFFFF, np.uint16))
        self.gpu.launch("x0ne_panel_bf16", (rows * cols // 8 + 255) // 256 or 1, 256,
                        [Arg.ptr(a.ptr(src)), Arg.ptr(a.ptr(dst)), Arg.u32(rows), Arg.u32(cols)])
        self.gpu.sync()
        return a.read_array(dst, 0, m.size, np.uint16)

    def attention_prefill_at(self, q, k, v, t: int, pos0: int, h: Heads, rows, page_of=None, pool=None,
                             grouped=False, panel=False, exact=False):
        """Causal attention for positions pos0..t of a t-position cache in one launch at pos0
        (ops.rs:724-775); q holds those t - pos0 rows; returns the rows asked for. grouped: the
        matrix-core kernel for the geometry's group size (x0ne_attention_prefill_g*_bf16);
        panel: its variant writing out in 16-row panels (x0ne_attention_prefill_panel_g*_bf16),
        read back row-major; exact: the exact mode's f64 kernel (x0ne_attention_prefill_exact_g*_bf16)."""
        h.check()
        m = t - pos0
        if m <= 0 or q.size != m * h.q_dim or k.size != t * h.kv_dim or v.size != t * h.kv_dim or \
                any(r >= m for r in rows):
            raise FormatError("attention_prefill_at: lengths")
        g = h.q_heads // h.kv_heads
        if (grouped or panel or exact) and g not in (1, 2, 4, 8):
            raise FormatError(f"attention_prefill_at: no grouped kernel for group {g}")
        mp = -(-m // 16) * 16 if panel else m
        a, s = self._kv_arena(q, k, v, t, h, page_of, pool, [("out", mp * h.q_dim * 2)])
        a.write(s["pos"], 0, np.array([pos0], np.uint32))
        kind = "prefill_panel" if panel else "prefill"
        if exact:
            name, grid, block = (f"x0ne_attention_prefill_exact_g{g}_bf16",
                                 (h.kv_heads, (m + PREFILL_EXACT_COLS // g - 1) // (PREFILL_EXACT_COLS // g)),
                                 PREFILL_EXACT_THREADS)
        elif grouped or panel:
            name, grid, block = (f"x0ne_attention_{kind}_g{g}_bf16",
                                 (h.kv_heads, (m + PREFILL_COLS // g - 1) // (PREFILL_COLS // g)), PREFILL_THREADS)
        else:
            name, grid, block = "x0ne_attention_prefill_bf16", (h.q_heads, m), 256
        self.gpu.launch(name, grid, block,
                        [Arg.ptr(a.ptr(s["q"])), Arg.ptr(a.ptr(s["k"])), Arg.ptr(a.ptr(s["v"])),
                         Arg.ptr(a.ptr(s["pt"])), Arg.ptr(a.ptr(s["out"])), Arg.ptr(a.ptr(s["pos"])), Arg.u32(m),
                         Arg.u32(h.q_heads), Arg.u32(h.kv_heads), Arg.u32(t), Arg.f32(attn_scale(h.head_dim))])
        self.gpu.sync()
        out = a.read_array(s["out"], 0, mp * h.q_dim, np.uint16)
        out = from_panels(out, m, h.q_dim) if panel else out.reshape(m, h.q_dim)
        return [out[r].copy() for r in rows]

    def attention_prefill_rows(self, q, k, v, t: int, h: Heads, rows, page_of=None, pool=None, grouped=False,
                               panel=False, exact=False):
        """ops.rs:683-722: causal attention over t positions, the rows asked for."""
        if t == 0:
            raise FormatError("attention_prefill_rows: lengths")
        return self.attention_prefill_at(q, k, v, t, 0, h, rows, page_of, pool, grouped, panel, exact)

    # -- swiglu (ops.rs:777-795, :978-1001) --
    def swiglu_rows(self, gate_up, rows: int, panel: bool = False) -> np.ndarray:
        """x0ne_swiglu_bf16 over rows of [gate; up]; panel: x0ne_swiglu_panel_bf16 (out in
        16-row panels, read back row-major). Returns [rows][inter] flattened."""
        if rows == 0 or gate_up.size == 0 or gate_up.size % (2 * rows):
            raise FormatError("swiglu_rows: length is not rows x 2 x inter")
        inter = gate_up.size // rows // 2
        if panel and inter % 8:
            raise FormatError("swiglu_rows: panels need inter a multiple of 8")
        rp = -(-rows // 16) * 16 if panel else rows
        a = self._arena()
        gu = a.alloc("gate_up", gate_up.size * 2, Class.CLIENT_DATA)
        out = a.alloc("out", rp * inter * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(gu, 0, gate_up.astype(np.uint16))
        self.gpu.launch("x0ne_swiglu_panel_bf16" if panel else "x0ne_swiglu_bf16", ((inter + 2047) // 2048, rows), 256,
                        [Arg.ptr(a.ptr(gu)), Arg.ptr(a.ptr(out)), Arg.u32(inter)])
        self.gpu.sync()
        got = a.read_array(out, 0, rp * inter, np.uint16)
        return from_panels(got, rows, inter).reshape(-1) if panel else got

    def swiglu(self, gate_up) -> np.ndarray:
        if gate_up.size == 0 or gate_up.size % 2:
            raise FormatError("swiglu: odd length")
        return self.swiglu_rows(gate_up, 1)

    # -- the MoE block (ops.rs:796-920) --
    MOE_MAX_EXPERTS = 1024
    MOE_NO_EXPERT = 0xFFFFFFFF

    def moe_route(self, logits, experts: int, top_k: int):
        """x0ne_moe_route_f32 over rows of `experts` f32 router logits: (ids, weights), each
        [rows][top_k] flattened (ops.rs:796-842, the same refusals)."""
        lg = np.ascontiguousarray(logits, np.float32).ravel()
        if experts == 0 or experts > self.MOE_MAX_EXPERTS or top_k == 0 or top_k > 32 or top_k > experts or \
                lg.size == 0 or lg.size % experts:
            raise FormatError(f"moe_route: {lg.size} logits, {experts} experts, top {top_k}")
        rows = lg.size // experts
        a = self._arena()
        ls = a.alloc("logits", lg.size * 4, Class.CLIENT_DATA)
        ids = a.alloc("ids", rows * top_k * 4, Class.CLIENT_DATA)
        ws = a.alloc("weights", rows * top_k * 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ls, 0, lg)
        self.gpu.launch("x0ne_moe_route_f32", rows, 64,
                        [Arg.ptr(a.ptr(ls)), Arg.u32(experts), Arg.u32(top_k), Arg.ptr(a.ptr(ids)),
                         Arg.ptr(a.ptr(ws))])
        self.gpu.sync()
        return a.read_array(ids, 0, rows * top_k, np.uint32), a.read_array(ws, 0, rows * top_k, np.float32)

    def moe_gemv(self, w, experts: int, rows: int, cols: int, ids, x, x_group: int, f32_out: bool) -> np.ndarray:
        """x0ne_moe_gemv_{bf16,f32}: y[s] = W[ids[s]] x[s / x_group] for bf16 bits W
        [experts][rows][cols] and x [slots / x_group][cols]; [slots][rows] as f32 values
        (ops.rs:844-907, the same refusals)."""
        w = np.ascontiguousarray(w, np.uint16).ravel()
        x = np.ascontiguousarray(x, np.uint16).ravel()
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        slots = ids.size
        if experts == 0 or rows == 0 or cols == 0 or cols % 8 or w.size != experts * rows * cols or slots == 0 or \
                x_group == 0 or slots % x_group or x.size != slots // x_group * cols:
            raise FormatError(f"moe_gemv: W {w.size} for {experts}x{rows}x{cols}, {slots} slots, x {x.size}")
        ob = 4 if f32_out else 2
        a = self._arena()
        ws = a.alloc("w", w.size * 2, Class.WEIGHTS)
        is_ = a.alloc("ids", slots * 4, Class.CLIENT_DATA)
        xs = a.alloc("x", x.size * 2, Class.CLIENT_DATA)
        ys = a.alloc("y", slots * rows * ob, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ws, 0, w)
        a.write(is_, 0, ids)
        a.write(xs, 0, x)
        self.gpu.launch("x0ne_moe_gemv_f32" if f32_out else "x0ne_moe_gemv_bf16", ((rows + 7) // 8, slots), 256,
                        [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(is_)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(ys)),
                         Arg.u32(rows), Arg.u32(cols), Arg.u32(experts), Arg.u32(x_group), Arg.u32(cols)])
        self.gpu.sync()
        if f32_out:
            return a.read_array(ys, 0, slots * rows, np.float32)
        y = a.read_array(ys, 0, slots * rows, np.uint16)
        return (y.astype(np.uint32) << 16).view(np.float32)

    def moe_combine(self, y, weights, hidden: int, top_k: int) -> np.ndarray:
        """x0ne_moe_combine_bf16: out[r] = bf16(sum_s weights[r][s] y[r][s]) for y
        [rows][top_k][hidden] f32; bf16 bits [rows][hidden] (ops.rs:909-920)."""
        y = np.ascontiguousarray(y, np.float32).ravel()
        wt = np.ascontiguousarray(weights, np.float32).ravel()
        if hidden == 0 or top_k == 0 or wt.size == 0 or wt.size % top_k or y.size != wt.size * hidden:
            raise FormatError(f"moe_combine: y {y.size}, weights {wt.size}, hidden {hidden}, top {top_k}")
        rows = wt.size // top_k
        a = self._arena()
        ys = a.alloc("y", y.size * 4, Class.CLIENT_DATA)
        ws = a.alloc("weights", wt.size * 4, Class.CLIENT_DATA)
        out = a.alloc("out", rows * hidden * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ys, 0, y)
        a.write(ws, 0, wt)
        self.gpu.launch("x0ne_moe_combine_bf16", ((hidden + 255) // 256, rows), 256,
                        [Arg.ptr(a.ptr(ys)), Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(out)), Arg.u32(hidden), Arg.u32(top_k)])
        self.gpu.sync()
        return a.read_array(out, 0, rows * hidden, np.uint16)

    def moe_gate_up_swiglu(self, w, experts: int, inter: int, cols: int, ids, x, exact: bool = False) -> np.ndarray:
        """x0ne_moe_gate_up_swiglu_bf16 (exact: _exact_bf16, the sums in f64): act[s] =
        bf16(silu(bf16 g) bf16 u) for the gate and up rows of expert ids[s] (W [experts][2
        inter][cols] bf16 bits) against x; [slots][inter] bf16 bits."""
        w = np.ascontiguousarray(w, np.uint16).ravel()
        x = np.ascontiguousarray(x, np.uint16).ravel()
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        if experts == 0 or inter == 0 or cols % 8 or w.size != experts * 2 * inter * cols or x.size != cols or \
                ids.size == 0 or ids.size > 32:
            raise FormatError("moe_gate_up_swiglu: shapes")
        a = self._arena()
        ws, is_ = a.alloc("w", w.size * 2, Class.WEIGHTS), a.alloc("ids", ids.size * 4, Class.CLIENT_DATA)
        xs, act = a.alloc("x", x.size * 2, Class.CLIENT_DATA), a.alloc("act", ids.size * inter * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ws, 0, w)
        a.write(is_, 0, ids)
        a.write(xs, 0, x)
        self.gpu.launch("x0ne_moe_gate_up_swiglu_exact_bf16" if exact else "x0ne_moe_gate_up_swiglu_bf16",
                        ((inter + 7) // 8, ids.size), 256,
                        [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(is_)), Arg.ptr(a.ptr(xs)), Arg.ptr(a.ptr(act)),
                         Arg.u32(inter), Arg.u32(cols), Arg.u32(experts)])
        self.gpu.sync()
        return a.read_array(act, 0, ids.size * inter, np.uint16)

    def moe_down_combine(self, w, experts: int, hidden: int, inter: int, ids, weights, act,
                         exact: bool = False) -> np.ndarray:
        """x0ne_moe_down_combine_bf16 (exact: _exact_bf16, the sums and the combination in f64):
        out = bf16(sum_s weights[s] W[ids[s]] act[s]) (the down rows rounded to f32, the
        combination in slot order); W [experts][hidden][inter] bf16 bits, act [slots][inter] bf16
        bits; hidden bf16 bits."""
        w = np.ascontiguousarray(w, np.uint16).ravel()
        act = np.ascontiguousarray(act, np.uint16).ravel()
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        wt = np.ascontiguousarray(weights, np.float32).ravel()
        k = ids.size
        if experts == 0 or hidden == 0 or inter % 8 or w.size != experts * hidden * inter or act.size != k * inter or \
                wt.size != k or k == 0 or k > 32:
            raise FormatError("moe_down_combine: shapes")
        a = self._arena()
        ws, is_ = a.alloc("w", w.size * 2, Class.WEIGHTS), a.alloc("ids", k * 4, Class.CLIENT_DATA)
        wts, xs = a.alloc("weights", k * 4, Class.CLIENT_DATA), a.alloc("act", act.size * 2, Class.CLIENT_DATA)
        out = a.alloc("out", hidden * 2, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ws, 0, w)
        a.write(is_, 0, ids)
        a.write(wts, 0, wt)
        a.write(xs, 0, act)
        self.gpu.launch("x0ne_moe_down_combine_exact_bf16" if exact else "x0ne_moe_down_combine_bf16",
                        (hidden + 7) // 8, 256,
                        [Arg.ptr(a.ptr(ws)), Arg.ptr(a.ptr(is_)), Arg.ptr(a.ptr(wts)), Arg.ptr(a.ptr(xs)),
                         Arg.ptr(a.ptr(out)), Arg.u32(hidden), Arg.u32(inter), Arg.u32(experts), Arg.u32(k)])
        self.gpu.sync()
        return a.read_array(out, 0, hidden, np.uint16)

    # -- advance, argmax (ops.rs:925-976) --
    def advance(self, value: int) -> int:
        a = self._arena()
        pos = a.alloc("pos", 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(pos, 0, np.array([value & 0xFFFFFFFF], np.uint32))
        self.gpu.launch("x0ne_advance_u32", 1, 64, [Arg.ptr(a.ptr(pos))])
        self.gpu.sync()
        return int(a.read_array(pos, 0, 1, np.uint32)[0])

    def argmax_rows_sliced(self, logits, slices: int, pos):
        """The batched step's two-launch pick over rows of logits ([rows][n] f32): each row cut
        in `slices` blocks, then the pick and the advance; returns (tokens, positions after).
        A token 0xFFFFFFFF marks a row holding a NaN."""
        logits = np.ascontiguousarray(logits, np.float32)
        rows, n = logits.shape
        a = self._arena()
        ls = a.alloc("logits", logits.nbytes, Class.CLIENT_DATA)
        part = a.alloc("partial", rows * slices * 12, Class.CLIENT_DATA)
        toks = a.alloc("tokens", rows * 4, Class.CLIENT_DATA)
        ps = a.alloc("pos", rows * 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ls, 0, logits)
        a.write(ps, 0, np.asarray(pos, np.uint32))
        self.gpu.launch("x0ne_argmax_slices_f32", (rows, slices), 256,
                        [Arg.ptr(a.ptr(ls)), Arg.u32(n), Arg.u32(slices), Arg.ptr(a.ptr(part))])
        self.gpu.launch("x0ne_argmax_pick_advance", rows, 64,
                        [Arg.ptr(a.ptr(part)), Arg.u32(slices), Arg.ptr(a.ptr(toks)), Arg.ptr(a.ptr(ps))])
        self.gpu.sync()
        return a.read_array(toks, 0, rows, np.uint32), a.read_array(ps, 0, rows, np.uint32)

    def argmax(self, logits) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        if logits.size == 0:
            raise FormatError("argmax: empty")
        a = self._arena()
        ls = a.alloc("logits", logits.size * 4, Class.CLIENT_DATA)
        out = a.alloc("out", 4, Class.CLIENT_DATA)
        self._freeze(a)
        a.write(ls, 0, logits)
        self.gpu.launch("x0ne_argmax_f32", 1, 1024, [Arg.ptr(a.ptr(ls)), Arg.u32(logits.size), Arg.ptr(a.ptr(out))])
        self.gpu.sync()
        v = int(a.read_array(out, 0, 1, np.uint32)[0])
        if v >= logits.size:
            raise GpuError("argmax: no finite maximum (NaN row)")
        return v
